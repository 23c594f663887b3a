// LDS tile staging and MFMA operand fetch shared by the attention kernels.
//
// A tile holds ROWS token rows of D elements.  It is staged through registers
// (16-byte global loads, coalesced along D) and written to LDS either
// row-major [ROWS][D + RPAD] or transposed [D][ROWS + TPAD].
//
// Operand conventions for the 16x16 MFMA (see common.h): with rows of the
// output as "keys" and columns as "queries", lane l = 16*g + c works on
// column c and on rows 4g..4g+3.
//  * row_op16(): 8 consecutive D elements of one row (A or B operand over D),
//    D-chunk dc covers elements 32*dc + 8g .. +7.
//  * col_op16(): elements of one D index at token offsets kb + 4g + 0..3 and
//    kb + 16 + 4g + 0..3 of a transposed tile -- the permuted K order that
//    matches two stacked 16x16 accumulator tiles used as the other operand.
//  * fp32: K = 4 per instruction; row_op32 gives D/4 consecutive elements
//    (lane g covers D indices g*D/4 .. +D/4-1, one per instruction) and
//    col_op32 the 4 token offsets kb + 4g + 0..3 of one D index.
#pragma once

#include "common.h"

namespace dsalt {

template <typename T> struct Pad;
template <> struct Pad<bf16> { static constexpr int R = 8, C = 4; };
template <> struct Pad<f16> { static constexpr int R = 8, C = 4; };
template <> struct Pad<float> { static constexpr int R = 4, C = 4; };

template <typename T, int D, int ROWS>
struct Tile {
    static constexpr int VW = 16 / (int)sizeof(T);  // elements per 16-byte vector
    static constexpr int CPR = D / VW;               // vectors per row
    static constexpr int NV = ROWS * CPR / 256;      // vectors per thread (256 threads)
    static_assert(ROWS * CPR % 256 == 0, "tile must split evenly over 256 threads");
    static constexpr int RS = D + Pad<T>::R;         // row-major row stride (elements)
    static constexpr int TS = ROWS + Pad<T>::C;      // transposed row stride (elements)
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    u4 r[NV];

    // row(rr) returns the global pointer of tile row rr or nullptr (zero row)
    template <typename RowFn>
    __device__ __forceinline__ void load(int tid, RowFn row) {
#pragma unroll
        for (int n = 0; n < NV; ++n) {
            int vi = tid + 256 * n, rr = vi / CPR, c = vi % CPR;
            const T* src = row(rr);
            r[n] = src ? *(const u4*)(src + c * VW) : u4{0u, 0u, 0u, 0u};
        }
    }
    __device__ __forceinline__ void store_rows(T* lds, int tid) const {
#pragma unroll
        for (int n = 0; n < NV; ++n) {
            int vi = tid + 256 * n, rr = vi / CPR, c = vi % CPR;
            *(u4*)(lds + rr * RS + c * VW) = r[n];
        }
    }
    __device__ __forceinline__ void store_cols(T* lds, int tid) const {
#pragma unroll
        for (int n = 0; n < NV; ++n) {
            int vi = tid + 256 * n, rr = vi / CPR, c = vi % CPR;
            const T* e = (const T*)&r[n];
#pragma unroll
            for (int i = 0; i < VW; ++i) lds[(c * VW + i) * TS + rr] = e[i];
        }
    }
};

template <typename T>
__device__ __forceinline__ typename Vec8<T>::type row_op16(const T* lds, int rs, int row, int dc, int g) {
    return *(const typename Vec8<T>::type*)(lds + row * rs + dc * 32 + 8 * g);
}

template <typename T>
__device__ __forceinline__ typename Vec8<T>::type col_op16(const T* lds, int ts, int drow, int kb, int g) {
    typedef typename Vec8<T>::half H4;
    H4 lo = *(const H4*)(lds + drow * ts + kb + 4 * g);
    H4 hi = *(const H4*)(lds + drow * ts + kb + 16 + 4 * g);
    typename Vec8<T>::type v;
    v[0] = lo[0]; v[1] = lo[1]; v[2] = lo[2]; v[3] = lo[3];
    v[4] = hi[0]; v[5] = hi[1]; v[6] = hi[2]; v[7] = hi[3];
    return v;
}

__device__ __forceinline__ floatx4 col_op32(const float* lds, int ts, int drow, int kb, int g) {
    return *(const floatx4*)(lds + drow * ts + kb + 4 * g);
}

// D/4 consecutive fp32 of a row starting at g*D/4
template <int D>
__device__ __forceinline__ void row_op32(const float* lds, int rs, int row, int g, float (&out)[D / 4]) {
#pragma unroll
    for (int m = 0; m < D / 16; ++m) {
        floatx4 v = *(const floatx4*)(lds + row * rs + g * (D / 4) + 4 * m);
        out[4 * m] = v[0]; out[4 * m + 1] = v[1]; out[4 * m + 2] = v[2]; out[4 * m + 3] = v[3];
    }
}

// Register copy of one token row in operand layout (queries in the forward
// and dq kernels, keys/values in the dk/dv kernels).
template <typename T, int D>
struct RowReg {
    typename Vec8<T>::type x[D / 32];
    __device__ __forceinline__ void load(const T* src, int g) {
#pragma unroll
        for (int dc = 0; dc < D / 32; ++dc) {
            if (src) x[dc] = *(const typename Vec8<T>::type*)(src + dc * 32 + 8 * g);
            else for (int e = 0; e < 8; ++e) x[dc][e] = from_float<T>(0.f);
        }
    }
};
template <int D>
struct RowReg<float, D> {
    float x[D / 4];
    __device__ __forceinline__ void load(const float* src, int g) {
#pragma unroll
        for (int m = 0; m < D / 16; ++m) {
            floatx4 v = src ? *(const floatx4*)(src + g * (D / 4) + 4 * m) : floatx4{0.f, 0.f, 0.f, 0.f};
            x[4 * m] = v[0]; x[4 * m + 1] = v[1]; x[4 * m + 2] = v[2]; x[4 * m + 3] = v[3];
        }
    }
};

// acc = sum over D of A-rows (from LDS, row-major) times the register row:
// output tile (16 LDS rows) x (16 register rows).
template <typename T, int D>
__device__ __forceinline__ floatx4 dot_rows(const T* lds, int rs, int row0, int lane, const RowReg<T, D>& reg,
                                            floatx4 acc) {
    const int g = lane >> 4, rr = row0 + (lane & 15);
#pragma unroll
    for (int dc = 0; dc < D / 32; ++dc) acc = mma(row_op16<T>(lds, rs, rr, dc, g), reg.x[dc], acc);
    return acc;
}
template <>
__device__ __forceinline__ floatx4 dot_rows<float, 64>(const float* lds, int rs, int row0, int lane,
                                                       const RowReg<float, 64>& reg, floatx4 acc) {
    float a[16];
    row_op32<64>(lds, rs, row0 + (lane & 15), lane >> 4, a);
#pragma unroll
    for (int m = 0; m < 16; ++m) acc = mma(a[m], reg.x[m], acc);
    return acc;
}
template <>
__device__ __forceinline__ floatx4 dot_rows<float, 128>(const float* lds, int rs, int row0, int lane,
                                                        const RowReg<float, 128>& reg, floatx4 acc) {
    float a[32];
    row_op32<128>(lds, rs, row0 + (lane & 15), lane >> 4, a);
#pragma unroll
    for (int m = 0; m < 32; ++m) acc = mma(a[m], reg.x[m], acc);
    return acc;
}

// Same product with the operands swapped: the register row is the A operand
// (output rows = 16 register rows), LDS rows are B (output cols = LDS rows).
template <typename T, int D>
__device__ __forceinline__ floatx4 dot_rows_t(const T* lds, int rs, int row0, int lane, const RowReg<T, D>& reg,
                                              floatx4 acc) {
    const int g = lane >> 4, rr = row0 + (lane & 15);
#pragma unroll
    for (int dc = 0; dc < D / 32; ++dc) acc = mma(reg.x[dc], row_op16<T>(lds, rs, rr, dc, g), acc);
    return acc;
}
template <>
__device__ __forceinline__ floatx4 dot_rows_t<float, 64>(const float* lds, int rs, int row0, int lane,
                                                         const RowReg<float, 64>& reg, floatx4 acc) {
    float a[16];
    row_op32<64>(lds, rs, row0 + (lane & 15), lane >> 4, a);
#pragma unroll
    for (int m = 0; m < 16; ++m) acc = mma(reg.x[m], a[m], acc);
    return acc;
}
template <>
__device__ __forceinline__ floatx4 dot_rows_t<float, 128>(const float* lds, int rs, int row0, int lane,
                                                          const RowReg<float, 128>& reg, floatx4 acc) {
    float a[32];
    row_op32<128>(lds, rs, row0 + (lane & 15), lane >> 4, a);
#pragma unroll
    for (int m = 0; m < 32; ++m) acc = mma(reg.x[m], a[m], acc);
    return acc;
}

// acc[dt] += (transposed LDS tile rows dt*16.., token cols kb..kb+31) x P,
// where P is two stacked 16-token accumulator tiles (p0: tokens kb..kb+15,
// p1: kb+16..kb+31) used as the K x 16 operand.
template <typename T, int D>
__device__ __forceinline__ void acc_cols(const T* ldsT, int ts, int kb, int lane, floatx4 p0, floatx4 p1,
                                         floatx4 (&acc)[D / 16]) {
    const int g = lane >> 4, c = lane & 15;
    typename Vec8<T>::type b = pack8<T>(p0, p1);
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) acc[dt] = mma(col_op16<T>(ldsT, ts, dt * 16 + c, kb, g), b, acc[dt]);
}

// fp32 variant: one 16-token accumulator tile p (tokens kb..kb+15)
template <int D>
__device__ __forceinline__ void acc_cols32(const float* ldsT, int ts, int kb, int lane, floatx4 p,
                                           floatx4 (&acc)[D / 16]) {
    const int g = lane >> 4, c = lane & 15;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
        floatx4 a = col_op32(ldsT, ts, dt * 16 + c, kb, g);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[dt] = mma(a[r], p[r], acc[dt]);
    }
}

}  // namespace dsalt
