// LDS tile staging and MFMA operand fetch shared by the attention kernels.
//
// A tile holds ROWS token rows of D elements, staged through registers
// (16-byte global loads along D, branch-free zero fill for missing rows) and
// stored row-major in LDS as [ROWS][D + pad].  Both operand orientations come
// from that one copy:
//  * row_op16(): 8 consecutive D elements of one row -- the A or B operand of
//    a product that reduces over D (lane l: row l & 15, D chunk 32*dc + 8*(l>>4)).
//  * tr_op16(): the operand that reduces over tokens: lane l = 16g + i gets
//    elements (token kb + 4g + r, column c0 + i) for r = 0..3, then the same
//    for tokens kb + 16 + 4g + r.  gfx950's ds_read_b64_tr_b16 transposes
//    within each 16-lane group: lane i receives element (i & 3) of the 8-byte
//    rows addressed by lanes 4r + (i >> 2), so lane j of group g addresses
//    row kb + 4g + (j >> 2), columns c0 + 4 (j & 3) .. +3.
//    That token order (4g..4g+3, 16+4g..16+4g+3) is the one in which two
//    stacked 16x16 accumulator tiles sit in a lane, so accumulators feed the
//    other MFMA operand directly (pack8).
//  * fp32 (K = 4 per instruction): row_op32() gives D/4 consecutive elements
//    (lane group g covers D indices g*D/4 ..), col_f32() the element
//    (token kb + 4g + r, column c) for instruction r.
#pragma once

#include "common.h"

namespace dsalt {

// Row padding (elements) of an LDS tile.  16-bit rows take 16 (160- / 288-byte rows: both
// the row-operand and the transposed reads free of bank conflicts); the forward's and dQ's
// 64-key chunks take 8 (the 16-element padding would cost those blocks a block per CU of LDS).
template <typename T, int D> struct Pad { static constexpr int R = 16; };
template <int D> struct Pad<float, D> { static constexpr int R = 4; };

typedef uint32_t u4v __attribute__((ext_vector_type(4)));

// Raw buffer resource (stride 0, gfx9 word 3): loads at byte offsets >= bytes
// return zero without touching memory, so rows past a bound need no select.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// rsrc over `rows` consecutive token rows from `base` (row stride `row_bytes`,
// `row_len` meaningful bytes per row); rows >= rows read as zero.
__device__ __forceinline__ rsrc_t rows_rsrc(const void* base, int rows, uint32_t row_bytes, uint32_t row_len) {
    const uint32_t n = rows > 0 ? (uint32_t)(rows - 1) * row_bytes + row_len : 0u;
    return make_rsrc(base, n);
}

// Gathered-row offset of a missing row: beyond every resource of at most 2^31 bytes.
constexpr uint32_t kNoRow = 0x80000000u;
// Byte extent of `rows` token rows (stride row_bytes, row_len bytes used), or 0 when
// it exceeds 2^31 - 1 and gathered rows must take 64-bit addresses instead.
__device__ __forceinline__ uint32_t gather_extent(int rows, uint32_t row_bytes, uint32_t row_len) {
    const int64_t n = rows > 0 ? (int64_t)(rows - 1) * row_bytes + row_len : 0;
    return n <= 0x7fffffff ? (uint32_t)n : 0u;
}

template <typename T, int D, int ROWS, int NT = 256, int PAD = Pad<T, D>::R>
struct Tile {
    static constexpr int VW = 16 / (int)sizeof(T);  // elements per 16-byte vector
    static constexpr int CPR = D / VW;               // vectors per row
    static constexpr int NV = ROWS * CPR / NT;       // vectors per thread (NT threads)
    static_assert(ROWS * CPR % NT == 0, "tile must split evenly over the block's threads");
    static constexpr int RS = D + PAD;                // LDS row stride (elements)
    static constexpr int ELEMS = ROWS * RS;
    u4v r[NV];

    // row(rr) returns the global pointer of tile row rr, or nullptr for a zero row
    template <typename RowFn>
    __device__ __forceinline__ void load(int tid, RowFn row, const T* any_valid) {
#pragma unroll
        for (int n = 0; n < NV; ++n) {
            const int vi = tid + NT * n, rr = vi / CPR, c = vi % CPR;
            const T* src = row(rr);
            const bool ok = src != nullptr;
            u4v v = *(const u4v*)((ok ? src : any_valid) + c * VW);
            r[n] = ok ? v : u4v{0u, 0u, 0u, 0u};
        }
    }
    // byte offsets of this thread's vectors in a tile of consecutive rows
    __device__ __forceinline__ static uint32_t row_offset(int tid, int n, uint32_t row_bytes) {
        const int vi = tid + NT * n;
        return (uint32_t)(vi / CPR) * row_bytes + (uint32_t)(vi % CPR) * 16u;
    }
    // byte offsets of this thread's vectors for gathered rows of two tensors (row
    // strides rb0, rb1): row(rr) is the token row of tile row rr, or -1 for a zero
    // row, which gets kNoRow (past any resource of at most 2^31 bytes)
    template <typename RowFn>
    __device__ __forceinline__ static void gather_offsets(int tid, RowFn row, uint32_t rb0, uint32_t rb1,
                                                          uint32_t (&o0)[NV], uint32_t (&o1)[NV]) {
#pragma unroll
        for (int n = 0; n < NV; ++n) {
            const int vi = tid + NT * n, rr = vi / CPR, c = vi % CPR;
            const int j = row(rr);
            o0[n] = j >= 0 ? (uint32_t)j * rb0 + (uint32_t)c * 16u : kNoRow;
            o1[n] = j >= 0 ? (uint32_t)j * rb1 + (uint32_t)c * 16u : kNoRow;
        }
    }
    // rows through a buffer resource at per-thread offsets (zero past its bound)
    __device__ __forceinline__ void load_rows(rsrc_t rs, const uint32_t (&off)[NV]) {
#pragma unroll
        for (int n = 0; n < NV; ++n) r[n] = __builtin_amdgcn_raw_buffer_load_b128(rs, off[n], 0, 0);
    }
    __device__ __forceinline__ void store(T* lds, int tid) const {
#pragma unroll
        for (int n = 0; n < NV; ++n) {
            const int vi = tid + NT * n, rr = vi / CPR, c = vi % CPR;
            *(u4v*)(lds + rr * RS + c * VW) = r[n];
        }
    }
};

template <typename T>
__device__ __forceinline__ typename Vec8<T>::type row_op16(const T* lds, int rs, int row, int dc, int g) {
    return *(const typename Vec8<T>::type*)(lds + row * rs + dc * 32 + 8 * g);
}

__device__ __forceinline__ bf16x4 tr_read(const bf16* p) {
    typedef __attribute__((address_space(3))) bf16x4* lp;
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lp)p);
}
__device__ __forceinline__ f16x4 tr_read(const f16* p) {
    typedef __fp16 h4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) h4* lp;
    return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lp)p));
}

template <typename T>
__device__ __forceinline__ typename Vec8<T>::type tr_op16(const T* lds, int rs, int c0, int kb, int lane) {
    const int g = lane >> 4, j = lane & 15;
    const T* p = lds + (kb + 4 * g + (j >> 2)) * rs + c0 + 4 * (j & 3);
    typename Vec8<T>::half lo = tr_read(p), hi = tr_read(p + 16 * rs);
    typename Vec8<T>::type v;
    v[0] = lo[0]; v[1] = lo[1]; v[2] = lo[2]; v[3] = lo[3];
    v[4] = hi[0]; v[5] = hi[1]; v[6] = hi[2]; v[7] = hi[3];
    return v;
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
// and dq kernels, keys/values in the key-parallel kernels).
template <typename T, int D>
struct RowReg {
    typename Vec8<T>::type x[D / 32];
    __device__ __forceinline__ void load(const T* src, const T* any_valid, int g) {
        const bool ok = src != nullptr;
        const T* p = ok ? src : any_valid;
#pragma unroll
        for (int dc = 0; dc < D / 32; ++dc) {
            typename Vec8<T>::type v = *(const typename Vec8<T>::type*)(p + dc * 32 + 8 * g);
            if (!ok) v = typename Vec8<T>::type{};
            x[dc] = v;
        }
    }
};
template <int D>
struct RowReg<float, D> {
    float x[D / 4];
    __device__ __forceinline__ void load(const float* src, const float* any_valid, int g) {
        const bool ok = src != nullptr;
        const float* p = ok ? src : any_valid;
#pragma unroll
        for (int m = 0; m < D / 16; ++m) {
            floatx4 v = *(const floatx4*)(p + g * (D / 4) + 4 * m);
            if (!ok) v = floatx4{0.f, 0.f, 0.f, 0.f};
            x[4 * m] = v[0]; x[4 * m + 1] = v[1]; x[4 * m + 2] = v[2]; x[4 * m + 3] = v[3];
        }
    }
};

// acc + (16 LDS rows from row0) x (16 register rows), reduced over D:
// output row = LDS row (4g + r), output column = register row (lane & 15).
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

// acc[dt] += (row-major LDS tile, tokens kb..kb+31, columns 16dt..16dt+15)^T
//            x P, with P two stacked 16-token accumulator tiles (p0: tokens
// kb..kb+15, p1: kb+16..kb+31).  Returns the packed P operand so callers can
// reuse it (row sums through a ones operand).
template <typename T, int D>
__device__ __forceinline__ typename Vec8<T>::type acc_tr(const T* lds, int rs, int kb, int lane, floatx4 p0,
                                                         floatx4 p1, floatx4 (&acc)[D / 16]) {
    typename Vec8<T>::type b = pack8<T>(p0, p1);
    typename Vec8<T>::type a[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) a[dt] = tr_op16<T>(lds, rs, dt * 16, kb, lane);
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) acc[dt] = mma(a[dt], b, acc[dt]);
    return b;
}

// fp32: acc[dt] += (tokens kb..kb+15 of the row-major tile)^T x p (one 16-token tile)
template <int D>
__device__ __forceinline__ void acc_rm32(const float* lds, int rs, int kb, int lane, floatx4 p,
                                         floatx4 (&acc)[D / 16]) {
    const int g = lane >> 4, c = lane & 15;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[dt] = mma(lds[(kb + 4 * g + r) * rs + dt * 16 + c], p[r], acc[dt]);
}

// The LDS operand of one 16-row subtile for products reduced over D, fetched
// once and applied to several register row sets (row groups of a wave).
template <typename T, int D>
struct KOp {
    typename Vec8<T>::type a[D / 32];
    __device__ __forceinline__ void load(const T* lds, int rs, int row0, int lane) {
#pragma unroll
        for (int dc = 0; dc < D / 32; ++dc) a[dc] = row_op16<T>(lds, rs, row0 + (lane & 15), dc, lane >> 4);
    }
    __device__ __forceinline__ floatx4 dot(const RowReg<T, D>& reg, floatx4 acc) const {
#pragma unroll
        for (int dc = 0; dc < D / 32; ++dc) acc = mma(a[dc], reg.x[dc], acc);
        return acc;
    }
};
template <int D>
struct KOp<float, D> {
    float a[D / 4];
    __device__ __forceinline__ void load(const float* lds, int rs, int row0, int lane) {
        row_op32<D>(lds, rs, row0 + (lane & 15), lane >> 4, a);
    }
    __device__ __forceinline__ floatx4 dot(const RowReg<float, D>& reg, floatx4 acc) const {
#pragma unroll
        for (int m = 0; m < D / 4; ++m) acc = mma(a[m], reg.x[m], acc);
        return acc;
    }
};

// The transposed LDS operand of a slab of tokens for products reduced over
// tokens (P V, dS K, ...): 16-bit types take 32 tokens kb..kb+31 through the
// transpose read, fp32 16 tokens kb..kb+15 element by element.
template <typename T, int D>
struct VOp {
    static constexpr int TOK = 32;
    typename Vec8<T>::type a[D / 16];
    __device__ __forceinline__ void load(const T* lds, int rs, int kb, int lane) {
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) a[dt] = tr_op16<T>(lds, rs, dt * 16, kb, lane);
    }
    // acc += slab^T x (p0 | p1); returns the packed P operand
    __device__ __forceinline__ typename Vec8<T>::type acc(floatx4 p0, floatx4 p1, floatx4 (&c)[D / 16]) const {
        const typename Vec8<T>::type b = pack8<T>(p0, p1);
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) c[dt] = mma(a[dt], b, c[dt]);
        return b;
    }
};
template <int D>
struct VOp<float, D> {
    static constexpr int TOK = 16;
    float a[D / 16][4];
    __device__ __forceinline__ void load(const float* lds, int rs, int kb, int lane) {
        const int g = lane >> 4, c = lane & 15;
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r) a[dt][r] = lds[(kb + 4 * g + r) * rs + dt * 16 + c];
    }
    __device__ __forceinline__ void acc(floatx4 p, floatx4 (&c)[D / 16]) const {
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r) c[dt] = mma(a[dt][r], p[r], c[dt]);
    }
};

template <typename T> __device__ __forceinline__ typename Vec8<T>::type ones8() {
    typename Vec8<T>::type v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = from_float<T>(1.0f);
    return v;
}

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Whole-row output of a wave's 16 rows held in the accumulator layout (acc[dt][r]: column
// 16 dt + 4 (lane >> 4) + r of the row of lane & 15), times `mul`: the values go through
// `stage` (LDS private to the wave, StoreRows::ELEMS elements) and leave as 16-byte pieces,
// D * sizeof(T) / 16 lanes per row, so each store instruction writes whole rows (stores of
// 8-byte pieces, four instructions per row, cost the kernels up to a tenth of their time).
// dst(rr) is row rr's destination (rr = 0..15, the row of accumulator lane rr), nullptr for
// a row not written.  Every lane of the wave calls it.
template <typename T, int D>
struct StoreRows {
    static constexpr int RS = D + 16 / (int)sizeof(T);  // row stride in LDS: 16 bytes of padding
    static constexpr int ELEMS = 16 * RS;
    template <typename Dst>
    __device__ __forceinline__ static void run(T* stage, const floatx4 (&acc)[D / 16], float mul, int lane, Dst dst) {
        const int j = lane & 15, g = lane >> 4;
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) {
            T v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = from_float<T>(acc[dt][r] * mul);
            T* at = stage + j * RS + dt * 16 + 4 * g;
            if constexpr (sizeof(T) == 2) *(uint2*)at = *(const uint2*)v;
            else *(floatx4*)at = *(const floatx4*)v;
        }
        // the wave's LDS writes are seen by its reads below (no other wave touches `stage`)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        constexpr int VE = 16 / (int)sizeof(T);  // elements per 16 bytes
        constexpr int LPR = D / VE;              // lanes per row
        constexpr int RPI = 64 / LPR;            // rows per store instruction
#pragma unroll
        for (int u = 0; u < 16 / RPI; ++u) {
            const int rr = u * RPI + lane / LPR, c = (lane % LPR) * VE;
            const uint4 val = *(const uint4*)(stage + rr * RS + c);
            T* d = dst(rr);
            if (d) *(uint4*)(d + c) = val;
        }
    }
};

}  // namespace dsalt
