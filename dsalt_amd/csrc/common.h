// Shared device helpers for the gfx950 DSALT kernels: element types, MFMA
// wrappers, wave reductions and the canonical fp64 helpers of landmark selection.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dsalt_amd.h"

namespace dsalt {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
// Landmark slots per set: at most kMaxLandmarks.  The single-set attention kernels keep a set
// of up to kSetSlots in LDS; larger sets, and the several sets a 64-row tile's rows use when
// a block-causal block_size is not a multiple of 64 (at most kMaxTileSets, staged side by
// side: sets x k_lmk at most kMultiSetSlots), take the wide instantiations.
constexpr int kMaxLandmarks = 2048;
constexpr int kSetSlots = 512;
constexpr int kMaxTileSets = 64;
constexpr int kMultiSetSlots = 2048;

__device__ __forceinline__ float to_float(float x) { return x; }
__device__ __forceinline__ float to_float(bf16 x) { return (float)x; }
__device__ __forceinline__ float to_float(f16 x) { return (float)x; }

template <typename T> __device__ __forceinline__ T from_float(float x);
template <> __device__ __forceinline__ float from_float<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_float<bf16>(float x) { return (bf16)x; }
template <> __device__ __forceinline__ f16 from_float<f16>(float x) { return (f16)x; }

// ---------------------------------------------------------------- wave ops
__device__ __forceinline__ float wave_xor(float v, int off) { return __shfl_xor(v, off, kWave); }
__device__ __forceinline__ int wave_xor(int v, int off) { return __shfl_xor(v, off, kWave); }
__device__ __forceinline__ double wave_xor(double v, int off) { return __shfl_xor(v, off, kWave); }

// reductions over the 16 lanes that share (lane & 15) groups: xor 1,2,4,8
__device__ __forceinline__ int min16(int v) {
    for (int o = 1; o < 16; o <<= 1) v = min(v, wave_xor(v, o));
    return v;
}
__device__ __forceinline__ int max16(int v) {
    for (int o = 1; o < 16; o <<= 1) v = max(v, wave_xor(v, o));
    return v;
}
// reductions within each 16-lane row through DPP row rotations (VALU only)
__device__ __forceinline__ int dpp_ror(int v, int n) {
    switch (n) {
        case 1: return __builtin_amdgcn_update_dpp(0, v, 0x121, 0xf, 0xf, false);
        case 2: return __builtin_amdgcn_update_dpp(0, v, 0x122, 0xf, 0xf, false);
        case 4: return __builtin_amdgcn_update_dpp(0, v, 0x124, 0xf, 0xf, false);
        default: return __builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, false);
    }
}
__device__ __forceinline__ int row_min16(int v) {
    v = min(v, dpp_ror(v, 1));
    v = min(v, dpp_ror(v, 2));
    v = min(v, dpp_ror(v, 4));
    return min(v, dpp_ror(v, 8));
}
__device__ __forceinline__ int row_max16(int v) {
    v = max(v, dpp_ror(v, 1));
    v = max(v, dpp_ror(v, 2));
    v = max(v, dpp_ror(v, 4));
    return max(v, dpp_ror(v, 8));
}

// maximum over the wave (every lane gets it)
__device__ __forceinline__ int wave_max(int v) {
    const int m = row_max16(v);
    return max(max(__builtin_amdgcn_readlane(m, 0), __builtin_amdgcn_readlane(m, 16)),
               max(__builtin_amdgcn_readlane(m, 32), __builtin_amdgcn_readlane(m, 48)));
}

// reductions over the 4 lanes l, l^16, l^32, l^48, with gfx950's lane-swap
// instructions (VALU, no LDS round trip): permlane32_swap(x, x) yields the lower
// and the upper 32 lanes each broadcast to both halves; permlane16_swap(y, y)
// the even and the odd 16-lane rows each broadcast over their pair.
__device__ __forceinline__ float max_g4(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const float m = fmaxf(__builtin_bit_cast(float, (uint32_t)a[0]), __builtin_bit_cast(float, (uint32_t)a[1]));
    const uint32_t um = __builtin_bit_cast(uint32_t, m);
    auto b = __builtin_amdgcn_permlane16_swap(um, um, false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)b[0]), __builtin_bit_cast(float, (uint32_t)b[1]));
}
__device__ __forceinline__ float sum_g4(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const float m = __builtin_bit_cast(float, (uint32_t)a[0]) + __builtin_bit_cast(float, (uint32_t)a[1]);
    const uint32_t um = __builtin_bit_cast(uint32_t, m);
    auto b = __builtin_amdgcn_permlane16_swap(um, um, false, false);
    return __builtin_bit_cast(float, (uint32_t)b[0]) + __builtin_bit_cast(float, (uint32_t)b[1]);
}

// ------------------------------------------------------------------- MFMA
// 16x16 output tile D = A(16 x K) * B(K x 16) + C with fp32 accumulation.
// Lane l holds A row (l & 15), B column (l & 15) and D column (l & 15),
// D rows 4*(l >> 4) + r for r = 0..3.  For 16-bit types one instruction
// reduces K = 32 (lane holds k = 8*(l >> 4) + e, e = 0..7); for fp32 K = 4
// (lane holds k = l >> 4).
__device__ __forceinline__ floatx4 mma(bf16x8 a, bf16x8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mma(f16x8 a, f16x8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mma(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <typename T> struct Vec8;
template <> struct Vec8<bf16> { typedef bf16x8 type; typedef bf16x4 half; };
template <> struct Vec8<f16> { typedef f16x8 type; typedef f16x4 half; };

// pack two groups of 4 fp32 values into one 8-element 16-bit operand
template <typename T>
__device__ __forceinline__ typename Vec8<T>::type pack8(floatx4 lo, floatx4 hi) {
    typename Vec8<T>::type r;
    r[0] = from_float<T>(lo[0]); r[1] = from_float<T>(lo[1]);
    r[2] = from_float<T>(lo[2]); r[3] = from_float<T>(lo[3]);
    r[4] = from_float<T>(hi[0]); r[5] = from_float<T>(hi[1]);
    r[6] = from_float<T>(hi[2]); r[7] = from_float<T>(hi[3]);
    return r;
}

// ------------------------------------------------------- canonical numbers
// Heron square root from an exponent-halving seed: IEEE add/mul/div only, so
// the host oracle and the device produce identical bits.
__device__ __forceinline__ double canon_sqrt64(double x) {
    if (!(x > 0.0)) return 0.0;
    unsigned long long b = (unsigned long long)__double_as_longlong(x);
    b = (b >> 1) + 0x1ff8000000000000ull;
    double y = __longlong_as_double((long long)b);
#pragma unroll
    for (int it = 0; it < 6; ++it) y = __dmul_rn(0.5, __dadd_rn(y, __ddiv_rn(x, y)));
    return y;
}

__device__ __forceinline__ float round_bf16_value(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7fffu + ((u >> 16) & 1u);
    return __uint_as_float(u & 0xffff0000u);
}

template <typename T> __device__ __forceinline__ float round_norm(float f);
template <> __device__ __forceinline__ float round_norm<float>(float f) { return f; }
template <> __device__ __forceinline__ float round_norm<bf16>(float f) { return round_bf16_value(f); }
template <> __device__ __forceinline__ float round_norm<f16>(float f) { return (float)(f16)f; }

__host__ __device__ __forceinline__ int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Start and length of sequence s, clamped to the packed buffer [0, total) and to
// max_len, so malformed offsets can never address rows outside the tensors.
__device__ __forceinline__ void seq_bounds(const int32_t* cu, int s, int total, int max_len, int& st, int& len) {
    st = min(max(cu[s], 0), total);
    int en = min(max(cu[s + 1], st), total);
    len = min(en - st, max_len);
}

// XCD-aware block index: the hardware deals blocks round-robin to 8 XCDs;
// remap so each XCD walks a contiguous range of logical tiles (L2 reuse of
// the shared key band between neighbouring query tiles).
__device__ __forceinline__ int xcd_swizzle(int b, int n) {
    int x = b & 7, y = b >> 3, q = n >> 3, r = n & 7;
    return x * q + (x < r ? x : r) + y;
}

}  // namespace dsalt
