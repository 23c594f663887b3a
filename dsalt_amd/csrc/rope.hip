// Rotary position embedding, half-split convention, in place on the query and key
// heads of a packed projection output (e.g. the fused QKV GEMM result read through
// strides).  For the pair (x1, x2) = (x[j], x[j + D/2]) of a token at sequence
// position p:
//   x[j]       <- x1 * cos[p][j]       + (-x2) * sin[p][j]
//   x[j + D/2] <- x2 * cos[p][j + D/2] +   x1  * sin[p][j + D/2]
// with cos/sin rounded to the tensor type first and every product and the sum rounded
// to the tensor type, the arithmetic of the elementwise expression
// q * cos + rotate_half(q) * sin evaluated one operation at a time in that type.
// HBM-bound: one read and one write of every q/k element, cos/sin rows from cache.
#include "common.h"
#include "rope.h"
#include "timing.h"

namespace dsalt {

namespace {

template <typename T>
__device__ __forceinline__ float rnd(float x) {
    return to_float(from_float<T>(x));
}

// product and sum rounded separately (no fused multiply-add)
template <typename T>
__device__ __forceinline__ float rot_term(float x, float c, float y, float s) {
    const float a = rnd<T>(__fmul_rn(x, c));
    const float b = rnd<T>(__fmul_rn(y, s));
    return __fadd_rn(a, b);
}

__device__ __forceinline__ int seq_of(const int* cu, int num_seqs, int t) {
    int lo = 0, hi = num_seqs - 1;  // last s with cu[s] <= t
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (cu[mid] <= t) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// one thread: one (token, head, 8-element chunk of the first half)
template <typename T>
__global__ __launch_bounds__(256) void rope_kernel(RopeParams p) {
    const int half = p.head_dim >> 1;
    const int nch = half >> 3;
    const int nh = p.n_q_heads + p.n_k_heads;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t per_tok = (int64_t)nh * nch;
    if (gid >= (int64_t)p.total_len * per_tok) return;
    const int t = (int)(gid / per_tok);
    const int rem = (int)(gid - (int64_t)t * per_tok);
    const int hh = rem / nch, ch = rem - hh * nch;
    const int pos = t - p.cu[seq_of(p.cu, p.num_seqs, t)];
    T* const row = hh < p.n_q_heads ? (T*)p.q + (int64_t)t * p.q_st + (int64_t)hh * p.q_sh
                              : (T*)p.k + (int64_t)t * p.k_st + (int64_t)(hh - p.n_q_heads) * p.k_sh;
    if (pos >= p.max_pos) return;  // excluded by the host check max_seqlen <= max_pos
    const int j0 = ch * 8;
    typedef T vec8 __attribute__((ext_vector_type(8), aligned(16)));
    typedef float f32x8 __attribute__((ext_vector_type(8), aligned(16)));
    const f32x8 c1 = *(const f32x8*)(p.cos + (int64_t)pos * p.head_dim + j0);
    const f32x8 c2 = *(const f32x8*)(p.cos + (int64_t)pos * p.head_dim + half + j0);
    const f32x8 s1 = *(const f32x8*)(p.sin + (int64_t)pos * p.head_dim + j0);
    const f32x8 s2 = *(const f32x8*)(p.sin + (int64_t)pos * p.head_dim + half + j0);
    const vec8 a = *(const vec8*)(row + j0);
    const vec8 b = *(const vec8*)(row + half + j0);
    vec8 o1, o2;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float x1 = to_float(a[e]), x2 = to_float(b[e]);
        o1[e] = from_float<T>(rot_term<T>(x1, rnd<T>(c1[e]), -x2, rnd<T>(s1[e])));
        o2[e] = from_float<T>(rot_term<T>(x2, rnd<T>(c2[e]), x1, rnd<T>(s2[e])));
    }
    *(vec8*)(row + j0) = o1;
    *(vec8*)(row + half + j0) = o2;
}

}  // namespace

hipError_t rope_launch(const RopeParams& p, hipStream_t stream) {
    const int64_t n = (int64_t)p.total_len * (p.n_q_heads + p.n_k_heads) * (p.head_dim / 16);
    if (n == 0) return hipSuccess;
    const dim3 grid((unsigned)((n + 255) / 256));
    switch (p.dtype) {
        case 0: DSALT_LAUNCH("rope", rope_kernel<float>, grid, dim3(256), 0, stream, p); break;
        case 1: DSALT_LAUNCH("rope", rope_kernel<bf16>, grid, dim3(256), 0, stream, p); break;
        default: DSALT_LAUNCH("rope", rope_kernel<f16>, grid, dim3(256), 0, stream, p); break;
    }
    return hipGetLastError();
}

}  // namespace dsalt
