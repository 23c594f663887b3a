// Attention probabilities of one sequence over its attended keys A(i) = W(i) U L(i), in
// banded form: p_win[h][i][c] = P(i, i - c) for the window keys c < min(w_i, i + 1),
// p_lmk[h][i][slot] = P(i, landmark slot) for the landmarks the row sees, zero elsewhere.
// P = exp(scale * q_i . k_j + bias_j - lse_i) with the forward's log-sum-exp, so the
// values are the probabilities the forward used (O(L (w + k)) memory instead of the
// O(L^2) dense matrix).  One wave per (head, row): lanes over keys, q in LDS.
#include "attn.h"
#include "common.h"
#include "probs.h"
#include "timing.h"

namespace dsalt {

namespace {

template <typename T, int D>
__device__ __forceinline__ float row_dot(const float* qs, const T* krow) {
    typedef T vec8 __attribute__((ext_vector_type(8), aligned(16)));
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < D / 8; ++c) {
        const vec8 kv = *(const vec8*)(krow + c * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += qs[c * 8 + e] * to_float(kv[e]);
    }
    return acc;
}

template <typename T, int D>
__global__ __launch_bounds__(256) void probs_kernel(ProbsParams pp) {
    const AttnParams& p = pp.a;
    __shared__ float qs[4][D];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int h = blockIdx.y;
    const int i = blockIdx.x * 4 + wave;
    int st, len;
    seq_bounds(p.cu, pp.seq, p.total_len, p.max_seqlen, st, len);
    const int rows = min(len, pp.out_rows);
    const bool active = i < rows;
    const T* qrow = (const T*)p.q + (int64_t)(st + (active ? i : 0)) * p.q_st + (int64_t)h * p.q_sh;
    for (int d = lane; d < D; d += 64) qs[wave][d] = active ? to_float(qrow[d]) : 0.f;
    __syncthreads();
    if (!active) return;
    const int kvh = h / (p.n_heads / p.n_kv_heads);
    const float lse = p.lse_out[(int64_t)(st + i) * p.n_heads + h];
    const int wi = max(p.w[st + i], 1);
    const int lo = max(i - wi + 1, 0);
    const int nb = i - lo + 1;
    const T* kbase = (const T*)p.k + (int64_t)st * p.k_st + (int64_t)kvh * p.k_sh;
    float* prow = pp.p_win + ((int64_t)h * pp.out_rows + i) * pp.w_cap;
    for (int c = lane; c < pp.w_cap; c += 64) {
        float v = 0.f;
        if (c < nb) v = __expf(row_dot<T, D>(qs[wave], kbase + (int64_t)(i - c) * p.k_st) * p.scale - lse);
        prow[c] = v;
    }
    if (pp.p_lmk) {
        const int K = p.k_lmk;
        const int set = p.block_size ? i / p.block_size : 0;
        const int64_t set_off = (((int64_t)h * p.num_seqs + pp.seq) * p.n_sets + set) * K;
        float* lrow = pp.p_lmk + ((int64_t)h * pp.out_rows + i) * K;
        for (int sl = lane; sl < K; sl += 64) {
            const int pos = p.lmk[set_off + sl];
            float v = 0.f;
            if (pos >= 0 && pos < lo && pos < len) {
                const float b = p.lbias ? p.lbias[set_off + sl] : 0.f;
                v = __expf(row_dot<T, D>(qs[wave], kbase + (int64_t)pos * p.k_st) * p.scale + b - lse);
            }
            lrow[sl] = v;
        }
    }
}

}  // namespace

hipError_t probs_launch(const ProbsParams& pp, hipStream_t stream) {
    const AttnParams& p = pp.a;
    const dim3 grid((unsigned)((pp.out_rows + 3) / 4), (unsigned)p.n_heads);
    if (pp.out_rows == 0) return hipSuccess;
#define DSALT_PROBS(T, D) DSALT_LAUNCH("probs", (probs_kernel<T, D>), grid, dim3(256), 0, stream, pp)
    const bool d64 = p.head_dim == 64;
    switch (p.dtype) {
        case 0: if (d64) DSALT_PROBS(float, 64); else DSALT_PROBS(float, 128); break;
        case 1: if (d64) DSALT_PROBS(bf16, 64); else DSALT_PROBS(bf16, 128); break;
        default: if (d64) DSALT_PROBS(f16, 64); else DSALT_PROBS(f16, 128); break;
    }
#undef DSALT_PROBS
    return hipGetLastError();
}

}  // namespace dsalt
