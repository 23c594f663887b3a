// Landmark selection for gfx950.
//
// Replaces hybrid_scores_per_head (dsalt/kernels/landmark_tokens_ker.py:19-61),
// _compute_landmark_indices (dsalt/kernels/selectors.py:75-134) and the
// block-causal _select (results/causal_landmark_check.py:82-113).
//
// Pipeline (all stream-ordered, no host sync):
//   sel_norms   one wave per token: |h_t| and |v_{t,g}| as fp64 sums of squares
//               (lane-strided 16-byte chunks + xor butterfly); the block then
//               takes the square roots of its tokens' sums lane-parallel and
//               rounds them to fp32 and then to the input dtype.
//   sel_sums    one 256-thread block per (range, signal): fp64 S1, S2 by 256
//               strided partials and a halving tree; in the global variant the
//               same block turns them into mean / unbiased std (global sets of up
//               to 32768 tokens without z or scores for the caller: each top-k
//               part computes them itself, in the same order, and sel_sums is
//               not launched).
//   sel_stats   (block-causal) mean / std per prefix by adding whole-block sums
//               in block order.
//   sel_z       (global) z = fp32((a - mean)/std) in fp64, one thread per
//               (token, signal); sel_scores the optional per-head scores.
//   top-k on the 64-bit key (order(score) << 32 | ~index), so ties go to the
//   lower index; output ascending indices:
//     global:   sel_part keeps the best pow2(k) keys of each part of a set's
//               candidates (the order statistic by radix passes, kth_desc);
//               sel_merge does the same over the survivors of up to G parts per
//               block, level by level, and the last level writes the indices in
//               ascending order (by ranks).
//     block:    (bf16, sequences of 65536+ tokens) sel_prune_* list per kv head
//               the candidates that fewer than k earlier candidates can dominate
//               in both norms (a lower bound from 2D bin histograms); the others
//               are in no set's top k.  sel_topk, one 256/512-thread block per
//               landmark set (largest sets first), scans the listed candidates
//               below the set's start (or the whole prefix).  Sets of at most 2048:
//               every key in LDS and one order statistic.  Larger sets (8192+
//               unlisted candidates): a threshold key, the order
//               statistic of a strided sample of 2048 (1024 of a list) found by radix passes
//               (kth_desc), one pass screening every candidate with a float32 affine
//               form of its score (exact keys only near the threshold; bf16 inputs
//               read both norms from one packed word), then the K-th largest survivor
//               by the same radix passes and the K survivors at or above it, output
//               in index order by ranks; when the sample misplaces the threshold,
//               and for smaller sets: radix select 8 bits per pass until the boundary
//               bin fits in LDS, then its order statistic by kth_desc.
// The arithmetic order above is the canonical one that the CPU oracle
// restates; this file is compiled with -ffp-contract=off.
#include "common.h"
#include "plan.h"
#include "select.h"
#include "timing.h"

namespace dsalt {

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / kWave;
// block-causal sets (sel_topk): blocks smaller than the global top-k's put more sets in
// flight per CU; 256 threads when the sets scan pruned lists (a few thousand candidates
// each), 512 for whole prefixes
constexpr int kTopkThreads = 512;
constexpr int kTopkThreadsPruned = 256;
constexpr int kBorderCap = 2048;

__device__ __forceinline__ int pow2ceil64(int n) {
    int g = 1;
    while (g < n && g < 64) g <<= 1;
    return g;
}

// ------------------------------------------------------------------ norms
constexpr int kNormTPW = 1;              // tokens per wave
constexpr int kNormTB = 4 * kNormTPW;    // tokens per 256-thread block

// bf16 inputs: the norms are non-negative bf16 values, so a token's |h| and |v_g| pack
// losslessly into one word, pk[g][t] = bf16(|v_g|) << 16 | bf16(|h|), whose bit 15 (the
// sign of |h|) instead flags a token that is never a candidate (its own window reaches
// its sequence start, j_rel < w_j).  The block-causal top-k reads only that word per
// candidate in its prefix scans: no window load, and exact keys straight from it.
constexpr uint32_t kExcluded = 0x8000u;
__device__ __forceinline__ uint32_t pack_norms(float nx, float nv, bool excluded) {
    return (__float_as_uint(nv) & 0xffff0000u) | (__float_as_uint(nx) >> 16) | (excluded ? kExcluded : 0u);
}
__device__ __forceinline__ float packed_nx(uint32_t w) { return __uint_as_float((w << 16) & 0x7fff0000u); }
__device__ __forceinline__ float packed_nv(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// sequence of packed token t: the last s whose (clamped) start is <= t
__device__ __forceinline__ int seq_of(const SelectParams& p, int t) {
    int lo = 0, hi = p.num_seqs - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (min(max(p.cu[mid], 0), p.total_len) <= t) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// Blocks past the norms' `nblk` (when the caller asked for the forward's row plan) plan four
// 64-row tiles each, one per wave: independent work that rides in the same launch.
template <typename T>
__global__ __launch_bounds__(256) void sel_norms_kernel(SelectParams p, float* nx, float* nv, uint32_t* pk, int nblk) {
    constexpr int VW = 16 / (int)sizeof(T);
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    extern __shared__ double ss[];  // [kNormTB][1 + n_kv] sums of squares
    const int nsig = 1 + p.n_kv_heads;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if ((int)blockIdx.x >= nblk) {
        __shared__ int sp[4][64], slo[4][64];
        const int tile = ((int)blockIdx.x - nblk) * 4 + wave;
        row_plan_tile(p.w, p.cu, p.total_len, p.max_seqlen, p.n_tiles, tile, tile < p.num_seqs * p.n_tiles, lane,
                      sp[wave], slo[wave], PlanOut{p.plan_perm, p.plan_bounds, p.tile_wmax});
        return;
    }
    const int t0 = blockIdx.x * kNormTB;
    const int hch = p.hidden / VW, gh = pow2ceil64(hch);
    const int vch = p.head_dim / VW, gv = pow2ceil64(vch);
    const int hpp = 64 / gv;  // value heads per pass
    for (int i = 0; i < kNormTPW; ++i) {
        const int tl = wave * kNormTPW + i, t = t0 + tl;
        if (t >= p.total_len) break;
        // hidden-state norm
        const T* hr = (const T*)p.h + (int64_t)t * p.h_stride_t;
        double acc = 0.0;
        if (lane < gh) {
            for (int ch = lane; ch < hch; ch += gh) {
                u4 raw = *(const u4*)(hr + ch * VW);
                const T* e = (const T*)&raw;
#pragma unroll
                for (int q = 0; q < VW; ++q) {
                    double x = (double)to_float(e[q]);
                    acc = __dadd_rn(acc, __dmul_rn(x, x));
                }
            }
        }
        for (int off = gh >> 1; off >= 1; off >>= 1) acc = __dadd_rn(acc, wave_xor(acc, off));
        if (lane == 0) ss[tl * nsig] = acc;
        // value-vector norms, gv lanes per kv head
        for (int g0 = 0; g0 < p.n_kv_heads; g0 += hpp) {
            int g = g0 + lane / gv, sub = lane % gv;
            double a2 = 0.0;
            if (g < p.n_kv_heads && sub < vch) {
                const T* vr = (const T*)p.v + (int64_t)t * p.v_stride_t + (int64_t)g * p.v_stride_h;
                u4 raw = *(const u4*)(vr + sub * VW);
                const T* e = (const T*)&raw;
#pragma unroll
                for (int q = 0; q < VW; ++q) {
                    double x = (double)to_float(e[q]);
                    a2 = __dadd_rn(a2, __dmul_rn(x, x));
                }
            }
            for (int off = gv >> 1; off >= 1; off >>= 1) a2 = __dadd_rn(a2, wave_xor(a2, off));
            if (sub == 0 && g < p.n_kv_heads) ss[tl * nsig + 1 + g] = a2;
        }
    }
    __shared__ bool excl[kNormTB];
    if (pk && threadIdx.x < kNormTB && t0 + (int)threadIdx.x < p.total_len) {
        const int t = t0 + threadIdx.x;
        const int st = min(max(p.cu[seq_of(p, t)], 0), p.total_len);
        excl[threadIdx.x] = t - st < p.w[t];
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < kNormTB * nsig; idx += 256) {
        const int tl = idx / nsig, sig = idx % nsig, t = t0 + tl;
        if (t >= p.total_len) continue;
        const float nr = round_norm<T>((float)canon_sqrt64(ss[idx]));
        if (sig == 0) nx[t] = nr;
        else nv[(int64_t)(sig - 1) * p.total_len + t] = nr;
        if (pk && sig > 0)
            pk[(int64_t)(sig - 1) * p.total_len + t] =
                pack_norms(round_norm<T>((float)canon_sqrt64(ss[tl * nsig])), nr, excl[tl]);
    }
}

// ------------------------------------------------------------- statistics
// Range r of signal sig: global/packed r=0 -> [0,T); global/sequence r=s ->
// sequence s; block r = s*n_sets + b -> block b of sequence s.
__device__ __forceinline__ void range_of(const SelectParams& p, int r, int& r0, int& r1) {
    if (p.select_mode == DSALT_SELECT_GLOBAL) {
        if (p.stats_scope == DSALT_STATS_PACKED) {
            r0 = 0;
            r1 = p.total_len;
        } else {
            int len;
            seq_bounds(p.cu, r, p.total_len, p.max_seqlen, r0, len);
            r1 = r0 + len;
        }
    } else {
        int s = r / p.n_sets, b = r % p.n_sets;
        int st, len;
        seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
        r0 = min(st + b * p.block_size, st + len);
        r1 = min(r0 + p.block_size, st + len);
    }
}

__device__ __forceinline__ void mean_std(double s1, double s2, int n, double& mean, double& sd) {
    double m = __ddiv_rn(s1, (double)n);
    double den = (double)(n - 1 > 1 ? n - 1 : 1);
    double var = __ddiv_rn(__dadd_rn(s2, -__dmul_rn(__dmul_rn((double)n, m), m)), den);
    if (!(var > 0.0)) var = 0.0;
    double s = canon_sqrt64(var);
    if (s < 1e-6) s = 1e-6;
    mean = m;
    sd = s;
}

// The canonical sum of a range: kSumParts strided partials (partial t adds elements
// r0 + t + kSumParts m in increasing m), then a halving tree.
constexpr int kSumParts = 1024;

__global__ __launch_bounds__(256) void sel_sums_kernel(SelectParams p, const float* nx, const float* nv,
                                                       double* sums, double* stats) {
    // thread t owns partials t + 256 q (q = 0..3), U chain steps of each in flight; reads past
    // the range return zero, and adding +0 to these sums of non-negative norms changes no bit
    constexpr int Q = kSumParts / 256, U = 8;
    __shared__ double a1[kSumParts], a2[kSumParts];
    const int r = blockIdx.x, sig = blockIdx.y, t = threadIdx.x;
    const float* x = sig == 0 ? nx : nv + (int64_t)(sig - 1) * p.total_len;
    int r0, r1;
    range_of(p, r, r0, r1);
    double s1[Q], s2[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) s1[q] = s2[q] = 0.0;
    for (int j0 = r0; j0 < r1; j0 += kSumParts * U) {
        const int n = min(kSumParts * U, r1 - j0);
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc((void*)(x + j0), (short)0, (int)(n * sizeof(float)), 0x00020000);
        float xv[U][Q];
#pragma unroll
        for (int m = 0; m < U; ++m)
#pragma unroll
            for (int q = 0; q < Q; ++q)
                xv[m][q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                          rs, (uint32_t)(t + 256 * q + kSumParts * m) * 4u, 0, 0));
#pragma unroll
        for (int m = 0; m < U; ++m)
#pragma unroll
            for (int q = 0; q < Q; ++q) {
                const double v = (double)xv[m][q];
                s1[q] = __dadd_rn(s1[q], v);
                s2[q] = __dadd_rn(s2[q], __dmul_rn(v, v));
            }
    }
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        a1[t + 256 * q] = s1[q];
        a2[t + 256 * q] = s2[q];
    }
    __syncthreads();
    for (int off = kSumParts / 2; off >= 1; off >>= 1) {
        for (int i = t; i < off; i += 256) {
            a1[i] = __dadd_rn(a1[i], a1[i + off]);
            a2[i] = __dadd_rn(a2[i], a2[i + off]);
        }
        __syncthreads();
    }
    if (t == 0) {
        const int nsig = 1 + p.n_kv_heads;
        const int64_t o = ((int64_t)r * nsig + sig) * 2;
        sums[o] = a1[0];
        sums[o + 1] = a2[0];
        if (stats) {  // global variant: statistics of this range
            double m = 0.0, sd = 1.0;
            if (r1 > r0) mean_std(a1[0], a2[0], r1 - r0, m, sd);
            stats[o] = m;
            stats[o + 1] = sd;
        }
    }
}

// stats[(r * nsig + sig) * 2] = {mean, std} of the block-causal prefixes: r
// indexes (sequence, block) sets, statistics over the blocks before it.
// one thread per (sequence, signal, block): the block's prefix sums are accumulated in block
// order (the same additions, in the same order, for every block), then its mean and std
__global__ void sel_stats_kernel(SelectParams p, const double* sums, double* stats) {
    const int nsig = 1 + p.n_kv_heads;
    const int id = blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= p.num_seqs * nsig * p.n_sets) return;
    const int b = id % p.n_sets;
    const int sig = (id / p.n_sets) % nsig;
    const int s = id / (p.n_sets * nsig);
    int st, len;
    seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
    double p1 = 0.0, p2 = 0.0;
    for (int bb = 0; bb < b; ++bb) {
        if (bb * p.block_size >= len) break;
        const int64_t o = ((int64_t)(s * p.n_sets + bb) * nsig + sig) * 2;
        p1 = __dadd_rn(p1, sums[o]);
        p2 = __dadd_rn(p2, sums[o + 1]);
    }
    const int64_t o = ((int64_t)(s * p.n_sets + b) * nsig + sig) * 2;
    const int b0 = b * p.block_size;
    double m = 0.0, sd = 1.0;
    if (b0 >= 2 && b0 < len) mean_std(p1, p2, b0, m, sd);
    stats[o] = m;
    stats[o + 1] = sd;
}

// One block per (sequence, signal) when the sets fit in LDS: the block sums staged once,
// then each thread adds the prefix of its sets in block order (the order above: same bits).
constexpr int kStatsLdsSets = 2048;
__global__ __launch_bounds__(256) void sel_stats_lds_kernel(SelectParams p, const double* sums, double* stats) {
    extern __shared__ double bs[];  // [n_sets][2]
    const int nsig = 1 + p.n_kv_heads;
    const int sig = blockIdx.x % nsig, s = blockIdx.x / nsig;
    int st, len;
    seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
    const int nb = min(p.n_sets, ceil_div(len, p.block_size));  // blocks holding tokens
    for (int b = threadIdx.x; b < nb; b += 256) {
        const int64_t o = ((int64_t)(s * p.n_sets + b) * nsig + sig) * 2;
        bs[2 * b] = sums[o];
        bs[2 * b + 1] = sums[o + 1];
    }
    __syncthreads();
    for (int b = threadIdx.x; b < p.n_sets; b += 256) {
        double p1 = 0.0, p2 = 0.0;
        const int e = min(b, nb);
        for (int bb = 0; bb < e; ++bb) {
            p1 = __dadd_rn(p1, bs[2 * bb]);
            p2 = __dadd_rn(p2, bs[2 * bb + 1]);
        }
        const int64_t o = ((int64_t)(s * p.n_sets + b) * nsig + sig) * 2;
        const int b0 = b * p.block_size;
        double m = 0.0, sd = 1.0;
        if (b0 >= 2 && b0 < len) mean_std(p1, p2, b0, m, sd);
        stats[o] = m;
        stats[o + 1] = sd;
    }
}

__device__ __forceinline__ float zscore(float a, double mean, double sd) {
    return (float)__ddiv_rn(__dadd_rn((double)a, -mean), sd);
}

// zscore from a precomputed reciprocal rsd = 1/sd (rounded): q = (a - mean) * rsd is within
// 2^-51 (relative) of the quotient, so when q widened by 2^-48 either way rounds to one fp32
// value, that value is the quotient's rounding; otherwise (q within 2^-48 of an fp32
// rounding midpoint, about once in 2^24 draws) the division decides.  Same result as zscore.
__device__ __forceinline__ float zscore_rcp(float a, double mean, double sd, double rsd) {
    const double d = __dadd_rn((double)a, -mean);
    const double q = __dmul_rn(d, rsd);
    const float lo = (float)__dmul_rn(q, 1.0 - 0x1p-48), hi = (float)__dmul_rn(q, 1.0 + 0x1p-48);
    return lo == hi ? lo : (float)__ddiv_rn(d, sd);
}

__device__ __forceinline__ float mix_score(float alpha, float zv, float zx) {
    float t1 = __fmul_rn(alpha, zv);
    float om = __fsub_rn(1.0f, alpha);
    float t2 = __fmul_rn(om, zx);
    float s = __fadd_rn(t1, t2);
    return s == 0.0f ? 0.0f : s;
}

__device__ __forceinline__ uint32_t order_key(float s) {
    uint32_t u = __float_as_uint(s);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float from_order_key(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// global variant: z per (token, signal), head-major zv for the selection, API outputs
__global__ __launch_bounds__(256) void sel_z_kernel(SelectParams p, const float* nx, const float* nv,
                                                    const double* stats, float* zx, float* zv) {
    const int s = blockIdx.y, sig = blockIdx.z;
    const int nsig = 1 + p.n_kv_heads;
    int st, len;
    seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
    const int t = st + blockIdx.x * 256 + threadIdx.x;
    if (t >= st + len) return;
    const int r = p.stats_scope == DSALT_STATS_PACKED ? 0 : s;
    const double* sr = stats + ((int64_t)r * nsig + sig) * 2;
    if (sig == 0) {
        const float z = zscore(nx[t], sr[0], sr[1]);
        zx[t] = z;
        if (p.z_x) p.z_x[t] = z;
    } else {
        const int g = sig - 1;
        const float z = zscore(nv[(int64_t)g * p.total_len + t], sr[0], sr[1]);
        zv[(int64_t)g * p.total_len + t] = z;
        if (p.z_v) p.z_v[(int64_t)t * p.n_kv_heads + g] = z;
    }
}

// global variant, optional output: per-head scores [T, H]
__global__ __launch_bounds__(256) void sel_scores_kernel(SelectParams p, const float* nx, const float* nv,
                                                         const double* stats) {
    const int s = blockIdx.y;
    const int nsig = 1 + p.n_kv_heads;
    int st, len;
    seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
    const int t = st + blockIdx.x * 256 + threadIdx.x;
    if (t >= st + len) return;
    const int r = p.stats_scope == DSALT_STATS_PACKED ? 0 : s;
    const double* sr = stats + (int64_t)r * nsig * 2;
    const float zxt = zscore(nx[t], sr[0], sr[1]);
    const int rep = p.n_heads / p.n_kv_heads;
    for (int h = 0; h < p.n_heads; ++h) {
        const int g = h / rep;
        const float zvt = zscore(nv[(int64_t)g * p.total_len + t], sr[2 * (g + 1)], sr[2 * (g + 1) + 1]);
        p.scores[(int64_t)t * p.n_heads + h] = mix_score(p.alpha[h], zvt, zxt);
    }
}

// ------------------------------------------------------------------ top-k
constexpr int kSample = 2048;      // candidates sampled for the threshold of large block-causal sets
constexpr int kSampleMin = 8192;   // sets of fewer candidates take the radix path directly
constexpr int kSampleList = 1024;  // sample of a pruned list (its candidates are near the top)

constexpr int kKthCand = 64;       // radix passes of kth_desc stop once the bin holds at most this many keys

// KCAP: the largest set size the block writes (kSetSlots, or kMaxLandmarks for large sets)
template <int NT_, int KCAP>
struct TopkShared {
    static constexpr int NT = NT_;
    uint32_t hist[NT_ / kWave][256];
    unsigned long long border[kBorderCap > kSample ? kBorderCap : kSample];
    int sel[KCAP];
    unsigned long long cand[kKthCand];
    unsigned long long kth;
    uint32_t total;
    int digit;
    uint32_t above;
    uint32_t nsure;
    uint32_t nborder;
    uint32_t ncand;
};

// LDS of kth_desc alone (the global top-k parts and merges)
struct KthShared {
    static constexpr int NT = kSelThreads;
    uint32_t hist[kSelWaves][256];
    unsigned long long cand[kKthCand];
    unsigned long long kth;
    int digit;
    uint32_t above;
    uint32_t ncand;
};

// The r-th largest (0-based) of the n keys a[0..n) in LDS, for the whole block: radix
// passes over 8-bit digits from the top (per-wave LDS histograms, as in the selection
// below) narrow the keys to one digit prefix until at most kKthCand remain; those are
// gathered and the answer is the candidate c with #{> c} <= r < #{>= c} (equal keys all
// qualify and write the same value).  Exact for any keys; replaces a full sort where only
// one order statistic is needed.
template <class Sh>
__device__ unsigned long long kth_desc(Sh& sh, const unsigned long long* a, int n, int r, int tid) {
    const int wave = tid >> 6, lane = tid & 63;
    unsigned long long prefix = 0ull;
    int plen = 0;
    uint32_t rem = (uint32_t)r;
    for (;;) {
        for (int i = tid; i < (Sh::NT / kWave) * 256; i += Sh::NT) (&sh.hist[0][0])[i] = 0u;
        __syncthreads();
        const int shift = 56 - plen;
        for (int i = tid; i < n; i += Sh::NT) {
            const unsigned long long k = a[i];
            if (plen > 0 && (k >> (64 - plen)) != prefix) continue;
            atomicAdd(&sh.hist[wave][(uint32_t)(k >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid < 256) {
            uint32_t c = 0;
            for (int w2 = 0; w2 < (Sh::NT / kWave); ++w2) c += sh.hist[w2][tid];
            sh.hist[0][tid] = c;
        }
        __syncthreads();
        if (wave == 0) {  // the digit whose bin holds rank rem, counting from the top bin
            const uint32_t c0 = sh.hist[0][4 * lane], c1 = sh.hist[0][4 * lane + 1];
            const uint32_t c2 = sh.hist[0][4 * lane + 2], c3 = sh.hist[0][4 * lane + 3];
            const uint32_t loc = c0 + c1 + c2 + c3;
            uint32_t suf = loc;
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t o = __shfl_down(suf, off, 64);
                if (lane + off < 64) suf += o;
            }
            const uint32_t cs[4] = {c0, c1, c2, c3};
            uint32_t above = suf - loc;  // keys in bins >= 4 lane + 4
            for (int b = 3; b >= 0; --b) {
                if (above <= rem && rem < above + cs[b]) {
                    sh.digit = 4 * lane + b;
                    sh.above = above;
                }
                above += cs[b];
            }
        }
        __syncthreads();
        const int d = sh.digit;
        const uint32_t inbin = sh.hist[0][d];
        rem -= sh.above;
        prefix = (prefix << 8) | (unsigned long long)d;
        plen += 8;
        if (plen == 64) return prefix;  // every bit fixed
        if (inbin <= (uint32_t)kKthCand) break;
        __syncthreads();  // hist and digit are rewritten by the next pass
    }
    if (tid == 0) sh.ncand = 0u;
    __syncthreads();
    for (int i = tid; i < n; i += Sh::NT) {
        const unsigned long long k = a[i];
        if ((k >> (64 - plen)) == prefix) sh.cand[atomicAdd(&sh.ncand, 1u)] = k;
    }
    __syncthreads();
    const int m = (int)sh.ncand;
    if (tid < m) {
        const unsigned long long c = sh.cand[tid];
        uint32_t gt = 0u, ge = 0u;
        for (int u = 0; u < m; ++u) {
            const unsigned long long o = sh.cand[u];
            gt += o > c ? 1u : 0u;
            ge += o >= c ? 1u : 0u;
        }
        if (gt <= rem && rem < ge) sh.kth = c;
    }
    __syncthreads();
    const unsigned long long res = sh.kth;
    __syncthreads();
    return res;
}

// out[0..m) = the m distinct values v[0..m) (LDS) in ascending order: each value's rank
// is the number of smaller values (m <= the set size, one thread per value)
template <int NT>
__device__ void rank_sort_asc(const int* v, int m, int32_t* out, int tid) {
    for (int t = tid; t < m; t += NT) {
        const int x = v[t];
        int rank = 0;
        for (int u = 0; u < m; ++u) rank += v[u] < x ? 1 : 0;
        out[rank] = x;
    }
}

// key of candidate j_rel, or 0 when j_rel is not a candidate
struct KeyFn {
    const int32_t* w;
    int total_len;
    int st, rep_g, h;
    float alpha;
    bool block;
    const float *zx, *zv, *nx, *nv;
    const uint32_t* pk;  // packed norms (bf16 inputs), or null
    double mx, sx, mv, sv, rsx, rsv;
    __device__ __forceinline__ unsigned long long operator()(int j) const {
        if (block && pk) return packed(j, pk[(int64_t)rep_g * total_len + st + j]);
        if (j < w[st + j]) return 0ull;
        float zxj, zvj;
        if (zx) {
            zxj = zx[st + j];
            zvj = zv[(int64_t)rep_g * total_len + st + j];
        } else {  // from the norms: zscore_rcp gives zscore's bits
            zxj = zscore_rcp(nx[st + j], mx, sx, rsx);
            zvj = zscore_rcp(nv[(int64_t)rep_g * total_len + st + j], mv, sv, rsv);
        }
        return of_score(j, mix_score(alpha, zvj, zxj));
    }
    // block-causal key of candidate j from its packed norms word
    __device__ __forceinline__ unsigned long long packed(int j, uint32_t wd) const {
        if (wd & kExcluded) return 0ull;
        return of_score(j, mix_score(alpha, zscore_rcp(packed_nv(wd), mv, sv, rsv),
                                     zscore_rcp(packed_nx(wd), mx, sx, rsx)));
    }
    __device__ __forceinline__ static unsigned long long of_score(int j, float sc) {
        return ((unsigned long long)order_key(sc) << 32) | (unsigned long long)(0xffffffffu - (uint32_t)j);
    }
};



// ------------------------------------------------ block-causal pruning
// With bf16 norms, a candidate t that at least k earlier candidates q dominate
// (bf16 |v_q| >= |v_t| and |h_q| >= |h_t|, q < t) is in no set's top k: for alpha in
// [0, 1] the key's score is non-decreasing in both norms (zscore_rcp and mix_score are
// compositions of monotone roundings) and an equal score goes to the lower index, and
// every set holding t holds its earlier candidates.  The dominators are counted from
// below: tokens of earlier kPruneSB-token super-blocks whose bins (monotone in each norm)
// are strictly higher in both.  Survivors are listed per (kv head, sequence) in token
// order; a set scans the prefix of that list instead of its whole prefix.
constexpr int kPruneSB = 4096;  // tokens per super-block
constexpr int kPruneNB = 32;    // bins per norm: quarter standard deviations, clamped
constexpr int kPruneRS = kPruneNB + 1;  // LDS row stride of the bin table
// Pruning pays from this sequence length on (its four launches cost ~45 us; at 32768
// tokens the scans it saves are shorter than that, at 131072 it saves ~190 us)
constexpr int kPruneMinLen = 65536;

struct PruneBins {
    float mx, ix, mv, iv;
    // z-scaled bins of the sequence's longest prefix statistics (any monotone binning
    // is exact; these spread the tokens)
    __device__ PruneBins(const SelectParams& p, const double* stats, int s, int g, int len) {
        const int nsig = 1 + p.n_kv_heads;
        const int b = min(max((len - 1) / p.block_size, 0), p.n_sets - 1);
        const double* sr = stats + (int64_t)(s * p.n_sets + b) * nsig * 2;
        auto inv = [](double sd) { return (sd > 1e-30 && sd < 1e30) ? (float)(4.0 / sd) : 0.f; };
        mx = (float)sr[0];
        ix = inv(sr[1]);
        mv = (float)sr[2 * (g + 1)];
        iv = inv(sr[2 * (g + 1) + 1]);
        if (!(mx == mx) || !(mv == mv)) ix = iv = mx = mv = 0.f;
    }
    // in [0, kPruneNB) for every input (NaN -> 0: still monotone, it arises only at a == m)
    __device__ static int bin(float a, float m, float i) {
        const float z = floorf(__fmul_rn(__fsub_rn(a, m), i));
        if (!(z >= -(float)(kPruneNB / 2))) return 0;
        if (z >= (float)(kPruneNB / 2)) return kPruneNB - 1;
        return (int)z + kPruneNB / 2;
    }
    __device__ int v(uint32_t wd) const { return bin(packed_nv(wd), mv, iv); }
    __device__ int x(uint32_t wd) const { return bin(packed_nx(wd), mx, ix); }
};

// per (super-block, sequence, kv head): 2D histogram of the candidates' bins
__global__ __launch_bounds__(256) void sel_prune_hist_kernel(SelectParams p, const uint32_t* pk, const double* stats,
                                                             uint32_t* hist) {
    __shared__ uint32_t hs[kPruneNB * kPruneNB];
    const int M = blockIdx.x, s = blockIdx.y, g = blockIdx.z, tid = threadIdx.x;
    int st, len;
    seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
    for (int i = tid; i < kPruneNB * kPruneNB; i += 256) hs[i] = 0u;
    __syncthreads();
    const int t0 = M * kPruneSB;
    if (t0 < len) {
        const PruneBins bins(p, stats, s, g, len);
        const uint32_t* w = pk + (int64_t)g * p.total_len + st;
        constexpr int PER = kPruneSB / 256;
        uint32_t wd[PER];  // all of the thread's words in flight before any bin
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int t = t0 + tid + 256 * u;
            wd[u] = t < len ? w[t] : kExcluded;
        }
#pragma unroll
        for (int u = 0; u < PER; ++u)
            if (!(wd[u] & kExcluded)) atomicAdd(&hs[bins.v(wd[u]) * kPruneNB + bins.x(wd[u])], 1u);
    }
    __syncthreads();
    uint32_t* o = hist + (((int64_t)g * p.num_seqs + s) * gridDim.x + M) * (kPruneNB * kPruneNB);
    for (int i = tid; i < kPruneNB * kPruneNB; i += 256) o[i] = hs[i];
}

// per (bin group, sequence, kv head), in place: each bin's count becomes the sum over the
// earlier super-blocks (exclusive prefix along the super-blocks)
__global__ __launch_bounds__(256) void sel_prune_prefix_kernel(SelectParams p, uint32_t* hist, int nsb) {
    constexpr int NB2 = kPruneNB * kPruneNB, U = 8;
    const int bin = blockIdx.x * 256 + threadIdx.x, s = blockIdx.y, g = blockIdx.z;
    uint32_t* h = hist + ((int64_t)g * p.num_seqs + s) * nsb * NB2 + bin;
    uint32_t run = 0u;
    for (int m0 = 0; m0 < nsb; m0 += U) {
        uint32_t c[U];
#pragma unroll
        for (int u = 0; u < U; ++u) c[u] = m0 + u < nsb ? h[(int64_t)(m0 + u) * NB2] : 0u;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (m0 + u < nsb) h[(int64_t)(m0 + u) * NB2] = run;
            run += c[u];
        }
    }
}

// per (super-block, sequence, kv head): keep flag of each token (a candidate whose lower
// bound of earlier dominators is below k) and the super-block's survivor count; hist
// holds the earlier super-blocks' sums by now
__global__ __launch_bounds__(256) void sel_prune_mark_kernel(SelectParams p, const uint32_t* pk, const double* stats,
                                                             const uint32_t* hist, uint8_t* keep, int* cnt) {
    __shared__ uint32_t sf[kPruneNB * kPruneRS];
    __shared__ int wsum[4];
    const int M = blockIdx.x, s = blockIdx.y, g = blockIdx.z, tid = threadIdx.x;
    int st, len;
    seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
    const int64_t gs = (int64_t)g * p.num_seqs + s;
    const uint32_t* h0 = hist + (gs * gridDim.x + M) * (kPruneNB * kPruneNB);  // earlier super-blocks' sums
    for (int i = tid; i < kPruneNB * kPruneNB; i += 256) sf[(i / kPruneNB) * kPruneRS + i % kPruneNB] = h0[i];
    __syncthreads();
    // inclusive suffix sums along x, then along v: sf[a][b] = tokens in bins >= a, >= b
    if (tid < kPruneNB) {
        uint32_t r = 0u;
        for (int b = kPruneNB - 1; b >= 0; --b) r = sf[tid * kPruneRS + b] += r;
    }
    __syncthreads();
    if (tid < kPruneNB) {
        uint32_t r = 0u;
        for (int a = kPruneNB - 1; a >= 0; --a) r = sf[a * kPruneRS + tid] += r;
    }
    __syncthreads();
    const int t0 = M * kPruneSB;
    int n = 0;
    if (t0 < len) {
        const PruneBins bins(p, stats, s, g, len);
        const uint32_t* w = pk + (int64_t)g * p.total_len + st;
        uint8_t* kp = keep + (int64_t)g * p.total_len + st;
        constexpr int PER = kPruneSB / 256;
        uint32_t wd[PER];
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int t = t0 + tid + 256 * u;
            wd[u] = t < len ? w[t] : kExcluded;
        }
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int t = t0 + tid + 256 * u;
            bool k = false;
            if (!(wd[u] & kExcluded)) {
                const int a = bins.v(wd[u]), b = bins.x(wd[u]);
                const uint32_t dom = (a + 1 < kPruneNB && b + 1 < kPruneNB) ? sf[(a + 1) * kPruneRS + b + 1] : 0u;
                k = dom < (uint32_t)p.k_lmk;
            }
            if (t < len) kp[t] = k ? 1 : 0;
            n += k ? 1 : 0;
        }
    }
    for (int off = 32; off >= 1; off >>= 1) n += __shfl_xor(n, off);
    if ((tid & 63) == 0) wsum[tid >> 6] = n;
    __syncthreads();
    if (tid == 0) cnt[gs * gridDim.x + M] = wsum[0] + wsum[1] + wsum[2] + wsum[3];
}

// per (super-block, sequence, kv head): the survivors' in-sequence indices, in token order,
// at the super-block's offset of the (kv head, sequence) list, and at every token of the
// sequence the number of survivors below it (a block of any size starts at any token)
__global__ __launch_bounds__(256) void sel_prune_list_kernel(SelectParams p, const uint8_t* keep, const int* cnt,
                                                             int32_t* list, int32_t* below) {
    __shared__ int wsum[4], woff[4];
    const int M = blockIdx.x, s = blockIdx.y, g = blockIdx.z, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int st, len;
    seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
    const int t0 = M * kPruneSB;
    if (t0 >= len) return;
    const int64_t gs = (int64_t)g * p.num_seqs + s;
    // thread tid takes tokens t0 + 16 tid .. + 15 (flags loaded together): counts, block
    // exclusive scan, writes; the earlier super-blocks' counts are summed by the block
    constexpr int PER = kPruneSB / 256;
    const uint8_t* kp = keep + (int64_t)g * p.total_len + st;
    const int a = t0 + PER * tid;
    uint8_t kb[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) kb[u] = a + u < len ? kp[a + u] : (uint8_t)0;
    int prev = 0;
    for (int m = tid; m < M; m += 256) prev += cnt[gs * gridDim.x + m];
    int c = 0;
#pragma unroll
    for (int u = 0; u < PER; ++u) c += kb[u];
    for (int o = 32; o >= 1; o >>= 1) prev += __shfl_xor(prev, o);
    int inc = c;
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(inc, o);
        if (lane >= o) inc += y;
    }
    if (lane == 63) {
        wsum[wave] = inc;
        woff[wave] = prev;
    }
    __syncthreads();
    int base = woff[0] + woff[1] + woff[2] + woff[3] + inc - c;
    for (int w2 = 0; w2 < wave; ++w2) base += wsum[w2];
    int32_t* lo = list + (int64_t)g * p.total_len + st;
    int32_t* bl = below + (int64_t)g * p.total_len + st;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        if (a + u < len) bl[a + u] = base;  // survivors below token a + u
        if (kb[u]) lo[base++] = a + u;
    }
}

// ------------------------------------------- global variant: parts + merges
constexpr int kPartMax = 2048;   // candidates per part (keys in LDS)
constexpr int kMergeMax = 4096;  // keys per merge block

// key of set (h, sequence s starting at st): z-scores from the norms and the range's
// statistics (mean, std of the hidden-state and value-vector norms; the same values sel_z
// stores)
__device__ __forceinline__ KeyFn global_key_of(const SelectParams& p, const float* nx, const float* nv, int st, int h,
                                               double mx, double sx, double mv, double sv) {
    KeyFn key;
    key.w = p.w;
    key.total_len = p.total_len;
    key.st = st;
    key.h = h;
    key.rep_g = h / (p.n_heads / p.n_kv_heads);
    key.alpha = p.alpha[h];
    key.block = false;
    key.zx = nullptr;
    key.zv = nullptr;
    key.nx = nx;
    key.nv = nv;
    key.pk = nullptr;
    key.mx = mx;
    key.sx = sx;
    key.mv = mv;
    key.sv = sv;
    key.rsx = __ddiv_rn(1.0, key.sx);
    key.rsv = __ddiv_rn(1.0, key.sv);
    return key;
}

// Each global top-k part reads its whole range's norms to compute the statistics itself, which
// saves the sel_sums launch but costs parts x length reads, growing with the square of the
// length: past kPartStatsMaxLen tokens per sequence sel_sums computes them once per range, in the
// same order (selection of H16, 32768 tokens: 50.4 us in the parts, 51.6 through sel_sums;
// 65536 tokens: 89.3 against 84.0 us).
constexpr int kPartStatsMaxLen = 32768;
inline bool parts_own_stats(const SelectParams& p) {
    return !p.z_x && !p.z_v && !p.scores && p.max_seqlen <= kPartStatsMaxLen;
}

__device__ __forceinline__ int global_range(const SelectParams& p, int s) {
    return p.stats_scope == DSALT_STATS_PACKED ? 0 : s;
}

// Statistics of range r for the hidden-state norms (q = 0) and the norms of value head g
// (q = 1), computed by one 1024-thread block in sel_sums' canonical order: thread t sums
// partial t of both signals, then the halving tree, then mean_std.  The global top-k parts
// use it when no caller asked for z or scores, so no sel_sums launch precedes them.
__device__ void pair_stats(const SelectParams& p, const float* nx, const float* nv, int r, int g, double (&mean)[2],
                           double (&sd)[2]) {
    static_assert(kSelThreads == kSumParts, "one partial per thread");
    constexpr int U = 16;
    __shared__ double a1[2][kSumParts], a2[2][kSumParts];
    const int t = threadIdx.x;
    int r0, r1;
    range_of(p, r, r0, r1);
    const float* xs[2] = {nx, nv + (int64_t)g * p.total_len};
    double s1[2] = {0.0, 0.0}, s2[2] = {0.0, 0.0};
    for (int j0 = r0; j0 < r1; j0 += kSumParts * U) {
        const int n = min(kSumParts * U, r1 - j0);
        float xv[2][U];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const __amdgpu_buffer_rsrc_t rs =
                __builtin_amdgcn_make_buffer_rsrc((void*)(xs[q] + j0), (short)0, (int)(n * sizeof(float)), 0x00020000);
#pragma unroll
            for (int m = 0; m < U; ++m)
                xv[q][m] = __builtin_bit_cast(float,
                                              __builtin_amdgcn_raw_buffer_load_b32(rs, (uint32_t)(t + kSumParts * m) * 4u, 0, 0));
        }
#pragma unroll
        for (int m = 0; m < U; ++m)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const double v = (double)xv[q][m];
                s1[q] = __dadd_rn(s1[q], v);
                s2[q] = __dadd_rn(s2[q], __dmul_rn(v, v));
            }
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        a1[q][t] = s1[q];
        a2[q][t] = s2[q];
    }
    __syncthreads();
    for (int off = kSumParts / 2; off >= 1; off >>= 1) {
        if (t < off) {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                a1[q][t] = __dadd_rn(a1[q][t], a1[q][t + off]);
                a2[q][t] = __dadd_rn(a2[q][t], a2[q][t + off]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        mean[u] = 0.0;
        sd[u] = 1.0;
        if (r1 > r0) mean_std(a1[u][0], a2[u][0], r1 - r0, mean[u], sd[u]);
    }
}

// Writes the kpad largest of the n keys a[0..n) (LDS) to o, in no particular order: the keys
// above the kpad-th largest, then copies of it (several only when it is 0, the key of no
// candidate); with n <= kpad, every key and zeros after them.
__device__ void keep_largest(KthShared& sh, const unsigned long long* a, int n, int kpad, unsigned long long* o,
                             int tid) {
    if (n <= kpad) {
        for (int i = tid; i < kpad; i += kSelThreads) o[i] = i < n ? a[i] : 0ull;
        return;
    }
    const unsigned long long kk = kth_desc(sh, a, n, kpad - 1, tid);
    if (tid == 0) sh.ncand = 0u;
    __syncthreads();
    for (int i = tid; i < n; i += kSelThreads)
        if (a[i] > kk) o[atomicAdd(&sh.ncand, 1u)] = a[i];
    __syncthreads();
    for (int i = (int)sh.ncand + tid; i < kpad; i += kSelThreads) o[i] = kk;
}

// part q of set (h, s): candidates [q*psize, (q+1)*psize); writes its kpad best keys
// (zero keys where it has fewer)
constexpr int kSortThreads = kSelThreads;

__global__ __launch_bounds__(kSortThreads) void sel_part_kernel(SelectParams p, const float* nx, const float* nv,
                                                                const double* stats, int psize, int nparts, int kpad,
                                                                unsigned long long* out) {
    __shared__ KthShared sh;
    __shared__ unsigned long long keys[kPartMax];
    const int tid = threadIdx.x;
    const int part = blockIdx.x % nparts, sidx = blockIdx.x / nparts;
    const int s = sidx % p.num_seqs, h = sidx / p.num_seqs;
    int st, len;
    seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
    const int g = h / (p.n_heads / p.n_kv_heads), r = global_range(p, s);
    double mean[2], sd[2];
    if (stats) {  // written by sel_sums
        const int nsig = 1 + p.n_kv_heads;
        const double* sx = stats + (int64_t)r * nsig * 2;
        const double* sv = stats + ((int64_t)r * nsig + 1 + g) * 2;
        mean[0] = sx[0];
        sd[0] = sx[1];
        mean[1] = sv[0];
        sd[1] = sv[1];
    } else {
        pair_stats(p, nx, nv, r, g, mean, sd);
    }
    const KeyFn key = global_key_of(p, nx, nv, st, h, mean[0], sd[0], mean[1], sd[1]);
    const int j0 = part * psize;
    const int n = max(0, min(psize, len - j0));
    for (int i = tid; i < n; i += kSortThreads) keys[i] = key(j0 + i);
    __syncthreads();
    keep_largest(sh, keys, n, kpad, out + ((int64_t)sidx * nparts + part) * kpad, tid);
}

// merge parts [op*G, op*G+G) of set sidx (G*kpad <= kMergeMax keys): with `out`, keep
// the kpad best keys; without, write the set's landmark indices (ascending, -1 padded)
template <int KCAP>
__global__ __launch_bounds__(kSortThreads) void sel_merge_kernel(SelectParams p, const unsigned long long* in,
                                                                 int nin, int G, int kpad, unsigned long long* out,
                                                                 int nout) {
    __shared__ KthShared sh;
    __shared__ unsigned long long keys[kMergeMax];
    __shared__ int sel[KCAP];
    const int tid = threadIdx.x;
    const int op = blockIdx.x % nout, sidx = blockIdx.x / nout;
    const int q0 = op * G, q1 = min(nin, q0 + G);
    const int m = (q1 - q0) * kpad;
    const unsigned long long* src = in + ((int64_t)sidx * nin + q0) * kpad;
    for (int i = tid; i < m; i += kSortThreads) keys[i] = src[i];
    __syncthreads();
    if (out) {
        keep_largest(sh, keys, m, kpad, out + ((int64_t)sidx * nout + op) * kpad, tid);
        return;
    }
    // the K largest keys: those above the K-th largest, and it when it is a candidate's
    // key (keys of candidates are distinct; fewer than K candidates leave it 0)
    const int K = p.k_lmk;
    const unsigned long long kk = kth_desc(sh, keys, m, K - 1, tid);
    if (tid == 0) sh.ncand = 0u;
    __syncthreads();
    for (int i = tid; i < m; i += kSortThreads) {
        const unsigned long long kj = keys[i];
        if (kj > kk || (kj == kk && kk != 0ull))
            sel[atomicAdd(&sh.ncand, 1u)] = (int)(0xffffffffu - (uint32_t)(kj & 0xffffffffull));
    }
    __syncthreads();
    const int nsel = (int)sh.ncand;
    int32_t* o = p.lmk_idx + (int64_t)sidx * K;
    rank_sort_asc<kSelThreads>(sel, nsel, o, tid);
    for (int i = nsel + tid; i < K; i += kSortThreads) o[i] = -1;
}

template <int NT, int KCAP>
__global__ __launch_bounds__(NT) void sel_topk_kernel(SelectParams p, const float* zx, const float* zv,
                                                               const float* nx, const float* nv, const uint32_t* pk,
                                                               const double* stats, int border_cap,
                                                               const int32_t* plist, const int32_t* pbelow) {
    __shared__ TopkShared<NT, KCAP> sh;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // blocks of one (head, sequence) are contiguous in the XCD-swizzled order, so each XCD's
    // L2 holds the norms of few heads; within them later sets, which scan longer prefixes,
    // come first (largest sets first balances the tail)
    const int Lb = xcd_swizzle(blockIdx.x, p.n_heads * p.num_seqs * p.n_sets);
    const int set = p.n_sets - 1 - Lb % p.n_sets;
    const int s = (Lb / p.n_sets) % p.num_seqs;
    const int h = (Lb / p.n_sets) / p.num_seqs;
    const int K = p.k_lmk;
    int32_t* out = p.lmk_idx + (((int64_t)h * p.num_seqs + s) * p.n_sets + set) * K;
    int st, len;
    seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
    const bool block = p.select_mode == DSALT_SELECT_BLOCK;
    int n = len;
    KeyFn key;
    key.w = p.w;
    key.total_len = p.total_len;
    key.st = st;
    key.h = h;
    key.rep_g = h / (p.n_heads / p.n_kv_heads);
    key.alpha = p.alpha[h];
    key.block = block;
    key.zx = zx;
    key.zv = zv;
    key.nx = nx;
    key.nv = nv;
    key.pk = pk;
    if (block) {
        int b0 = set * p.block_size;
        if (b0 < 2 || b0 >= len) {
            for (int i = tid; i < K; i += NT) out[i] = -1;
            return;
        }
        n = b0;
        const int nsig = 1 + p.n_kv_heads;
        const double* sr = stats + (int64_t)(s * p.n_sets + set) * nsig * 2;
        key.mx = sr[0];
        key.sx = sr[1];
        key.mv = sr[2 * (key.rep_g + 1)];
        key.sv = sr[2 * (key.rep_g + 1) + 1];
        key.rsx = __ddiv_rn(1.0, key.sx);
        key.rsv = __ddiv_rn(1.0, key.sv);
    }
    // candidates e < n are the in-sequence indices cand(e): the pruned survivor list's
    // entries below b0 where it applies to this head (alpha in [0, 1]), else 0 .. b0-1
    const int32_t* cl = nullptr;
    if (block && plist && key.alpha >= 0.f && key.alpha <= 1.f) {
        cl = plist + (int64_t)key.rep_g * p.total_len + st;
        n = pbelow[(int64_t)key.rep_g * p.total_len + st + n];  // survivors below b0
    }
    auto cand = [&](int e) { return cl ? cl[e] : e; };
    const int cap = min(border_cap, kBorderCap);

    // Sets of at most kSample candidates: every key in LDS, the K-th largest by kth_desc,
    // the keys at or above it (zero keys, of excluded tokens, never) by ascending index.
    if (n <= kSample && border_cap >= kBorderCap) {
        for (int i = tid; i < n; i += NT) sh.border[i] = key(cand(i));
        __syncthreads();
        const unsigned long long kk = n > K ? kth_desc(sh, sh.border, n, K - 1, tid) : 0ull;
        if (tid == 0) sh.nsure = 0u;
        __syncthreads();
        for (int i = tid; i < n; i += NT) {
            const unsigned long long kj = sh.border[i];
            if (kj != 0ull && kj >= kk) sh.sel[atomicAdd(&sh.nsure, 1u)] = (int)(0xffffffffu - (uint32_t)(kj & 0xffffffffull));
        }
        __syncthreads();
        const int nsel = (int)sh.nsure;
        rank_sort_asc<NT>(sh.sel, nsel, out, tid);
        for (int i = nsel + tid; i < K; i += NT) out[i] = -1;
        return;
    }

    // Large sets: a threshold from an evenly strided sample of the candidates, then one pass
    // that keeps every key at or above it.  When that keeps between K and cap keys, their
    // top K are the set's top K; otherwise (an unrepresentative sample) the radix path
    // below runs from scratch.
    // (a pruned list takes it from kSample candidates: its candidates are all near the top)
    const int ns = cl ? kSampleList : kSample;
    if (n >= (cl ? kSample : kSampleMin) && border_cap >= kBorderCap) {
        for (int i = tid; i < ns; i += NT) sh.border[i] = key(cand((int)((int64_t)i * n / ns)));
        __syncthreads();
        // aim at about 1.6 K + 128 keys above the threshold (the sample's spread leaves
        // fewer than K above it in a small fraction of the sets: those take the radix path)
        const long long want = ((long long)K * 16 / 10 + 128) * ns / n;
        const int rank = (int)min((long long)ns - 1, max(want, 1ll));
        const unsigned long long thr = kth_desc(sh, sh.border, ns, rank, tid);
        if (tid == 0) sh.nborder = 0u;
        __syncthreads();
        if (thr != 0ull) {
            // Screen with the score as one float32 affine form of the two norms,
            // s' = A nv + B nx + C; it differs from the canonical score by less than
            // 16 * 2^-24 * M (M: the magnitudes of the terms), so keys at or above the
            // threshold all pass s' + 2^-19 M >= thr_score and only those get exact keys.
            const float thr_s = from_order_key((uint32_t)(thr >> 32));
            float A = 0.f, B = 0.f, Cv = 0.f, Cx = 0.f;
            if (block) {
                const double al = (double)key.alpha, om = 1.0 - al;
                A = (float)(al / key.sv);
                B = (float)(om / key.sx);
                Cv = (float)(al * key.mv / key.sv);
                Cx = (float)(om * key.mx / key.sx);
            }
            // U candidates per thread per step, all loads issued before any screen
            constexpr int U = 8;
            const float* nvg = nv + (int64_t)key.rep_g * p.total_len + st;
            const float* nxs = nx + st;
            const uint32_t* pkg = pk ? pk + (int64_t)key.rep_g * p.total_len + st : nullptr;
            const float C = -(Cv + Cx), Cm = fabsf(Cv) + fabsf(Cx);
            for (int j0 = tid; j0 < n; j0 += NT * U) {
                float av[U], bv[U];
                uint32_t wds[U];
                if (block) {
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const int j = cand(min(j0 + u * NT, n - 1));
                        if (pkg) {
                            wds[u] = pkg[j];
                            av[u] = packed_nx(wds[u]);
                            bv[u] = packed_nv(wds[u]);
                        } else {
                            wds[u] = 0u;
                            av[u] = nxs[j];
                            bv[u] = nvg[j];
                        }
                    }
                }
                uint32_t pass = 0u;
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int j = j0 + u * NT;
                    bool maybe = j < n;
                    if (pkg) maybe = maybe && !(wds[u] & kExcluded);
                    if (block && maybe) {
                        const float sa = fmaf(A, bv[u], fmaf(B, av[u], C));
                        const float M = fabsf(A * bv[u]) + fabsf(B * av[u]) + Cm;
                        maybe = sa + 0x1p-19f * M >= thr_s;
                    }
                    pass |= maybe ? 1u << u : 0u;
                }
                while (pass) {  // exact keys of the few survivors (one copy of the key code)
                    const int u = __builtin_ctz(pass);
                    pass &= pass - 1u;
                    const int j = j0 + u * NT;
                    uint32_t wd = 0u;
#pragma unroll
                    for (int v = 0; v < U; ++v) wd = v == u ? wds[v] : wd;
                    const unsigned long long kj = pkg ? key.packed(cand(j), wd) : key(cand(j));
                    if (kj >= thr) {
                        const uint32_t slot = atomicAdd(&sh.nborder, 1u);
                        if (slot < (uint32_t)cap) sh.border[slot] = kj;
                    }
                }
            }
        }
        __syncthreads();
        const int nb = (int)sh.nborder;
        if (thr != 0ull && nb >= K && nb <= cap) {
            // the survivors' keys are distinct (one per candidate index): the K at or above
            // the K-th largest are the set, output by ascending index
            const unsigned long long kk = kth_desc(sh, sh.border, nb, K - 1, tid);
            if (tid == 0) sh.nsure = 0u;
            __syncthreads();
            for (int i = tid; i < nb; i += NT) {
                const unsigned long long kj = sh.border[i];
                if (kj >= kk) sh.sel[atomicAdd(&sh.nsure, 1u)] = (int)(0xffffffffu - (uint32_t)(kj & 0xffffffffull));
            }
            __syncthreads();
            rank_sort_asc<NT>(sh.sel, K, out, tid);
            return;
        }
        __syncthreads();
    }

    unsigned long long prefix = 0ull;
    int plen = 0;
    uint32_t k_rem = (uint32_t)K;
    bool all_sure = false;
    for (;;) {
        for (int i = tid; i < (NT / kWave) * 256; i += NT) (&sh.hist[0][0])[i] = 0u;
        __syncthreads();
        const int shift = 56 - plen;
        for (int j = tid; j < n; j += NT) {
            unsigned long long kj = key(cand(j));
            if (kj == 0ull) continue;
            if (plen > 0 && (kj >> (64 - plen)) != prefix) continue;
            atomicAdd(&sh.hist[wave][(uint32_t)(kj >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid < 256) {
            uint32_t c = 0;
            for (int w2 = 0; w2 < (NT / kWave); ++w2) c += sh.hist[w2][tid];
            sh.hist[0][tid] = c;
        }
        __syncthreads();
        if (wave == 0) {
            uint32_t c0 = sh.hist[0][4 * lane], c1 = sh.hist[0][4 * lane + 1];
            uint32_t c2 = sh.hist[0][4 * lane + 2], c3 = sh.hist[0][4 * lane + 3];
            uint32_t loc = c0 + c1 + c2 + c3, suf = loc;
            for (int off = 1; off < 64; off <<= 1) {
                uint32_t o = __shfl_down(suf, off, 64);
                if (lane + off < 64) suf += o;
            }
            uint32_t excl = suf - loc;  // bins >= 4*lane+4
            if (plen == 0 && lane == 0) sh.total = suf;
            uint32_t cs[4] = {c0, c1, c2, c3};
            uint32_t above = excl;
            for (int b = 3; b >= 0; --b) {
                if (above < k_rem && above + cs[b] >= k_rem) {
                    sh.digit = 4 * lane + b;
                    sh.above = above;
                }
                above += cs[b];
            }
        }
        __syncthreads();
        if (plen == 0 && sh.total <= k_rem) {
            all_sure = true;
            break;
        }
        const int d = sh.digit;
        const uint32_t above = sh.above;
        const uint32_t inbin = sh.hist[0][d];
        __syncthreads();
        k_rem -= above;
        prefix = (prefix << 8) | (unsigned long long)d;
        plen += 8;
        if ((int)inbin <= cap || plen == 64) break;
    }

    // collect: sure candidates (prefix above) and the boundary bin
    if (tid == 0) {
        sh.nsure = 0u;
        sh.nborder = 0u;
    }
    __syncthreads();
    for (int e = tid; e < n; e += NT) {
        const int j = cand(e);
        unsigned long long kj = key(j);
        if (kj == 0ull) continue;
        if (all_sure) {
            sh.sel[atomicAdd(&sh.nsure, 1u)] = j;
            continue;
        }
        unsigned long long top = kj >> (64 - plen);
        if (top > prefix) sh.sel[atomicAdd(&sh.nsure, 1u)] = j;
        else if (top == prefix) sh.border[atomicAdd(&sh.nborder, 1u)] = kj;
    }
    __syncthreads();
    if (!all_sure) {
        // the k_rem largest of the boundary bin (distinct candidate keys): at or above its
        // k_rem-th largest
        const int nb = (int)sh.nborder;
        const unsigned long long kk = kth_desc(sh, sh.border, nb, (int)k_rem - 1, tid);
        for (int i = tid; i < nb; i += NT) {
            const unsigned long long kj = sh.border[i];
            if (kj >= kk) sh.sel[atomicAdd(&sh.nsure, 1u)] = (int)(0xffffffffu - (uint32_t)(kj & 0xffffffffull));
        }
        __syncthreads();
    }
    const int nsel = (int)sh.nsure;
    rank_sort_asc<NT>(sh.sel, nsel, out, tid);
    for (int i = nsel + tid; i < K; i += NT) out[i] = -1;
}

// --------------------------------------------------------------- gather
template <typename T>
__global__ __launch_bounds__(256) void gather_kernel(GatherParams p) {
    constexpr int VW = 16 / (int)sizeof(T);
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    const int vpr = p.head_dim / VW;  // vectors per row
    const int64_t nrows = (int64_t)p.n_heads * p.num_seqs * p.n_sets * p.k_lmk;
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= nrows * vpr) return;
    const int c = (int)(id % vpr);
    const int64_t row = id / vpr;
    const int s = (int)((row / ((int64_t)p.n_sets * p.k_lmk)) % p.num_seqs);
    const int h = (int)(row / ((int64_t)p.num_seqs * p.n_sets * p.k_lmk));
    const int g = h / (p.n_heads / p.n_kv_heads);
    const int pos = p.lmk_idx[row];
    int st, len;
    seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
    u4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
    if (pos >= 0 && pos < len) {
        kv = *(const u4*)((const T*)p.k + (int64_t)(st + pos) * p.k_stride_t + (int64_t)g * p.k_stride_h + c * VW);
        vv = *(const u4*)((const T*)p.v + (int64_t)(st + pos) * p.v_stride_t + (int64_t)g * p.v_stride_h + c * VW);
    }
    *(u4*)((T*)p.lmk_k + row * p.head_dim + c * VW) = kv;
    *(u4*)((T*)p.lmk_v + row * p.head_dim + c * VW) = vv;
}

// ------------------------------------------------------------- launchers
namespace {

struct TopkPlan {
    int psize, nparts, kpad, G;
};

// global variant: part size and merge fan-in (the testing hook's border_cap
// shrinks both, to drive many parts and several merge levels)
TopkPlan topk_plan(const SelectParams& p, int border_cap) {
    TopkPlan t;
    t.kpad = 1;
    while (t.kpad < p.k_lmk) t.kpad <<= 1;
    const int full = border_cap >= (1 << 20);
    t.psize = kPartMax;
    if (!full) {
        t.psize = 16;
        while (t.psize < border_cap && t.psize < kPartMax) t.psize <<= 1;
    }
    t.nparts = ceil_div(p.max_seqlen, t.psize);
    t.G = kMergeMax / t.kpad;
    if (!full) t.G = max(2, min(t.G, border_cap));
    return t;
}

int n_ranges(const SelectParams& p) {
    return p.select_mode == DSALT_SELECT_GLOBAL ? (p.stats_scope == DSALT_STATS_PACKED ? 1 : p.num_seqs)
                                                : p.num_seqs * p.n_sets;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

size_t select_workspace(const SelectParams& p) {
    return select_workspace_cap(p, 1 << 30);
}

size_t select_workspace_cap(const SelectParams& p, int border_cap) {
    const int nsig = 1 + p.n_kv_heads;
    const int nranges = n_ranges(p);
    size_t b = 0;
    b += align256(sizeof(float) * (size_t)p.total_len * nsig);           // norms
    b += align256(sizeof(double) * 2 * (size_t)nranges * nsig);          // sums
    b += align256(sizeof(double) * 2 * (size_t)nranges * nsig);          // stats
    if (p.select_mode != DSALT_SELECT_GLOBAL && p.dtype == DSALT_DTYPE_BF16) {
        const size_t tg = (size_t)p.total_len * p.n_kv_heads;
        const size_t gsb = (size_t)p.n_kv_heads * p.num_seqs * ceil_div(p.max_seqlen, kPruneSB);
        b += align256(sizeof(uint32_t) * tg);                            // packed norms
        b += align256(sizeof(uint32_t) * gsb * kPruneNB * kPruneNB);     // pruning histograms
        b += align256(tg) + align256(sizeof(int) * gsb);                 // keep flags, survivor counts
        b += 2 * align256(sizeof(int32_t) * tg);                         // survivor lists, counts below
    }
    if (p.select_mode == DSALT_SELECT_GLOBAL) {
        b += align256(sizeof(float) * (size_t)p.total_len * nsig);       // z
        if (p.k_lmk > 0) {
            const TopkPlan t = topk_plan(p, border_cap);
            b += 2 * align256(sizeof(unsigned long long) * (size_t)p.n_heads * p.num_seqs * t.nparts * t.kpad);
        }
    }
    return b;
}

hipError_t select_launch(const SelectParams& p, void* ws, hipStream_t stream, int border_cap) {
    const int nsig = 1 + p.n_kv_heads;
    const int nranges = n_ranges(p);
    const bool global = p.select_mode == DSALT_SELECT_GLOBAL;
    char* w = (char*)ws;
    float* nx = (float*)w;
    float* nv = nx + p.total_len;
    w += align256(sizeof(float) * (size_t)p.total_len * nsig);
    double* sums = (double*)w;
    w += align256(sizeof(double) * 2 * (size_t)nranges * nsig);
    double* stats = (double*)w;
    w += align256(sizeof(double) * 2 * (size_t)nranges * nsig);
    uint32_t* pk = nullptr;
    uint32_t* phist = nullptr;
    uint8_t* pkeep = nullptr;
    int* pcnt = nullptr;
    int32_t* plist = nullptr;
    int32_t* pbelow = nullptr;
    const int nsb = ceil_div(p.max_seqlen, kPruneSB);
    if (!global && p.dtype == DSALT_DTYPE_BF16) {
        const size_t tg = (size_t)p.total_len * p.n_kv_heads;
        const size_t gsb = (size_t)p.n_kv_heads * p.num_seqs * nsb;
        pk = (uint32_t*)w;
        w += align256(sizeof(uint32_t) * tg);
        phist = (uint32_t*)w;
        w += align256(sizeof(uint32_t) * gsb * kPruneNB * kPruneNB);
        pkeep = (uint8_t*)w;
        w += align256(tg);
        pcnt = (int*)w;
        w += align256(sizeof(int) * gsb);
        plist = (int32_t*)w;
        w += align256(sizeof(int32_t) * tg);
        pbelow = (int32_t*)w;
        w += align256(sizeof(int32_t) * tg);
    }
    float* zx = nullptr;
    float* zv = nullptr;
    if (global) {
        zx = (float*)w;
        zv = zx + p.total_len;
        w += align256(sizeof(float) * (size_t)p.total_len * nsig);
    }
    if (p.total_len > 0) {
        const int blocks = ceil_div(p.total_len, kNormTB);
        const int plan_blocks = p.plan_perm ? ceil_div(p.num_seqs * p.n_tiles, 4) : 0;
        const dim3 grid(blocks + plan_blocks);
        const size_t shm = sizeof(double) * kNormTB * nsig;
        if (p.dtype == DSALT_DTYPE_BF16)
            DSALT_LAUNCH("sel_norms", sel_norms_kernel<bf16>, grid, dim3(256), shm, stream, p, nx, nv, pk, blocks);
        else if (p.dtype == DSALT_DTYPE_F16)
            DSALT_LAUNCH("sel_norms", sel_norms_kernel<f16>, grid, dim3(256), shm, stream, p, nx, nv, nullptr, blocks);
        else
            DSALT_LAUNCH("sel_norms", sel_norms_kernel<float>, grid, dim3(256), shm, stream, p, nx, nv, nullptr, blocks);
        // the global top-k parts compute the statistics they need themselves (the same order)
        // unless z or scores are written for the caller, or the sequences are long
        const bool global_parts_only = global && parts_own_stats(p);
        if (!global_parts_only)
            DSALT_LAUNCH("sel_sums", sel_sums_kernel, dim3(nranges, nsig), dim3(256), 0, stream, p, nx, nv, sums,
                         global ? stats : nullptr);
        if (global) {
            // z-scores are stored only for the caller (the selection recomputes them from the norms)
            if (p.z_x || p.z_v)
                DSALT_LAUNCH("sel_z", sel_z_kernel, dim3(ceil_div(p.max_seqlen, 256), p.num_seqs, nsig), dim3(256), 0,
                             stream, p, nx, nv, stats, zx, zv);
            if (p.scores)
                DSALT_LAUNCH("sel_scores", sel_scores_kernel, dim3(ceil_div(p.max_seqlen, 256), p.num_seqs),
                             dim3(256), 0, stream, p, nx, nv, stats);
        } else {
            if (p.n_sets <= kStatsLdsSets)
                DSALT_LAUNCH("sel_stats", sel_stats_lds_kernel, dim3(p.num_seqs * nsig), dim3(256),
                             sizeof(double) * 2 * p.n_sets, stream, p, sums, stats);
            else
                DSALT_LAUNCH("sel_stats", sel_stats_kernel, dim3(ceil_div(p.num_seqs * nsig * p.n_sets, 64)), dim3(64),
                             0, stream, p, sums, stats);
        }
    }
    const int nsets_total = p.n_heads * p.num_seqs * p.n_sets;
    if (nsets_total == 0 || p.k_lmk == 0) return hipGetLastError();
    if (!global) {
        const bool prune = pk && p.total_len > 0 && nsb > 1 &&
                           (p.max_seqlen >= kPruneMinLen || border_cap == DSALT_SELECT_FORCE_PRUNE);
        if (prune) {
            const dim3 pg(nsb, p.num_seqs, p.n_kv_heads);
            DSALT_LAUNCH("sel_prune_hist", sel_prune_hist_kernel, pg, dim3(256), 0, stream, p, pk, stats, phist);
            DSALT_LAUNCH("sel_prune_prefix", sel_prune_prefix_kernel, dim3(kPruneNB * kPruneNB / 256, p.num_seqs,
                         p.n_kv_heads), dim3(256), 0, stream, p, phist, nsb);
            DSALT_LAUNCH("sel_prune_mark", sel_prune_mark_kernel, pg, dim3(256), 0, stream, p, pk, stats, phist, pkeep,
                         pcnt);
            DSALT_LAUNCH("sel_prune_list", sel_prune_list_kernel, pg, dim3(256), 0, stream, p, pkeep, pcnt, plist,
                         pbelow);
        }
        // sets of more than kSetSlots take instantiations with a larger output buffer in LDS
        const bool lk = p.k_lmk > kSetSlots;
        if (prune && lk)
            DSALT_LAUNCH("sel_topk", (sel_topk_kernel<kTopkThreadsPruned, kMaxLandmarks>), dim3(nsets_total),
                         dim3(kTopkThreadsPruned), 0, stream, p, zx, zv, nx, nv, pk, stats, border_cap, plist, pbelow);
        else if (prune)
            DSALT_LAUNCH("sel_topk", (sel_topk_kernel<kTopkThreadsPruned, kSetSlots>), dim3(nsets_total),
                         dim3(kTopkThreadsPruned), 0, stream, p, zx, zv, nx, nv, pk, stats, border_cap, plist, pbelow);
        else if (lk)
            DSALT_LAUNCH("sel_topk", (sel_topk_kernel<kTopkThreads, kMaxLandmarks>), dim3(nsets_total),
                         dim3(kTopkThreads), 0, stream, p, zx, zv, nx, nv, pk, stats, border_cap, nullptr, nullptr);
        else
            DSALT_LAUNCH("sel_topk", (sel_topk_kernel<kTopkThreads, kSetSlots>), dim3(nsets_total), dim3(kTopkThreads),
                         0, stream, p, zx, zv, nx, nv, pk, stats, border_cap, nullptr, nullptr);
        return hipGetLastError();
    }
    const TopkPlan t = topk_plan(p, border_cap);
    const size_t kb = align256(sizeof(unsigned long long) * (size_t)nsets_total * t.nparts * t.kpad);
    unsigned long long* ka = (unsigned long long*)w;
    unsigned long long* kb2 = (unsigned long long*)(w + kb);
    const bool stats_written = !parts_own_stats(p);
    DSALT_LAUNCH("sel_part", sel_part_kernel, dim3(nsets_total * t.nparts), dim3(kSortThreads), 0, stream, p, nx, nv,
                 stats_written ? stats : nullptr, t.psize, t.nparts, t.kpad, ka);
    // keys per merge block <= kMergeMax
    auto merge = [&](int nin, unsigned long long* out, int nout) {
        if (p.k_lmk > kSetSlots)
            DSALT_LAUNCH("sel_merge", sel_merge_kernel<kMaxLandmarks>, dim3(nsets_total * nout), dim3(kSortThreads), 0,
                         stream, p, ka, nin, t.G, t.kpad, out, nout);
        else
            DSALT_LAUNCH("sel_merge", sel_merge_kernel<kSetSlots>, dim3(nsets_total * nout), dim3(kSortThreads), 0,
                         stream, p, ka, nin, t.G, t.kpad, out, nout);
    };
    int nin = t.nparts;
    while (nin > t.G) {
        const int nout = ceil_div(nin, t.G);
        merge(nin, kb2, nout);
        unsigned long long* tmp = ka;
        ka = kb2;
        kb2 = tmp;
        nin = nout;
    }
    merge(nin, nullptr, 1);
    return hipGetLastError();
}

hipError_t gather_launch(const GatherParams& p, hipStream_t stream) {
    const int vw = p.dtype == DSALT_DTYPE_F32 ? 4 : 8;
    int64_t n = (int64_t)p.n_heads * p.num_seqs * p.n_sets * p.k_lmk * (p.head_dim / vw);
    if (n == 0) return hipSuccess;
    dim3 grid((unsigned)((n + 255) / 256));
    if (p.dtype == DSALT_DTYPE_BF16)
        DSALT_LAUNCH("gather", gather_kernel<bf16>, grid, dim3(256), 0, stream, p);
    else if (p.dtype == DSALT_DTYPE_F16)
        DSALT_LAUNCH("gather", gather_kernel<f16>, grid, dim3(256), 0, stream, p);
    else
        DSALT_LAUNCH("gather", gather_kernel<float>, grid, dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace dsalt
