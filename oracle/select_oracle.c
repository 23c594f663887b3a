/*
 * CPU restatement of DSALT landmark selection - TEST INFRASTRUCTURE ONLY.
 *
 * This file is the oracle that the HIP selection kernels are checked against.
 * Nothing in the product links it; only tests/, the smoke check and the CPU
 * baseline of bench.py load it.
 *
 * Reference algorithm restated here:
 *   hybrid_scores_per_head   dsalt/kernels/landmark_tokens_ker.py:19-61
 *     norms of x and of x W_V^T per kv head (:47,:52), z-score with unbiased std
 *     clamped at 1e-6 (:48,:53-55), GQA repeat (:56-58), s = a z_v + (1-a) z_x (:60)
 *   _compute_landmark_indices dsalt/kernels/selectors.py:75-134
 *     exclusion j_rel < w(j) (:105-107), per (head, seq) top-k (:120,:129),
 *     -1 where fewer than k candidates (:121-123,:130-133)
 *   block-causal _select      results/causal_landmark_check.py:82-113
 *     fp64 prefix sums (:82-85), mean/unbiased std at n (:88-92),
 *     z in fp64 then fp32 (:104-105), n < 2 -> no landmarks (:100-101)
 *
 * Canonical arithmetic (the reference leaves reduction order and tie order to
 * torch; this restatement fixes both, and the GPU kernels follow it exactly):
 *   - row norm: fp64 sum of squares, lane-strided over 16-byte chunks with
 *     G = min(64, pow2ceil(n_chunks)) lanes, then an xor butterfly
 *     (offsets G/2 .. 1); sqrt by canon_sqrt64 (Heron iteration, IEEE ops
 *     only); rounded to fp32, then to the input dtype (torch computes the norm
 *     of a bf16 tensor in bf16).
 *   - statistics: fp64 sums over a range by 1024 strided partial sums (partial
 *     t adds elements r0 + t + 1024 m in increasing m) followed by a halving
 *     tree (offsets 512 .. 1); mean = S1/n, var = (S2 - (n*mean)*mean)/max(n-1,1)
 *     clamped at 0, std = max(canon_sqrt64(var), 1e-6).  Block-causal prefix
 *     sums add whole-block sums in block order.
 *   - z = fp32((a - mean) / std) computed in fp64, for both variants.
 *   - score = fp32(fp32(alpha*z_v) + fp32(fp32(1-alpha)*z_x)), no fused
 *     multiply-add; -0 is replaced by +0.
 *   - top-k by (score descending, index ascending); output ascending indices.
 * Build with -ffp-contract=off.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../include/dsalt_amd.h"

/* ------------------------------------------------------------------ numbers */
static float bf16_bits_to_float(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float f16_bits_to_float(uint16_t h) {
    int sign = h >> 15, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    double v;
    if (e == 0) v = ldexp((double)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexp((double)(m | 0x400), e - 25);
    return (float)(sign ? -v : v);
}

static double load_elem(const void* base, int dtype, int64_t i) {
    if (dtype == DSALT_DTYPE_F32) return (double)((const float*)base)[i];
    uint16_t b = ((const uint16_t*)base)[i];
    return dtype == DSALT_DTYPE_BF16 ? (double)bf16_bits_to_float(b) : (double)f16_bits_to_float(b);
}

/* round-to-nearest-even of a finite fp32 value to bf16, returned as fp32 */
static float round_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    memcpy(&f, &u, 4);
    return f;
}

/* round-to-nearest-even of a finite non-negative fp32 value to fp16, as fp32 */
static float round_f16(float f) {
    if (f == 0.0f) return f;
    double a = fabs((double)f);
    int e;
    frexp(a, &e);           /* a = m * 2^e, m in [0.5,1) -> unit exponent e-1 */
    int ue = e - 1;
    if (ue < -14) ue = -14; /* subnormal quantum 2^-24 */
    double q = ldexp(1.0, ue - 10);
    double r = nearbyint(a / q) * q; /* default rounding mode: nearest-even */
    if (r > 65504.0) r = INFINITY;
    return (float)(f < 0 ? -r : r);
}

static float round_to_dtype(float f, int dtype) {
    if (dtype == DSALT_DTYPE_BF16) return round_bf16(f);
    if (dtype == DSALT_DTYPE_F16) return round_f16(f);
    return f;
}

/* Heron iteration from an exponent-halving seed; uses only IEEE-exact ops so
 * every conforming platform produces the same bits. */
double oracle_canon_sqrt64(double x) {
    if (!(x > 0.0)) return 0.0;
    uint64_t b;
    memcpy(&b, &x, 8);
    b = (b >> 1) + 0x1ff8000000000000ull;
    double y;
    memcpy(&y, &b, 8);
    for (int it = 0; it < 6; ++it) y = 0.5 * (y + x / y);
    return y;
}

/* ------------------------------------------------------------------- norms */
double oracle_row_sumsq(const void* row, int dtype, int n) {
    /* 16-byte vectors of vw elements; a row that is not whole vectors is summed as if
       zero-padded to them (the zeros add exactly nothing: the operator pads such rows) */
    int vw = dtype == DSALT_DTYPE_F32 ? 4 : 8;
    int nch = (n + vw - 1) / vw;
    int g = 1;
    while (g < nch && g < 64) g <<= 1;
    double a[64], b[64];
    for (int l = 0; l < g; ++l) {
        double acc = 0.0;
        for (int ch = l; ch < nch; ch += g)
            for (int e = 0; e < vw; ++e) {
                int64_t i = (int64_t)ch * vw + e;
                double x = i < n ? load_elem(row, dtype, i) : 0.0;
                acc = acc + x * x;
            }
        a[l] = acc;
    }
    for (int off = g / 2; off >= 1; off >>= 1) {
        for (int l = 0; l < g; ++l) b[l] = a[l] + a[l ^ off];
        memcpy(a, b, sizeof(double) * g);
    }
    return a[0];
}

float oracle_row_norm(const void* row, int dtype, int n) {
    double ss = oracle_row_sumsq(row, dtype, n);
    return round_to_dtype((float)oracle_canon_sqrt64(ss), dtype);
}

static size_t esize(int dtype) { return dtype == DSALT_DTYPE_F32 ? 4 : 2; }

/* nx[T], nv[n_kv][T] */
void oracle_norms(const dsalt_select_args* a, float* nx, float* nv) {
    const dsalt_problem* p = &a->p;
    size_t es = esize(p->dtype);
    for (int64_t t = 0; t < p->total_len; ++t) {
        const char* hr = (const char*)a->h + (size_t)(t * a->h_stride_t) * es;
        nx[t] = oracle_row_norm(hr, p->dtype, a->hidden);
        for (int g = 0; g < p->n_kv_heads; ++g) {
            const char* vr = (const char*)a->v + (size_t)(t * a->v_stride_t + g * a->v_stride_h) * es;
            nv[(int64_t)g * p->total_len + t] = oracle_row_norm(vr, p->dtype, p->head_dim);
        }
    }
}

/* -------------------------------------------------------------- statistics */
#define SUM_PARTS 1024
void oracle_range_sums(const float* x, int64_t r0, int64_t r1, double* s1_out, double* s2_out) {
    static _Thread_local double a1[SUM_PARTS], a2[SUM_PARTS];
    for (int t = 0; t < SUM_PARTS; ++t) {
        double s1 = 0.0, s2 = 0.0;
        for (int64_t j = r0 + t; j < r1; j += SUM_PARTS) {
            double v = (double)x[j];
            s1 = s1 + v;
            s2 = s2 + v * v;
        }
        a1[t] = s1;
        a2[t] = s2;
    }
    for (int off = SUM_PARTS / 2; off >= 1; off >>= 1)
        for (int t = 0; t < off; ++t) {
            a1[t] = a1[t] + a1[t + off];
            a2[t] = a2[t] + a2[t + off];
        }
    *s1_out = a1[0];
    *s2_out = a2[0];
}

void oracle_mean_std(double s1, double s2, int64_t n, double* mean, double* sd) {
    double m = s1 / (double)n;
    double den = (double)(n - 1 > 1 ? n - 1 : 1);
    double var = (s2 - ((double)n * m) * m) / den;
    if (!(var > 0.0)) var = 0.0;
    double s = oracle_canon_sqrt64(var);
    if (s < 1e-6) s = 1e-6;
    *mean = m;
    *sd = s;
}

static float zscore(float a, double mean, double sd) {
    return (float)(((double)a - mean) / sd);
}

static float mix_score(float alpha, float zv, float zx) {
    float t1 = alpha * zv;
    float om = 1.0f - alpha;
    float t2 = om * zx;
    float s = t1 + t2;
    if (s == 0.0f) s = 0.0f;
    return s;
}

static uint32_t order_key(float s) {
    uint32_t u;
    memcpy(&u, &s, 4);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* ------------------------------------------------------------------ top-k */
typedef struct { uint32_t key; int32_t idx; } cand_t;

static int cmp_cand(const void* x, const void* y) {
    const cand_t* a = (const cand_t*)x;
    const cand_t* b = (const cand_t*)y;
    if (a->key != b->key) return a->key > b->key ? -1 : 1;
    return a->idx < b->idx ? -1 : (a->idx > b->idx);
}

static int cmp_int(const void* x, const void* y) {
    int a = *(const int*)x, b = *(const int*)y;
    return (a > b) - (a < b);
}

static void topk_write(cand_t* c, int n, int k, int32_t* out) {
    qsort(c, (size_t)n, sizeof(cand_t), cmp_cand);
    int m = n < k ? n : k;
    int* sel = (int*)malloc(sizeof(int) * (size_t)(m > 0 ? m : 1));
    for (int i = 0; i < m; ++i) sel[i] = c[i].idx;
    qsort(sel, (size_t)m, sizeof(int), cmp_int);
    for (int i = 0; i < k; ++i) out[i] = i < m ? sel[i] : -1;
    free(sel);
}

int oracle_n_sets(const dsalt_problem* p) {
    if (p->select_mode == DSALT_SELECT_GLOBAL) return 1;
    return (p->max_seqlen + p->block_size - 1) / p->block_size;
}

/* Full selection with host pointers; same argument struct as dsalt_select. */
int oracle_select(const dsalt_select_args* a) {
    const dsalt_problem* p = &a->p;
    int T = p->total_len, S = p->num_seqs, H = p->n_heads, G = p->n_kv_heads, K = p->k_lmk;
    int rep = H / G;
    int nsets = oracle_n_sets(p);
    float* nx = (float*)malloc(sizeof(float) * (size_t)T);
    float* nv = (float*)malloc(sizeof(float) * (size_t)T * (size_t)G);
    oracle_norms(a, nx, nv);
    const int32_t* cu = a->cu_seqlens;
    int maxlen = 1;
    for (int s = 0; s < S; ++s)
        if (cu[s + 1] - cu[s] > maxlen) maxlen = cu[s + 1] - cu[s];
    cand_t* cand = (cand_t*)malloc(sizeof(cand_t) * (size_t)maxlen);

    if (p->select_mode == DSALT_SELECT_GLOBAL) {
        float* zx = (float*)malloc(sizeof(float) * (size_t)T);
        float* zv = (float*)malloc(sizeof(float) * (size_t)T * (size_t)G);
        int nscope = a->stats_scope == DSALT_STATS_PACKED ? 1 : S;
        for (int r = 0; r < nscope; ++r) {
            int64_t r0 = a->stats_scope == DSALT_STATS_PACKED ? 0 : cu[r];
            int64_t r1 = a->stats_scope == DSALT_STATS_PACKED ? T : cu[r + 1];
            if (r1 <= r0) continue;
            double s1, s2, m, sd;
            oracle_range_sums(nx, r0, r1, &s1, &s2);
            oracle_mean_std(s1, s2, r1 - r0, &m, &sd);
            for (int64_t t = r0; t < r1; ++t) zx[t] = zscore(nx[t], m, sd);
            for (int g = 0; g < G; ++g) {
                const float* col = nv + (int64_t)g * T;
                oracle_range_sums(col, r0, r1, &s1, &s2);
                oracle_mean_std(s1, s2, r1 - r0, &m, &sd);
                for (int64_t t = r0; t < r1; ++t) zv[(int64_t)g * T + t] = zscore(col[t], m, sd);
            }
        }
        for (int h = 0; h < H; ++h) {
            int g = h / rep;
            float al = a->alpha[h];
            for (int s = 0; s < S; ++s) {
                int st = cu[s], len = cu[s + 1] - cu[s], n = 0;
                for (int j = 0; j < len; ++j) {
                    if (j < a->w[st + j]) continue; /* covered by its own window */
                    float sc = mix_score(al, zv[(int64_t)g * T + st + j], zx[st + j]);
                    cand[n].key = order_key(sc);
                    cand[n].idx = j;
                    ++n;
                }
                topk_write(cand, n, K, a->lmk_idx + ((int64_t)h * S + s) * K);
            }
        }
        if (a->z_x) memcpy(a->z_x, zx, sizeof(float) * (size_t)T);
        if (a->z_v)
            for (int64_t t = 0; t < T; ++t)
                for (int g = 0; g < G; ++g) a->z_v[t * G + g] = zv[(int64_t)g * T + t];
        if (a->scores)
            for (int64_t t = 0; t < T; ++t)
                for (int h = 0; h < H; ++h)
                    a->scores[t * H + h] = mix_score(a->alpha[h], zv[(int64_t)(h / rep) * T + t], zx[t]);
        free(zx);
        free(zv);
    } else {
        int B = p->block_size;
        for (int s = 0; s < S; ++s) {
            int st = cu[s], len = cu[s + 1] - cu[s];
            /* running fp64 prefix sums over whole blocks, per signal */
            double* p1 = (double*)calloc((size_t)(G + 1), sizeof(double));
            double* p2 = (double*)calloc((size_t)(G + 1), sizeof(double));
            for (int b = 0; b < nsets; ++b) {
                int b0 = b * B;
                for (int h = 0; h < H; ++h) {
                    int32_t* out = a->lmk_idx + (((int64_t)h * S + s) * nsets + b) * K;
                    if (b0 < 2 || b0 >= len) {
                        for (int i = 0; i < K; ++i) out[i] = -1;
                        continue;
                    }
                    int g = h / rep;
                    double mx, sx, mv, sv;
                    oracle_mean_std(p1[0], p2[0], b0, &mx, &sx);
                    oracle_mean_std(p1[1 + g], p2[1 + g], b0, &mv, &sv);
                    float al = a->alpha[h];
                    int n = 0;
                    for (int j = 0; j < b0; ++j) {
                        if (j < a->w[st + j]) continue;
                        float zxj = zscore(nx[st + j], mx, sx);
                        float zvj = zscore(nv[(int64_t)g * T + st + j], mv, sv);
                        cand[n].key = order_key(mix_score(al, zvj, zxj));
                        cand[n].idx = j;
                        ++n;
                    }
                    topk_write(cand, n, K, out);
                }
                /* add block b to the prefix */
                if (b0 < len) {
                    int64_t r0 = st + b0, r1 = st + (b0 + B < len ? b0 + B : len);
                    double c1, c2;
                    oracle_range_sums(nx, r0, r1, &c1, &c2);
                    p1[0] = p1[0] + c1;
                    p2[0] = p2[0] + c2;
                    for (int g = 0; g < G; ++g) {
                        oracle_range_sums(nv + (int64_t)g * T, r0, r1, &c1, &c2);
                        p1[1 + g] = p1[1 + g] + c1;
                        p2[1 + g] = p2[1 + g] + c2;
                    }
                }
            }
            free(p1);
            free(p2);
        }
    }
    free(cand);
    free(nx);
    free(nv);
    return 0;
}

/* Flat-argument entry for ctypes callers (host pointers). h/v hold raw element
 * bits of `dtype`; strides in elements.  Outputs may be NULL except lmk_idx. */
int oracle_select_flat(int total_len, int num_seqs, int max_seqlen, int n_heads, int n_kv_heads,
                       int head_dim, int k_lmk, int select_mode, int block_size, int dtype,
                       int hidden, int stats_scope,
                       const void* h, int64_t h_stride_t,
                       const void* v, int64_t v_stride_t, int64_t v_stride_h,
                       const float* alpha, const int32_t* w, const int32_t* cu_seqlens,
                       int32_t* lmk_idx, float* z_x, float* z_v, float* scores) {
    dsalt_select_args a;
    memset(&a, 0, sizeof(a));
    a.p.total_len = total_len;
    a.p.num_seqs = num_seqs;
    a.p.max_seqlen = max_seqlen;
    a.p.n_heads = n_heads;
    a.p.n_kv_heads = n_kv_heads;
    a.p.head_dim = head_dim;
    a.p.k_lmk = k_lmk;
    a.p.select_mode = select_mode;
    a.p.block_size = block_size;
    a.p.dtype = dtype;
    a.hidden = hidden;
    a.stats_scope = stats_scope;
    a.h = h;
    a.h_stride_t = h_stride_t;
    a.v = v;
    a.v_stride_t = v_stride_t;
    a.v_stride_h = v_stride_h;
    a.alpha = alpha;
    a.w = w;
    a.cu_seqlens = cu_seqlens;
    a.lmk_idx = lmk_idx;
    a.z_x = z_x;
    a.z_v = z_v;
    a.scores = scores;
    return oracle_select(&a);
}

/* Row norms only (nx [T], nv [n_kv][T]) for the norm-level checks. */
void oracle_norms_flat(int total_len, int n_kv_heads, int head_dim, int dtype, int hidden,
                       const void* h, int64_t h_stride_t,
                       const void* v, int64_t v_stride_t, int64_t v_stride_h,
                       float* nx, float* nv) {
    dsalt_select_args a;
    memset(&a, 0, sizeof(a));
    a.p.total_len = total_len;
    a.p.n_kv_heads = n_kv_heads;
    a.p.head_dim = head_dim;
    a.p.dtype = dtype;
    a.hidden = hidden;
    a.h = h;
    a.h_stride_t = h_stride_t;
    a.v = v;
    a.v_stride_t = v_stride_t;
    a.v_stride_h = v_stride_h;
    oracle_norms(&a, nx, nv);
}
