// DSALT attention backward for gfx950, deterministic (no float atomics).
//
// Replaces _dsalt_bwd_preprocess and _dsalt_bwd_kernel
// (dsalt/kernels/dsalt_triton_bwd.py:17-216), which accumulate dK/dV with
// atomic_add.  Here every output element has exactly one writer:
//   bwd_rowinfo  per sequence: min/max window start of each 16-row tile and
//                the largest window (bounds of the key-parallel sweep).
//   bwd_delta    delta = rowsum(O * dO) from the stored O (:44).
//   bwd_dq       query-parallel, like the forward: dQ = scale * dS K over the
//                band and the landmark slots (:148,:196).
//   bwd_dkdv     key-parallel over the band: 16 keys per wave, query rows
//                staged in LDS; dV = P^T dO, dK = scale * dS^T Q (:198-199).
//   bwd_lmk      landmark slots x row chunks: partial dK/dV/d_bias of each
//                (head, sequence, slot) over 1024 rows (:150-155).
//   bwd_lmk_sum  sums the partials in chunk order and adds them into the dK/dV
//                rows at the landmark positions.
// P = exp(q.k * scale + bias - LSE) is recomputed in base 2 from the forward's
// LSE; dS = P (dP - delta), dP = dO V^T.
#include "attn.h"
#include "tiles.h"
#include "timing.h"

namespace dsalt {

constexpr float kLog2eB = 1.4426950408889634f;
constexpr int kRowChunk = 1024;

template <typename T, int D> struct BwdShape;
template <> struct BwdShape<bf16, 64> { static constexpr int BN = 64, BQ = 32, NBUF = 2; };
template <> struct BwdShape<bf16, 128> { static constexpr int BN = 32, BQ = 32, NBUF = 1; };
template <> struct BwdShape<f16, 64> { static constexpr int BN = 64, BQ = 32, NBUF = 2; };
template <> struct BwdShape<f16, 128> { static constexpr int BN = 32, BQ = 32, NBUF = 1; };
template <> struct BwdShape<float, 64> { static constexpr int BN = 32, BQ = 16, NBUF = 2; };
template <> struct BwdShape<float, 128> { static constexpr int BN = 16, BQ = 16, NBUF = 1; };

__device__ __forceinline__ int seq_start_of(const AttnParams& p, int s) {
    int st, len;
    seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
    return st;
}
__device__ __forceinline__ int seq_len_of(const AttnParams& p, int s) {
    int st, len;
    seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
    return len;
}

__device__ __forceinline__ int lower_bound_i(const int* a, int n, int x) {
    int lo = 0, hi = n;
    while (lo < hi) {
        int mid = (lo + hi) >> 1;
        if (a[mid] < x) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// ------------------------------------------------------------------ prep
__global__ __launch_bounds__(256) void bwd_rowinfo_kernel(AttnParams p) {
    __shared__ int wm[256];
    const int s = blockIdx.x, tid = threadIdx.x;
    const int st = seq_start_of(p, s), len = seq_len_of(p, s);
    const int nt16 = ceil_div(p.max_seqlen, 16);
    int wmax = 1;
    for (int t16 = tid; t16 < nt16; t16 += 256) {
        int mn = 0x7fffffff, mx = -1;
        for (int r = 0; r < 16; ++r) {
            int i = t16 * 16 + r;
            if (i >= len) {
                mx = 0x7fffffff;  // padding rows: never "fully valid"
                continue;
            }
            int wi = max(p.w[st + i], 1);
            wmax = max(wmax, min(wi, len));
            int lo = max(i - wi + 1, 0);
            mn = min(mn, lo);
            mx = max(mx, lo);
        }
        p.tile_minlo[((int64_t)s * nt16 + t16) * 2] = mn;
        p.tile_minlo[((int64_t)s * nt16 + t16) * 2 + 1] = mx;
    }
    wm[tid] = wmax;
    __syncthreads();
    for (int off = 128; off >= 1; off >>= 1) {
        if (tid < off) wm[tid] = max(wm[tid], wm[tid + off]);
        __syncthreads();
    }
    if (tid == 0) p.seq_wmax[s] = wm[0];
}

template <typename T, int D>
__global__ __launch_bounds__(256) void bwd_delta_kernel(AttnParams p) {
    constexpr int VW = 16 / (int)sizeof(T);
    constexpr int LPR = D / VW;  // lanes per row
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    const int64_t nrows = (int64_t)p.total_len * p.n_heads;
    const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) / LPR;
    const int sub = threadIdx.x % LPR;
    float acc = 0.f;
    if (row < nrows) {
        const int64_t t = row / p.n_heads;
        const int h = (int)(row % p.n_heads);
        u4 a = *(const u4*)((const T*)p.o + t * p.o_st + (int64_t)h * p.o_sh + sub * VW);
        u4 b = *(const u4*)((const T*)p.dout + t * p.do_st + (int64_t)h * p.do_sh + sub * VW);
        const T* ea = (const T*)&a;
        const T* eb = (const T*)&b;
#pragma unroll
        for (int i = 0; i < VW; ++i) acc += to_float(ea[i]) * to_float(eb[i]);
    }
    for (int off = LPR >> 1; off >= 1; off >>= 1) acc += wave_xor(acc, off);
    if (row < nrows && sub == 0) p.delta[row] = acc;
}

// -------------------------------------------------------------------- dQ
template <typename T, int D>
__global__ __launch_bounds__(256, 2) void bwd_dq_kernel(AttnParams p) {
    constexpr int BN = BwdShape<T, D>::BN;
    constexpr int NST = BN / 16;
    typedef Tile<T, D, BN> KT;
    __shared__ __attribute__((aligned(16))) T Ks[BN * KT::RS];
    __shared__ __attribute__((aligned(16))) T Kt[D * KT::TS];
    __shared__ __attribute__((aligned(16))) T Vs[BN * KT::RS];
    __shared__ int lpos[kMaxLandmarks];
    __shared__ float lb[kMaxLandmarks + 64];
    __shared__ int red[4][3];
    __shared__ int nvalid_s;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4;
    const int total = p.n_heads * p.num_seqs * p.n_tiles;
    const int L = xcd_swizzle(blockIdx.x, total);
    const int t = L % p.n_tiles;
    const int s = (L / p.n_tiles) % p.num_seqs;
    const int h = L / (p.n_tiles * p.num_seqs);
    const int st = seq_start_of(p, s);
    const int len = seq_len_of(p, s);
    const int r0 = t * 64;
    if (r0 >= len) return;
    const int kvh = h / (p.n_heads / p.n_kv_heads);
    const int K = p.k_lmk;
    const int64_t set_off = (((int64_t)h * p.num_seqs + s) * p.n_sets) * K;
    const float c2 = p.scale * kLog2eB;
    const float inv_scale = 1.0f / p.scale;

    if (tid == 0) nvalid_s = 0;
    __syncthreads();
    for (int i = tid; i < K; i += 256) {
        int v = p.lmk[set_off + i];
        lpos[i] = v;
        if (v >= 0 && (i + 1 == K || p.lmk[set_off + i + 1] < 0)) nvalid_s = i + 1;
    }
    for (int i = tid; i < K + 64; i += 256) lb[i] = (i < K && p.lbias) ? p.lbias[set_off + i] * inv_scale : 0.f;
    __syncthreads();
    const int nvalid = nvalid_s;

    const int i = r0 + wave * 16 + (lane & 15);
    const bool valid = i < len;
    int lo = 0x7fffffff, hi = -1, cnt = 0;
    float lse2 = 0.f, dlt = 0.f;
    if (valid) {
        int wi = max(p.w[st + i], 1);
        lo = max(i - wi + 1, 0);
        hi = i;
        cnt = lower_bound_i(lpos, nvalid, lo);
        lse2 = p.lse[(int64_t)(st + i) * p.n_heads + h] * kLog2eB;
        dlt = p.delta[(int64_t)(st + i) * p.n_heads + h];
    }
    const int wlo = min16(lo), whi = max16(hi), wLmax = max16(lo), wHmin = min16(hi);
    const int wcmax = max16(cnt), wcmin = min16(valid ? cnt : 0);
    if (lane == 0) {
        red[wave][0] = wlo;
        red[wave][1] = whi;
        red[wave][2] = wcmax;
    }
    __syncthreads();
    int blo = red[0][0], bhi = red[0][1], bcm = red[0][2];
    for (int w2 = 1; w2 < 4; ++w2) {
        blo = min(blo, red[w2][0]);
        bhi = max(bhi, red[w2][1]);
        bcm = max(bcm, red[w2][2]);
    }
    const int cs = (blo / BN) * BN;
    const int nband = (bhi - cs) / BN + 1;
    const int nchunks = nband + ceil_div(bcm, BN);

    RowReg<T, D> qr, dor;
    qr.load(valid ? (const T*)p.q + (int64_t)(st + i) * p.q_st + (int64_t)h * p.q_sh : nullptr, g);
    dor.load(valid ? (const T*)p.dout + (int64_t)(st + i) * p.do_st + (int64_t)h * p.do_sh : nullptr, g);

    const T* kbase = (const T*)p.k + (int64_t)st * p.k_st + (int64_t)kvh * p.k_sh;
    const T* vbase = (const T*)p.v + (int64_t)st * p.v_st + (int64_t)kvh * p.v_sh;
    auto rowpos = [&](int c, int rr) -> int {
        if (c < nband) {
            int j = cs + c * BN + rr;
            return j <= bhi ? j : -1;
        }
        int sl = (c - nband) * BN + rr;
        int pos = sl < bcm ? lpos[sl] : -1;
        return pos < len ? pos : -1;
    };

    floatx4 acc[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) acc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    const float NEG = -INFINITY;
    KT kt, vt;
    for (int c = 0; c < nchunks; ++c) {
        kt.load(tid, [&](int rr) {
            int j = rowpos(c, rr);
            return j >= 0 ? kbase + (int64_t)j * p.k_st : (const T*)nullptr;
        });
        vt.load(tid, [&](int rr) {
            int j = rowpos(c, rr);
            return j >= 0 ? vbase + (int64_t)j * p.v_st : (const T*)nullptr;
        });
        __syncthreads();
        kt.store_rows(Ks, tid);
        kt.store_cols(Kt, tid);
        vt.store_rows(Vs, tid);
        __syncthreads();
        const bool band = c < nband;
        const int base = band ? cs + c * BN : (c - nband) * BN;
        floatx4 P[NST];
        bool act[NST];
#pragma unroll
        for (int stt = 0; stt < NST; ++stt) {
            const int a = base + stt * 16;
            act[stt] = band ? (a <= whi && a + 15 >= wlo) : (a < wcmax);
            if (!act[stt]) {
                P[stt] = floatx4{0.f, 0.f, 0.f, 0.f};
                continue;
            }
            floatx4 ci;
            if (band) {
                if (a >= wLmax && a + 15 <= wHmin) {
                    ci = floatx4{0.f, 0.f, 0.f, 0.f};
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        int j = a + 4 * g + r;
                        ci[r] = (j >= lo && j <= hi) ? 0.f : NEG;
                    }
                }
            } else {
                const bool full = a + 15 < wcmin;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    int sl = a + 4 * g + r;
                    ci[r] = (full || sl < cnt) ? lb[sl] : NEG;
                }
            }
            floatx4 sc = dot_rows<T, D>(Ks, KT::RS, stt * 16, lane, qr, ci);
            floatx4 dp = dot_rows<T, D>(Vs, KT::RS, stt * 16, lane, dor, floatx4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float pr = __builtin_amdgcn_exp2f(sc[r] * c2 - lse2);
                P[stt][r] = pr * (dp[r] - dlt);  // dS (without scale)
            }
        }
        if constexpr (sizeof(T) == 2) {
#pragma unroll
            for (int hp = 0; hp < NST / 2; ++hp)
                if (act[2 * hp] || act[2 * hp + 1])
                    acc_cols<T, D>(Kt, KT::TS, hp * 32, lane, P[2 * hp], P[2 * hp + 1], acc);
        } else {
#pragma unroll
            for (int stt = 0; stt < NST; ++stt)
                if (act[stt]) acc_cols32<D>((const float*)Kt, KT::TS, stt * 16, lane, P[stt], acc);
        }
    }
    if (valid) {
        T* drow = (T*)p.dq + (int64_t)(st + i) * p.n_heads * D + (int64_t)h * D;
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) {
            T ov[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) ov[r] = from_float<T>(acc[dt][r] * p.scale);
            if constexpr (sizeof(T) == 2) *(uint2*)(drow + dt * 16 + 4 * g) = *(const uint2*)ov;
            else *(floatx4*)(drow + dt * 16 + 4 * g) = *(const floatx4*)ov;
        }
    }
}

// ----------------------------------------------------- query-row staging
// Query rows i0..i0+BQ-1 of one (head, sequence): Q and dO row-major and
// transposed, plus per-row LSE (base 2), delta, window start and landmark count.
template <typename T, int D, int BQ>
struct QStage {
    typedef Tile<T, D, BQ> QT;
    T qs[BQ * QT::RS];
    T qt[D * QT::TS];
    T ds[BQ * QT::RS];
    T dt[D * QT::TS];
    float lse2[BQ];
    float dlt[BQ];
    int lo[BQ];   // window start, INT_MAX for rows past the end
    int cnt[BQ];  // visible landmark slots
};

// -------------------------------------------------------------- band dK/dV
template <typename T, int D>
__global__ __launch_bounds__(256, 2) void bwd_dkdv_kernel(AttnParams p) {
    constexpr int BQ = BwdShape<T, D>::BQ;
    constexpr int NB = BwdShape<T, D>::NBUF;
    constexpr int NQS = BQ / 16;
    typedef QStage<T, D, BQ> QS;
    typedef typename QS::QT QT;
    __shared__ __attribute__((aligned(16))) QS sq[NB];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4;
    const int total = p.n_heads * p.num_seqs * p.n_tiles;
    const int L = xcd_swizzle(blockIdx.x, total);
    const int t = L % p.n_tiles;
    const int s = (L / p.n_tiles) % p.num_seqs;
    const int h = L / (p.n_tiles * p.num_seqs);
    const int st = seq_start_of(p, s);
    const int len = seq_len_of(p, s);
    const int j0 = t * 64;
    if (j0 >= len) return;
    const int nt16 = ceil_div(p.max_seqlen, 16);
    const int* tinfo = p.tile_minlo + (int64_t)s * nt16 * 2;
    const float c2 = p.scale * kLog2eB;

    const int wj0 = j0 + wave * 16;
    const int j = wj0 + (lane & 15);
    const bool jvalid = j < len;
    RowReg<T, D> kr, vr;
    kr.load(jvalid ? (const T*)p.k + (int64_t)(st + j) * p.k_st + (int64_t)h * p.k_sh : nullptr, g);
    vr.load(jvalid ? (const T*)p.v + (int64_t)(st + j) * p.v_st + (int64_t)h * p.v_sh : nullptr, g);

    // rows that can see keys j0..j0+63: i in [j0, min(len, j0 + 63 + wmax))
    const int iend = min(len, j0 + 63 + p.seq_wmax[s]);
    const int nq = ceil_div(iend - j0, BQ);
    const T* qb = (const T*)p.q + (int64_t)st * p.q_st + (int64_t)h * p.q_sh;
    const T* db = (const T*)p.dout + (int64_t)st * p.do_st + (int64_t)h * p.do_sh;
    auto chunk_needed = [&](int c) {
        int i0 = j0 + c * BQ;
        for (int q16 = 0; q16 < NQS; ++q16) {
            int ti = i0 / 16 + q16;
            if (i0 + q16 * 16 < iend && tinfo[ti * 2] <= j0 + 63) return true;
        }
        return false;
    };
    QT tq, tdo;
    auto load_chunk = [&](int c) {
        int i0 = j0 + c * BQ;
        tq.load(tid, [&](int rr) { return i0 + rr < iend ? qb + (int64_t)(i0 + rr) * p.q_st : (const T*)nullptr; });
        tdo.load(tid, [&](int rr) { return i0 + rr < iend ? db + (int64_t)(i0 + rr) * p.do_st : (const T*)nullptr; });
    };
    auto store_chunk = [&](int c, QS& q) {
        int i0 = j0 + c * BQ;
        tq.store_rows(q.qs, tid);
        tq.store_cols(q.qt, tid);
        tdo.store_rows(q.ds, tid);
        tdo.store_cols(q.dt, tid);
        if (tid < BQ) {
            int i = i0 + tid;
            if (i < iend) {
                int wi = max(p.w[st + i], 1);
                q.lo[tid] = max(i - wi + 1, 0);
                q.lse2[tid] = p.lse[(int64_t)(st + i) * p.n_heads + h] * kLog2eB;
                q.dlt[tid] = p.delta[(int64_t)(st + i) * p.n_heads + h];
            } else {
                q.lo[tid] = 0x7fffffff;
                q.lse2[tid] = 0.f;
                q.dlt[tid] = 0.f;
            }
        }
    };

    floatx4 adk[D / 16], adv[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
        adk[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
        adv[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    const float NEG = -INFINITY;
    int c = 0;
    while (c < nq && !chunk_needed(c)) ++c;
    if (c < nq) {
        load_chunk(c);
        store_chunk(c, sq[0]);
    }
    __syncthreads();
    int buf = 0;
    while (c < nq) {
        int cn = c + 1;
        while (cn < nq && !chunk_needed(cn)) ++cn;
        if (cn < nq) load_chunk(cn);
        QS& q = sq[buf];
        const int i0 = j0 + c * BQ;
        floatx4 P[NQS], dS[NQS];
        bool act[NQS];
#pragma unroll
        for (int qs = 0; qs < NQS; ++qs) {
            const int qa = i0 + qs * 16;
            const int ti = qa / 16;
            const int tmin = qa < iend ? tinfo[ti * 2] : 0x7fffffff;
            const int tmax = qa < iend ? tinfo[ti * 2 + 1] : 0x7fffffff;
            act[qs] = qa < iend && tmin <= wj0 + 15 && qa + 15 >= wj0 && wj0 < len;
            if (!act[qs]) {
                P[qs] = floatx4{0.f, 0.f, 0.f, 0.f};
                dS[qs] = P[qs];
                continue;
            }
            floatx4 ci;
            const bool full = tmax <= wj0 && qa >= wj0 + 15 && qa + 15 < iend && wj0 + 15 < len;
            if (full) {
                ci = floatx4{0.f, 0.f, 0.f, 0.f};
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    int rr = qs * 16 + 4 * g + r;
                    int i = i0 + rr;
                    ci[r] = (jvalid && j >= q.lo[rr] && j <= i) ? 0.f : NEG;
                }
            }
            floatx4 sc = dot_rows<T, D>(q.qs, QT::RS, qs * 16, lane, kr, ci);
            floatx4 dp = dot_rows<T, D>(q.ds, QT::RS, qs * 16, lane, vr, floatx4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                int rr = qs * 16 + 4 * g + r;
                float pr = __builtin_amdgcn_exp2f(sc[r] * c2 - q.lse2[rr]);
                P[qs][r] = pr;
                dS[qs][r] = pr * (dp[r] - q.dlt[rr]);
            }
        }
        if constexpr (sizeof(T) == 2) {
#pragma unroll
            for (int hp = 0; hp < NQS / 2; ++hp)
                if (act[2 * hp] || act[2 * hp + 1]) {
                    acc_cols<T, D>(q.dt, QT::TS, hp * 32, lane, P[2 * hp], P[2 * hp + 1], adv);
                    acc_cols<T, D>(q.qt, QT::TS, hp * 32, lane, dS[2 * hp], dS[2 * hp + 1], adk);
                }
        } else {
#pragma unroll
            for (int qs = 0; qs < NQS; ++qs)
                if (act[qs]) {
                    acc_cols32<D>((const float*)q.dt, QT::TS, qs * 16, lane, P[qs], adv);
                    acc_cols32<D>((const float*)q.qt, QT::TS, qs * 16, lane, dS[qs], adk);
                }
        }
        if constexpr (NB == 2) {
            if (cn < nq) store_chunk(cn, sq[buf ^ 1]);
            __syncthreads();
            buf ^= 1;
        } else {
            __syncthreads();
            if (cn < nq) store_chunk(cn, sq[0]);
            __syncthreads();
        }
        c = cn;
    }
    if (jvalid) {
        T* kd = (T*)p.dk + (int64_t)(st + j) * p.n_heads * D + (int64_t)h * D;
        T* vd = (T*)p.dv + (int64_t)(st + j) * p.n_heads * D + (int64_t)h * D;
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) {
            T ok[4], ov[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                ok[r] = from_float<T>(adk[dt][r] * p.scale);
                ov[r] = from_float<T>(adv[dt][r]);
            }
            if constexpr (sizeof(T) == 2) {
                *(uint2*)(kd + dt * 16 + 4 * g) = *(const uint2*)ok;
                *(uint2*)(vd + dt * 16 + 4 * g) = *(const uint2*)ov;
            } else {
                *(floatx4*)(kd + dt * 16 + 4 * g) = *(const floatx4*)ok;
                *(floatx4*)(vd + dt * 16 + 4 * g) = *(const floatx4*)ov;
            }
        }
    }
}

// -------------------------------------------------------- landmark dK/dV
// Block = (head, sequence, 1024-row chunk, group of 128 slots); wave w owns
// slots grp*128 + 32w .. +31 as two 16-slot subtiles.
template <typename T, int D>
__global__ __launch_bounds__(256, 2) void bwd_lmk_kernel(AttnParams p) {
    constexpr int BQ = BwdShape<T, D>::BQ;
    constexpr int NQS = BQ / 16;
    typedef QStage<T, D, BQ> QS;
    typedef typename QS::QT QT;
    __shared__ __attribute__((aligned(16))) QS q;
    __shared__ int lpos[kMaxLandmarks];
    __shared__ float lb[kMaxLandmarks + 64];
    __shared__ int cmin_s[BQ / 16], cmax_s[BQ / 16];
    __shared__ int nvalid_s;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4;
    const int K = p.k_lmk;
    const int ngrp = ceil_div(K, 128);
    int b = blockIdx.x;
    const int grp = b % ngrp;
    b /= ngrp;
    const int chunk = b % p.n_chunks;
    b /= p.n_chunks;
    const int s = b % p.num_seqs;
    const int h = b / p.num_seqs;
    const int st = seq_start_of(p, s);
    const int len = seq_len_of(p, s);
    const int kvh = h / (p.n_heads / p.n_kv_heads);
    const int64_t set_off = (((int64_t)h * p.num_seqs + s) * p.n_sets) * K;
    const float c2 = p.scale * kLog2eB;
    const float inv_scale = 1.0f / p.scale;
    const int rbeg = chunk * kRowChunk, rend = min(len, rbeg + kRowChunk);

    if (tid == 0) nvalid_s = 0;
    __syncthreads();
    for (int i = tid; i < K; i += 256) {
        int v = p.lmk[set_off + i];
        lpos[i] = v;
        if (v >= 0 && (i + 1 == K || p.lmk[set_off + i + 1] < 0)) nvalid_s = i + 1;
    }
    for (int i = tid; i < K + 64; i += 256) lb[i] = (i < K && p.lbias) ? p.lbias[set_off + i] * inv_scale : 0.f;
    __syncthreads();
    const int nvalid = nvalid_s;

    // slots of this lane (two subtiles)
    const int sl0 = grp * 128 + wave * 32;
    RowReg<T, D> kr[2], vr[2];
    int slot[2];
    bool sval[2];
    const T* kbase = (const T*)p.k + (int64_t)st * p.k_st + (int64_t)kvh * p.k_sh;
    const T* vbase = (const T*)p.v + (int64_t)st * p.v_st + (int64_t)kvh * p.v_sh;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        slot[u] = sl0 + u * 16 + (lane & 15);
        sval[u] = slot[u] < nvalid && lpos[slot[u]] < len;
        kr[u].load(sval[u] ? kbase + (int64_t)lpos[slot[u]] * p.k_st : nullptr, g);
        vr[u].load(sval[u] ? vbase + (int64_t)lpos[slot[u]] * p.v_st : nullptr, g);
    }
    floatx4 adk[2][D / 16], adv[2][D / 16];
    float dbias[2] = {0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) {
            adk[u][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
            adv[u][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
    const T* qb = (const T*)p.q + (int64_t)st * p.q_st + (int64_t)h * p.q_sh;
    const T* db = (const T*)p.dout + (int64_t)st * p.do_st + (int64_t)h * p.do_sh;
    const float NEG = -INFINITY;
    // first row with any visible landmark: lo_i > lpos[0]  =>  i > lpos[0]
    const int first_row = nvalid > 0 ? lpos[0] + 1 : 0x7fffffff;
    const int istart = max(rbeg, (first_row / BQ) * BQ);
    QT tq, tdo;
    // the loop bound is uniform over the block (every wave reaches each barrier);
    // waves whose slots are all empty skip their products through act[] below
    const bool any_slot = grp * 128 < nvalid;
    for (int i0 = istart; any_slot && i0 < rend; i0 += BQ) {
        tq.load(tid, [&](int rr) { return i0 + rr < rend ? qb + (int64_t)(i0 + rr) * p.q_st : (const T*)nullptr; });
        tdo.load(tid, [&](int rr) { return i0 + rr < rend ? db + (int64_t)(i0 + rr) * p.do_st : (const T*)nullptr; });
        __syncthreads();
        tq.store_rows(q.qs, tid);
        tq.store_cols(q.qt, tid);
        tdo.store_rows(q.ds, tid);
        tdo.store_cols(q.dt, tid);
        if (tid < BQ) {
            int i = i0 + tid;
            if (i < rend) {
                int wi = max(p.w[st + i], 1);
                q.cnt[tid] = lower_bound_i(lpos, nvalid, max(i - wi + 1, 0));
                q.lse2[tid] = p.lse[(int64_t)(st + i) * p.n_heads + h] * kLog2eB;
                q.dlt[tid] = p.delta[(int64_t)(st + i) * p.n_heads + h];
            } else {
                q.cnt[tid] = 0;
                q.lse2[tid] = 0.f;
                q.dlt[tid] = 0.f;
            }
        }
        __syncthreads();
        if (tid < NQS) {
            int mn = 0x7fffffff, mx = 0;
            for (int r = 0; r < 16; ++r) {
                mn = min(mn, q.cnt[tid * 16 + r]);
                mx = max(mx, q.cnt[tid * 16 + r]);
            }
            cmin_s[tid] = mn;
            cmax_s[tid] = mx;
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int a = sl0 + u * 16;
            floatx4 P[NQS], dS[NQS];
            bool act[NQS];
#pragma unroll
            for (int qs = 0; qs < NQS; ++qs) {
                act[qs] = cmax_s[qs] > a;
                if (!act[qs]) {
                    P[qs] = floatx4{0.f, 0.f, 0.f, 0.f};
                    dS[qs] = P[qs];
                    continue;
                }
                floatx4 ci;
                const bool full = cmin_s[qs] > a + 15;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    int rr = qs * 16 + 4 * g + r;
                    ci[r] = (full || slot[u] < q.cnt[rr]) ? lb[slot[u]] : NEG;
                }
                floatx4 sc = dot_rows<T, D>(q.qs, QT::RS, qs * 16, lane, kr[u], ci);
                floatx4 dp = dot_rows<T, D>(q.ds, QT::RS, qs * 16, lane, vr[u], floatx4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    int rr = qs * 16 + 4 * g + r;
                    float pr = __builtin_amdgcn_exp2f(sc[r] * c2 - q.lse2[rr]);
                    float d = pr * (dp[r] - q.dlt[rr]);
                    P[qs][r] = pr;
                    dS[qs][r] = d;
                    dbias[u] += d;
                }
            }
            if constexpr (sizeof(T) == 2) {
#pragma unroll
                for (int hp = 0; hp < NQS / 2; ++hp)
                    if (act[2 * hp] || act[2 * hp + 1]) {
                        acc_cols<T, D>(q.dt, QT::TS, hp * 32, lane, P[2 * hp], P[2 * hp + 1], adv[u]);
                        acc_cols<T, D>(q.qt, QT::TS, hp * 32, lane, dS[2 * hp], dS[2 * hp + 1], adk[u]);
                    }
            } else {
#pragma unroll
                for (int qs = 0; qs < NQS; ++qs)
                    if (act[qs]) {
                        acc_cols32<D>((const float*)q.dt, QT::TS, qs * 16, lane, P[qs], adv[u]);
                        acc_cols32<D>((const float*)q.qt, QT::TS, qs * 16, lane, dS[qs], adk[u]);
                    }
            }
        }
    }
    // partials: [chunk][h][s][slot][D]
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        float db2 = sum_g4(dbias[u]);
        if (slot[u] >= K) continue;
        const int64_t row = (((int64_t)chunk * p.n_heads + h) * p.num_seqs + s) * K + slot[u];
        float* pk = p.part_k + row * D;
        float* pv = p.part_v + row * D;
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) {
            *(floatx4*)(pk + dt * 16 + 4 * g) = adk[u][dt] * p.scale;
            *(floatx4*)(pv + dt * 16 + 4 * g) = adv[u][dt];
        }
        if (g == 0) p.part_b[row] = db2;
    }
}

template <typename T, int D>
__global__ __launch_bounds__(256) void bwd_lmk_sum_kernel(AttnParams p) {
    const int K = p.k_lmk;
    const int64_t nrow = (int64_t)p.n_heads * p.num_seqs * K;
    const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= nrow * D) return;
    const int d = (int)(id % D);
    const int64_t row = id / D;  // (h, s, slot)
    const int sl = (int)(row % K);
    const int s = (int)((row / K) % p.num_seqs);
    const int h = (int)(row / ((int64_t)K * p.num_seqs));
    const int pos = p.lmk[(((int64_t)h * p.num_seqs + s) * p.n_sets) * K + sl];
    const int len = seq_len_of(p, s);
    float sk = 0.f, sv = 0.f, sb = 0.f;
    for (int ch = 0; ch < p.n_chunks; ++ch) {
        const int64_t pr = ((int64_t)ch * p.n_heads + h) * p.num_seqs * K + (int64_t)s * K + sl;
        sk += p.part_k[pr * D + d];
        sv += p.part_v[pr * D + d];
        if (d == 0) sb += p.part_b[pr];
    }
    if (d == 0 && p.d_bias) p.d_bias[(((int64_t)h * p.num_seqs + s) * p.n_sets) * K + sl] = sb;
    if (pos < 0 || pos >= len) return;
    const int64_t o = (int64_t)(seq_start_of(p, s) + pos) * p.n_heads * D + (int64_t)h * D + d;
    T* dk = (T*)p.dk;
    T* dv = (T*)p.dv;
    dk[o] = from_float<T>(to_float(dk[o]) + sk);
    dv[o] = from_float<T>(to_float(dv[o]) + sv);
}

// ---------------------------------------------------------------- launch
size_t bwd_workspace(const AttnParams& p) {
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const int nt16 = ceil_div(p.max_seqlen, 16);
    const int nch = ceil_div(p.max_seqlen, kRowChunk);
    size_t b = 0;
    b += al(sizeof(float) * (size_t)p.total_len * p.n_heads);
    b += al(sizeof(int) * 2 * (size_t)p.num_seqs * nt16);
    b += al(sizeof(int) * (size_t)p.num_seqs);
    b += 2 * al(sizeof(float) * (size_t)nch * p.n_heads * p.num_seqs * p.k_lmk * p.head_dim);
    b += al(sizeof(float) * (size_t)nch * p.n_heads * p.num_seqs * p.k_lmk);
    return b;
}

template <typename T, int D>
static void bwd_run(const AttnParams& p, hipStream_t stream) {
    const int total = p.n_heads * p.num_seqs * p.n_tiles;
    DSALT_LAUNCH("bwd_rowinfo", bwd_rowinfo_kernel, dim3(p.num_seqs), dim3(256), 0, stream, p);
    constexpr int LPR = D / (16 / (int)sizeof(T));
    const int64_t nrows = (int64_t)p.total_len * p.n_heads;
    DSALT_LAUNCH("bwd_delta", (bwd_delta_kernel<T, D>), dim3((unsigned)((nrows * LPR + 255) / 256)), dim3(256), 0, stream,
                       p);
    DSALT_LAUNCH("bwd_dq", (bwd_dq_kernel<T, D>), dim3(total), dim3(256), 0, stream, p);
    DSALT_LAUNCH("bwd_dkdv", (bwd_dkdv_kernel<T, D>), dim3(total), dim3(256), 0, stream, p);
    if (p.k_lmk > 0) {
        const int ngrp = ceil_div(p.k_lmk, 128);
        DSALT_LAUNCH("bwd_lmk", (bwd_lmk_kernel<T, D>), dim3(p.n_heads * p.num_seqs * p.n_chunks * ngrp), dim3(256), 0,
                           stream, p);
        const int64_t n = (int64_t)p.n_heads * p.num_seqs * p.k_lmk * D;
        DSALT_LAUNCH("bwd_lmk_sum", (bwd_lmk_sum_kernel<T, D>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p);
    }
}

hipError_t bwd_launch(AttnParams p, void* ws, hipStream_t stream) {
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const int nt16 = ceil_div(p.max_seqlen, 16);
    p.n_chunks = ceil_div(p.max_seqlen, kRowChunk);
    char* w = (char*)ws;
    p.delta = (float*)w;
    w += al(sizeof(float) * (size_t)p.total_len * p.n_heads);
    p.tile_minlo = (int*)w;
    w += al(sizeof(int) * 2 * (size_t)p.num_seqs * nt16);
    p.seq_wmax = (int*)w;
    w += al(sizeof(int) * (size_t)p.num_seqs);
    const size_t npart = (size_t)p.n_chunks * p.n_heads * p.num_seqs * p.k_lmk;
    p.part_k = (float*)w;
    w += al(sizeof(float) * npart * p.head_dim);
    p.part_v = (float*)w;
    w += al(sizeof(float) * npart * p.head_dim);
    p.part_b = (float*)w;
    if (p.total_len == 0 || p.num_seqs == 0) return hipSuccess;
    if (p.dtype == DSALT_DTYPE_BF16) {
        if (p.head_dim == 64) bwd_run<bf16, 64>(p, stream);
        else bwd_run<bf16, 128>(p, stream);
    } else if (p.dtype == DSALT_DTYPE_F16) {
        if (p.head_dim == 64) bwd_run<f16, 64>(p, stream);
        else bwd_run<f16, 128>(p, stream);
    } else {
        if (p.head_dim == 64) bwd_run<float, 64>(p, stream);
        else bwd_run<float, 128>(p, stream);
    }
    return hipGetLastError();
}

}  // namespace dsalt
