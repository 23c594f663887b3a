// DSALT attention forward for gfx950.
//
// Replaces _dsalt_fwd_kernel (dsalt/kernels/dsalt_triton_attn.py:27-169).
// One 256-thread block (4 waves) owns 64 query rows of one (head, sequence);
// wave w owns rows 16w..16w+15 and each lane one query row (column of the
// transposed score tile S^T = K Q^T).  The block walks the union of its rows'
// windows [min_i lo_i, max_i i] in BN-key chunks staged row-major in LDS
// (double-buffered), then the landmark slots of its set through the same
// buffers.  Masks are folded into the MFMA accumulator initialisation (0 or
// -inf, bias/scale for landmarks); 16-key subtiles outside a wave's own range
// are skipped with scalar branches.  Landmarks arrive sorted, so the landmarks
// visible to row i are exactly the first cnt_i = #{p < i - w_i + 1} slots -- a
// landmark inside the window is never counted twice.  Online softmax in base 2
// with a lazy rescale (the running max moves only when a row max grows by more
// than 2^8); P is rounded to the input dtype before P V as in the reference
// (:115,:147), V^T comes from the row-major tile through the transpose read,
// and the row sums come from the same packed P through a ones operand.
#include "attn.h"
#include "tiles.h"
#include "timing.h"

namespace dsalt {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kBM = 64;

template <typename T, int D> struct FwdShape;
template <> struct FwdShape<bf16, 64> { static constexpr int BN = 64; };
template <> struct FwdShape<bf16, 128> { static constexpr int BN = 32; };
template <> struct FwdShape<f16, 64> { static constexpr int BN = 64; };
template <> struct FwdShape<f16, 128> { static constexpr int BN = 32; };
template <> struct FwdShape<float, 64> { static constexpr int BN = 32; };
template <> struct FwdShape<float, 128> { static constexpr int BN = 16; };

__device__ __forceinline__ int lower_bound_lds(const int* a, int n, int x) {
    int lo = 0, hi = n;
    while (lo < hi) {
        int mid = (lo + hi) >> 1;
        if (a[mid] < x) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

template <typename T, int D>
__global__ __launch_bounds__(256, 2) void fwd_kernel(AttnParams p) {
    constexpr int BN = FwdShape<T, D>::BN;
    constexpr int NST = BN / 16;
    constexpr bool kHalf = sizeof(T) == 2;
    typedef Tile<T, D, BN> KT;
    __shared__ __attribute__((aligned(16))) T Ks[2][KT::ELEMS];
    __shared__ __attribute__((aligned(16))) T Vs[2][KT::ELEMS];
    __shared__ int lpos[kMaxLandmarks];
    __shared__ int red[4][3];
    __shared__ int nvalid_s;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4;
    const int total = p.n_heads * p.num_seqs * p.n_tiles;
    const int L = xcd_swizzle(blockIdx.x, total);
    const int t = L % p.n_tiles;
    const int s = (L / p.n_tiles) % p.num_seqs;
    const int h = L / (p.n_tiles * p.num_seqs);
    int st, len;
    seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
    const int r0 = t * kBM;
    if (r0 >= len) return;
    const int kvh = h / (p.n_heads / p.n_kv_heads);
    const int set = p.block_size ? r0 / p.block_size : 0;
    const int K = p.k_lmk;
    const int64_t set_off = (((int64_t)h * p.num_seqs + s) * p.n_sets + set) * K;
    const float c2 = p.scale * kLog2e;
    const float inv_scale = 1.0f / p.scale;
    const bool has_bias = p.lbias != nullptr;

    if (tid == 0) nvalid_s = 0;
    __syncthreads();
    for (int i = tid; i < K; i += 256) {
        int v = p.lmk[set_off + i];
        lpos[i] = v;
        if (v >= 0 && (i + 1 == K || p.lmk[set_off + i + 1] < 0)) nvalid_s = i + 1;
    }
    __syncthreads();
    const int nvalid = nvalid_s;

    // the row of this lane: window [lo, hi] and visible landmark count
    const int i = r0 + wave * 16 + (lane & 15);
    const bool valid = i < len;
    int lo = 0x7fffffff, hi = -1, cnt = 0;
    if (valid) {
        const int wi = max(p.w[st + i], 1);
        lo = max(i - wi + 1, 0);
        hi = i;
        cnt = lower_bound_lds(lpos, nvalid, lo);
    }
    // wave-uniform bounds (scalar registers: the subtile branches below are scalar)
    const int wlo = uniform(min16(lo)), whi = uniform(max16(hi));
    const int wLmax = uniform(max16(lo)), wHmin = uniform(min16(hi));
    const int wcmax = uniform(max16(cnt)), wcmin = uniform(min16(valid ? cnt : 0));
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
    blo = uniform(blo);
    bhi = uniform(bhi);
    bcm = uniform(bcm);
    const int cs = (blo / BN) * BN;
    const int nband = (bhi - cs) / BN + 1;
    const int nchunks = nband + ceil_div(bcm, BN);

    const T* qhead = (const T*)p.q + (int64_t)st * p.q_st + (int64_t)h * p.q_sh;
    RowReg<T, D> qr;
    qr.load(valid ? qhead + (int64_t)i * p.q_st : nullptr, qhead, g);

    const T* kbase = (const T*)p.k + (int64_t)st * p.k_st + (int64_t)kvh * p.k_sh;
    const T* vbase = (const T*)p.v + (int64_t)st * p.v_st + (int64_t)kvh * p.v_sh;
    // band chunks: consecutive rows through buffer resources bounded at bhi
    // (loop-invariant per-thread offsets); landmark chunks: gathered rows
    const uint32_t krb = (uint32_t)(p.k_st * (int64_t)sizeof(T)), vrb = (uint32_t)(p.v_st * (int64_t)sizeof(T));
    uint32_t koff[KT::NV], voff[KT::NV];
#pragma unroll
    for (int n = 0; n < KT::NV; ++n) {
        koff[n] = KT::row_offset(tid, n, krb);
        voff[n] = KT::row_offset(tid, n, vrb);
    }
    KT kt, vt;
    auto load_chunk = [&](int c) {
        if (c < nband) {
            const int j0 = cs + c * BN;
            const int rows = min(BN, bhi + 1 - j0);
            kt.load_rows(rows_rsrc(kbase + (int64_t)j0 * p.k_st, rows, krb, D * sizeof(T)), koff);
            vt.load_rows(rows_rsrc(vbase + (int64_t)j0 * p.v_st, rows, vrb, D * sizeof(T)), voff);
        } else {
            auto pos = [&](int rr) -> int {
                const int sl = (c - nband) * BN + rr;
                const int q = sl < bcm ? lpos[sl] : -1;
                return q < len ? q : -1;
            };
            kt.load(tid, [&](int rr) { int j = pos(rr); return j >= 0 ? kbase + (int64_t)j * p.k_st : (const T*)nullptr; },
                    kbase);
            vt.load(tid, [&](int rr) { int j = pos(rr); return j >= 0 ? vbase + (int64_t)j * p.v_st : (const T*)nullptr; },
                    vbase);
        }
    };
    load_chunk(0);
    kt.store(Ks[0], tid);
    vt.store(Vs[0], tid);
    __syncthreads();

    floatx4 acc[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) acc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    floatx4 lacc = floatx4{0.f, 0.f, 0.f, 0.f};  // row sums (16-bit path: ones x P)
    float l_run = 0.f;                             // row sums (fp32 path)
    float m_run = -INFINITY;
    const float thr = 8.0f / c2;
    const float NEG = -INFINITY;
    const int lane_off = 4 * g;

    for (int c = 0; c < nchunks; ++c) {
        const int buf = c & 1;
        if (c + 1 < nchunks) load_chunk(c + 1);
        const bool band = c < nband;
        const int base = band ? cs + c * BN : (c - nband) * BN;
        floatx4 S[NST];
        bool act[NST];
#pragma unroll
        for (int stt = 0; stt < NST; ++stt) {
            const int a = base + stt * 16;
            act[stt] = band ? (a <= whi && a + 15 >= wlo) : (a < wcmax);
            if (!act[stt]) {
                S[stt] = floatx4{NEG, NEG, NEG, NEG};
                continue;
            }
            floatx4 ci;
            if (band) {
                if (a >= wLmax && a + 15 <= wHmin) {
                    ci = floatx4{0.f, 0.f, 0.f, 0.f};
                } else if (a + 15 <= wHmin) {  // below every row's diagonal: lower bound only
                    const int tl = lo - a - lane_off;
#pragma unroll
                    for (int r = 0; r < 4; ++r) ci[r] = r < tl ? NEG : 0.f;
                } else {
                    const int tl = lo - a - lane_off, th = hi - a - lane_off;
#pragma unroll
                    for (int r = 0; r < 4; ++r) ci[r] = (r < tl || r > th) ? NEG : 0.f;
                }
            } else {
                floatx4 bv = floatx4{0.f, 0.f, 0.f, 0.f};
                if (has_bias) {
                    float braw[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) braw[r] = p.lbias[set_off + min(a + lane_off + r, K - 1)];
#pragma unroll
                    for (int r = 0; r < 4; ++r) bv[r] = a + lane_off + r < K ? braw[r] * inv_scale : 0.f;
                }
                if (a + 15 < wcmin) {
                    ci = bv;
                } else {
                    const int tc = cnt - a - lane_off;
#pragma unroll
                    for (int r = 0; r < 4; ++r) ci[r] = r < tc ? bv[r] : NEG;
                }
            }
            S[stt] = dot_rows<T, D>(Ks[buf], KT::RS, stt * 16, lane, qr, ci);
        }
        // online softmax over the chunk
        float mx = NEG;
#pragma unroll
        for (int stt = 0; stt < NST; ++stt)
#pragma unroll
            for (int r = 0; r < 4; ++r) mx = fmaxf(mx, S[stt][r]);
        mx = max_g4(mx);
        const float mnew = fmaxf(m_run, mx);
        if (__any(mnew > m_run + thr)) {
            const float alpha = m_run == NEG ? 0.f : __builtin_amdgcn_exp2f((m_run - mnew) * c2);
#pragma unroll
            for (int dt = 0; dt < D / 16; ++dt) acc[dt] *= alpha;
            lacc *= alpha;
            l_run *= alpha;
            m_run = mnew;
        }
        const float msc = m_run == NEG ? 0.f : m_run * c2;
#pragma unroll
        for (int stt = 0; stt < NST; ++stt)
#pragma unroll
            for (int r = 0; r < 4; ++r) S[stt][r] = __builtin_amdgcn_exp2f(S[stt][r] * c2 - msc);
        if constexpr (kHalf) {
            const typename Vec8<T>::type ones = ones8<T>();
#pragma unroll
            for (int hp = 0; hp < NST / 2; ++hp)
                if (act[2 * hp] || act[2 * hp + 1]) {
                    auto b = acc_tr<T, D>(Vs[buf], KT::RS, hp * 32, lane, S[2 * hp], S[2 * hp + 1], acc);
                    lacc = mma(ones, b, lacc);
                }
        } else {
#pragma unroll
            for (int stt = 0; stt < NST; ++stt)
                if (act[stt]) {
                    l_run += S[stt][0] + S[stt][1] + S[stt][2] + S[stt][3];
                    acc_rm32<D>((const float*)Vs[buf], KT::RS, stt * 16, lane, S[stt], acc);
                }
        }
        if (c + 1 < nchunks) {
            kt.store(Ks[buf ^ 1], tid);
            vt.store(Vs[buf ^ 1], tid);
        }
        __syncthreads();
    }

    const float l_tot = kHalf ? lacc[0] : sum_g4(l_run);
    if (valid) {
        const float inv = 1.0f / l_tot;
        T* orow = (T*)p.o + (int64_t)(st + i) * p.o_st + (int64_t)h * p.o_sh;
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) {
            T ov[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) ov[r] = from_float<T>(acc[dt][r] * inv);
            if constexpr (kHalf) *(uint2*)(orow + dt * 16 + lane_off) = *(const uint2*)ov;
            else *(floatx4*)(orow + dt * 16 + lane_off) = *(const floatx4*)ov;
        }
        if (g == 0) p.lse_out[(int64_t)(st + i) * p.n_heads + h] = m_run * p.scale + __logf(l_tot);
    }
}

template <typename T>
static hipError_t fwd_dispatch(const AttnParams& p, hipStream_t stream) {
    const int total = p.n_heads * p.num_seqs * p.n_tiles;
    if (total == 0) return hipSuccess;
    if (p.head_dim == 64)
        DSALT_LAUNCH("attn_fwd", (fwd_kernel<T, 64>), dim3(total), dim3(256), 0, stream, p);
    else
        DSALT_LAUNCH("attn_fwd", (fwd_kernel<T, 128>), dim3(total), dim3(256), 0, stream, p);
    return hipGetLastError();
}

hipError_t fwd_launch(const AttnParams& p, hipStream_t stream) {
    if (p.dtype == DSALT_DTYPE_BF16) return fwd_dispatch<bf16>(p, stream);
    if (p.dtype == DSALT_DTYPE_F16) return fwd_dispatch<f16>(p, stream);
    return fwd_dispatch<float>(p, stream);
}

}  // namespace dsalt
