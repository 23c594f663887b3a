// DSALT attention backward for gfx950, deterministic (no float atomics).
//
// Replaces _dsalt_bwd_preprocess and _dsalt_bwd_kernel
// (dsalt/kernels/dsalt_triton_bwd.py:17-216), which accumulate dK/dV with
// atomic_add.  Here every output element has exactly one writer:
//   bwd_dq       query-parallel, like the forward (64 rows per block, one row
//                per lane): delta = rowsum(O dO) from the stored O (:44),
//                dQ = scale * dS K over the band and the landmark slots
//                (:148,:196); also records each row's LSE, delta and visible
//                landmark count for the passes below.
//   bwd_dkdv     key-parallel over the band: 16 keys per wave, the query rows
//                that can see them staged row-major in LDS (double-buffered);
//                dV = P^T dO, dK = scale * dS^T Q (:198-199); the rows to sweep end
//                at the sequence's largest window (from the row plan's tile maxima),
//                and a key that is a landmark row leaves its sums in fp32 for the
//                landmark pass (its owner: the first (head, slot) of the group holding it).
//   bwd_lmk      landmark slots x 1024-row chunks: partial dK/dV/d_bias of each
//                (head, sequence, slot) (:150-155).
//   bwd_lmk_sum  per landmark row: the band sums the dK/dV pass left in fp32
//                plus the partials of every head holding the row, in head and
//                chunk order, rounded once into the dK/dV row.
// Grouped heads: dQ and the landmark pass run per query head; the dK/dV pass
// runs per key/value head and sweeps the group's query heads in order.
// P = exp(q.k * scale + bias - LSE) is recomputed in base 2 from the forward's
// LSE; dS = P (dP - delta), dP = dO V^T.  Products over tokens read their
// transposed operand from the row-major tiles with ds_read_b64_tr_b16.
#include <type_traits>

#include "attn.h"
#include "tiles.h"
#include "timing.h"

namespace dsalt {

constexpr float kLog2eB = 1.4426950408889634f;
constexpr int kRowChunk = 1024;  // rows per landmark-backward block, at most
constexpr int kSeg = 512;  // rows compacted at a time in the dK/dV sweep

template <typename T, int D> struct BwdShape;
// BN: keys per staged chunk of the query-parallel dQ kernel (32 for 16-bit head_dim 64:
// the shorter chunk brings the kernel to 78 registers, six waves per SIMD, and the
// kernel is bound by the latency of its chunk loop, not by issue); BQ: query rows per
// staged chunk of the key-parallel dK/dV kernel (32 for 16-bit head_dim 64: four waves
// per SIMD without spills, also in the training variant); BL: the same for the landmark
// kernel
template <> struct BwdShape<bf16, 64> { static constexpr int BN = 32, BQ = 32, BL = 64; };
template <> struct BwdShape<bf16, 128> { static constexpr int BN = 32, BQ = 32, BL = 32; };
template <> struct BwdShape<f16, 64> { static constexpr int BN = 32, BQ = 32, BL = 64; };
template <> struct BwdShape<f16, 128> { static constexpr int BN = 32, BQ = 32, BL = 32; };
template <> struct BwdShape<float, 64> { static constexpr int BN = 32, BQ = 32, BL = 32; };
template <> struct BwdShape<float, 128> { static constexpr int BN = 16, BQ = 16, BL = 16; };

__device__ __forceinline__ int lower_bound_i(const int* a, int n, int x) {
    int lo = 0, hi = n;
    while (lo < hi) {
        int mid = (lo + hi) >> 1;
        if (a[mid] < x) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// loads a landmark set into LDS; returns the number of valid (non -1) slots
__device__ __forceinline__ int load_set(const AttnParams& p, int64_t set_off, int* lpos, int* nvalid_s, int tid,
                                        float* lbs = nullptr, int nthreads = 256) {
    if (tid == 0) *nvalid_s = 0;
    __syncthreads();
    for (int i = tid; i < p.k_lmk; i += nthreads) {
        int v = p.lmk[set_off + i];
        lpos[i] = v;
        if (v >= 0 && (i + 1 == p.k_lmk || p.lmk[set_off + i + 1] < 0)) *nvalid_s = i + 1;
        if (lbs) lbs[i] = p.lbias[set_off + i] * p.inv_scale;  // landmark bias in raw-score units
    }
    __syncthreads();
    return *nvalid_s;
}

// -------------------------------------------------------------------- dQ
// TR: training variant -- band keys near the window start carry the soft edge bias,
// and the lane also sums dS * d(bias)/d(w~) of its row into dw_h.
// LK: sets of more than kSetSlots landmarks (inference operator), staged by a loop.
template <typename T, int D, int BN, bool TR, bool LK = false>
__global__ __launch_bounds__(256, (sizeof(T) == 2 && D == 64) ? (BN == 32 ? (TR ? 5 : 6) : 4) : 2) void bwd_dq_kernel(AttnParams p) {
    static_assert(!(LK && TR), "large sets: inference operator");
    constexpr int NST = BN / 16;
    constexpr bool kHalf = sizeof(T) == 2;
    constexpr int LCAP = LK ? kMaxLandmarks : kSetSlots;
    typedef Tile<T, D, BN, 256, (BN == 64 ? 8 : Pad<T, D>::R)> KT;
    __shared__ __attribute__((aligned(16))) T Ks[2][KT::ELEMS];
    __shared__ __attribute__((aligned(16))) T Vs[2][KT::ELEMS];
    __shared__ int lpos[LCAP];
    __shared__ __attribute__((aligned(16))) float lbs[LCAP];
    // block scalars live in the second K buffer until the first chunk is staged there
    int* red = (int*)Ks[1];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4;
    const int total = p.n_heads * p.num_seqs * p.n_tiles;
    const int L = xcd_swizzle(blockIdx.x, total);
    // each XCD sweeps whole heads, the last tiles of a sequence (most landmarks) first
    const int t = p.n_tiles - 1 - L % p.n_tiles;
    const int s = (L / p.n_tiles) % p.num_seqs;
    const int h = L / (p.n_tiles * p.num_seqs);
    int st, len;
    seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
    const int r0 = t * 64;
    if (r0 >= len) return;
    const int kvh = h / (p.n_heads / p.n_kv_heads);
    const int K = p.k_lmk;
    const int64_t set_off = (((int64_t)h * p.num_seqs + s) * p.n_sets) * K;
    const float c2 = p.c2;
    const float inv_scale = p.inv_scale;
    const bool has_bias = p.lbias != nullptr;

    // Prologue: the loads that depend on no other load -- the landmark set, the row plan's
    // bounds and rows -- are issued together (every lane loads, from clamped addresses, so no
    // load waits on a branch), then the rows' windows, LSE and row vectors; the block's
    // largest visible landmark count follows from the tile's largest window start, so one
    // barrier (the set in LDS) precedes the counts and the first chunk.
    constexpr int NLV = LK ? 1 : kSetSlots / 256;  // LK: the set is staged by a loop below
    int lv[NLV], ln[NLV];
    float lb[NLV];
#pragma unroll
    for (int u = 0; u < NLV; ++u) {
        lv[u] = -1;
        ln[u] = -1;
        lb[u] = 0.f;
        if (!LK && u * 256 < K) {
            lv[u] = p.lmk[set_off + min(u * 256 + tid, K - 1)];
            ln[u] = p.lmk[set_off + min(u * 256 + tid + 1, K - 1)];
            if (has_bias) lb[u] = p.lbias[set_off + min(u * 256 + tid, K - 1)];
        }
    }
    // this wave's rows (ordered by window start) and their bounds, from the row plan
    const int uw = uniform(wave);
    const int64_t tile = (int64_t)s * p.n_tiles + t;
    const int* bnd = p.plan_bounds + tile * 16;
    const int wlo = bnd[uw * 4], wLmax = bnd[uw * 4 + 1], whi = bnd[uw * 4 + 2], wHmin = bnd[uw * 4 + 3];
    int blo = 0x7fffffff, bhi = -1, blmax = (int)0x80000000;
    if (lane < 4) {
        blo = bnd[lane * 4];
        blmax = bnd[lane * 4 + 1];
        bhi = bnd[lane * 4 + 2];
    }
    const int pm = p.plan_perm[tile * 64 + uw * 16 + (lane & 15)];
    __builtin_amdgcn_sched_barrier(0);  // the independent loads above issued before any is used
    const int i = r0 + pm;
    const bool valid = i < len;
    const int at = st + (valid ? i : 0);  // loads by every lane (a row past the end reads row 0)
    const int wi = max(p.w[at], 1);
    const float lse_raw = p.lse[(int64_t)at * p.n_heads + h];
    const float wt_raw = TR ? train_wt(p, p.w_cont[at]) : 0.f;
    const T* qhead = (const T*)p.q + (int64_t)st * p.q_st + (int64_t)h * p.q_sh;
    const T* dohead = (const T*)p.dout + (int64_t)st * p.do_st + (int64_t)h * p.do_sh;
    const T* ohead = (const T*)p.o + (int64_t)st * p.o_st + (int64_t)h * p.o_sh;
    RowReg<T, D> qr, dor, orr;
    qr.load(valid ? qhead + (int64_t)i * p.q_st : nullptr, qhead, g);
    dor.load(valid ? dohead + (int64_t)i * p.do_st : nullptr, dohead, g);
    orr.load(valid ? ohead + (int64_t)i * p.o_st : nullptr, ohead, g);
    // the band's key range, clamped to the sequence: a plan made for other windows or offsets
    // gives wrong values, never reads outside the sequence's rows
    blo = max(uniform(-wave_max(-blo)), 0);
    bhi = min(uniform(wave_max(bhi)), len - 1);
    blmax = uniform(wave_max(blmax));

    int nvalid;
    if constexpr (!LK) {
        int nv_loc = 0;  // one past the last valid slot (sets are ascending, -1 after the valid slots)
#pragma unroll
        for (int u = 0; u < NLV; ++u) {
            const int sl = u * 256 + tid;
            if (sl < K) {
                lpos[sl] = lv[u];
                if (has_bias) lbs[sl] = lb[u] * inv_scale;  // landmark bias in raw-score units
                if (lv[u] >= 0 && (sl + 1 == K || ln[u] < 0)) nv_loc = sl + 1;
            }
        }
        nv_loc = wave_max(nv_loc);
        if (lane == 0) red[4 + uw] = nv_loc;
        __syncthreads();
        nvalid = uniform(max(max(red[4], red[5]), max(red[6], red[7])));
    } else {
        nvalid = uniform(load_set(p, set_off, lpos, red + 4, tid, has_bias ? lbs : nullptr));
    }

    int lo = 0x7fffffff, hi = -1, cnt = 0, lou = 0x7fffffff;
    float wt = 0.f;
    if (valid) {
        lo = max(i - wi + 1, 0);
        lou = i - (wi - 1);
        hi = i;
        cnt = lower_bound_i(lpos, nvalid, lo);
        if (TR) wt = wt_raw;
    }
    // soft-edge bias and window gradient of keys lou .. lou+3 (training variant)
    float etb[TR ? kEdgeTab : 1], etg[TR ? kEdgeTab : 1];
    if (TR) edge_table(p, wt, etb, etg);
    const int lo_edge = TR ? wLmax + p.edge_keys : wLmax;  // keys from here on carry no edge bias
    float dwacc = 0.f;
    // per-row data of the key-parallel passes, head-major: a head's rows are contiguous
    const int64_t hrow = (int64_t)h * p.total_len + st + i;
    if (valid && g == 0 && p.cnt) p.cnt[hrow] = cnt;
    const int wcmax = uniform(row_max16(cnt)), wcmin = uniform(row_min16(valid ? cnt : 0));
    // the block's largest visible count: that of its largest window start (counts grow with it)
    const int bcm = uniform(lower_bound_i(lpos, nvalid, blmax));
    const int cs = (blo / BN) * BN;
    const int nband = (bhi - cs) / BN + 1;
    const int nchunks = nband + ceil_div(bcm, BN);

    // delta = rowsum(O * dO) over the stored (rounded) O
    float dpart = 0.f;
    if constexpr (kHalf) {
#pragma unroll
        for (int dc = 0; dc < D / 32; ++dc)
#pragma unroll
            for (int e = 0; e < 8; ++e) dpart += to_float(orr.x[dc][e]) * to_float(dor.x[dc][e]);
    } else {
#pragma unroll
        for (int m = 0; m < D / 4; ++m) dpart += orr.x[m] * dor.x[m];
    }
    const float dlt = sum_g4(dpart);
    float lse2 = 0.f;
    if (valid) {
        lse2 = lse_raw * kLog2eB;
        if (g == 0) {
            p.delta[hrow] = -dlt;
            p.lse2t[hrow] = lse2;
        }
    }

    const T* kbase = (const T*)p.k + (int64_t)st * p.k_st + (int64_t)kvh * p.k_sh;
    const T* vbase = (const T*)p.v + (int64_t)st * p.v_st + (int64_t)kvh * p.v_sh;
    // band chunks through buffer resources bounded at bhi, landmark chunks gathered
    const uint32_t krb = (uint32_t)(p.k_st * (int64_t)sizeof(T)), vrb = (uint32_t)(p.v_st * (int64_t)sizeof(T));
    uint32_t koff[KT::NV], voff[KT::NV];
#pragma unroll
    for (int n = 0; n < KT::NV; ++n) {
        koff[n] = KT::row_offset(tid, n, krb);
        voff[n] = KT::row_offset(tid, n, vrb);
    }
    // landmark rows: 32-bit offsets into resources over the sequence's rows when the
    // sequence spans less than 2 GiB of K and of V, else 64-bit row addresses (always
    // for D128, where the offsets would cost a wave of occupancy)
    const uint32_t kext = gather_extent(len, krb, D * sizeof(T)), vext = gather_extent(len, vrb, D * sizeof(T));
    const bool lmk32 = (D == 64) && kext != 0u && vext != 0u;
    const rsrc_t krs = make_rsrc(kbase, kext), vrs = make_rsrc(vbase, vext);
    KT kt, vt;
    // band rows [cs, bhi]: one resource per tensor over the whole band (rows past bhi read
    // zero), chunk c at byte offset c * BN * row bytes -- no per-chunk address arithmetic
    const rsrc_t kband = rows_rsrc(kbase + (int64_t)cs * p.k_st, bhi + 1 - cs, krb, D * sizeof(T));
    const rsrc_t vband = rows_rsrc(vbase + (int64_t)cs * p.v_st, bhi + 1 - cs, vrb, D * sizeof(T));
    // band chunks are loaded in order: the per-thread offsets advance by one chunk per load
    auto load_band = [&](int) {
        kt.load_rows(kband, koff);
        vt.load_rows(vband, voff);
#pragma unroll
        for (int n = 0; n < KT::NV; ++n) {
            koff[n] += (uint32_t)BN * krb;
            voff[n] += (uint32_t)BN * vrb;
        }
    };
    auto load_lmk = [&](int c) {  // landmark chunk c (slots c*BN ..)
        auto pos = [&](int rr) -> int {
            const int sl = c * BN + rr;
            const int q = sl < bcm ? lpos[sl] : -1;
            return q < len ? q : -1;
        };
        if (lmk32) {
            uint32_t ko[KT::NV], vo[KT::NV];
            KT::gather_offsets(tid, pos, krb, vrb, ko, vo);
            kt.load_rows(krs, ko);
            vt.load_rows(vrs, vo);
        } else {
            kt.load(tid, [&](int rr) { int j = pos(rr); return j >= 0 ? kbase + (int64_t)j * p.k_st : (const T*)nullptr; },
                    kbase);
            vt.load(tid, [&](int rr) { int j = pos(rr); return j >= 0 ? vbase + (int64_t)j * p.v_st : (const T*)nullptr; },
                    vbase);
        }
    };
    // landmark chunks first (their gathers only in the first loop), then the band
    const int nlmk = nchunks - nband;
    if (nlmk > 0) load_lmk(0);
    else load_band(0);
    kt.store(Ks[0], tid);
    vt.store(Vs[0], tid);
    __syncthreads();

    floatx4 acc[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) acc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    const float NEG = -INFINITY;
    const int lane_off = 4 * g;
    // one chunk; `band` is a compile-time tag, so the band and landmark loops below are
    // separate straight-line code
    // chunk n of the sweep: landmark chunk n (n < nlmk), else band chunk n - nlmk
    auto process = [&](int n, auto band_tag) {
        constexpr bool band = decltype(band_tag)::value;
        const int buf = n & 1;
        const int c = band ? n - nlmk : n;
        if (!band) {
            if (n + 1 < nlmk) load_lmk(n + 1);
            else if (nband > 0) load_band(0);
        } else if (c + 1 < nband) {
            load_band(c + 1);
        }
        const int base = band ? cs + c * BN : c * BN;
        floatx4 dS[NST];
        bool act[NST];
        // a band chunk some row sees is computed whole under the window mask (a subtile wholly
        // outside every window scores -inf and adds zeros: cheaper than the branches that
        // would skip it; the training variant, whose edge terms cost more, skips it);
        // landmark subtiles past the largest visible count are skipped
        const bool cact = band ? (base <= whi && base + BN - 1 >= wlo) : true;
#pragma unroll
        for (int stt = 0; stt < NST; ++stt) {
            const int a = base + stt * 16;
            act[stt] = band ? (TR ? (a <= whi && a + 15 >= wlo) : cact) : (a < wcmax);
            if (!act[stt]) {
                // an inactive band chunk of the inference variant adds nothing (both subtiles
                // share its activity, so its dS is never read); a skipped subtile beside an
                // active one adds zeros
                if (!band || TR) dS[stt] = floatx4{0.f, 0.f, 0.f, 0.f};
                continue;
            }
            floatx4 ci;
            floatx4 eg = floatx4{0.f, 0.f, 0.f, 0.f};  // d(bias)/d(w~) per key (training variant)
            if (band) {
                const int tl = lo - a - lane_off, th = hi - a - lane_off;
                if (TR && a >= lo_edge && a + 15 <= wHmin) {  // training: no edge bias, no mask
                    ci = floatx4{0.f, 0.f, 0.f, 0.f};
                } else {
                    // below every row's diagonal only the window start masks; the soft
                    // edge only reaches subtiles before lo_edge (wave-uniform tests)
                    // key a + lane_off + r in [lo, hi] (hi ignored below every row's diagonal): one
                    // unsigned compare of r - tl (a row past the end has lo > hi and fails it)
                    const bool upper = a + 15 > wHmin;
                    const int x0 = a + lane_off - lo;
                    const unsigned wd = upper ? (unsigned)hi - (unsigned)lo : 0x7fffffffu;
#pragma unroll
                    for (int r = 0; r < 4; ++r) ci[r] = (unsigned)(x0 + r) <= wd ? 0.f : NEG;
                    if (TR && a < lo_edge) {
                        if (p.edge_keys <= kEdgeTab) {
                            const int k0 = a + lane_off - lou;
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                const bool out = r < tl || r > th;
                                ci[r] = out ? NEG : edge_lookup(etb, k0 + r);
                                eg[r] = out ? 0.f : edge_lookup(etg, k0 + r);
                            }
                        } else {
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                float b, gr;
                                edge_terms(p, wt, th - r, b, gr);
                                const bool out = r < tl || r > th;
                                ci[r] = out ? NEG : b;
                                eg[r] = out ? 0.f : gr;
                            }
                        }
                    }
                }
            } else {
                // slots past the set's valid count are masked below (a + 15 < 512)
                const floatx4 bv = has_bias ? *(const floatx4*)(lbs + a + lane_off) : floatx4{0.f, 0.f, 0.f, 0.f};
                if (a + 15 < wcmin) {
                    ci = bv;
                } else {
                    const int tc = cnt - a - lane_off;
#pragma unroll
                    for (int r = 0; r < 4; ++r) ci[r] = r < tc ? bv[r] : NEG;
                }
            }
            const floatx4 sc = dot_rows<T, D>(Ks[buf], KT::RS, stt * 16, lane, qr, ci);
            const floatx4 dp = dot_rows<T, D>(Vs[buf], KT::RS, stt * 16, lane, dor, floatx4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int r = 0; r < 4; ++r) dS[stt][r] = __builtin_amdgcn_exp2f(sc[r] * c2 - lse2) * (dp[r] - dlt);
            if (TR && band)
#pragma unroll
                for (int r = 0; r < 4; ++r) dwacc += dS[stt][r] * eg[r];
        }
        if constexpr (kHalf) {
#pragma unroll
            for (int hp = 0; hp < NST / 2; ++hp)
                if (act[2 * hp] || act[2 * hp + 1])
                    acc_tr<T, D>(Ks[buf], KT::RS, hp * 32, lane, dS[2 * hp], dS[2 * hp + 1], acc);
        } else {
#pragma unroll
            for (int stt = 0; stt < NST; ++stt)
                if (act[stt]) acc_rm32<D>((const float*)Ks[buf], KT::RS, stt * 16, lane, dS[stt], acc);
        }
        if (n + 1 < nchunks) {
            kt.store(Ks[buf ^ 1], tid);
            vt.store(Vs[buf ^ 1], tid);
        }
        __syncthreads();
    };
    for (int n = 0; n < nlmk; ++n) process(n, std::false_type{});
    for (int n = nlmk; n < nchunks; ++n) process(n, std::true_type{});
    if (TR) {
        const float dw = sum_g4(dwacc);
        if (valid && g == 0) p.dw_h[(int64_t)(st + i) * p.n_heads + h] = dw;
    }
    const int64_t rstride = (int64_t)p.n_heads * D;
    T* dq0 = (T*)p.dq + (int64_t)st * rstride + (int64_t)h * D;
    if constexpr (!TR) {
        // dQ rows whole, staged in the idle K/V buffers (waves 0-1 in Ks, 2-3 in Vs)
        typedef StoreRows<T, D> SR;
        static_assert(KT::ELEMS >= SR::ELEMS, "row staging does not fit the chunk buffers");
        T* stage = (wave < 2 ? &Ks[0][0] : &Vs[0][0]) + (wave & 1) * SR::ELEMS;
        const int vi = valid ? i : -1;
        SR::run(stage, acc, p.scale, lane, [&](int rr) {
            const int ir = __shfl(vi, rr);
            return ir >= 0 ? dq0 + ir * rstride : (T*)nullptr;
        });
    } else if (valid) {  // (the training variant's registers leave no room for the staging)
        T* drow = dq0 + i * rstride;
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) {
            T ov[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) ov[r] = from_float<T>(acc[dt][r] * p.scale);
            if constexpr (kHalf) *(uint2*)(drow + dt * 16 + lane_off) = *(const uint2*)ov;
            else *(floatx4*)(drow + dt * 16 + lane_off) = *(const floatx4*)ov;
        }
    }
}

// ----------------------------------------------------- query-row staging
// BQ query rows of one (head, sequence): Q and dO row-major, plus per-row LSE
// (base 2), delta, and a per-row key: the window start in the dK/dV sweep, the
// visible landmark count in the landmark sweep (0 past the end).  Rows past
// the end are zero with LSE 0 and delta 0, so they contribute exactly zero.
template <typename T, int D, int BQ, bool TR = false, int NT = 256>
struct QStage {
    typedef Tile<T, D, BQ, NT> QT;
    T q[QT::ELEMS];
    T d[QT::ELEMS];
    float lse2[BQ];
    float dlt[BQ];  // -delta
    int key[BQ];
    float wt[TR ? BQ : 4];  // training variant: continuous window of the row
    int ri[TR ? BQ : 4];    // training variant: row index
};

template <typename T, int D, int BQ, int NT = 256>
struct QLoader {
    typedef Tile<T, D, BQ, NT> QT;
    QT tq, tdo;
    uint32_t qoff[QT::NV], doff[QT::NV];
    uint32_t qrb, drb;
    __device__ __forceinline__ QLoader(const AttnParams& p, int tid) {
        qrb = (uint32_t)(p.q_st * (int64_t)sizeof(T));
        drb = (uint32_t)(p.do_st * (int64_t)sizeof(T));
#pragma unroll
        for (int n = 0; n < QT::NV; ++n) {
            qoff[n] = QT::row_offset(tid, n, qrb);
            doff[n] = QT::row_offset(tid, n, drb);
        }
    }
    // resources over rows [i0, iend) of q and dO (later rows read as zero)
    __device__ __forceinline__ void span(const AttnParams& p, const T* qb, const T* db, int i0, int iend, rsrc_t& rq,
                                         rsrc_t& rd) const {
        rq = rows_rsrc(qb + (int64_t)i0 * p.q_st, iend - i0, qrb, D * sizeof(T));
        rd = rows_rsrc(db + (int64_t)i0 * p.do_st, iend - i0, drb, D * sizeof(T));
    }
    // rows c*BQ .. c*BQ + BQ - 1 of a span
    __device__ __forceinline__ void load(rsrc_t rq, rsrc_t rd, int c) {
        uint32_t q2[QT::NV], d2[QT::NV];
#pragma unroll
        for (int v = 0; v < QT::NV; ++v) {
            q2[v] = qoff[v] + (uint32_t)(c * BQ) * qrb;
            d2[v] = doff[v] + (uint32_t)(c * BQ) * drb;
        }
        tq.load_rows(rq, q2);
        tdo.load_rows(rd, d2);
    }
    // rows list[rr] (rr < BQ) of a span, a negative entry reading zero
    __device__ __forceinline__ void gather_list(rsrc_t rq, rsrc_t rd, const short* list, int tid) {
#pragma unroll
        for (int v = 0; v < QT::NV; ++v) {
            const int vi = tid + 256 * v;
            const uint32_t cb = (uint32_t)(vi % QT::CPR) * 16u;
            const int row = list[vi / QT::CPR];
            tq.r[v] = __builtin_amdgcn_raw_buffer_load_b128(rq, row >= 0 ? (uint32_t)row * qrb + cb : 0x80000000u, 0, 0);
            tdo.r[v] = __builtin_amdgcn_raw_buffer_load_b128(rd, row >= 0 ? (uint32_t)row * drb + cb : 0x80000000u, 0, 0);
        }
    }
    template <class QS>
    __device__ __forceinline__ void store(QS& q, int tid) const {
        tq.store(q.q, tid);
        tdo.store(q.d, tid);
    }
};

// -------------------------------------------------------------- band dK/dV
// Block = 64 keys j0..j0+63 of one (head, sequence); wave w owns keys
// j0+16w..+15, one key per lane (column of the transposed tiles).  Query rows
// that see any of these keys are i in [j0, j0 + 63 + largest window).  They are
// taken in three kinds:
//   diagonal rows j0..j0+63 (contiguous; window start and causal masks),
//   then, per segment of kSeg rows after the diagonal, the rows compacted
//   by their window start lo_i into
//     full rows    lo_i <= j0           (see all 64 keys: no mask), and
//     partial rows j0 < lo_i <= j0+63   (see keys >= lo_i: one-sided mask);
// rows with lo_i > j0 + 63 are skipped.  List order is row order, so the sum
// order is fixed and results are deterministic.
// four waves per SIMD for 16-bit head_dim 64 (32-row stages keep it free of spills; three with
// grouped heads or the training variant, which need more registers), two otherwise.
// TR: training variant -- fully visible rows must also see every key of the block
// past their edge_keys edge-bias keys; other rows add the soft edge bias.
// GQA: the key/value head has several query heads (swept in order); without it the
// sweep is straight-line code for one head.
template <typename T, int D, int BQ, int NT = 256>
struct QTiles {  // one staged chunk of the dK/dV sweep: BQ rows of Q and of dO
    typedef Tile<T, D, BQ, NT> QT;
    T q[QT::ELEMS];
    T d[QT::ELEMS];
};

template <typename T, int D, bool TR, bool GQA>
__global__ __launch_bounds__(256, (sizeof(T) == 2 && D == 64) ? ((GQA || TR) ? 3 : 4) : 2) void bwd_dkdv_kernel(AttnParams p) {
    constexpr int BQ = BwdShape<T, D>::BQ;
    constexpr int NQS = BQ / 16;
    constexpr int NDIAG = 64 / BQ;
    constexpr bool kHalf = sizeof(T) == 2;
    // list positions of a segment: full rows from 0, partial rows from the next chunk
    // boundary, each list padded to whole chunks
    constexpr int kLst = kSeg + 2 * BQ;
    typedef QTiles<T, D, BQ> QS;
    typedef typename QS::QT QT;
    __shared__ __attribute__((aligned(16))) QS sq[2];
    __shared__ int wcnt[4][8];
    // per-row data of the rows a chunk covers, in chunk order, read by the products straight
    // from these tables: window start (0x7fffffff for no row), LSE in base 2, -delta (0 for
    // no row)[, continuous window, row index]; a segment's rows in list order with their row
    // offsets (-1 for padding) for the gathers, the 64 diagonal rows in row order
    __shared__ short lrw[kLst];
    __shared__ __attribute__((aligned(16))) int lt_lo[kLst];
    __shared__ __attribute__((aligned(16))) float lt_l[kLst], lt_d[kLst];
    __shared__ __attribute__((aligned(16))) float lt_wt[TR ? kLst : 4];
    __shared__ __attribute__((aligned(16))) int lt_ri[TR ? kLst : 4];
    __shared__ __attribute__((aligned(16))) int dt_lo[64];
    __shared__ __attribute__((aligned(16))) float dt_l[64], dt_d[64];
    __shared__ __attribute__((aligned(16))) float dt_wt[TR ? 64 : 4];
    __shared__ int own_s[64];  // per key of the block: h * K + slot of its owner, or kNoOwner
    __shared__ int wmax_s[4];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4;
    const int total = p.n_kv_heads * p.num_seqs * p.n_tiles;
    const int L = xcd_swizzle(blockIdx.x, total);
    const int t = L % p.n_tiles;
    const int s = (L / p.n_tiles) % p.num_seqs;
    const int kvh = L / (p.n_tiles * p.num_seqs);
    const int rep = GQA ? p.n_heads / p.n_kv_heads : 1;
    int st, len;
    seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
    const int j0 = t * 64;
    if (j0 >= len) return;
    const float c2 = p.scale * kLog2eB;

    const int wj0 = uniform(j0 + wave * 16);
    const int j = wj0 + (lane & 15);
    const bool jvalid = j < len;
    const int jj = jvalid ? j : -1;  // below every window start when past the end
    const T* khead = (const T*)p.k + (int64_t)st * p.k_st + (int64_t)kvh * p.k_sh;
    const T* vhead = (const T*)p.v + (int64_t)st * p.v_st + (int64_t)kvh * p.v_sh;
    RowReg<T, D> kr, vr;
    kr.load(jvalid ? khead + (int64_t)j * p.k_st : nullptr, khead, g);
    vr.load(jvalid ? vhead + (int64_t)j * p.v_st : nullptr, vhead, g);

    // The sequence's largest window, from the row plan's tile maxima, bounds the rows to
    // sweep (known after the first barrier; the diagonal rows end at dend <= iend).  Keys of
    // the block that are landmark rows get their owner: the first (head, slot) of the group
    // holding the row (first copy of a repeated position, heads in order; an integer
    // minimum over LDS atomics, so the same whatever their order).
    const int dend = min(len, j0 + 64);
    int iend = dend;
    const int* wrow = p.w + st;
    QLoader<T, D, BQ> ld(p, tid);
    floatx4 adk[D / 16], adv[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
        adk[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
        adv[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    const float NEG = -INFINITY;
    const int lane_off = 4 * g;
    const int seg0 = j0 + 64;  // first row after the diagonal
    // one query head per key/value head: the first segment is prepared in the prologue and its
    // first chunk fetched under the last diagonal stage; grouped heads (more registers live
    // across the head loop) take every segment in the sweep after the diagonal
    constexpr bool kPre = !GQA;
    // the query heads of this key/value head are swept one after the other (head order),
    // all adding into the same dK/dV registers
    for (int hh = 0; hh < rep; ++hh) {
    const int h = kvh * rep + hh;
    const T* qb = (const T*)p.q + (int64_t)st * p.q_st + (int64_t)h * p.q_sh;
    const T* db = (const T*)p.dout + (int64_t)st * p.do_st + (int64_t)h * p.do_sh;
    const float* lrow = p.lse2t + (int64_t)h * p.total_len + st;
    const float* drow = p.delta + (int64_t)h * p.total_len + st;
    // a row's data: window start, LSE, -delta[, continuous window]
    struct RowData {
        int lo;
        float l, d, wt;
    };
    auto load_row = [&](int i) {
        RowData r;
        const int wi = max(wrow[i], 1);
        r.lo = max(i - wi + 1, 0);
        r.l = lrow[i];
        r.d = drow[i];
        r.wt = TR ? train_wt(p, p.w_cont[st + i]) : 0.f;
        return r;
    };

    // one staged chunk; kind 0: diagonal rows from i0, 1: full rows, 2: partial rows; its
    // per-row data at position `pos` of the diagonal table (dg) or the segment's list table.
    // Query subtiles are taken in the groups one accumulation consumes (two 16-row
    // subtiles for 16-bit types), so only one group's P and dS are live at a time.
    constexpr int GQ = kHalf ? 2 : 1;
    auto compute = [&](auto diag_tag, const QS& q, int kind, int i0, int pos) {
        constexpr bool dg = decltype(diag_tag)::value;
#pragma unroll
        for (int hp = 0; hp < NQS / GQ; ++hp) {
            floatx4 P[GQ], dS[GQ];
            bool act[GQ];
            bool any = false;
#pragma unroll
            for (int u = 0; u < GQ; ++u) {
                const int qs = hp * GQ + u;
                const int qa = i0 + qs * 16;
                const int e = pos + qs * 16 + lane_off;  // table entry of the lane's first row
                act[u] = kind != 0 || qa + 15 >= wj0;
                any |= act[u];
                if (!act[u]) {
                    P[u] = floatx4{0.f, 0.f, 0.f, 0.f};
                    dS[u] = P[u];
                    continue;
                }
                floatx4 ci = floatx4{0.f, 0.f, 0.f, 0.f};
                if (kind != 1) {
                    const int4 lo4 = *(const int4*)((dg ? dt_lo : lt_lo) + e);
                    floatx4 eb = floatx4{0.f, 0.f, 0.f, 0.f};
                    // the soft edge reaches this key only for rows with jj < lo + edge_keys:
                    // skipped unless some lane of the wave has such a row
                    if (TR && __builtin_amdgcn_ballot_w64(jj < lo4.x + p.edge_keys || jj < lo4.y + p.edge_keys ||
                                                          jj < lo4.z + p.edge_keys || jj < lo4.w + p.edge_keys)) {
                        const floatx4 w4 = *(const floatx4*)((dg ? dt_wt : lt_wt) + e);
                        const int4 i4 = dg ? int4{qa + lane_off, qa + lane_off + 1, qa + lane_off + 2, qa + lane_off + 3}
                                           : *(const int4*)(lt_ri + e);
                        eb[0] = edge_bias(p, w4[0], i4.x - jj);
                        eb[1] = edge_bias(p, w4[1], i4.y - jj);
                        eb[2] = edge_bias(p, w4[2], i4.z - jj);
                        eb[3] = edge_bias(p, w4[3], i4.w - jj);
                    }
                    if (kind == 2 || qa >= wj0 + 15) {
                        ci[0] = jj >= lo4.x ? eb[0] : NEG;
                        ci[1] = jj >= lo4.y ? eb[1] : NEG;
                        ci[2] = jj >= lo4.z ? eb[2] : NEG;
                        ci[3] = jj >= lo4.w ? eb[3] : NEG;
                    } else {
                        const int qd = qa + lane_off - jj;  // row index minus key index, r = 0
                        ci[0] = (jj >= lo4.x && qd >= 0) ? eb[0] : NEG;
                        ci[1] = (jj >= lo4.y && qd + 1 >= 0) ? eb[1] : NEG;
                        ci[2] = (jj >= lo4.z && qd + 2 >= 0) ? eb[2] : NEG;
                        ci[3] = (jj >= lo4.w && qd + 3 >= 0) ? eb[3] : NEG;
                    }
                }
                const floatx4 nd4 = *(const floatx4*)((dg ? dt_d : lt_d) + e);  // -delta
                const floatx4 sc = dot_rows<T, D>(q.q, QT::RS, qs * 16, lane, kr, ci);
                const floatx4 dp = dot_rows<T, D>(q.d, QT::RS, qs * 16, lane, vr, nd4);  // dP - delta
                const floatx4 l4 = *(const floatx4*)((dg ? dt_l : lt_l) + e);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float pr = __builtin_amdgcn_exp2f(sc[r] * c2 - l4[r]);
                    P[u][r] = pr;
                    dS[u][r] = pr * dp[r];
                }
            }
            if (!any) continue;
            if constexpr (kHalf) {
                acc_tr<T, D>(q.d, QT::RS, hp * 32, lane, P[0], P[1], adv);
                acc_tr<T, D>(q.q, QT::RS, hp * 32, lane, dS[0], dS[1], adk);
            } else {
                acc_rm32<D>((const float*)q.d, QT::RS, hp * 16, lane, P[0], adv);
                acc_rm32<D>((const float*)q.q, QT::RS, hp * 16, lane, dS[0], adk);
            }
        }
    };

    // A segment's rows in two lists (row order within each): full rows lo <= j0 (no mask)
    // and partial rows j0 < lo <= j0 + 63; rows with lo > j0 + 63 are skipped.  The per-wave
    // counts of flags bf / bp go to wcnt; list_rows writes the lists' row offsets and row data
    // once the counts are visible, and pads each list to whole chunks.
    auto flag_rows = [&](int lo, bool ok, bool& f, bool& pp) {
        f = ok && lo <= j0 - (TR ? p.edge_keys : 0);
        pp = ok && !f && lo <= j0 + 63;
    };
    auto count_rows = [&](const uint64_t* bf, const uint64_t* bp) {
        if (lane == 0) {
#pragma unroll
            for (int u = 0; u < kSeg / 256; ++u) {
                wcnt[wave][u] = __popcll(bf[u]);
                wcnt[wave][4 + u] = __popcll(bp[u]);
            }
        }
    };
    int nfc = 0, nc = 0;
    auto list_rows = [&](const uint64_t* bf, const uint64_t* bp, auto row_data, int seg) {
        int basef[kSeg / 256], basep[kSeg / 256];
        int nf = 0, np = 0;
#pragma unroll
        for (int u = 0; u < kSeg / 256; ++u) {
            basef[u] = nf;
            basep[u] = np;
            for (int w2 = 0; w2 < 4; ++w2) {
                const int cf = wcnt[w2][u], cp = wcnt[w2][4 + u];
                if (w2 < wave) {
                    basef[u] += cf;
                    basep[u] += cp;
                }
                nf += cf;
                np += cp;
            }
        }
        nf = uniform(nf);
        np = uniform(np);
        nfc = ceil_div(nf, BQ);
        nc = nfc + ceil_div(np, BQ);
        const int pbase = nfc * BQ;
#pragma unroll
        for (int u = 0; u < kSeg / 256; ++u) {
            const uint32_t flo = (uint32_t)bf[u], fhi = (uint32_t)(bf[u] >> 32);
            const uint32_t plo = (uint32_t)bp[u], phi = (uint32_t)(bp[u] >> 32);
            const int rf = __builtin_amdgcn_mbcnt_hi(fhi, __builtin_amdgcn_mbcnt_lo(flo, 0));
            const int rp = __builtin_amdgcn_mbcnt_hi(phi, __builtin_amdgcn_mbcnt_lo(plo, 0));
            const uint64_t me = 1ull << lane;
            const bool inf = (bf[u] & me) != 0, inp = (bp[u] & me) != 0;
            if (inf || inp) {
                const int at = inf ? basef[u] + rf : pbase + basep[u] + rp;
                const int r = u * 256 + tid;
                const RowData x = row_data(u);
                lrw[at] = (short)r;
                lt_lo[at] = x.lo;
                lt_l[at] = x.l;
                lt_d[at] = x.d;
                if (TR) {
                    lt_wt[at] = x.wt;
                    lt_ri[at] = seg + r;
                }
            }
        }
        // padding: rows of no list (zero Q and dO rows, LSE and -delta 0, no key visible)
        if (tid < 2 * BQ) {
            const int at = tid < BQ ? nf + tid : pbase + np + (tid - BQ);
            const int lim = tid < BQ ? pbase : nc * BQ;
            if (at < lim) {
                lrw[at] = -1;
                lt_lo[at] = 0x7fffffff;
                lt_l[at] = 0.f;
                lt_d[at] = 0.f;
                if (TR) {
                    lt_wt[at] = 0.f;
                    lt_ri[at] = 0;
                }
            }
        }
    };
    int seg = seg0;
    rsrc_t rqs, rds;  // rows of the current segment
    auto gather_chunk = [&](int c) { ld.gather_list(rqs, rds, lrw + c * BQ, tid); };

    // ---- prologue: the diagonal rows' first tile and data, the first segment's row data and
    // flags (rows seg0 .. seg0 + kSeg - 1 below the sequence end; rows past the largest
    // window reach are never flagged), the window bound and the landmark owners' positions:
    // every load here depends on no other; all are issued (by every lane, from clamped
    // addresses, so no load waits on a branch) before any is used, and waited for at one
    // barrier
    const int ndiag = uniform(min(NDIAG, ceil_div(dend - j0, BQ)));
    rsrc_t rq, rd;
    ld.span(p, qb, db, j0, dend, rq, rd);
    ld.load(rq, rd, 0);
    const RowData dgr = load_row(min(j0 + (tid & 63), len - 1));
    RowData rdat[kSeg / 256];
#pragma unroll
    for (int u = 0; u < kSeg / 256; ++u) rdat[u] = load_row(min(seg0 + u * 256 + tid, len - 1));
    constexpr int kWm = 4;  // tile maxima read before the barrier by each thread (more: a loop)
    int wmv[kWm];
    int ov = -1, ovp = -1;  // this thread's landmark slot among the first 256 of the group, and the one before
    const int K = p.k_lmk;
    const int nown = rep * K;
    const int32_t* oset = p.lmk + (((int64_t)(kvh * rep + min(tid, max(nown, 1) - 1) / max(K, 1)) * p.num_seqs + s) *
                                   p.n_sets) * K;
    const int osl = K > 0 ? min(tid, nown - 1) % K : 0;
    if (hh == 0) {
#pragma unroll
        for (int k = 0; k < kWm; ++k) wmv[k] = p.tile_wmax[(int64_t)s * p.n_tiles + min(tid + 256 * k, p.n_tiles - 1)];
        if (nown > 0) {
            ov = oset[osl];
            ovp = oset[max(osl - 1, 0)];
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // the loads above issued before any is used
    if (tid < 64) {
        const bool ok = j0 + tid < dend;
        dt_lo[tid] = ok ? dgr.lo : 0x7fffffff;
        dt_l[tid] = ok ? dgr.l : 0.f;
        dt_d[tid] = ok ? dgr.d : 0.f;
        if (TR) dt_wt[tid] = ok ? dgr.wt : 0.f;
    }
    uint64_t bf[kSeg / 256], bp[kSeg / 256];
#pragma unroll
    for (int u = 0; u < kSeg / 256; ++u) {
        const bool ok = kPre && seg0 + u * 256 + tid < len;
        bool f, pp;
        flag_rows(rdat[u].lo, ok, f, pp);
        bf[u] = __ballot(f);
        bp[u] = __ballot(pp);
    }
    if (kPre) count_rows(bf, bp);
    int own_at = -1, own_id = 0;
    if (hh == 0) {
        if (tid < 64) own_s[tid] = kNoOwner;
        int wm = 1;
#pragma unroll
        for (int k = 0; k < kWm; ++k) wm = max(wm, wmv[k]);
        for (int u = tid + 256 * kWm; u < p.n_tiles; u += 256) wm = max(wm, p.tile_wmax[(int64_t)s * p.n_tiles + u]);
        wm = wave_max(wm);
        if (lane == 0) wmax_s[wave] = wm;
        // the slot values are first used here (not where they were loaded)
        asm volatile("" : "+v"(ov), "+v"(ovp));
        if (tid < nown && ov >= j0 && ov < dend && (osl == 0 || ovp != ov)) {
            own_at = ov - j0;
            own_id = (kvh * rep + tid / K) * K + osl;
        }
    }
    __syncthreads();
    iend = uniform(min(len, j0 + 63 + max(max(wmax_s[0], wmax_s[1]), max(wmax_s[2], wmax_s[3]))));
    if (hh == 0) {
        if (own_at >= 0) atomicMin(own_s + own_at, own_id);
        for (int e = tid + 256; e < rep * K; e += 256) {  // groups of more than 256 slots
            const int hs = e / K, sl = e % K;
            const int32_t* set = p.lmk + (((int64_t)(kvh * rep + hs) * p.num_seqs + s) * p.n_sets) * K;
            const int v = set[sl];
            if (v >= j0 && v < dend && (sl == 0 || set[sl - 1] != v)) atomicMin(own_s + (v - j0), (kvh * rep + hs) * K + sl);
        }
    }
    if (kPre) list_rows(bf, bp, [&](int u) { return rdat[u]; }, seg0);
    ld.span(p, qb, db, seg0, min(len, seg0 + kSeg), rqs, rds);
    ld.store(sq[0], tid);
    __syncthreads();

    // ---- diagonal rows j0 .. j0+63, then the first segment's chunks: one double-buffered
    // sweep (the last diagonal stage fetches the segment's first chunk)
    for (int c = 0; c < ndiag; ++c) {
        const int buf = c & 1;
        const bool last = c + 1 == ndiag;
        if (!last) ld.load(rq, rd, c + 1);
        else if (nc > 0) gather_chunk(0);
        compute(std::true_type{}, sq[buf], 0, j0 + c * BQ, c * BQ);
        if (!last || nc > 0) ld.store(sq[buf ^ 1], tid);
        __syncthreads();
    }
    for (int c = 0; c < nc; ++c) {
        const int buf = (ndiag + c) & 1;
        if (c + 1 < nc) gather_chunk(c + 1);
        compute(std::false_type{}, sq[buf], c < nfc ? 1 : 2, 0, c * BQ);
        if (c + 1 < nc) ld.store(sq[buf ^ 1], tid);
        __syncthreads();
    }

    // ---- later segments (windows longer than kSeg - 63 rows), one at a time; their rows'
    // data wait for the list positions in the second tile buffer (free until the segment's
    // second chunk), not in registers
    static_assert(sizeof(QS) >= sizeof(float) * (TR ? 4 : 3) * kSeg, "row scratch does not fit a tile buffer");
    float* scr = (float*)&sq[1];
    for (seg = kPre ? seg0 + kSeg : seg0; seg < iend; seg += kSeg) {
        const int nrows = uniform(min(kSeg, iend - seg));
#pragma unroll
        for (int u = 0; u < kSeg / 256; ++u) {
            const int r = u * 256 + tid;
            const bool ok = r < nrows;
            const RowData x = ok ? load_row(seg + r) : RowData{0x7fffffff, 0.f, 0.f, 0.f};
            scr[r] = __int_as_float(x.lo);
            scr[kSeg + r] = x.l;
            scr[2 * kSeg + r] = x.d;
            if (TR) scr[3 * kSeg + r] = x.wt;
            bool f, pp;
            flag_rows(x.lo, ok, f, pp);
            bf[u] = __ballot(f);
            bp[u] = __ballot(pp);
        }
        count_rows(bf, bp);
        __syncthreads();
        list_rows(bf, bp, [&](int u) {
            const int r = u * 256 + tid;
            return RowData{__float_as_int(scr[r]), scr[kSeg + r], scr[2 * kSeg + r], TR ? scr[3 * kSeg + r] : 0.f};
        }, seg);
        __syncthreads();
        ld.span(p, qb, db, seg, seg + nrows, rqs, rds);
        if (nc > 0) {
            gather_chunk(0);
            ld.store(sq[0], tid);
        }
        __syncthreads();
        for (int c = 0; c < nc; ++c) {
            const int buf = c & 1;
            if (c + 1 < nc) gather_chunk(c + 1);
            compute(std::false_type{}, sq[buf], c < nfc ? 1 : 2, 0, c * BQ);
            if (c + 1 < nc) ld.store(sq[buf ^ 1], tid);
            __syncthreads();
        }
    }
    }  // query heads of the group

    bool owner = false;
    if (jvalid && p.k_lmk > 0) {
        // a landmark row: its band sums go to the landmark pass's final sum in fp32, which
        // rounds the total once (and writes the row)
        const int own = own_s[j - j0];
        if (own != kNoOwner) {
            owner = true;
            const int64_t so = (((int64_t)(own / p.k_lmk) * p.num_seqs + s) * p.k_lmk + own % p.k_lmk) * D;
            const int64_t half = (int64_t)p.n_heads * p.num_seqs * p.k_lmk * D;
#pragma unroll
            for (int dt = 0; dt < D / 16; ++dt) {
                *(floatx4*)(p.lmk_stage + so + dt * 16 + lane_off) = adk[dt] * p.scale;
                *(floatx4*)(p.lmk_stage + half + so + dt * 16 + lane_off) = adv[dt];
            }
        }
    }
    // the other rows: dK, then dV, as whole rows staged in the wave's part of the query tile
    // buffers (idle after the last barrier)
    typedef StoreRows<T, D> SR;
    static_assert(sizeof(sq) >= sizeof(T) * 4 * SR::ELEMS, "row staging does not fit the tile buffers");
    T* stage = (T*)&sq[0] + wave * SR::ELEMS;
    const int wr = jvalid && !owner;
    const int64_t rstride = (int64_t)p.n_kv_heads * D;
    T* kd0 = (T*)p.dk + (int64_t)(st + wj0) * rstride + (int64_t)kvh * D;
    T* vd0 = (T*)p.dv + (int64_t)(st + wj0) * rstride + (int64_t)kvh * D;
    SR::run(stage, adk, p.scale, lane, [&](int rr) { return __shfl(wr, rr) ? kd0 + rr * rstride : (T*)nullptr; });
    SR::run(stage, adv, 1.0f, lane, [&](int rr) { return __shfl(wr, rr) ? vd0 + rr * rstride : (T*)nullptr; });
}

// -------------------------------------------------------- landmark dK/dV
// Block = (head, sequence, chunk c, group of 16*NW slots) with NW waves; wave w owns slots
// grp*16*NW + 16*w .. +15.  Chunk c takes the BQ-row tiles c, c + n_chunks, c + 2 n_chunks,
// ... of the sequence: a row sees more landmarks the later it is, so strided tiles give
// every block the same work (the kernel lasts as long as its longest block).  Each row tile
// is read from memory once per slot group: eight waves (128 slots) where a set has more
// than 64 slots and the registers allow four waves per SIMD (16-bit, head_dim 64), else four.
template <typename T, int D>
constexpr int lmk_waves(int k_lmk) { return (sizeof(T) == 2 && D == 64 && k_lmk > 64) ? 8 : 4; }

// LK: sets of more than kSetSlots landmarks (the set's positions in a larger LDS copy).
// (16-bit head_dim 128 in four-wave blocks is held to three waves per SIMD: 166 VGPRs, no
// spills, from 170 at two)
template <typename T, int D, int NW, bool LK = false>
__global__ __launch_bounds__(64 * NW, (NW == 8 && sizeof(T) == 2 && D == 64) ? 4
                                      : (NW == 4 && sizeof(T) == 2 && D == 128) ? 3 : 2) void bwd_lmk_kernel(AttnParams p) {
    constexpr int NT = 64 * NW;
    constexpr int kLmkGroup = 16 * NW;
    constexpr int BQ = BwdShape<T, D>::BL;
    constexpr int NQS = BQ / 16;
    constexpr bool kHalf = sizeof(T) == 2;
    typedef QStage<T, D, BQ, false, NT> QS;
    typedef typename QS::QT QT;
    __shared__ __attribute__((aligned(16))) QS q;
    __shared__ int lpos[LK ? kMaxLandmarks : kSetSlots];
    __shared__ int cmax_s[NQS];
    __shared__ int nvalid_s;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4;
    const int K = p.k_lmk;
    const int ngrp = ceil_div(K, kLmkGroup);
    int b = blockIdx.x;
    const int grp = b % ngrp;
    b /= ngrp;
    const int chunk = b % p.n_chunks;
    b /= p.n_chunks;
    const int s = b % p.num_seqs;
    const int h = b / p.num_seqs;
    int st, len;
    seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
    const int kvh = h / (p.n_heads / p.n_kv_heads);
    const int64_t set_off = (((int64_t)h * p.num_seqs + s) * p.n_sets) * K;
    const float c2 = p.c2;
    const float inv_scale = p.inv_scale;
    const int nvalid = load_set(p, set_off, lpos, &nvalid_s, tid, nullptr, NT);

    // slots of this lane
    constexpr int kLmkSub = 1;
    const int sl0 = uniform(grp * kLmkGroup + wave * 16);
    RowReg<T, D> kr[kLmkSub], vr[kLmkSub];
    int slot[kLmkSub];
    float bsl[kLmkSub];
    const T* kbase = (const T*)p.k + (int64_t)st * p.k_st + (int64_t)kvh * p.k_sh;
    const T* vbase = (const T*)p.v + (int64_t)st * p.v_st + (int64_t)kvh * p.v_sh;
#pragma unroll
    for (int u = 0; u < kLmkSub; ++u) {
        slot[u] = sl0 + u * 16 + (lane & 15);
        const bool sval = slot[u] < nvalid && lpos[slot[u]] < len;
        kr[u].load(sval ? kbase + (int64_t)lpos[slot[u]] * p.k_st : nullptr, kbase, g);
        vr[u].load(sval ? vbase + (int64_t)lpos[slot[u]] * p.v_st : nullptr, vbase, g);
        bsl[u] = (p.lbias && slot[u] < K) ? p.lbias[set_off + slot[u]] * inv_scale : 0.f;
    }
    floatx4 adk[kLmkSub][D / 16], adv[kLmkSub][D / 16];
    float dbias[kLmkSub];
#pragma unroll
    for (int u = 0; u < kLmkSub; ++u) dbias[u] = 0.f;
#pragma unroll
    for (int u = 0; u < kLmkSub; ++u)
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) {
            adk[u][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
            adv[u][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
    const T* qb = (const T*)p.q + (int64_t)st * p.q_st + (int64_t)h * p.q_sh;
    const T* db = (const T*)p.dout + (int64_t)st * p.do_st + (int64_t)h * p.do_sh;
    const float NEG = -INFINITY;
    const int lane_off = 4 * g;
    // first row with any visible landmark: lo_i > lpos[0]  =>  i > lpos[0]; tiles wholly
    // before it are skipped
    const int first_row = nvalid > 0 ? lpos[0] + 1 : 0x7fffffff;
    const int ntile = ceil_div(len, BQ);
    int t0 = chunk;
    if (nvalid > 0 && t0 < first_row / BQ) t0 += ceil_div(first_row / BQ - t0, p.n_chunks) * p.n_chunks;
    // the loop bound is uniform over the block (every wave reaches each barrier);
    // waves whose slots are all empty skip their products through act[] below
    const bool any_slot = grp * kLmkGroup < nvalid;
    QLoader<T, D, BQ, NT> ld(p, tid);
    // row tile t (q, dO and per-row data) fetched into registers one tile ahead: its memory
    // latency overlaps the products of the tile before
    int c = 0;
    float rl = 0.f, rd = 0.f;
    auto fetch = [&](int t) {
        const int i0 = t * BQ;
        rsrc_t rq, rdo;
        ld.span(p, qb, db, i0, min(len, i0 + BQ), rq, rdo);
        ld.load(rq, rdo, 0);
        c = 0;
        rl = rd = 0.f;
        if (tid < BQ && i0 + tid < len) {
            const int64_t hr = (int64_t)h * p.total_len + st + i0 + tid;
            c = p.cnt[hr];
            rl = p.lse2t[hr];
            rd = p.delta[hr];
        }
    };
    if (any_slot && t0 < ntile) fetch(t0);
    // rows staged in LDS; visible landmark counts come from the dQ pass
    for (int t = t0; any_slot && t < ntile; t += p.n_chunks) {
        __syncthreads();
        ld.store(q, tid);
        if (tid < BQ) {
            q.lse2[tid] = rl;
            q.dlt[tid] = rd;
            q.key[tid] = c;
            const int mx = row_max16(c);
            if ((tid & 15) == 0) cmax_s[tid >> 4] = mx;
        }
        __syncthreads();
        if (t + p.n_chunks < ntile) fetch(t + p.n_chunks);
#pragma unroll
        for (int u = 0; u < kLmkSub; ++u) {
            const int a = sl0 + u * 16;
            floatx4 P[NQS], dS[NQS];
            bool act[NQS];
            // a tile with some row seeing one of the wave's slots is computed whole under the
            // count mask (subtiles whose rows see none of them add zeros: cheaper than the
            // branches that would skip them or drop the mask)
            int tmx = cmax_s[0];
#pragma unroll
            for (int qs = 1; qs < NQS; ++qs) tmx = max(tmx, cmax_s[qs]);
            const bool tact = uniform(tmx) > a;
#pragma unroll
            for (int qs = 0; qs < NQS; ++qs) {
                act[qs] = tact;
                if (!act[qs]) {
                    P[qs] = floatx4{0.f, 0.f, 0.f, 0.f};
                    dS[qs] = P[qs];
                    continue;
                }
                floatx4 ci;
                const int4 c4 = *(const int4*)(q.key + qs * 16 + lane_off);
                ci[0] = slot[u] < c4.x ? bsl[u] : NEG;
                ci[1] = slot[u] < c4.y ? bsl[u] : NEG;
                ci[2] = slot[u] < c4.z ? bsl[u] : NEG;
                ci[3] = slot[u] < c4.w ? bsl[u] : NEG;
                const floatx4 sc = dot_rows<T, D>(q.q, QT::RS, qs * 16, lane, kr[u], ci);
                const floatx4 dp = dot_rows<T, D>(q.d, QT::RS, qs * 16, lane, vr[u], floatx4{0.f, 0.f, 0.f, 0.f});
                const floatx4 l4 = *(const floatx4*)(q.lse2 + qs * 16 + lane_off);
                const floatx4 nd4 = *(const floatx4*)(q.dlt + qs * 16 + lane_off);  // -delta
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float pr = __builtin_amdgcn_exp2f(sc[r] * c2 - l4[r]);
                    const float dd = pr * (dp[r] + nd4[r]);
                    P[qs][r] = pr;
                    dS[qs][r] = dd;
                    dbias[u] += dd;
                }
            }
            if constexpr (kHalf) {
#pragma unroll
                for (int hp = 0; hp < NQS / 2; ++hp)
                    if (act[2 * hp] || act[2 * hp + 1]) {
                        acc_tr<T, D>(q.d, QT::RS, hp * 32, lane, P[2 * hp], P[2 * hp + 1], adv[u]);
                        acc_tr<T, D>(q.q, QT::RS, hp * 32, lane, dS[2 * hp], dS[2 * hp + 1], adk[u]);
                    }
            } else {
#pragma unroll
                for (int qs = 0; qs < NQS; ++qs)
                    if (act[qs]) {
                        acc_rm32<D>((const float*)q.d, QT::RS, qs * 16, lane, P[qs], adv[u]);
                        acc_rm32<D>((const float*)q.q, QT::RS, qs * 16, lane, dS[qs], adk[u]);
                    }
            }
        }
    }
    // partials: [chunk][h][s][slot][D]
#pragma unroll
    for (int u = 0; u < kLmkSub; ++u) {
        const float db2 = sum_g4(dbias[u]);
        if (slot[u] >= K) continue;
        const int64_t row = (((int64_t)chunk * p.n_heads + h) * p.num_seqs + s) * K + slot[u];
        float* pk = p.part_k + row * D;
        float* pv = p.part_v + row * D;
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) {
            *(floatx4*)(pk + dt * 16 + lane_off) = adk[u][dt] * p.scale;
            *(floatx4*)(pv + dt * 16 + lane_off) = adv[u][dt];
        }
        if (g == 0) p.part_b[row] = db2;
    }
}

// Position of `pos` in a landmark set (ascending, -1 padding after the valid slots), or -1.
__device__ __forceinline__ int find_slot(const int32_t* set, int K, int pos) {
    int lo = 0, hi = K;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        const int v = set[mid];
        if (v >= 0 && v < pos) lo = mid + 1;
        else hi = mid;
    }
    return lo < K && set[lo] == pos ? lo : -1;
}

// One thread per (head, sequence, slot, column): d_bias from the slot's chunk partials in
// chunk order; the owner of a landmark row (the first (head, slot) of the key/value head's
// group holding it) writes the row's dK/dV once: its band sums from the dK/dV pass, then
// the chunk partials of every head of the group holding the row, heads and chunks in
// order, rounded to the output type once.
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
    const int rep = p.n_heads / p.n_kv_heads, kvh = h / rep;
    const int32_t* set = p.lmk + (((int64_t)h * p.num_seqs + s) * p.n_sets) * K;
    const int pos = set[sl];
    int st, len;
    seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
    const int64_t cstride = (int64_t)p.n_heads * p.num_seqs * K;
    auto prow = [&](int hh, int slot) { return (int64_t)hh * p.num_seqs * K + (int64_t)s * K + slot; };
    if (d == 0 && p.d_bias) {
        float sb = 0.f;
        constexpr int U = 8;  // eight chunks' loads in flight at a time, summed in chunk order
        for (int ch0 = 0; ch0 < p.n_chunks; ch0 += U) {
            float ab[U];
#pragma unroll
            for (int u = 0; u < U; ++u) ab[u] = p.part_b[min(ch0 + u, p.n_chunks - 1) * cstride + prow(h, sl)];
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (ch0 + u < p.n_chunks) sb += ab[u];
        }
        p.d_bias[(((int64_t)h * p.num_seqs + s) * p.n_sets) * K + sl] = sb;
    }
    if (pos < 0 || pos >= len) return;
    // only the owner of the row goes on: the first copy of the position in this set, and no
    // earlier head of the group holding it
    if (sl > 0 && set[sl - 1] == pos) return;
    for (int hh = kvh * rep; hh < h; ++hh)
        if (find_slot(p.lmk + (((int64_t)hh * p.num_seqs + s) * p.n_sets) * K, K, pos) >= 0) return;
    const int64_t half = (int64_t)p.n_heads * p.num_seqs * K * D;
    const int64_t so = prow(h, sl) * D + d;
    float sk = p.lmk_stage[so], sv = p.lmk_stage[half + so];
    for (int hh = h; hh < (kvh + 1) * rep; ++hh) {
        const int32_t* hset = p.lmk + (((int64_t)hh * p.num_seqs + s) * p.n_sets) * K;
        // a set may repeat a position (each copy counts, as in the forward): its copies
        // are adjacent in the ascending set
        for (int slot = hh == h ? sl : find_slot(hset, K, pos); slot >= 0 && slot < K && hset[slot] == pos; ++slot) {
            const int64_t pr0 = prow(hh, slot);
            // chunk partials in chunk order; eight chunks' loads in flight at a time
            constexpr int U = 8;
            for (int ch0 = 0; ch0 < p.n_chunks; ch0 += U) {
                float ak[U], av[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int ch = min(ch0 + u, p.n_chunks - 1);
                    const int64_t pr = ch * cstride + pr0;
                    ak[u] = p.part_k[pr * D + d];
                    av[u] = p.part_v[pr * D + d];
                }
#pragma unroll
                for (int u = 0; u < U; ++u)
                    if (ch0 + u < p.n_chunks) {
                        sk += ak[u];
                        sv += av[u];
                    }
            }
        }
    }
    const int64_t o = (int64_t)(st + pos) * p.n_kv_heads * D + (int64_t)kvh * D + d;
    ((T*)p.dk)[o] = from_float<T>(sk);
    ((T*)p.dv)[o] = from_float<T>(sv);
}

// training variant: d w~ per token, the per-head sums added in head order
__global__ __launch_bounds__(256) void train_dw_kernel(AttnParams p) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t >= p.total_len) return;
    float s = 0.f;
    for (int h = 0; h < p.n_heads; ++h) s += p.dw_h[(int64_t)t * p.n_heads + h];
    p.d_w[t] = s;
}

hipError_t train_dw_launch(const AttnParams& p, hipStream_t stream) {
    if (p.total_len == 0) return hipSuccess;
    DSALT_LAUNCH("train_dw", train_dw_kernel, dim3(ceil_div(p.total_len, 256)), dim3(256), 0, stream, p);
    return hipGetLastError();
}

// ---------------------------------------------------------------- launch
// blocks of the landmark backward per (head, sequence, slot group): at most kRowChunk rows
// each, and more (down to one 64-row tile each) until the launch has about sixteen waves
// per CU, since a block's rows are one dependent chain of staged tiles
static int lmk_chunks(const AttnParams& p) {
    const int nw = p.dtype != DSALT_DTYPE_F32 && p.head_dim == 64 && p.k_lmk > 64 ? 8 : 4;  // as lmk_waves
    const int ngrp = ceil_div(p.k_lmk, 16 * nw);
    const int sets = max(1, p.n_heads * p.num_seqs * ngrp);
    const int fill = ceil_div(4096 / nw, sets);
    const int rows = (p.variant & DSALT_VARIANT_LMK_SHORT) ? kRowChunk / 2 : kRowChunk;
    return max(ceil_div(p.max_seqlen, rows), min(fill, ceil_div(p.max_seqlen, 64)));
}

size_t bwd_workspace(const AttnParams& p, bool plan_given) {
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const int nch = lmk_chunks(p);
    size_t b = plan_given ? 0 : plan_bytes(p);
    b += al(sizeof(float) * (size_t)p.total_len * p.n_heads);
    b += al(sizeof(int) * (size_t)p.total_len * p.n_heads);
    b += al(sizeof(float) * (size_t)p.total_len * p.n_heads);
    b += 2 * al(sizeof(float) * (size_t)nch * p.n_heads * p.num_seqs * p.k_lmk * p.head_dim);
    b += al(sizeof(float) * (size_t)nch * p.n_heads * p.num_seqs * p.k_lmk);
    b += al(sizeof(float) * 2 * (size_t)p.n_heads * p.num_seqs * p.k_lmk * p.head_dim);
    return b;
}

template <typename T, int D>
static hipError_t bwd_run(const AttnParams& p, bool plan_given, hipStream_t stream) {
    const int total = p.n_heads * p.num_seqs * p.n_tiles;
    const int total_kv = p.n_kv_heads * p.num_seqs * p.n_tiles;
    if (!plan_given) {
        const hipError_t e = plan_launch(p, stream);
        if (e != hipSuccess) return e;
    }
    constexpr int BN = BwdShape<T, D>::BN;
    constexpr bool kBn64 = sizeof(T) == 2 && D == 64;  // the only shape with a 64-key dQ tiling
    const bool lk = p.k_lmk > kSetSlots;               // large sets (inference operator only)
    if (lk) {
        DSALT_LAUNCH("bwd_dq", (bwd_dq_kernel<T, D, BN, false, true>), dim3(total), dim3(256), 0, stream, p);
    } else if (kBn64 && (p.variant & DSALT_VARIANT_DQ_BN64)) {
        if constexpr (kBn64) {
            if (p.w_cont) DSALT_LAUNCH("bwd_dq", (bwd_dq_kernel<T, D, 64, true>), dim3(total), dim3(256), 0, stream, p);
            else DSALT_LAUNCH("bwd_dq", (bwd_dq_kernel<T, D, 64, false>), dim3(total), dim3(256), 0, stream, p);
        }
    } else {
        if (p.w_cont) DSALT_LAUNCH("bwd_dq", (bwd_dq_kernel<T, D, BN, true>), dim3(total), dim3(256), 0, stream, p);
        else DSALT_LAUNCH("bwd_dq", (bwd_dq_kernel<T, D, BN, false>), dim3(total), dim3(256), 0, stream, p);
    }
    if (p.n_kv_heads != p.n_heads) {
        if (p.w_cont) DSALT_LAUNCH("bwd_dkdv", (bwd_dkdv_kernel<T, D, true, true>), dim3(total_kv), dim3(256), 0, stream, p);
        else DSALT_LAUNCH("bwd_dkdv", (bwd_dkdv_kernel<T, D, false, true>), dim3(total_kv), dim3(256), 0, stream, p);
    } else {
        if (p.w_cont) DSALT_LAUNCH("bwd_dkdv", (bwd_dkdv_kernel<T, D, true, false>), dim3(total_kv), dim3(256), 0, stream, p);
        else DSALT_LAUNCH("bwd_dkdv", (bwd_dkdv_kernel<T, D, false, false>), dim3(total_kv), dim3(256), 0, stream, p);
    }
    if (p.k_lmk > 0) {
        if (lmk_waves<T, D>(p.k_lmk) == 8) {
            const dim3 grid(p.n_heads * p.num_seqs * p.n_chunks * ceil_div(p.k_lmk, 128));
            if (lk) DSALT_LAUNCH("bwd_lmk", (bwd_lmk_kernel<T, D, 8, true>), grid, dim3(512), 0, stream, p);
            else DSALT_LAUNCH("bwd_lmk", (bwd_lmk_kernel<T, D, 8>), grid, dim3(512), 0, stream, p);
        } else {
            const dim3 grid(p.n_heads * p.num_seqs * p.n_chunks * ceil_div(p.k_lmk, 64));
            if (lk) DSALT_LAUNCH("bwd_lmk", (bwd_lmk_kernel<T, D, 4, true>), grid, dim3(256), 0, stream, p);
            else DSALT_LAUNCH("bwd_lmk", (bwd_lmk_kernel<T, D, 4>), grid, dim3(256), 0, stream, p);
        }
        const int64_t n = (int64_t)p.n_heads * p.num_seqs * p.k_lmk * D;
        DSALT_LAUNCH("bwd_lmk_sum", (bwd_lmk_sum_kernel<T, D>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     stream, p);
    }
    return hipGetLastError();
}

hipError_t bwd_launch(AttnParams p, void* ws, const void* plan, hipStream_t stream) {
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    p.n_chunks = lmk_chunks(p);
    char* w = (char*)ws;
    if (plan) {
        char* pw = (char*)const_cast<void*>(plan);  // read only: the kernels never write it
        plan_carve(p, pw);
    } else {
        plan_carve(p, w);  // advances w past the plan
    }
    p.delta = (float*)w;
    w += al(sizeof(float) * (size_t)p.total_len * p.n_heads);
    p.cnt = (int*)w;
    w += al(sizeof(int) * (size_t)p.total_len * p.n_heads);
    p.lse2t = (float*)w;
    w += al(sizeof(float) * (size_t)p.total_len * p.n_heads);
    const size_t npart = (size_t)p.n_chunks * p.n_heads * p.num_seqs * p.k_lmk;
    p.part_k = (float*)w;
    w += al(sizeof(float) * npart * p.head_dim);
    p.part_v = (float*)w;
    w += al(sizeof(float) * npart * p.head_dim);
    p.part_b = (float*)w;
    w += al(sizeof(float) * npart);
    p.lmk_stage = (float*)w;
    w += al(sizeof(float) * 2 * (size_t)p.n_heads * p.num_seqs * p.k_lmk * p.head_dim);
    if (p.total_len == 0 || p.num_seqs == 0) return hipSuccess;
    const bool pg = plan != nullptr;
    if (p.dtype == DSALT_DTYPE_BF16) return p.head_dim == 64 ? bwd_run<bf16, 64>(p, pg, stream) : bwd_run<bf16, 128>(p, pg, stream);
    if (p.dtype == DSALT_DTYPE_F16) return p.head_dim == 64 ? bwd_run<f16, 64>(p, pg, stream) : bwd_run<f16, 128>(p, pg, stream);
    return p.head_dim == 64 ? bwd_run<float, 64>(p, pg, stream) : bwd_run<float, 128>(p, pg, stream);
}

}  // namespace dsalt
