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
#include <type_traits>

#include "attn.h"
#include "plan.h"
#include "tiles.h"
#include "timing.h"

namespace dsalt {



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

// ------------------------------------------------------------- row plan
// (plan.h): one wave per 64-row tile
__global__ __launch_bounds__(64) void row_plan_kernel(AttnParams p) {
    __shared__ int sp[64], slo[64];
    row_plan_tile(p.w, p.cu, p.total_len, p.max_seqlen, p.n_tiles, blockIdx.x, true, threadIdx.x, sp, slo,
                  PlanOut{p.plan_perm, p.plan_bounds, p.tile_wmax});
}

size_t plan_bytes(const AttnParams& p) {
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t tiles = (size_t)p.num_seqs * p.n_tiles;
    return al(tiles * 64) + al(tiles * 16 * sizeof(int)) + al(tiles * sizeof(int));
}

void plan_carve(AttnParams& p, char*& ws) {
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t tiles = (size_t)p.num_seqs * p.n_tiles;
    p.plan_perm = (uint8_t*)ws;
    ws += al(tiles * 64);
    p.plan_bounds = (int*)ws;
    ws += al(tiles * 16 * sizeof(int));
    p.tile_wmax = (int*)ws;
    ws += al(tiles * sizeof(int));
}

hipError_t plan_launch(const AttnParams& p, hipStream_t stream) {
    const int tiles = p.num_seqs * p.n_tiles;
    if (tiles == 0) return hipSuccess;
    DSALT_LAUNCH("row_plan", row_plan_kernel, dim3(tiles), dim3(64), 0, stream, p);
    return hipGetLastError();
}

// ---------------------------------------------------------------- forward
// Rows of one 16-row group: per lane the row, its window [lo, hi] and visible
// landmark count; per group (wave-uniform) the bounds that classify subtiles.
struct RowGroup {
    int i, lo, hi, cnt;
    bool valid;
    float wt;  // continuous window of the row (training variant)
    int lou;   // unclamped window start i - floor(wt) (training variant)
    float eb[kEdgeTab];  // soft-edge bias of keys lou .. lou+3 (training variant, win_edge <= 4)
    int wlo, wLmax, whi, wHmin, wcmax, wcmin;
    // several landmark sets per block (block-causal, block_size not a multiple of 64): the
    // row's set starts at slot ls of the staged sets, its visible slots are ls .. ls+cnt-1;
    // wcmax / wcmin then bound ls + cnt, wsmin / wsmax the set starts of the group's rows
    int ls, wsmin, wsmax;
};

// Block group (plan tile u, group within it) taken by wave w: groups are ordered
// by window start inside a plan tile, so wave w pairs the w-th group of tile 0
// with the (3-w)-th of tile 1 and the waves of a block get even work.
template <int RG>
__device__ __forceinline__ int group_of(int w, int u) {
    return RG == 1 ? w : 4 * u + (u & 1 ? 3 - w : w);
}

// Fills the lane's row of block group G (0 .. 4*RG-1) from the row plan: plan_rows the row
// and the group bounds, plan_window (after the rows of every group are requested) the
// window; the visible landmark counts need the block's landmark set in LDS (plan_counts).
struct PlanLoad {  // a group's plan entries as loaded
    int b0, b1, b2, b3, pm;
};
// loads from valid addresses whether or not the group exists (G past the block's tiles reads
// group 0), results selected in plan_rows: no load waits on a branch
__device__ __forceinline__ PlanLoad plan_load(const AttnParams& p, int64_t tile0, int ntl, int G, int lane) {
    const int Gc = G < 4 * ntl ? G : 0;
    const int* bnd = p.plan_bounds + (tile0 + Gc / 4) * 16 + (Gc % 4) * 4;
    return PlanLoad{bnd[0], bnd[1], bnd[2], bnd[3], (int)p.plan_perm[(tile0 + Gc / 4) * 64 + (Gc % 4) * 16 + (lane & 15)]};
}
__device__ __forceinline__ void plan_rows(const PlanLoad& l, int ntl, int G, int r0, int len, RowGroup& rg) {
    const bool has = G < 4 * ntl;
    const int Gc = has ? G : 0;
    rg.wlo = has ? l.b0 : 0x7fffffff;
    rg.wLmax = has ? l.b1 : (int)0x80000000;
    rg.whi = has ? l.b2 : -1;
    rg.wHmin = has ? l.b3 : 0x7fffffff;
    rg.i = has ? r0 + (Gc / 4) * 64 + l.pm : -1;
    rg.valid = has && rg.i < len;
    rg.lo = 0x7fffffff;
    rg.hi = -1;
    rg.cnt = 0;
    rg.wt = 0.f;
    rg.lou = 0x7fffffff;
}

__device__ __forceinline__ void plan_window(const AttnParams& p, int st, RowGroup& rg) {
    // loads issued by every lane (a row past the end reads the sequence's first row)
    const int at = st + (rg.valid ? rg.i : 0);
    const int wi = max(p.w[at], 1);
    const float wt = p.w_cont ? train_wt(p, p.w_cont[at]) : 0.f;
    if (rg.valid) {
        rg.lo = max(rg.i - wi + 1, 0);
        rg.hi = rg.i;
        rg.wt = wt;
        rg.lou = rg.i - (wi - 1);
    }
    if (p.w_cont) edge_table(p, rg.wt, rg.eb, nullptr);
}

// The group's visible landmark counts (the set's positions in LDS).
__device__ __forceinline__ void plan_counts(const int* lpos, int nvalid, RowGroup& rg) {
    rg.cnt = rg.valid ? lower_bound_lds(lpos, nvalid, rg.lo) : 0;
    rg.wcmax = uniform(row_max16(rg.cnt));
    rg.wcmin = uniform(row_min16(rg.valid ? rg.cnt : 0));
}

// The same with the block's sets staged side by side: set first + j at slots j*K .. j*K+K-1,
// nvs[j] valid positions (row i belongs to set i / block_size).
__device__ __forceinline__ void plan_counts_sets(const int* lpos, const int* nvs, int K, int block_size, int first,
                                                 int nsets, RowGroup& rg) {
    int ls = 0, cnt = 0;
    if (rg.valid) {
        const int j = block_size ? min(max(rg.i / block_size - first, 0), nsets - 1) : 0;
        ls = j * K;
        cnt = lower_bound_lds(lpos + ls, nvs[j], rg.lo);
    }
    rg.ls = ls;
    rg.cnt = cnt;
    rg.wcmax = uniform(row_max16(ls + cnt));
    rg.wcmin = uniform(row_min16(rg.valid ? ls + cnt : 0));
    rg.wsmin = uniform(row_min16(rg.valid ? ls : 0x7fffffff));
    rg.wsmax = uniform(row_max16(ls));
}

// Soft-edge bias of the lane's four keys a + lane_off + r of a band subtile (training
// variant), masked keys (r < tl, and r past the diagonal when `upper`) left at -inf.
__device__ __forceinline__ void band_edge(const AttnParams& p, const RowGroup& R, int a, int lane_off, int tl,
                                          bool upper, floatx4& ci) {
    const int th = R.hi - a - lane_off;
    if (p.edge_keys <= kEdgeTab) {
        const int k0 = a + lane_off - R.lou;  // key offset from the unclamped window start, r = 0
#pragma unroll
        for (int r = 0; r < 4; ++r) ci[r] = (r < tl || (upper && r > th)) ? -INFINITY : edge_lookup(R.eb, k0 + r);
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) ci[r] = (r < tl || (upper && r > th)) ? -INFINITY : edge_bias(p, R.wt, th - r);
    }
}

// One 256-thread block (4 waves; NW = 8 below: 512 threads) owns 64*RG query rows of one (head, sequence),
// (two 16-row groups with 32-key chunks, 16-bit head_dim 64: held at four waves per SIMD, 128
// VGPRs; the K and V^T operands of a chunk serve both groups of a wave)
// taken in the row plan's order; wave w owns the 16-row groups RG*w .. RG*w+RG-1
// (each lane one query row per group).  The K and V^T operands fetched from
// LDS for a subtile serve all of a wave's groups.
//
// TR: the training variant -- band keys near a row's window start carry the soft
// edge bias (edge_bias), so chunks classed "every row sees every key" must also
// lie past every row's first edge_keys band keys.
//
// MS: sets of more than kSetSlots landmarks, or block-causal sets with block_size not a
// multiple of 64 (one row group per wave, inference only): the block's rows may belong to
// several sets, all staged in LDS side by side; each row sees the slots of its own set only
// (a two-sided slot mask, like the band's key mask).
//
// NW = 8: eight waves, one row group each, over two plan tiles (128 rows): every staged chunk
// serves twice the rows (head_dim 128, where the chunks' staging is most of the time).
// (the 16-bit head_dim-128 training forward is held to four waves per SIMD: 128 VGPRs, no
// spills, from 132 at three)
// (head, sequence) pairs from which each XCD walks its pairs one at a time (fwd_kernel)
constexpr int kPairOrderMin = 256;

template <typename T, int D, int BN, int RG, bool TR, bool MS = false, int NW = 4>
__global__ __launch_bounds__(64 * NW, ((sizeof(T) == 2 && D == 64 && RG == 2 && BN == 32) ||
                                       (sizeof(T) == 2 && D == 128 && RG == 1 && BN == 32 && NW == 4 && TR))
                                          ? 4
                                          : 2) void fwd_kernel(AttnParams p) {
    static_assert(!MS || (RG == 1 && !TR), "several sets per block: one row group, inference");
    static_assert(NW == 4 || (NW == 8 && RG == 1 && !MS), "eight waves: one row group each, one set per block");
    constexpr int NT = 64 * NW;
    constexpr int TPB = RG * NW / 4;  // plan tiles (64 rows) per block
    constexpr int NST = BN / 16;
    constexpr bool kHalf = sizeof(T) == 2;
    constexpr int LCAP = MS ? kMultiSetSlots : kSetSlots;
    typedef Tile<T, D, BN, NT, (BN == 64 ? 8 : Pad<T, D>::R)> KT;
    __shared__ __attribute__((aligned(16))) T Ks[2][KT::ELEMS];
    __shared__ __attribute__((aligned(16))) T Vs[2][KT::ELEMS];
    __shared__ int lpos[LCAP];
    __shared__ __attribute__((aligned(16))) float lbs[LCAP];
    static_assert(KT::ELEMS * sizeof(T) >= sizeof(int) * (16 + kMaxTileSets), "block scalars fit a K buffer");
    // block scalars live in the second K buffer until the first chunk is staged there
    // (keeps the block at 40 KB of LDS: four blocks per CU)
    int* red = (int*)Ks[1];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4;
    const int nblk = ceil_div(p.n_tiles, TPB);
    // tile-major order, the last tiles of every sequence first (their rows see the most
    // landmarks: the longest blocks start first and short ones fill the end of the grid);
    // blocks reach the XCDs round-robin, so where 8 divides heads x sequences each XCD keeps
    // the same (head, sequence) pairs, and their K/V rows in its L2, throughout.  With many
    // pairs that order puts every block an XCD runs at once on another pair, and a pair's next
    // tile hundreds of blocks later: there each XCD walks its pairs one at a time instead, all
    // tiles of a pair (the last first) before the next, so neighbouring tiles share K/V in L2.
    const int nhs = p.n_heads * p.num_seqs;
    int hs, b;
    if (nhs % 8 == 0 && nhs >= kPairOrderMin) {
        const int x = (int)blockIdx.x % 8, j = (int)blockIdx.x / 8;
        hs = (j / nblk) * 8 + x;
        b = nblk - 1 - j % nblk;
    } else {
        hs = (int)blockIdx.x % nhs;
        b = nblk - 1 - (int)blockIdx.x / nhs;
    }
    const int h = hs % p.n_heads;
    const int s = hs / p.n_heads;
    int st, len;
    seq_bounds(p.cu, s, p.total_len, p.max_seqlen, st, len);
    const int r0 = b * 64 * TPB;
    if (r0 >= len) return;
    const int kvh = h / (p.n_heads / p.n_kv_heads);
    const int set = p.block_size ? r0 / p.block_size : 0;
    const int K = p.k_lmk;
    const int64_t set_off = (((int64_t)h * p.num_seqs + s) * p.n_sets + set) * K;
    // sets of the block's rows (MS): set .. set + nsets - 1, at most LCAP slots in all
    int nsets = 1;
    if (MS && p.block_size) {
        const int last = min(r0 + 63, len - 1) / p.block_size;
        nsets = min(min(last - set + 1, kMaxTileSets), LCAP / max(K, 1));
    }
    const int nslots = nsets * K;
    const float c2 = p.c2;
    const float inv_scale = p.inv_scale;
    const bool has_bias = p.lbias != nullptr;

    // Prologue: the loads that depend on no other load -- the landmark set, the row plan's
    // group bounds and rows -- are issued together, then the rows' windows and query rows;
    // the block's largest visible landmark count follows from the largest window start of
    // its groups, so one barrier (the set in LDS) precedes the first landmark chunk's fetch.
    // (MS: the sets are staged by a loop after the plan's loads)
    constexpr int NLV = MS ? 1 : kSetSlots / NT;
    int lv[NLV], ln[NLV];
    float lb[NLV];
#pragma unroll
    for (int u = 0; u < NLV; ++u) {
        lv[u] = -1;
        ln[u] = -1;
        lb[u] = 0.f;
        if (!MS && u * NT < K) {  // every lane loads (clamped slots), so no load waits on a branch
            lv[u] = p.lmk[set_off + min(u * NT + tid, K - 1)];
            ln[u] = p.lmk[set_off + min(u * NT + tid + 1, K - 1)];
            if (has_bias) lb[u] = p.lbias[set_off + min(u * NT + tid, K - 1)];
        }
    }

    // row groups of this wave, block-wide key range and largest window start, from the row plan
    const int uw = uniform(wave);
    const int64_t tile0 = (int64_t)s * p.n_tiles + (int64_t)b * TPB;
    const int ntl = min(TPB, p.n_tiles - b * TPB);
    int blo = 0x7fffffff, bhi = -1, blmax = (int)0x80000000;
    if (lane < 4 * ntl) {
        const int* bnd = p.plan_bounds + tile0 * 16 + lane * 4;
        blo = bnd[0];
        blmax = bnd[1];
        bhi = bnd[2];
    }
    PlanLoad pl[RG];
#pragma unroll
    for (int u = 0; u < RG; ++u) pl[u] = plan_load(p, tile0, ntl, group_of<RG>(uw, u), lane);
    __builtin_amdgcn_sched_barrier(0);  // every group's plan load issued before any is used
    RowGroup rg[RG];
#pragma unroll
    for (int u = 0; u < RG; ++u) plan_rows(pl[u], ntl, group_of<RG>(uw, u), r0, len, rg[u]);
#pragma unroll
    for (int u = 0; u < RG; ++u) plan_window(p, st, rg[u]);
    const T* qhead = (const T*)p.q + (int64_t)st * p.q_st + (int64_t)h * p.q_sh;
    RowReg<T, D> qr[RG];
#pragma unroll
    for (int u = 0; u < RG; ++u) qr[u].load(rg[u].valid ? qhead + (int64_t)rg[u].i * p.q_st : nullptr, qhead, g);
    // the band's key range, clamped to the sequence: a plan made for other windows or offsets
    // gives wrong values, never reads outside the sequence's rows
    blo = max(uniform(-wave_max(-blo)), 0);
    bhi = min(uniform(wave_max(bhi)), len - 1);
    blmax = uniform(wave_max(blmax));

    int nvalid;  // valid slots of the (first) set; MS: of any set, and nvs[j] per set
    int* nvs = red + 16;
    if constexpr (!MS) {
        int nv_loc = 0;  // one past the last valid slot (sets are ascending, -1 after the valid slots)
#pragma unroll
        for (int u = 0; u < NLV; ++u) {
            const int i = u * NT + tid;
            if (i < K) {
                lpos[i] = lv[u];
                if (has_bias) lbs[i] = lb[u] * inv_scale;  // raw-score units
                if (lv[u] >= 0 && (i + 1 == K || ln[u] < 0)) nv_loc = i + 1;
            }
        }
        nv_loc = wave_max(nv_loc);
        if (lane == 0) red[4 + uw] = nv_loc;
        __syncthreads();
        int nvm = red[4];
#pragma unroll
        for (int w2 = 1; w2 < NW; ++w2) nvm = max(nvm, red[4 + w2]);
        nvalid = uniform(nvm);
    } else {
        if (tid < kMaxTileSets) nvs[tid] = 0;
        __syncthreads();
        // slot e: position sl of set set + j (the block's sets are consecutive, K slots each)
        for (int e = tid; e < nslots; e += NT) {
            const int j = e / K, sl = e - j * K;
            const int64_t o = set_off + (int64_t)j * K;
            const int v = p.lmk[o + sl];
            const int vn = sl + 1 < K ? p.lmk[o + sl + 1] : -1;
            lpos[e] = v;
            if (has_bias) lbs[e] = p.lbias[o + sl] * inv_scale;
            if (v >= 0 && (sl + 1 == K || vn < 0)) nvs[j] = sl + 1;  // one writer per set
        }
        __syncthreads();
        int any = 0;
        for (int j = 0; j < nsets; ++j) any |= nvs[j];
        nvalid = uniform(any);
    }

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
    // landmark rows: 32-bit offsets into resources over the sequence's rows when the
    // sequence spans less than 2 GiB of K and of V, else 64-bit row addresses (always
    // for fp32 D128, where the offsets would cost a wave of occupancy)
    const uint32_t kext = gather_extent(len, krb, D * sizeof(T)), vext = gather_extent(len, vrb, D * sizeof(T));
    const bool lmk32 = (D == 64 || sizeof(T) == 2) && kext != 0u && vext != 0u;
    const rsrc_t krs = make_rsrc(kbase, kext), vrs = make_rsrc(vbase, vext);
    KT kt, vt;
    // landmark chunk c: slots c*BN .. below `lim` (slots past the block's largest count are
    // masked out of every product, so the first chunk, fetched before that count is known,
    // may take them from the set unmasked)
    auto load_lmk_lim = [&](int c, int lim) {
        auto pos = [&](int rr) -> int {
            const int sl = c * BN + rr;
            const int q = sl < lim ? lpos[sl] : -1;
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
    if (nvalid > 0) load_lmk_lim(0, MS ? nslots : nvalid);

    int bcm;
    if constexpr (!MS) {
#pragma unroll
        for (int u = 0; u < RG; ++u) plan_counts(lpos, nvalid, rg[u]);
        // the block's largest visible count: that of its largest window start (counts grow with it)
        bcm = uniform(lower_bound_lds(lpos, nvalid, blmax));
    } else {
#pragma unroll
        for (int u = 0; u < RG; ++u) plan_counts_sets(lpos, nvs, K, p.block_size, set, nsets, rg[u]);
        // the last set's rows end furthest: its count at the block's largest window start bounds
        // them; with every set empty there is no landmark chunk (and the first was not fetched)
        const int lj = (nsets - 1) * K;
        bcm = nvalid > 0 ? uniform(lj + lower_bound_lds(lpos + lj, nvs[nsets - 1], blmax)) : 0;
    }
    const int cs = (blo / BN) * BN;
    const int nband = bhi >= blo ? (bhi - cs) / BN + 1 : 0;
    const int nchunks = nband + ceil_div(bcm, BN);

    // band rows [cs, bhi]: one resource per tensor over the whole band (rows past bhi read
    // zero); band chunks are loaded in order, the per-thread offsets advancing one chunk per load
    const int brows = nband > 0 ? bhi + 1 - cs : 0;
    const rsrc_t kband = rows_rsrc(kbase + (int64_t)cs * p.k_st, brows, krb, D * sizeof(T));
    const rsrc_t vband = rows_rsrc(vbase + (int64_t)cs * p.v_st, brows, vrb, D * sizeof(T));
    auto load_band = [&]() {
        kt.load_rows(kband, koff);
        vt.load_rows(vband, voff);
#pragma unroll
        for (int n = 0; n < KT::NV; ++n) {
            koff[n] += (uint32_t)BN * krb;
            voff[n] += (uint32_t)BN * vrb;
        }
    };
    auto load_lmk = [&](int c) { load_lmk_lim(c, bcm); };
    // landmark chunks first (their gathers only in the first loop), then the band
    const int nlmk = nchunks - nband;
    if (nchunks > 0) {
        if (nlmk == 0) load_band();  // else the first landmark chunk is in flight
        kt.store(Ks[0], tid);
        vt.store(Vs[0], tid);
    }
    __syncthreads();

    floatx4 acc[RG][D / 16];
    floatx4 lacc[RG];  // row sums (16-bit path: ones x P)
    float l_run[RG];   // row sums (fp32 path)
    float m_run[RG];
#pragma unroll
    for (int u = 0; u < RG; ++u) {
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) acc[u][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
        lacc[u] = floatx4{0.f, 0.f, 0.f, 0.f};
        l_run[u] = 0.f;
        // a finite start below every score: the first rescale factor exp2((start - m) c2) is
        // exactly 0 and masked scores exp2(-inf) stay 0, with no test for an unset maximum
        m_run[u] = -1e30f;
    }
    const float thr = p.thr;
    const float NEG = -INFINITY;
    const int lane_off = 4 * g;

    // chunk n of the sweep: landmark chunk n (n < nlmk), else band chunk n - nlmk; `band` is a
    // compile-time tag, so the two loops below are separate straight-line code
    auto process = [&](int n, auto band_tag) {
        constexpr bool band = decltype(band_tag)::value;
        const int buf = n & 1;
        const int c = band ? n - nlmk : n;
        if (!band) {
            if (n + 1 < nlmk) load_lmk(n + 1);
            else if (nband > 0) load_band();
        } else if (c + 1 < nband) {
            load_band();
        }
        const int base = band ? cs + c * BN : c * BN;
        const T* kl = Ks[buf];
        floatx4 S[RG][NST];
        bool act[RG][NST];
        bool gact[RG];
#pragma unroll
        for (int u = 0; u < RG; ++u) {
            const RowGroup& R = rg[u];
            // chunk class for this group (wave-uniform): 0 no row sees it; 1 every row sees
            // every key; 2 (64-key chunks) every key at or below every row, window starts only;
            // 3 band keys under the two-sided window mask (subtiles wholly outside it included:
            // their scores are -inf and their products add zeros, cheaper than the branches
            // that would tell them apart); 4 landmarks all visible, no bias; 5 landmarks
            // subtile by subtile
            int kind;
            if (band) {
                const int last = base + BN - 1;
                if (base > R.whi || last < R.wlo) kind = 0;
                else if (base >= R.wLmax + (TR ? p.edge_keys : 0) && last <= R.wHmin) kind = 1;
                else if (BN > 32 && last <= R.wHmin) kind = 2;
                else kind = 3;
            } else if (!MS) {
                if (base >= R.wcmax) kind = 0;
                else if (base + BN - 1 < R.wcmin) kind = 4;
                else kind = 5;
            } else {
                if (base >= R.wcmax || base + BN - 1 < R.wsmin) kind = 0;
                else if (base >= R.wsmax && base + BN - 1 < R.wcmin) kind = 4;
                else kind = 5;
            }
            gact[u] = kind != 0;
#pragma unroll
            for (int stt = 0; stt < NST; ++stt) act[u][stt] = kind != 0;
            const floatx4 zero = floatx4{0.f, 0.f, 0.f, 0.f};
            if (kind == 1 || (kind == 4 && !has_bias)) {
#pragma unroll
                for (int stt = 0; stt < NST; ++stt) {
                    KOp<T, D> ko;
                    ko.load(kl, KT::RS, stt * 16, lane);
                    S[u][stt] = ko.dot(qr[u], zero);
                }
            } else if (!band && kind == 4) {  // every slot visible to every row, landmark bias only
#pragma unroll
                for (int stt = 0; stt < NST; ++stt) {
                    KOp<T, D> ko;
                    ko.load(kl, KT::RS, stt * 16, lane);
                    S[u][stt] = ko.dot(qr[u], *(const floatx4*)(lbs + base + stt * 16 + lane_off));
                }
            } else if (band && BN > 32 && kind == 2) {
#pragma unroll
                for (int stt = 0; stt < NST; ++stt) {
                    const int a = base + stt * 16;
                    const int tl = R.lo - a - lane_off;
                    floatx4 ci;
#pragma unroll
                    for (int r = 0; r < 4; ++r) ci[r] = r < tl ? NEG : 0.f;
                    if (TR && a < R.wLmax + p.edge_keys)  // the soft edge reaches this subtile
                        band_edge(p, R, a, lane_off, tl, false, ci);
                    KOp<T, D> ko;
                    ko.load(kl, KT::RS, stt * 16, lane);
                    S[u][stt] = ko.dot(qr[u], ci);
                }
            } else if (band && kind == 3) {
#pragma unroll
                for (int stt = 0; stt < NST; ++stt) {
                    const int a = base + stt * 16;
                    const int tl = R.lo - a - lane_off;
                    // key a + lane_off + r in [lo, hi]: one unsigned compare of r - tl against
                    // hi - lo (a row past the end has lo > hi and fails it)
                    const int x0 = a + lane_off - R.lo;
                    const unsigned wd = (unsigned)R.hi - (unsigned)R.lo;
                    floatx4 ci;
#pragma unroll
                    for (int r = 0; r < 4; ++r) ci[r] = (unsigned)(x0 + r) <= wd ? 0.f : NEG;
                    if (TR && a < R.wLmax + p.edge_keys) band_edge(p, R, a, lane_off, tl, true, ci);
                    KOp<T, D> ko;
                    ko.load(kl, KT::RS, stt * 16, lane);
                    S[u][stt] = ko.dot(qr[u], ci);
                }
            } else if (!band && kind == 5) {
#pragma unroll
                for (int stt = 0; stt < NST; ++stt) {
                    const int a = base + stt * 16;
                    act[u][stt] = a < R.wcmax && (!MS || a + 15 >= R.wsmin);
                    if (!act[u][stt]) {
                        S[u][stt] = floatx4{NEG, NEG, NEG, NEG};
                        continue;
                    }
                    // slots past the valid count are masked below (a + 15 < LCAP)
                    const floatx4 bv = has_bias ? *(const floatx4*)(lbs + a + lane_off) : zero;
                    floatx4 ci;
                    if constexpr (!MS) {
                        const int tc = R.cnt - a - lane_off;
#pragma unroll
                        for (int r = 0; r < 4; ++r) ci[r] = r < tc ? bv[r] : NEG;
                    } else {  // slot in [ls, ls + cnt): one unsigned compare
                        const int x0 = a + lane_off - R.ls;
#pragma unroll
                        for (int r = 0; r < 4; ++r) ci[r] = (unsigned)(x0 + r) < (unsigned)R.cnt ? bv[r] : NEG;
                    }
                    KOp<T, D> ko;
                    ko.load(kl, KT::RS, stt * 16, lane);
                    S[u][stt] = ko.dot(qr[u], ci);
                }
            }
        }
        // online softmax per group (skipped by groups with no row in the chunk)
#pragma unroll
        for (int u = 0; u < RG; ++u) {
            if (!gact[u]) continue;
            // the lane's own maximum decides whether the row maximum can move the running one past
            // the rescale threshold (the row maximum is the largest of its four lanes'), so the
            // cross-lane reduction runs only when some lane exceeds it
            float mx = NEG;
#pragma unroll
            for (int stt = 0; stt < NST; ++stt)
#pragma unroll
                for (int r = 0; r < 4; ++r) mx = fmaxf(mx, S[u][stt][r]);
            if (__any(mx > m_run[u] + thr)) {
                const float mnew = fmaxf(m_run[u], max_g4(mx));
                const float alpha = __builtin_amdgcn_exp2f((m_run[u] - mnew) * c2);
#pragma unroll
                for (int dt = 0; dt < D / 16; ++dt) acc[u][dt] *= alpha;
                lacc[u] *= alpha;
                l_run[u] *= alpha;
                m_run[u] = mnew;
            }
            const float msc = m_run[u] * c2;
#pragma unroll
            for (int stt = 0; stt < NST; ++stt)
#pragma unroll
                for (int r = 0; r < 4; ++r) S[u][stt][r] = __builtin_amdgcn_exp2f(S[u][stt][r] * c2 - msc);
        }
        if constexpr (kHalf) {
            const typename Vec8<T>::type ones = ones8<T>();
#pragma unroll
            for (int hp = 0; hp < NST / 2; ++hp) {
                bool pa[RG], any = false;
#pragma unroll
                for (int u = 0; u < RG; ++u) {
                    pa[u] = act[u][2 * hp] || act[u][2 * hp + 1];
                    any |= pa[u];
                }
                if (!any) continue;
                VOp<T, D> vo;
                vo.load(Vs[buf], KT::RS, hp * 32, lane);
#pragma unroll
                for (int u = 0; u < RG; ++u)
                    if (pa[u]) {
                        const auto bp = vo.acc(S[u][2 * hp], S[u][2 * hp + 1], acc[u]);
                        lacc[u] = mma(ones, bp, lacc[u]);
                    }
            }
        } else {
#pragma unroll
            for (int stt = 0; stt < NST; ++stt) {
                bool any = false;
#pragma unroll
                for (int u = 0; u < RG; ++u) any |= act[u][stt];
                if (!any) continue;
                VOp<T, D> vo;
                vo.load(Vs[buf], KT::RS, stt * 16, lane);
#pragma unroll
                for (int u = 0; u < RG; ++u)
                    if (act[u][stt]) {
                        l_run[u] += S[u][stt][0] + S[u][stt][1] + S[u][stt][2] + S[u][stt][3];
                        vo.acc(S[u][stt], acc[u]);
                    }
            }
        }
        if (n + 1 < nchunks) {
            kt.store(Ks[buf ^ 1], tid);
            vt.store(Vs[buf ^ 1], tid);
        }
        __syncthreads();
    };
    for (int n = 0; n < nlmk; ++n) process(n, std::false_type{});
    for (int n = nlmk; n < nchunks; ++n) process(n, std::true_type{});

    // output rows whole, staged in the idle K/V buffers (waves 0-1 in Ks, 2-3 in Vs; the
    // groups of a wave one after the other)
    typedef StoreRows<T, D> SR;
    static_assert(2 * KT::ELEMS >= (NW / 2) * SR::ELEMS, "row staging does not fit the chunk buffers");
    T* stage = (wave < NW / 2 ? &Ks[0][0] : &Vs[0][0]) + (wave % (NW / 2)) * SR::ELEMS;
    T* o0 = (T*)p.o + (int64_t)st * p.o_st + (int64_t)h * p.o_sh;
#pragma unroll
    for (int u = 0; u < RG; ++u) {
        const float l_tot = kHalf ? lacc[u][0] : sum_g4(l_run[u]);
        const int vi = rg[u].valid ? rg[u].i : -1;
        SR::run(stage, acc[u], rg[u].valid ? 1.0f / l_tot : 0.f, lane, [&](int rr) {
            const int ir = __shfl(vi, rr);
            return ir >= 0 ? o0 + (int64_t)ir * p.o_st : (T*)nullptr;
        });
        if (rg[u].valid && g == 0) p.lse_out[(int64_t)(st + rg[u].i) * p.n_heads + h] = m_run[u] * p.scale + __logf(l_tot);
    }
}

// Tilings (DSALT_VARIANT_* bits): for 16-bit head_dim 64, 32-key chunks instead of 64
// (FWD_BN32) and two 16-row groups per wave (FWD_RG2, 128 rows per block: the block must
// stay within one landmark set, block_size a multiple of 128); for 16-bit head_dim 128, two
// row groups per wave (FWD_RG2, same condition) or 64-key chunks instead of 32 (FWD_BN64;
// ignored with FWD_RG2);
// fp32 takes its single compiled tiling.  Sets of more than kSetSlots landmarks, and
// block-causal sets of a block_size that is not a multiple of 64, take the default tiling's
// wide instantiation (variant bits ignored).
template <typename T, int D, bool TR>
static void fwd_run(const AttnParams& p, hipStream_t stream) {
    constexpr int BN = FwdShape<T, D>::BN;
    if constexpr (!TR) {
        if (p.block_size % 64 || p.k_lmk > kSetSlots) {
            DSALT_LAUNCH("attn_fwd", (fwd_kernel<T, D, BN, 1, false, true>), dim3(p.n_heads * p.num_seqs * p.n_tiles),
                         dim3(256), 0, stream, p);
            return;
        }
    }
    if constexpr (sizeof(T) == 2) {
        const bool rg2 = (p.variant & DSALT_VARIANT_FWD_RG2) != 0 && (p.block_size == 0 || p.block_size % 128 == 0);
        const int total = p.n_heads * p.num_seqs * ceil_div(p.n_tiles, rg2 ? 2 : 1);
        if constexpr (D == 64) {
            const bool bn32 = (p.variant & DSALT_VARIANT_FWD_BN32) != 0;
            if (rg2) {
                if (bn32) DSALT_LAUNCH("attn_fwd", (fwd_kernel<T, D, 32, 2, TR>), dim3(total), dim3(256), 0, stream, p);
                else DSALT_LAUNCH("attn_fwd", (fwd_kernel<T, D, BN, 2, TR>), dim3(total), dim3(256), 0, stream, p);
                return;
            }
            if (bn32) {
                DSALT_LAUNCH("attn_fwd", (fwd_kernel<T, D, 32, 1, TR>), dim3(total), dim3(256), 0, stream, p);
                return;
            }
        } else if constexpr (!TR) {  // head_dim 128 (inference shapes)
            // two row groups keep 32-key chunks (with 64-key chunks they would spill at 256 VGPRs)
            const bool bn64 = (p.variant & DSALT_VARIANT_FWD_BN64) != 0;
            const bool w8 = (p.variant & DSALT_VARIANT_FWD_8W) != 0 && (p.block_size == 0 || p.block_size % 128 == 0);
            if (w8) {
                DSALT_LAUNCH("attn_fwd", (fwd_kernel<T, D, BN, 1, TR, false, 8>),
                             dim3(p.n_heads * p.num_seqs * ceil_div(p.n_tiles, 2)), dim3(512), 0, stream, p);
                return;
            }
            if (rg2) {
                DSALT_LAUNCH("attn_fwd", (fwd_kernel<T, D, BN, 2, TR>), dim3(total), dim3(256), 0, stream, p);
                return;
            }
            if (bn64) {
                DSALT_LAUNCH("attn_fwd", (fwd_kernel<T, D, 64, 1, TR>), dim3(total), dim3(256), 0, stream, p);
                return;
            }
        }
    }
    const int total = p.n_heads * p.num_seqs * p.n_tiles;
    DSALT_LAUNCH("attn_fwd", (fwd_kernel<T, D, BN, 1, TR>), dim3(total), dim3(256), 0, stream, p);
}

template <typename T>
static hipError_t fwd_dispatch(const AttnParams& p, bool plan_ready, hipStream_t stream) {
    if (p.n_heads * p.num_seqs * p.n_tiles == 0) return hipSuccess;
    if (!plan_ready) {
        const hipError_t e = plan_launch(p, stream);
        if (e != hipSuccess) return e;
    }
    const bool tr = p.w_cont != nullptr;
    if (p.head_dim == 64) {
        if (tr) fwd_run<T, 64, true>(p, stream);
        else fwd_run<T, 64, false>(p, stream);
    } else {
        if (tr) fwd_run<T, 128, true>(p, stream);
        else fwd_run<T, 128, false>(p, stream);
    }
    return hipGetLastError();
}

// training variant: integer windows floor(w~) + 1 (w~ below 0 as 0, at most max_seqlen);
// in the backward also clears the per-head window gradients
__global__ __launch_bounds__(256) void train_windows_kernel(AttnParams p, int* w_int) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t >= p.total_len) return;
    const float wt = train_wt(p, p.w_cont[t]);
    w_int[t] = (int)floorf(wt) + 1;
    if (p.dw_h)  // backward: rows outside every sequence keep a zero gradient
        for (int h = 0; h < p.n_heads; ++h) p.dw_h[(int64_t)t * p.n_heads + h] = 0.f;
}

hipError_t train_windows_launch(const AttnParams& p, int* w_int, hipStream_t stream) {
    if (p.total_len == 0) return hipSuccess;
    DSALT_LAUNCH("train_windows", train_windows_kernel, dim3(ceil_div(p.total_len, 256)), dim3(256), 0, stream, p,
                 w_int);
    return hipGetLastError();
}

hipError_t fwd_launch(AttnParams p, void* ws, void* plan, bool plan_ready, hipStream_t stream) {
    char* w = (char*)(plan ? plan : ws);
    plan_carve(p, w);
    const bool ready = plan_ready && plan != nullptr;
    if (p.dtype == DSALT_DTYPE_BF16) return fwd_dispatch<bf16>(p, ready, stream);
    if (p.dtype == DSALT_DTYPE_F16) return fwd_dispatch<f16>(p, ready, stream);
    return fwd_dispatch<float>(p, ready, stream);
}

}  // namespace dsalt
