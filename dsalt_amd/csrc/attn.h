// Internal launch interface of the attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dsalt_amd.h"

namespace dsalt {

constexpr int kNoOwner = 0x7fffffff;  // owner of a key that is no landmark row

struct AttnParams {
    int total_len, num_seqs, max_seqlen, n_heads, n_kv_heads, head_dim, k_lmk;
    int n_sets, block_size;  // block_size 0 in the global variant
    int dtype;
    int n_tiles;             // 64-row tiles per sequence, ceil(max_seqlen / 64)
    float scale;
    float c2;                // scale * log2(e)
    float inv_scale;         // 1 / scale
    float thr;               // lazy-rescale threshold in raw logits, 8 / c2
    const void* q;
    int64_t q_st, q_sh;
    const void* k;
    int64_t k_st, k_sh;
    const void* v;
    int64_t v_st, v_sh;
    const void* o;           // forward: output; backward: saved output
    int64_t o_st, o_sh;
    const void* dout;
    int64_t do_st, do_sh;
    const float* lse;        // [T, H]
    float* lse_out;
    const int32_t* w;
    const int32_t* cu;
    const int32_t* lmk;      // [H, S, n_sets, K]
    const float* lbias;      // same shape or null
    void* dq;
    void* dk;
    void* dv;
    float* d_bias;
    // training variant: soft window edge (w_cont null for the inference operator)
    const float* w_cont;     // [T] continuous windows w~ (values below 0 act as 0)
    float tau_inv;           // 1 / tau_win
    float edge;              // win_edge: band keys with d > w~ - edge carry log sigmoid((w~ - d) / tau)
    int edge_keys;           // ceil(win_edge): bound on the band keys of a row that carry the edge bias
    float* dw_h;             // [T, H] d loss / d w~ per head (training backward workspace)
    float* d_w;              // [T] d loss / d w~ summed over heads (training backward output)
    // row plan (forward and backward workspace), per 64-row tile of each sequence:
    // rows ordered by window start, and per 16-row group {min lo, max lo, max i, min i}
    uint8_t* plan_perm;      // [S * n_tiles * 64] row offset within the tile
    int* plan_bounds;        // [S * n_tiles * 4 * 4]
    int* tile_wmax;          // [S * n_tiles] largest clamped window of the tile's rows
    int variant;             // DSALT_VARIANT_* bits
    // backward workspace
    float* delta;            // [H, T] -rowsum(O * dO), head-major (written by the dQ pass; the
                             // key-parallel passes start their dP products from it)
    int* cnt;                // [H, T] landmarks visible to each row (written by the dQ pass)
    float* lse2t;            // [H, T] LSE * log2(e), head-major (written by the dQ pass)
    float* part_k;           // [n_chunks, H, S, K, D] landmark dK partials
    float* part_v;           // [n_chunks, H, S, K, D]
    float* part_b;           // [n_chunks, H, S, K]
    float* lmk_stage;        // [2, H, S, K, D] fp32 band dK / dV of landmark rows (dK/dV pass), at
                             // the row's owner: the first (head, slot) of its group holding it
    int n_chunks;            // row chunks of the landmark backward
};

// Training variant: a row's continuous window as the kernels take it, in [0, max_seqlen +
// ceil(win_edge)].  Above that bound every band key of any row (d <= max_seqlen - 1) lies in
// the core (wt - d > win_edge), no landmark is visible and d bias / d wt is 0, so the clamp
// changes no value; floor and fraction are both taken from the clamped window.
__device__ __forceinline__ float train_wt(const AttnParams& p, float w_cont) {
    return fminf(fmaxf(w_cont, 0.f), (float)(p.max_seqlen + p.edge_keys));
}

// Training variant, band key at distance d = i - j of a row with continuous window wt:
// logit bias log sigmoid((wt - d) / tau) outside the core d <= wt - edge, 0 inside,
// returned in raw-score units (divided by the logit scale).
__device__ __forceinline__ float edge_bias(const AttnParams& p, float wt, int d) {
    const float fd = wt - (float)d;
    return fd >= p.edge ? 0.f : -__logf(1.f + __expf(-fd * p.tau_inv)) * p.inv_scale;
}
// bias and d bias / d wt of the same key, sharing one exponential: d bias / d wt is
// (1 - sigmoid((wt - d) / tau)) / tau outside the core, 0 inside (keys outside the band
// get finite values; callers mask them)
__device__ __forceinline__ void edge_terms(const AttnParams& p, float wt, int d, float& bias, float& grad) {
    const float fd = fmaxf(wt - (float)d, 0.f);
    const float e = __expf(-fd * p.tau_inv);
    const bool inside = fd >= p.edge;
    bias = inside ? 0.f : -__logf(1.f + e) * p.inv_scale;
    grad = inside ? 0.f : e * __builtin_amdgcn_rcpf(1.f + e) * p.tau_inv;
}

// The soft edge of a row with continuous window wt covers at most ceil(win_edge) band
// keys from the unclamped window start lo_u = i - floor(wt): key lo_u + k sits at
// wt - d = frac(wt) + k.  For win_edge <= 4 the kernels read a row's edge terms from
// a four-entry table built once per row (no transcendentals per key).
constexpr int kEdgeTab = 4;
__device__ __forceinline__ void edge_table(const AttnParams& p, float wt, float* b, float* g) {
    const float fr = wt - floorf(wt);
#pragma unroll
    for (int k = 0; k < kEdgeTab; ++k) {
        float bb, gg;
        edge_terms(p, fr + (float)k, 0, bb, gg);
        b[k] = bb;
        if (g) g[k] = gg;
    }
}
// table entry for key offset k from lo_u (0 from kEdgeTab on: the core)
__device__ __forceinline__ float edge_lookup(const float* t, int k) {
    float v = 0.f;
#pragma unroll
    for (int e = 0; e < kEdgeTab; ++e) v = k == e ? t[e] : v;
    return v;
}

size_t plan_bytes(const AttnParams& p);
void plan_carve(AttnParams& p, char*& ws);  // assigns plan_perm / plan_bounds / tile_wmax from a buffer
hipError_t plan_launch(const AttnParams& p, hipStream_t stream);
// plan: a caller buffer of plan_bytes() that receives the row plan, or null (workspace);
// plan_ready: the buffer already holds the plan of these rows (not recomputed)
hipError_t fwd_launch(AttnParams p, void* ws, void* plan, bool plan_ready, hipStream_t stream);
// training variant: integer windows floor(w~) + 1 written into `w_int` ([T] int32)
hipError_t train_windows_launch(const AttnParams& p, int* w_int, hipStream_t stream);
// plan_given: the caller supplies the row plan (no room for it in the workspace)
size_t bwd_workspace(const AttnParams& p, bool plan_given);
// plan: the row plan the forward wrote for the same rows, or null (computed here)
hipError_t bwd_launch(AttnParams p, void* ws, const void* plan, hipStream_t stream);
// training variant: d_w[t] = sum over heads of dw_h[t, h], in head order
hipError_t train_dw_launch(const AttnParams& p, hipStream_t stream);

}  // namespace dsalt
