// Internal launch interface of the attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dsalt_amd.h"

namespace dsalt {

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
    // row plan (forward and backward workspace), per 64-row tile of each sequence:
    // rows ordered by window start, and per 16-row group {min lo, max lo, max i, min i}
    uint8_t* plan_perm;      // [S * n_tiles * 64] row offset within the tile
    int* plan_bounds;        // [S * n_tiles * 4 * 4]
    // backward workspace
    float* delta;            // [T, H]
    int* cnt;                // [T, H] landmarks visible to each row (written by the dQ pass)
    int* seq_wmax;           // [S] max clamped window per sequence
    float* part_k;           // [n_chunks, H, S, K, D] landmark dK partials
    float* part_v;           // [n_chunks, H, S, K, D]
    float* part_b;           // [n_chunks, H, S, K]
    int n_chunks;            // row chunks of the landmark backward
};

size_t plan_bytes(const AttnParams& p);
void plan_carve(AttnParams& p, char*& ws);  // assigns plan_perm / plan_bounds from a workspace
hipError_t plan_launch(const AttnParams& p, hipStream_t stream);
hipError_t fwd_launch(AttnParams p, void* ws, hipStream_t stream);
size_t bwd_workspace(const AttnParams& p);
hipError_t bwd_launch(AttnParams p, void* ws, hipStream_t stream);

}  // namespace dsalt
