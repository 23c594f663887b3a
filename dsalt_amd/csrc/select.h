// Internal launch interface of the selection and gather kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dsalt_amd.h"

namespace dsalt {

struct SelectParams {
    int total_len, num_seqs, max_seqlen, n_heads, n_kv_heads, head_dim, k_lmk;
    int select_mode, block_size, dtype, hidden, stats_scope, n_sets;
    const void* h;
    int64_t h_stride_t;
    const void* v;
    int64_t v_stride_t, v_stride_h;
    const float* alpha;
    const int32_t* w;
    const int32_t* cu;
    int32_t* lmk_idx;
    float* z_x;
    float* z_v;
    float* scores;
    // optional row plan of the forward (plan.h), written by extra blocks of the norms launch
    uint8_t* plan_perm;      // null: no plan
    int* plan_bounds;
    int* tile_wmax;
    int n_tiles;             // 64-row tiles per sequence, ceil(max_seqlen / 64)
};

struct GatherParams {
    int total_len, num_seqs, max_seqlen, n_heads, n_kv_heads, head_dim, k_lmk, n_sets, dtype;
    const void* k;
    int64_t k_stride_t, k_stride_h;
    const void* v;
    int64_t v_stride_t, v_stride_h;
    const int32_t* cu;
    const int32_t* lmk_idx;
    void* lmk_k;
    void* lmk_v;
};

size_t select_workspace(const SelectParams& p);
size_t select_workspace_cap(const SelectParams& p, int border_cap);  // workspace of a border_cap call
hipError_t select_launch(const SelectParams& p, void* ws, hipStream_t stream, int border_cap);
hipError_t gather_launch(const GatherParams& p, hipStream_t stream);

}  // namespace dsalt
