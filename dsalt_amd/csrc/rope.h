// Rotary position embedding applied in place to packed query and key heads.
#pragma once
#include <hip/hip_runtime.h>

#include <stdint.h>

namespace dsalt {

struct RopeParams {
    int total_len, num_seqs, n_q_heads, n_k_heads, head_dim, dtype;
    void* q;
    int64_t q_st, q_sh;
    void* k;
    int64_t k_st, k_sh;
    const int* cu;
    const float* cos;  // [max_pos, head_dim]
    const float* sin;
    int max_pos;
};

hipError_t rope_launch(const RopeParams& p, hipStream_t stream);

}  // namespace dsalt
