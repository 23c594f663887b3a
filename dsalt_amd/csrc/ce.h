// Row cross-entropy of the fused linear cross-entropy (loss and, in place, the gradient
// with respect to the logits).
#pragma once
#include <hip/hip_runtime.h>

#include <stdint.h>

namespace dsalt {

struct CeParams {
    int rows, n_cols, dtype;
    void* x;               // [rows, n_cols] logits, overwritten by the gradient when grads
    int64_t x_st;
    const int64_t* target; // [rows]
    const float* ce_weight;  // [n_cols] or null
    float* loss;           // [rows]
    void* z_loss;          // [rows] in the logits' type, or null
    float* accuracy;       // [rows] or null
    int64_t* predicted;    // [rows] or null
    int64_t ignore_index;
    float n_non_ignore, sum_non_ignore_weight, weight_sum;
    float lse_square_scale, label_smoothing, softcap;  // softcap 0: none
    int reduction;         // 0 none, 1 mean, 2 sum
    int grads, token_scaling;
};

hipError_t ce_launch(const CeParams& p, hipStream_t stream);

}  // namespace dsalt
