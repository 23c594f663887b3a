// Export of one sequence's attention probabilities in banded form.
#pragma once
#include "attn.h"

namespace dsalt {

struct ProbsParams {
    AttnParams a;     // q, k, w, cu, lmk, lbias, lse_out (forward LSE), scale, shape
    int seq;          // exported sequence
    int out_rows;     // rows of the outputs (the sequence length)
    int w_cap;        // columns of p_win
    float* p_win;     // [H, out_rows, w_cap]
    float* p_lmk;     // [H, out_rows, k_lmk] or null
};

hipError_t probs_launch(const ProbsParams& p, hipStream_t stream);

}  // namespace dsalt
