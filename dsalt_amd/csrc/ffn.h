// Gated activation of the SwiGLU feed-forward block.
#pragma once
#include <hip/hip_runtime.h>

#include <stdint.h>

namespace dsalt {

struct SiluMulParams {
    int rows, cols, dtype;
    const void* gate;
    int64_t gate_st;
    const void* up;
    int64_t up_st;
    void* out;
    int64_t out_st;
};

hipError_t silu_mul_launch(const SiluMulParams& p, hipStream_t stream);

}  // namespace dsalt
