// out = silu(gate) * up, row by row, for the SwiGLU feed-forward block whose gate and up
// projections come from one GEMM (gate and up then are column ranges of one buffer).
// Arithmetic of the elementwise pair silu(g) then * u in the tensor type: silu in float32
// as g / (1 + exp(-g)) rounded to the type, the product of two values of the type in
// float32 rounded to the type.  HBM-bound: two reads and one write per element.  A thread
// takes 8 columns (16-byte vectors); the last cols mod 8 columns of a row element by element.
#include "common.h"
#include "ffn.h"
#include "timing.h"

namespace dsalt {

namespace {

template <typename T>
__global__ __launch_bounds__(256) void silu_mul_kernel(SiluMulParams p) {
    const int per_row = (p.cols + 7) >> 3;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= (int64_t)p.rows * per_row) return;
    const int r = (int)(gid / per_row);
    const int c = (int)(gid - (int64_t)r * per_row) * 8;
    const T* gr = (const T*)p.gate + (int64_t)r * p.gate_st;
    const T* ur = (const T*)p.up + (int64_t)r * p.up_st;
    T* orow = (T*)p.out + (int64_t)r * p.out_st;
    auto one = [](float x, float u) {
        const float s = to_float(from_float<T>(x / (1.0f + expf(-x))));
        return from_float<T>(s * u);
    };
    if (c + 8 <= p.cols) {
        typedef T vec8 __attribute__((ext_vector_type(8), aligned(16)));
        const vec8 g = *(const vec8*)(gr + c);
        const vec8 u = *(const vec8*)(ur + c);
        vec8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = one(to_float(g[e]), to_float(u[e]));
        *(vec8*)(orow + c) = o;
    } else {
        for (int e = c; e < p.cols; ++e) orow[e] = one(to_float(gr[e]), to_float(ur[e]));
    }
}

}  // namespace

hipError_t silu_mul_launch(const SiluMulParams& p, hipStream_t stream) {
    const int64_t n = (int64_t)p.rows * ((p.cols + 7) / 8);
    if (n == 0) return hipSuccess;
    const dim3 grid((unsigned)((n + 255) / 256));
    switch (p.dtype) {
        case 0: DSALT_LAUNCH("silu_mul", silu_mul_kernel<float>, grid, dim3(256), 0, stream, p); break;
        case 1: DSALT_LAUNCH("silu_mul", silu_mul_kernel<bf16>, grid, dim3(256), 0, stream, p); break;
        default: DSALT_LAUNCH("silu_mul", silu_mul_kernel<f16>, grid, dim3(256), 0, stream, p); break;
    }
    return hipGetLastError();
}

}  // namespace dsalt
