// Row cross-entropy for the fused linear cross-entropy: one block per row of logits.
// Pass 1 streams the row once (8 elements per thread per step, then the last V mod 8
// elements one per thread: any vocabulary size, rows 16-byte aligned) for the running max and
// the sum of exponentials (rescaled once per 8-element step), the label-smoothing sum and
// the first index of the largest logit; the block combines them.  Pass 2 writes the
// gradient with respect to the logits in place.  Formulas (float32):
//   x <- softcap tanh(x / softcap) when softcapped; lse = m + log d;
//   loss = w_y (lse - x_y), with label smoothing eps = ls / V:
//          (1 - ls) loss + eps sum_c w_c (lse - x_c); z = zs lse^2;
//   "mean" divides the loss by the sum of w_y over kept rows and z by their count;
//   gradient, no class weights: softmax (1 + 2 zs lse) - eps - (1 - ls) [c == y] (/ n);
//   with class weights: (1 - ls) w_y (softmax - [c == y]) (/ sum w_y)
//                       + eps (softmax sum w - w_c) (/ sum w_y) + 2 zs lse softmax (/ n);
//   softcapped logits multiply the gradient by 1 - tanh^2; token scaling multiplies loss,
//   z and gradient by the row's probability of its target.
// HBM-bound: the row is read twice and written once.
#include "ce.h"
#include "common.h"
#include "timing.h"

namespace dsalt {

namespace {

constexpr int kCeThreads = 512;

struct RowStats {
    float m, d, sx;  // running max, sum of exp(x - m), label-smoothing sum
    float bv;        // largest logit
    int bi;          // its first index
};

__device__ __forceinline__ void merge(RowStats& a, const RowStats& b) {
    const float M = fmaxf(a.m, b.m);
    const float da = a.m == -INFINITY ? 0.f : a.d * __expf(a.m - M);
    const float db = b.m == -INFINITY ? 0.f : b.d * __expf(b.m - M);
    a.m = M;
    a.d = da + db;
    a.sx += b.sx;
    if (b.bv > a.bv || (b.bv == a.bv && b.bi < a.bi)) {
        a.bv = b.bv;
        a.bi = b.bi;
    }
}

__device__ __forceinline__ float capped(float x, float softcap) {
    return softcap > 0.f ? softcap * tanhf(x / softcap) : x;
}

template <typename T>
__global__ __launch_bounds__(kCeThreads) void ce_kernel(CeParams p) {
    typedef T vec8 __attribute__((ext_vector_type(8), aligned(16)));
    __shared__ RowStats red[kCeThreads / 64];
    __shared__ RowStats row;
    __shared__ float xy_s;  // the target's logit, read before any thread overwrites the row
    const int r = blockIdx.x, tid = threadIdx.x;
    T* X = (T*)p.x + (int64_t)r * p.x_st;
    const int64_t y = p.target[r];
    const int V = p.n_cols;
    const int V8 = V & ~7;  // whole 8-element vectors; the tail V8 .. V-1 one element per thread
    const bool has_w = p.ce_weight != nullptr;
    const float eps = p.label_smoothing / (float)V;
    if (y == p.ignore_index) {
        if (p.grads) {
            vec8 zero;
#pragma unroll
            for (int e = 0; e < 8; ++e) zero[e] = from_float<T>(0.f);
            for (int c = tid * 8; c < V8; c += kCeThreads * 8) *(vec8*)(X + c) = zero;
            for (int c = V8 + tid; c < V; c += kCeThreads) X[c] = from_float<T>(0.f);
        }
        if (tid == 0) {
            p.loss[r] = 0.f;
            if (p.z_loss) ((T*)p.z_loss)[r] = from_float<T>(0.f);
            if (p.accuracy) p.accuracy[r] = 0.f;
            if (p.predicted) p.predicted[r] = -1;
        }
        return;
    }
    RowStats s = {-INFINITY, 0.f, 0.f, -INFINITY, 0x7fffffff};
    for (int c = tid * 8; c < V8; c += kCeThreads * 8) {
        const vec8 v = *(const vec8*)(X + c);
        float xv[8];
        float m8 = -INFINITY;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            xv[e] = capped(to_float(v[e]), p.softcap);
            m8 = fmaxf(m8, xv[e]);
        }
        if (m8 > s.bv) {  // first index of the largest value in this step (earlier steps win ties)
            int bi = c;
#pragma unroll
            for (int e = 7; e >= 0; --e) bi = xv[e] == m8 ? c + e : bi;
            s.bv = m8;
            s.bi = bi;
        }
        if (m8 > s.m) {
            s.d = s.m == -INFINITY ? 0.f : s.d * __expf(s.m - m8);
            s.m = m8;
        }
        float d8 = 0.f, sx8 = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            d8 += __expf(xv[e] - s.m);
            sx8 += has_w ? xv[e] * p.ce_weight[c + e] : xv[e];
        }
        s.d += d8;
        s.sx += sx8;
    }
    for (int c = V8 + tid; c < V; c += kCeThreads) {  // the tail: indices past every vector's
        const float xv = capped(to_float(X[c]), p.softcap);
        if (xv > s.bv) {
            s.bv = xv;
            s.bi = c;
        }
        if (xv > s.m) {
            s.d = s.m == -INFINITY ? 0.f : s.d * __expf(s.m - xv);
            s.m = xv;
        }
        s.d += __expf(xv - s.m);
        s.sx += has_w ? xv * p.ce_weight[c] : xv;
    }
    // combine: lanes of a wave, then the waves
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        RowStats o;
        o.m = __shfl_xor(s.m, off);
        o.d = __shfl_xor(s.d, off);
        o.sx = __shfl_xor(s.sx, off);
        o.bv = __shfl_xor(s.bv, off);
        o.bi = __shfl_xor(s.bi, off);
        merge(s, o);
    }
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    if (tid == 0) {
        RowStats t = red[0];
        for (int w = 1; w < kCeThreads / 64; ++w) merge(t, red[w]);
        row = t;
        xy_s = capped(to_float(X[y]), p.softcap);
    }
    __syncthreads();
    const float m = row.m, d = row.d;
    const float lse = m + __logf(d);
    const float xy = xy_s;
    const float wy = has_w ? p.ce_weight[y] : 1.f;
    const float scale_tok = p.token_scaling ? __expf(xy - lse) : 1.f;
    const float zs = p.lse_square_scale, ls = p.label_smoothing;
    const bool mean = p.reduction == 1;
    if (p.grads) {
        const float inv_d = 1.f / d;
        // gradient of logit c (x0 as stored)
        auto grad = [&](float x0, int c) {
            const float th = p.softcap > 0.f ? tanhf(x0 / p.softcap) : 0.f;
            const float xv = p.softcap > 0.f ? p.softcap * th : x0;
            const float sm = __expf(xv - m) * inv_d;
            const bool is_y = c == y;
            float g;
            if (!has_w) {
                g = sm * (1.f + 2.f * zs * lse) - eps - (is_y ? 1.f - ls : 0.f);
                if (mean) g = g / p.n_non_ignore;
            } else {
                float go = (1.f - ls) * (sm - (is_y ? 1.f : 0.f)) * wy;
                float gs = eps * (sm * p.weight_sum - p.ce_weight[c]);
                float gz = 2.f * zs * lse * sm;
                if (mean) {
                    go = go / p.sum_non_ignore_weight;
                    gs = gs / p.sum_non_ignore_weight;
                    gz = gz / p.n_non_ignore;
                }
                g = go + gs + gz;
            }
            if (p.softcap > 0.f) g *= 1.f - th * th;
            return from_float<T>(g * scale_tok);
        };
        for (int c = tid * 8; c < V8; c += kCeThreads * 8) {
            vec8 v = *(const vec8*)(X + c);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = grad(to_float(v[e]), c + e);
            *(vec8*)(X + c) = v;
        }
        for (int c = V8 + tid; c < V; c += kCeThreads) X[c] = grad(to_float(X[c]), c);
    }
    if (tid == 0) {
        float loss = wy * (lse - xy);
        if (ls > 0.f) {
            const float smooth = has_w ? -eps * row.sx + eps * lse * p.weight_sum : -eps * row.sx + ls * lse;
            loss = loss * (1.f - ls) + smooth;
        }
        float z = zs * lse * lse;
        if (mean) {
            loss = loss / (has_w ? p.sum_non_ignore_weight : p.n_non_ignore);
            z = z / p.n_non_ignore;
        }
        loss *= scale_tok;
        z *= scale_tok;
        p.loss[r] = loss + z;
        if (p.z_loss) ((T*)p.z_loss)[r] = from_float<T>(z);
        if (p.accuracy) p.accuracy[r] = row.bi == y ? 1.f : 0.f;
        if (p.predicted) p.predicted[r] = row.bi;
    }
}

}  // namespace

hipError_t ce_launch(const CeParams& p, hipStream_t stream) {
    if (p.rows == 0) return hipSuccess;
    const dim3 grid((unsigned)p.rows);
    switch (p.dtype) {
        case 0: DSALT_LAUNCH("ce_rows", ce_kernel<float>, grid, dim3(kCeThreads), 0, stream, p); break;
        case 1: DSALT_LAUNCH("ce_rows", ce_kernel<bf16>, grid, dim3(kCeThreads), 0, stream, p); break;
        default: DSALT_LAUNCH("ce_rows", ce_kernel<f16>, grid, dim3(kCeThreads), 0, stream, p); break;
    }
    return hipGetLastError();
}

}  // namespace dsalt
