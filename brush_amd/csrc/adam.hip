// adam.hip — the AdamScaled optimizer step for gfx950.
//
// Restates AdamScaled::step and AdaptiveMomentum::transform
// (crates/brush-train/src/adam_scaled.rs:216-383): per element
//   m1 = m1 * b1 + g * (1 - b1)           (m1 = g * (1 - b1) on the first step)
//   m2 = m2 * b2 + g2 * (1 - b2)          (m2 = g2 * (1 - b2) on the first step)
//   step = (m1 / bc1) / (sqrt(m2 / bc2) + eps),  bc = 1 - b^t
//   param -= step * (scale[col] * lr)     (step * lr without a scale vector)
// where g2 = g * g, or, with reduce_moment_2, the mean of g * g over the row
// (the SH second moment kept as one value per splat, train.rs:966-990).
//
// One workgroup takes a contiguous run of rows; the element-wise work walks
// the run with consecutive threads on consecutive floats (coalesced), and the
// per-row mean of a reduced second moment goes through LDS, summed per row in
// index order.
#include <hip/hip_runtime.h>

#include "bh_internal.h"

namespace bh {

struct AdamParams {
    float b1, b2, one_minus_b1, one_minus_b2, bc1, bc2, eps, lr;
    uint32_t first;
};

constexpr uint32_t kAdamThreads = 256;
constexpr uint32_t kAdamChunk = 4096;  // floats of a reduced-moment run held in LDS

// Updates m1 in place and returns the parameter decrement of one element whose
// (already updated) second moment is m2.
__device__ __forceinline__ float adam_delta(const AdamParams& a, float g, float& m1, float m2,
                                            const float* __restrict__ scaling, uint32_t col) {
    m1 = a.first ? g * a.one_minus_b1 : m1 * a.b1 + g * a.one_minus_b1;
    const float m1c = m1 / a.bc1;
    const float m2c = m2 / a.bc2;
    const float step = m1c / (sqrtf(m2c) + a.eps);
    return scaling ? step * (scaling[col] * a.lr) : step * a.lr;
}

// Element-wise second moment (reduce_moment_2 off).
__global__ __launch_bounds__(kAdamThreads) void adam_elementwise_kernel(AdamParams a, float* __restrict__ param,
                                                                         const float* __restrict__ grad,
                                                                         float* __restrict__ m1,
                                                                         float* __restrict__ m2,
                                                                         const float* __restrict__ scaling,
                                                                         uint64_t count, uint32_t row_len) {
    const uint64_t stride = (uint64_t)gridDim.x * kAdamThreads;
    for (uint64_t e = (uint64_t)blockIdx.x * kAdamThreads + threadIdx.x; e < count; e += stride) {
        const float g = grad[e];
        const float g2 = g * g;
        const float v2 = a.first ? g2 * a.one_minus_b2 : m2[e] * a.b2 + g2 * a.one_minus_b2;
        float v1 = a.first ? 0.0f : m1[e];
        const float delta = adam_delta(a, g, v1, v2, scaling, (uint32_t)(e % row_len));
        param[e] = param[e] - delta;
        m1[e] = v1;
        m2[e] = v2;
    }
}

// Second moment reduced to one value per row: each workgroup takes
// rows_per_block rows (at most kAdamChunk floats).
__global__ __launch_bounds__(kAdamThreads) void adam_row_reduced_kernel(AdamParams a, float* __restrict__ param,
                                                                         const float* __restrict__ grad,
                                                                         float* __restrict__ m1,
                                                                         float* __restrict__ m2,
                                                                         const float* __restrict__ scaling,
                                                                         uint32_t rows, uint32_t row_len,
                                                                         uint32_t rows_per_block) {
    __shared__ float s_g2[kAdamChunk];
    __shared__ float s_m2[256];
    const uint64_t r0 = (uint64_t)blockIdx.x * rows_per_block;
    const uint32_t nrows = (uint32_t)min<uint64_t>(rows_per_block, rows - r0);
    const uint32_t count = nrows * row_len;
    const uint64_t base = r0 * row_len;
    for (uint32_t i = threadIdx.x; i < count; i += kAdamThreads) {
        const float g = grad[base + i];
        s_g2[i] = g * g;
    }
    __syncthreads();
    // mean_trailing_dims (adam_scaled.rs:287-300): row sum / row length
    for (uint32_t r = threadIdx.x; r < nrows; r += kAdamThreads) {
        float sum = 0.0f;
        for (uint32_t k = 0; k < row_len; k++) sum += s_g2[r * row_len + k];
        const float mean = sum / (float)row_len;
        const float v2 = a.first ? mean * a.one_minus_b2 : m2[r0 + r] * a.b2 + mean * a.one_minus_b2;
        m2[r0 + r] = v2;
        s_m2[r] = v2;
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < count; i += kAdamThreads) {
        const uint32_t r = i / row_len, col = i % row_len;
        const float g = grad[base + i];
        float v1 = a.first ? 0.0f : m1[base + i];
        const float delta = adam_delta(a, g, v1, s_m2[r], scaling, col);
        param[base + i] = param[base + i] - delta;
        m1[base + i] = v1;
    }
}

// b^t in f32 by binary exponentiation (the squaring loop of an integer power;
// t >= 1).
static float powi_f32(float b, uint32_t t) {
    float r = 1.0f;
    for (;;) {
        if (t & 1u) r *= b;
        t >>= 1;
        if (t == 0) break;
        b *= b;
    }
    return r;
}

bh_status launch_adam_step(bh_ctx* ctx, float* param, const float* grad, float* m1, float* m2,
                           const float* scaling, uint32_t rows, uint32_t row_len, bool reduce, float lr,
                           uint32_t time, const bh_adam_config& cfg) {
    AdamParams a;
    a.b1 = cfg.beta_1;
    a.b2 = cfg.beta_2;
    a.one_minus_b1 = 1.0f - cfg.beta_1;
    a.one_minus_b2 = 1.0f - cfg.beta_2;
    a.bc1 = 1.0f - powi_f32(cfg.beta_1, time);
    a.bc2 = 1.0f - powi_f32(cfg.beta_2, time);
    a.eps = cfg.epsilon;
    a.lr = lr;
    a.first = time == 1 ? 1u : 0u;
    const uint64_t count = (uint64_t)rows * row_len;
    if (count == 0) return BH_OK;
    KernelTimer t(ctx, "adam_step");
    if (reduce && row_len > 1) {
        if (row_len > kAdamChunk) return set_error(ctx, BH_ERR_INVALID_ARG, "adam: reduced rows longer than 4096");
        const uint32_t rpb = std::max<uint32_t>(1u, std::min<uint32_t>(kAdamChunk / row_len, 256u));
        adam_row_reduced_kernel<<<div_up(rows, rpb), kAdamThreads, 0, ctx->stream>>>(a, param, grad, m1, m2, scaling,
                                                                                       rows, row_len, rpb);
    } else {
        const uint32_t blocks = (uint32_t)std::min<uint64_t>(div_up(count, kAdamThreads), 8192);
        adam_elementwise_kernel<<<blocks, kAdamThreads, 0, ctx->stream>>>(a, param, grad, m1, m2, scaling, count,
                                                                           row_len);
    }
    return check_launch(ctx, "adam step");
}

}  // namespace bh
