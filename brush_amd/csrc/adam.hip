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

// Element-wise second moment (reduce_moment_2 off).  Each thread walks the
// parameter with a grid stride in groups of 4 floats (16-byte accesses when
// every array is 16-byte aligned); the column of an element for the scale
// vector is tracked incrementally, without a division per element.
template <bool VEC4>
__global__ __launch_bounds__(kAdamThreads) void adam_elementwise_kernel(AdamParams a, float* __restrict__ param,
                                                                         const float* __restrict__ grad,
                                                                         float* __restrict__ m1,
                                                                         float* __restrict__ m2,
                                                                         const float* __restrict__ scaling,
                                                                         uint64_t count, uint32_t row_len) {
    const uint64_t groups = VEC4 ? count / 4u : count;
    const uint64_t stride = (uint64_t)gridDim.x * kAdamThreads;
    uint64_t gi = (uint64_t)blockIdx.x * kAdamThreads + threadIdx.x;
    const uint32_t per = VEC4 ? 4u : 1u;
    // column of the first element of group gi, and how far it moves per stride
    uint32_t col = (uint32_t)((gi * per) % row_len);
    const uint32_t step_col = (uint32_t)((stride * per) % row_len);
    for (; gi < groups; gi += stride) {
        if (VEC4) {
            const uint64_t e = gi * 4u;
            const float4 g = reinterpret_cast<const float4*>(grad)[gi];
            float4 p = reinterpret_cast<float4*>(param)[gi];
            float4 v1 = a.first ? make_float4(0.0f, 0.0f, 0.0f, 0.0f) : reinterpret_cast<float4*>(m1)[gi];
            float4 v2 = a.first ? make_float4(0.0f, 0.0f, 0.0f, 0.0f) : reinterpret_cast<float4*>(m2)[gi];
            float* pg = &p.x;
            float* p1 = &v1.x;
            float* p2 = &v2.x;
            const float* gg = &g.x;
            uint32_t c = col;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float g2 = gg[j] * gg[j];
                p2[j] = a.first ? g2 * a.one_minus_b2 : p2[j] * a.b2 + g2 * a.one_minus_b2;
                pg[j] = pg[j] - adam_delta(a, gg[j], p1[j], p2[j], scaling, c);
                c = c + 1u == row_len ? 0u : c + 1u;
            }
            (void)e;
            reinterpret_cast<float4*>(param)[gi] = p;
            reinterpret_cast<float4*>(m1)[gi] = v1;
            reinterpret_cast<float4*>(m2)[gi] = v2;
        } else {
            const float g = grad[gi];
            const float g2 = g * g;
            const float v2 = a.first ? g2 * a.one_minus_b2 : m2[gi] * a.b2 + g2 * a.one_minus_b2;
            float v1 = a.first ? 0.0f : m1[gi];
            const float delta = adam_delta(a, g, v1, v2, scaling, col);
            param[gi] = param[gi] - delta;
            m1[gi] = v1;
            m2[gi] = v2;
        }
        col += step_col;
        if (col >= row_len) col -= row_len;
    }
    // the tail past the last group of four (VEC4 only)
    if (VEC4 && blockIdx.x == 0 && threadIdx.x < (uint32_t)(count - groups * 4u)) {
        const uint64_t e = groups * 4u + threadIdx.x;
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
// rows_per_block rows (at most kAdamChunk floats); the gradient run stays in
// LDS between the row sums and the update.
__global__ __launch_bounds__(kAdamThreads) void adam_row_reduced_kernel(AdamParams a, float* __restrict__ param,
                                                                         const float* __restrict__ grad,
                                                                         float* __restrict__ m1,
                                                                         float* __restrict__ m2,
                                                                         const float* __restrict__ scaling,
                                                                         uint32_t rows, uint32_t row_len,
                                                                         uint32_t rows_per_block) {
    __shared__ float s_g[kAdamChunk];
    __shared__ float s_m2[256];
    const uint64_t r0 = (uint64_t)blockIdx.x * rows_per_block;
    const uint32_t nrows = (uint32_t)min<uint64_t>(rows_per_block, rows - r0);
    const uint32_t count = nrows * row_len;
    const uint64_t base = r0 * row_len;
    for (uint32_t i = threadIdx.x; i < count; i += kAdamThreads) s_g[i] = grad[base + i];
    __syncthreads();
    // mean_trailing_dims (adam_scaled.rs:287-300): row sum of g^2 / row length
    for (uint32_t r = threadIdx.x; r < nrows; r += kAdamThreads) {
        float sum = 0.0f;
        for (uint32_t k = 0; k < row_len; k++) {
            const float g = s_g[r * row_len + k];
            sum += g * g;
        }
        const float mean = sum / (float)row_len;
        const float v2 = a.first ? mean * a.one_minus_b2 : m2[r0 + r] * a.b2 + mean * a.one_minus_b2;
        m2[r0 + r] = v2;
        s_m2[r] = v2;
    }
    __syncthreads();
    // element i of the run: row and column tracked as i advances by the block size
    uint32_t r = threadIdx.x / row_len, col = threadIdx.x % row_len;
    const uint32_t dr = kAdamThreads / row_len, dc = kAdamThreads % row_len;
    for (uint32_t i = threadIdx.x; i < count; i += kAdamThreads) {
        const float g = s_g[i];
        float v1 = a.first ? 0.0f : m1[base + i];
        const float delta = adam_delta(a, g, v1, s_m2[r], scaling, col);
        param[base + i] = param[base + i] - delta;
        m1[base + i] = v1;
        r += dr;
        col += dc;
        if (col >= row_len) {
            col -= row_len;
            r += 1u;
        }
    }
}

// The reduced second moment for rows of a multiple of 4 floats with 16-byte
// aligned arrays: each thread loads its (at most ITEMS) float4 groups of g,
// param and m1 up front, so the loads are in flight across the row sums; g
// also goes to LDS for the sums.  A group never straddles two rows.
template <int ITEMS>
__global__ __launch_bounds__(kAdamThreads) void adam_row_reduced_vec4_kernel(
    AdamParams a, float* __restrict__ param, const float* __restrict__ grad, float* __restrict__ m1,
    float* __restrict__ m2, const float* __restrict__ scaling, uint32_t rows, uint32_t row_len,
    uint32_t rows_per_block) {
    __shared__ float4 s_g[kAdamChunk / 4];
    __shared__ float s_m2[256];
    const uint64_t r0 = (uint64_t)blockIdx.x * rows_per_block;
    const uint32_t nrows = (uint32_t)min<uint64_t>(rows_per_block, rows - r0);
    const uint32_t quads = nrows * row_len / 4u, row_quads = row_len / 4u;
    const uint64_t base = r0 * row_quads;
    const float4* g4 = reinterpret_cast<const float4*>(grad) + base;
    float4* p4 = reinterpret_cast<float4*>(param) + base;
    float4* m14 = reinterpret_cast<float4*>(m1) + base;
    float4 g[ITEMS], pv[ITEMS], v1[ITEMS];
    // every load first (unconditional, at indices clamped into the block's
    // run: a load in a branch that also stores to LDS waits before the next
    // item's loads), then the LDS stores
#pragma unroll
    for (int i = 0; i < ITEMS; i++) {
        const uint32_t q = min(threadIdx.x + (uint32_t)i * kAdamThreads, quads - 1u);
        g[i] = g4[q];
        pv[i] = p4[q];
        v1[i] = a.first ? make_float4(0.0f, 0.0f, 0.0f, 0.0f) : m14[q];
    }
#pragma unroll
    for (int i = 0; i < ITEMS; i++) {
        const uint32_t q = threadIdx.x + (uint32_t)i * kAdamThreads;
        if (q < quads) s_g[q] = g[i];
    }
    __syncthreads();
    // mean_trailing_dims (adam_scaled.rs:287-300): row sum of g^2 in index order / row length
    for (uint32_t r = threadIdx.x; r < nrows; r += kAdamThreads) {
        float sum = 0.0f;
        for (uint32_t k = 0; k < row_quads; k++) {
            const float4 q = s_g[r * row_quads + k];
            sum += q.x * q.x;
            sum += q.y * q.y;
            sum += q.z * q.z;
            sum += q.w * q.w;
        }
        const float mean = sum / (float)row_len;
        const float v2 = a.first ? mean * a.one_minus_b2 : m2[r0 + r] * a.b2 + mean * a.one_minus_b2;
        m2[r0 + r] = v2;
        s_m2[r] = v2;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < ITEMS; i++) {
        const uint32_t q = threadIdx.x + (uint32_t)i * kAdamThreads;
        if (q < quads) {
            const uint32_t r = q / row_quads;
            const uint32_t col = (q - r * row_quads) * 4u;
            const float v2 = s_m2[r];
            pv[i].x = pv[i].x - adam_delta(a, g[i].x, v1[i].x, v2, scaling, col);
            pv[i].y = pv[i].y - adam_delta(a, g[i].y, v1[i].y, v2, scaling, col + 1u);
            pv[i].z = pv[i].z - adam_delta(a, g[i].z, v1[i].z, v2, scaling, col + 2u);
            pv[i].w = pv[i].w - adam_delta(a, g[i].w, v1[i].w, v2, scaling, col + 3u);
            p4[q] = pv[i];
            m14[q] = v1[i];
        }
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
        const bool vec4 = row_len % 4u == 0u && ((reinterpret_cast<uintptr_t>(param) |
                                                  reinterpret_cast<uintptr_t>(grad) |
                                                  reinterpret_cast<uintptr_t>(m1)) &
                                                 15u) == 0u;
        if (vec4)
            launch(ctx, adam_row_reduced_vec4_kernel<kAdamChunk / 4 / kAdamThreads>, dim3(div_up(rows, rpb)),
                   dim3(kAdamThreads), 0u, a, param, grad, m1, m2, scaling, rows, row_len, rpb);
        else
            launch(ctx, adam_row_reduced_kernel, dim3(div_up(rows, rpb)), dim3(kAdamThreads), 0u, a, param, grad, m1,
                   m2, scaling, rows, row_len, rpb);
    } else {
        const bool vec4 = count >= 4 && ((reinterpret_cast<uintptr_t>(param) | reinterpret_cast<uintptr_t>(grad) |
                                          reinterpret_cast<uintptr_t>(m1) | reinterpret_cast<uintptr_t>(m2)) &
                                         15u) == 0u;
        const uint32_t blocks =
            (uint32_t)std::max<uint64_t>(1u, std::min<uint64_t>(div_up(vec4 ? count / 4 : count, kAdamThreads), 1u << 20));
        if (vec4)
            launch(ctx, adam_elementwise_kernel<true>, dim3(blocks), dim3(kAdamThreads), 0u, a, param, grad, m1, m2,
                   scaling, count, row_len);
        else
            launch(ctx, adam_elementwise_kernel<false>, dim3(blocks), dim3(kAdamThreads), 0u, a, param, grad, m1, m2,
                   scaling, count, row_len);
    }
    return check_launch(ctx, "adam step");
}

}  // namespace bh
