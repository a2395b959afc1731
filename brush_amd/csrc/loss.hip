// loss.hip — fused L1 + SSIM image loss and its VJP for gfx950.
//
// Restates the image-loss kernels of crates/brush-loss/src/lib.rs:
//   image_l1_forward_kernel / image_loss_forward_kernel   (lib.rs:228-555)
//   image_l1_backward_kernel / image_loss_backward_kernel  (lib.rs:280-893)
// The loss map is l1_w * |pred - gt_eff| + ssim_w * SSIM(pred, gt_eff) per
// colour channel, with SSIM over an 11x11 Gaussian window (sigma 1.5) and
// zero padding outside the image; a 4th (alpha) channel gets |pred.a - gt.a|.
// GT stays packed RGBA8 ([H, W] u32, r in the low byte).  Optional compositing
// gt_eff = gt + (1 - gt.a) * bg and masking by gt.a as in the reference.
//
// Layout differs from the reference on purpose: the reference permutes the
// render to [C, H, W] before its kernels; here `pred` is read in the render's
// own [H, W, stride] layout (stride 4 reads RGB out of an RGBA image) and the
// gradient is written in that layout, zeros in the channels the loss does
// not see, so a training step hands the render's gradient straight to the
// rasterizer's backward.  One workgroup covers a 16x16 tile of one channel
// (grid z = channel); the separable blur is staged in LDS with a 5-pixel halo
// (10 for the backward, which recomputes the partials on a halo ring).
#include <hip/hip_runtime.h>

#include "bh_internal.h"

namespace bh {

constexpr int kLTile = 16;
constexpr int kHalo = 5;
constexpr int kShared = kLTile + 2 * kHalo;    // 26
constexpr int kExtended = kLTile + 4 * kHalo;  // 36

struct LossParams {
    uint32_t w, h, stride, channels;
    float l1_w, ssim_w, bg[3];
    uint32_t composite, mask;
    float taps[6];  // taps[5 - d] is the weight at distance d (taps[5] the centre)
};

constexpr float kC1 = 0.01f * 0.01f;
constexpr float kC2 = 0.03f * 0.03f;
constexpr float kInv255 = 1.0f / 255.0f;

// One packed GT byte as the reference's read_gt (lib.rs:140-159): colour byte c
// and alpha, both * 1/255.
__device__ __forceinline__ void gt_bytes(uint32_t v, uint32_t c, float& gc, float& ga) {
    gc = (float)((v >> (c * 8u)) & 0xFFu) * kInv255;
    ga = (float)((v >> 24u) & 0xFFu) * kInv255;
}

__device__ __forceinline__ float gt_effective(const LossParams& p, uint32_t v, uint32_t c, float& ga) {
    float gc;
    gt_bytes(v, c, gc, ga);
    return p.composite ? gc + (1.0f - ga) * p.bg[c] : gc;
}

// SSIM value and its partials from the five blurred moments (lib.rs:192-209,
// 502-520): returns the clamped SSIM; dmu1, dsigma1, dsigma12 zero when the
// raw value was clamped.
__device__ __forceinline__ float ssim_from_moments(float o0, float o1, float o2, float o3, float o4, float& dmu1,
                                                   float& dsigma1, float& dsigma12) {
    const float mu1 = o0, mu2 = o2;
    const float mu1_sq = mu1 * mu1, mu2_sq = mu2 * mu2;
    const float sigma1_sq = fmaxf(0.0f, o1 - mu1_sq);
    const float sigma2_sq = fmaxf(0.0f, o3 - mu2_sq);
    const float sigma12 = o4 - mu1 * mu2;
    const float a = mu1_sq + mu2_sq + kC1;
    const float b = sigma1_sq + sigma2_sq + kC2;
    const float c_top = 2.0f * mu1 * mu2 + kC1;
    const float d_top = 2.0f * sigma12 + kC2;
    const float inv_ab = 1.0f / (a * b);
    const float cd = c_top * d_top * inv_ab;
    const bool clamped = cd < -1.0f || cd > 1.0f;
    dmu1 = clamped ? 0.0f : 2.0f * mu2 * inv_ab * (d_top - c_top) - 2.0f * mu1 * cd * (1.0f / a - 1.0f / b);
    dsigma1 = clamped ? 0.0f : -cd / b;
    dsigma12 = clamped ? 0.0f : 2.0f * c_top * inv_ab;
    const float raw = (c_top * d_top) / (a * b);
    return fminf(fmaxf(raw, -1.0f), 1.0f);
}

__device__ __forceinline__ float l1_sign(float diff) { return diff > 0.0f ? 1.0f : (diff < 0.0f ? -1.0f : 0.0f); }

// ---- forward ----------------------------------------------------------------------

template <bool SSIM>
__global__ __launch_bounds__(256) void image_loss_forward_kernel(LossParams p, const float* __restrict__ pred,
                                                                  const uint32_t* __restrict__ gt,
                                                                  float* __restrict__ map) {
    __shared__ float s_tile[kShared * kShared * 2];       // (pred, gt_eff) with halo
    __shared__ float s_hconv[kShared * kLTile * 5];       // five horizontal sums
    const uint32_t c = blockIdx.z;
    const uint32_t tx = threadIdx.x & 15u, ty = threadIdx.x >> 4;
    const uint32_t x0 = blockIdx.x * kLTile, y0 = blockIdx.y * kLTile;
    const uint32_t px = x0 + tx, py = y0 + ty;
    const bool inside = px < p.w && py < p.h;
    if (c == 3u || !SSIM) {
        // alpha match (c == 3) and the L1-only specialisation: per pixel
        if (!inside) return;
        const size_t pix = (size_t)py * p.w + px;
        float ga;
        const float g = c == 3u ? (gt_bytes(gt[pix], 0u, ga, ga), ga) : gt_effective(p, gt[pix], c, ga);
        const float weight = c == 3u ? 1.0f : p.l1_w;
        float v = weight * fabsf(pred[pix * p.stride + c] - g);
        if (p.mask) v = v * ga;
        map[pix * p.channels + c] = v;
        return;
    }
    for (uint32_t i = threadIdx.x; i < (uint32_t)(kShared * kShared); i += 256u) {
        const uint32_t ly = i / kShared, lx = i % kShared;
        const int gy = (int)(y0 + ly) - kHalo, gx = (int)(x0 + lx) - kHalo;
        float pv = 0.0f, gv = 0.0f;
        if (gy >= 0 && gx >= 0 && gy < (int)p.h && gx < (int)p.w) {
            const size_t pix = (size_t)gy * p.w + gx;
            float ga;
            pv = pred[pix * p.stride + c];
            gv = gt_effective(p, gt[pix], c, ga);
        }
        s_tile[2 * i] = pv;
        s_tile[2 * i + 1] = gv;
    }
    __syncthreads();
    // horizontal 11-tap blur of (x, x^2, y, y^2, xy) for the 26 rows x 16 columns
    for (uint32_t i = threadIdx.x; i < (uint32_t)(kShared * kLTile); i += 256u) {
        const uint32_t ly = i / kLTile, lx = i % kLTile + kHalo;
        float sx = 0.0f, sx2 = 0.0f, sy = 0.0f, sy2 = 0.0f, sxy = 0.0f;
#pragma unroll
        for (int d = 1; d <= kHalo; d++) {
            const float wd = p.taps[kHalo - d];
            const uint32_t il = ly * kShared + lx - d, ir = ly * kShared + lx + d;
            const float xl = s_tile[2 * il], yl = s_tile[2 * il + 1], xr = s_tile[2 * ir], yr = s_tile[2 * ir + 1];
            sx += (xl + xr) * wd;
            sx2 += (xl * xl + xr * xr) * wd;
            sy += (yl + yr) * wd;
            sy2 += (yl * yl + yr * yr) * wd;
            sxy += (xl * yl + xr * yr) * wd;
        }
        const uint32_t ic = ly * kShared + lx;
        const float xc = s_tile[2 * ic], yc = s_tile[2 * ic + 1], wc = p.taps[kHalo];
        sx += xc * wc;
        sx2 += xc * xc * wc;
        sy += yc * wc;
        sy2 += yc * yc * wc;
        sxy += xc * yc * wc;
        float* o = s_hconv + (ly * kLTile + (lx - kHalo)) * 5;
        o[0] = sx;
        o[1] = sx2;
        o[2] = sy;
        o[3] = sy2;
        o[4] = sxy;
    }
    __syncthreads();
    if (!inside) return;
    float out[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t ly = ty + kHalo;
#pragma unroll
    for (int d = 1; d <= kHalo; d++) {
        const float wd = p.taps[kHalo - d];
        const float* t = s_hconv + ((ly - d) * kLTile + tx) * 5;
        const float* b = s_hconv + ((ly + d) * kLTile + tx) * 5;
#pragma unroll
        for (int k = 0; k < 5; k++) out[k] += (t[k] + b[k]) * wd;
    }
    {
        const float* m = s_hconv + (ly * kLTile + tx) * 5;
#pragma unroll
        for (int k = 0; k < 5; k++) out[k] += m[k] * p.taps[kHalo];
    }
    float dm, ds, dsc;
    const float ssim = ssim_from_moments(out[0], out[1], out[2], out[3], out[4], dm, ds, dsc);
    const uint32_t ic = (ty + kHalo) * kShared + (tx + kHalo);
    const float l1 = fabsf(s_tile[2 * ic] - s_tile[2 * ic + 1]);
    float v = p.l1_w * l1 + p.ssim_w * ssim;
    const size_t pix = (size_t)py * p.w + px;
    if (p.mask) {
        float gc, ga;
        gt_bytes(gt[pix], c, gc, ga);
        v = v * ga;
    }
    map[pix * p.channels + c] = v;
}

// ---- backward ------------------------------------------------------------------------

// dl_dpred has the layout of pred ([H, W, stride]); this kernel writes channel
// c of it, and the zero channels are written by the launcher's fill.
template <bool SSIM>
__global__ __launch_bounds__(256) void image_loss_backward_kernel(LossParams p, const float* __restrict__ pred,
                                                                   const uint32_t* __restrict__ gt,
                                                                   const float* __restrict__ dl_dmap,
                                                                   float* __restrict__ dl_dpred) {
    // buf_a: the (pred, gt_eff) tile with a 10-pixel halo, later the chained
    // partials on the 26x26 ring; buf_b: first-blur sums, later the second
    // horizontal blur (lib.rs:612-626 reuses its scratch the same way)
    __shared__ float buf_a[kExtended * kExtended * 2];
    __shared__ float buf_b[kExtended * kShared * 5];
    const uint32_t c = blockIdx.z;
    const uint32_t tx = threadIdx.x & 15u, ty = threadIdx.x >> 4;
    const uint32_t x0 = blockIdx.x * kLTile, y0 = blockIdx.y * kLTile;
    const uint32_t px = x0 + tx, py = y0 + ty;
    const bool inside = px < p.w && py < p.h;
    if (c == 3u || !SSIM) {
        if (!inside) return;
        const size_t pix = (size_t)py * p.w + px;
        float ga;
        const float g = c == 3u ? (gt_bytes(gt[pix], 0u, ga, ga), ga) : gt_effective(p, gt[pix], c, ga);
        const float weight = c == 3u ? 1.0f : p.l1_w;
        float chain = dl_dmap[pix * p.channels + c];
        if (p.mask) chain = chain * ga;
        dl_dpred[pix * p.stride + c] = weight * l1_sign(pred[pix * p.stride + c] - g) * chain;
        return;
    }
    for (uint32_t i = threadIdx.x; i < (uint32_t)(kExtended * kExtended); i += 256u) {
        const uint32_t ly = i / kExtended, lx = i % kExtended;
        const int gy = (int)(y0 + ly) - 2 * kHalo, gx = (int)(x0 + lx) - 2 * kHalo;
        float pv = 0.0f, gv = 0.0f;
        if (gy >= 0 && gx >= 0 && gy < (int)p.h && gx < (int)p.w) {
            const size_t pix = (size_t)gy * p.w + gx;
            float ga;
            pv = pred[pix * p.stride + c];
            gv = gt_effective(p, gt[pix], c, ga);
        }
        buf_a[2 * i] = pv;
        buf_a[2 * i + 1] = gv;
    }
    __syncthreads();
    // first horizontal blur over the 36 rows x 26 columns of the ring
    for (uint32_t i = threadIdx.x; i < (uint32_t)(kExtended * kShared); i += 256u) {
        const uint32_t row = i / kShared, col = i % kShared, centre = col + kHalo;
        float sx = 0.0f, sx2 = 0.0f, sy = 0.0f, sy2 = 0.0f, sxy = 0.0f;
#pragma unroll
        for (int d = 1; d <= kHalo; d++) {
            const float wd = p.taps[kHalo - d];
            const uint32_t il = row * kExtended + centre - d, ir = row * kExtended + centre + d;
            const float xl = buf_a[2 * il], yl = buf_a[2 * il + 1], xr = buf_a[2 * ir], yr = buf_a[2 * ir + 1];
            sx += (xl + xr) * wd;
            sx2 += (xl * xl + xr * xr) * wd;
            sy += (yl + yr) * wd;
            sy2 += (yl * yl + yr * yr) * wd;
            sxy += (xl * yl + xr * yr) * wd;
        }
        const uint32_t ic = row * kExtended + centre;
        const float xc = buf_a[2 * ic], yc = buf_a[2 * ic + 1], wc = p.taps[kHalo];
        sx += xc * wc;
        sx2 += xc * xc * wc;
        sy += yc * wc;
        sy2 += yc * yc * wc;
        sxy += xc * yc * wc;
        float* o = buf_b + (row * kShared + col) * 5;
        o[0] = sx;
        o[1] = sx2;
        o[2] = sy;
        o[3] = sy2;
        o[4] = sxy;
    }
    __syncthreads();
    // vertical blur on the 26x26 ring, SSIM partials times the chain (zero
    // outside the image)
    for (uint32_t i = threadIdx.x; i < (uint32_t)(kShared * kShared); i += 256u) {
        const uint32_t py2 = i / kShared, px2 = i % kShared, centre = py2 + kHalo;
        float out[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int d = 1; d <= kHalo; d++) {
            const float wd = p.taps[kHalo - d];
            const float* t = buf_b + ((centre - d) * kShared + px2) * 5;
            const float* b = buf_b + ((centre + d) * kShared + px2) * 5;
#pragma unroll
            for (int k = 0; k < 5; k++) out[k] += (t[k] + b[k]) * wd;
        }
        {
            const float* m = buf_b + (centre * kShared + px2) * 5;
#pragma unroll
            for (int k = 0; k < 5; k++) out[k] += m[k] * p.taps[kHalo];
        }
        float dm, ds, dsc;
        (void)ssim_from_moments(out[0], out[1], out[2], out[3], out[4], dm, ds, dsc);
        const int gy = (int)(y0 + py2) - kHalo, gx = (int)(x0 + px2) - kHalo;
        float chain = 0.0f;
        if (gy >= 0 && gx >= 0 && gy < (int)p.h && gx < (int)p.w) {
            const size_t pix = (size_t)gy * p.w + gx;
            chain = dl_dmap[pix * p.channels + c];
            if (p.mask) {
                float gc, ga;
                gt_bytes(gt[pix], c, gc, ga);
                chain = chain * ga;
            }
        }
        // buf_a's image tile is dead once buf_b holds the first blur
        float* o = buf_a + i * 3;
        o[0] = dm * chain;
        o[1] = ds * chain;
        o[2] = dsc * chain;
    }
    __syncthreads();
    // second horizontal blur: 26 rows x 16 columns into buf_b
    for (uint32_t i = threadIdx.x; i < (uint32_t)(kShared * kLTile); i += 256u) {
        const uint32_t row = i / kLTile, col = i % kLTile, centre = col + kHalo;
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f;
#pragma unroll
        for (int d = 1; d <= kHalo; d++) {
            const float wd = p.taps[kHalo - d];
            const float* l = buf_a + (row * kShared + centre - d) * 3;
            const float* r = buf_a + (row * kShared + centre + d) * 3;
            a0 += (l[0] + r[0]) * wd;
            a1 += (l[1] + r[1]) * wd;
            a2 += (l[2] + r[2]) * wd;
        }
        const float* m = buf_a + (row * kShared + centre) * 3;
        const float wc = p.taps[kHalo];
        a0 += m[0] * wc;
        a1 += m[1] * wc;
        a2 += m[2] * wc;
        float* o = buf_b + (row * kLTile + col) * 3;
        o[0] = a0;
        o[1] = a1;
        o[2] = a2;
    }
    __syncthreads();
    if (!inside) return;
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f;
    const uint32_t ly = ty + kHalo;
#pragma unroll
    for (int d = 1; d <= kHalo; d++) {
        const float wd = p.taps[kHalo - d];
        const float* t = buf_b + ((ly - d) * kLTile + tx) * 3;
        const float* b = buf_b + ((ly + d) * kLTile + tx) * 3;
        s0 += (t[0] + b[0]) * wd;
        s1 += (t[1] + b[1]) * wd;
        s2 += (t[2] + b[2]) * wd;
    }
    {
        const float* m = buf_b + (ly * kLTile + tx) * 3;
        const float wc = p.taps[kHalo];
        s0 += m[0] * wc;
        s1 += m[1] * wc;
        s2 += m[2] * wc;
    }
    const size_t pix = (size_t)py * p.w + px;
    const float p1 = pred[pix * p.stride + c];
    float ga;
    const float g = gt_effective(p, gt[pix], c, ga);
    const float ssim_grad = s0 + (2.0f * p1) * s1 + g * s2;
    float chain = dl_dmap[pix * p.channels + c];
    if (p.mask) chain = chain * ga;
    dl_dpred[pix * p.stride + c] = p.ssim_w * ssim_grad + p.l1_w * l1_sign(p1 - g) * chain;
}

// 11-tap Gaussian at sigma 1.5 normalised to sum 1, in f32 with the same
// operations as the reference's gauss_taps (lib.rs:86-100).
static void gauss_taps(float* taps6) {
    const float sigma = 1.5f;
    float w[11];
    float sum = 0.0f;
    for (int i = 0; i < 11; i++) {
        const float x = (float)i - 5.0f;
        w[i] = expf(-x * x / (2.0f * sigma * sigma));
        sum += w[i];
    }
    for (int i = 0; i < 11; i++) w[i] /= sum;
    for (int i = 0; i < 6; i++) taps6[i] = w[i];  // taps[5 - d] = weight at distance d
}

static LossParams loss_params(const bh_image_loss_config& cfg, uint32_t w, uint32_t h, uint32_t stride,
                              uint32_t channels) {
    LossParams p;
    p.w = w;
    p.h = h;
    p.stride = stride;
    p.channels = channels;
    p.l1_w = cfg.l1_weight;
    p.ssim_w = cfg.ssim_weight;
    p.composite = cfg.composite ? 1u : 0u;
    p.mask = cfg.mask ? 1u : 0u;
    for (int i = 0; i < 3; i++) p.bg[i] = cfg.composite ? cfg.background[i] : 0.0f;
    gauss_taps(p.taps);
    return p;
}

void launch_image_loss_forward(bh_ctx* ctx, const float* pred, uint32_t stride, uint32_t channels,
                               const uint32_t* gt, uint32_t w, uint32_t h, const bh_image_loss_config& cfg,
                               float* map) {
    const LossParams p = loss_params(cfg, w, h, stride, channels);
    const dim3 grid(div_up(w, kLTile), div_up(h, kLTile), channels);
    KernelTimer t(ctx, "image_loss_forward");
    if (cfg.ssim_weight != 0.0f)
        launch(ctx, image_loss_forward_kernel<true>, grid, dim3(256), 0u, p, pred, gt, map);
    else
        launch(ctx, image_loss_forward_kernel<false>, grid, dim3(256), 0u, p, pred, gt, map);
}

void launch_image_loss_backward(bh_ctx* ctx, const float* pred, uint32_t stride, uint32_t channels,
                                const uint32_t* gt, uint32_t w, uint32_t h, const bh_image_loss_config& cfg,
                                const float* dl_dmap, float* dl_dpred) {
    const LossParams p = loss_params(cfg, w, h, stride, channels);
    if (stride > channels) launch_fill_u32(ctx, (uint32_t*)dl_dpred, 0u, (uint64_t)w * h * stride);
    const dim3 grid(div_up(w, kLTile), div_up(h, kLTile), channels);
    KernelTimer t(ctx, "image_loss_backward");
    if (cfg.ssim_weight != 0.0f)
        launch(ctx, image_loss_backward_kernel<true>, grid, dim3(256), 0u, p, pred, gt, dl_dmap, dl_dpred);
    else
        launch(ctx, image_loss_backward_kernel<false>, grid, dim3(256), 0u, p, pred, gt, dl_dmap, dl_dpred);
}

}  // namespace bh
