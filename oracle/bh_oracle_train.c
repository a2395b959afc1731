/*
 * bh_oracle_train.c — CPU restatement of the training-step pieces downstream
 * of the rasterizer: the fused L1 + SSIM image loss (forward map and VJP) and
 * the AdamScaled optimizer step.  TEST INFRASTRUCTURE ONLY: the parity checker
 * for brush_amd/csrc/loss.hip and adam.hip and part of the CPU baseline.
 *
 * The image loss is written per pixel over whole images (separable blur with
 * zero padding), not in tiles; the float operations of every sum are in the
 * order of the reference kernels (crates/brush-loss/src/lib.rs).  All f32,
 * built with -ffp-contract=off.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "bh_oracle.h"

static const float kC1 = 0.01f * 0.01f;   /* lib.rs:112 */
static const float kC2 = 0.03f * 0.03f;   /* lib.rs:113 */
static const float kInv255 = 1.0f / 255.0f;

/* gauss_taps (lib.rs:86-100): 11 weights exp(-x^2 / (2 sigma^2)), sigma 1.5,
 * divided by their f32 sum.  taps6[5 - d] is the weight at distance d. */
void or_gauss_taps(float* taps6) {
    const float sigma = 1.5f;
    float w[11], sum = 0.0f;
    for (int i = 0; i < 11; i++) {
        const float x = (float)i - 5.0f;
        w[i] = expf(-x * x / (2.0f * sigma * sigma));
        sum += w[i];
    }
    for (int i = 0; i < 11; i++) w[i] /= sum;
    for (int i = 0; i < 6; i++) taps6[i] = w[i];
}

/* read_gt (lib.rs:140-159) and the gt_eff compositing (lib.rs:412-418). */
static float gt_eff(uint32_t v, uint32_t c, const bh_image_loss_config* cfg, float* alpha) {
    const float gc = (float)((v >> (c * 8u)) & 0xFFu) * kInv255;
    const float ga = (float)((v >> 24u) & 0xFFu) * kInv255;
    *alpha = ga;
    return cfg->composite ? gc + (1.0f - ga) * cfg->background[c] : gc;
}

static float sign1(float d) { return d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : 0.0f); }

/* 11-tap blur of `nch` interleaved planes along x then y, zero outside the
 * image, in the kernels' order: sum over d = 1..5 of (left + right) * w_d,
 * then + centre * w_c (lib.rs:432-465, 472-497). */
static void blur2d(const float* in, float* out, float* tmp, int w, int h, int nch, const float* taps) {
    for (int y = 0; y < h; y++)
        for (int x = 0; x < w; x++)
            for (int k = 0; k < nch; k++) {
                float s = 0.0f;
                for (int d = 1; d <= 5; d++) {
                    const float l = x - d >= 0 ? in[((size_t)y * w + x - d) * nch + k] : 0.0f;
                    const float r = x + d < w ? in[((size_t)y * w + x + d) * nch + k] : 0.0f;
                    s += (l + r) * taps[5 - d];
                }
                s += in[((size_t)y * w + x) * nch + k] * taps[5];
                tmp[((size_t)y * w + x) * nch + k] = s;
            }
    for (int y = 0; y < h; y++)
        for (int x = 0; x < w; x++)
            for (int k = 0; k < nch; k++) {
                float s = 0.0f;
                for (int d = 1; d <= 5; d++) {
                    const float t = y - d >= 0 ? tmp[((size_t)(y - d) * w + x) * nch + k] : 0.0f;
                    const float b = y + d < h ? tmp[((size_t)(y + d) * w + x) * nch + k] : 0.0f;
                    s += (t + b) * taps[5 - d];
                }
                s += tmp[((size_t)y * w + x) * nch + k] * taps[5];
                out[((size_t)y * w + x) * nch + k] = s;
            }
}

/* The five blurred moments (mu_x, E[x^2], mu_y, E[y^2], E[xy]) of one colour
 * channel.  The horizontal sums of the products are formed from the raw
 * values in the kernels' order ((xl*xl + xr*xr) * w), so the planes are the
 * raw pair and the products are taken inside the blur. */
static void moments(const float* px, const float* py, float* m5, int w, int h, const float* taps) {
    const size_t n = (size_t)w * h;
    float* tmp = (float*)malloc(n * 5 * sizeof(float));
    for (int y = 0; y < h; y++)
        for (int x = 0; x < w; x++) {
            float s[5] = {0, 0, 0, 0, 0};
            for (int d = 1; d <= 5; d++) {
                const int xl = x - d, xr = x + d;
                const float al = xl >= 0 ? px[(size_t)y * w + xl] : 0.0f, bl = xl >= 0 ? py[(size_t)y * w + xl] : 0.0f;
                const float ar = xr < w ? px[(size_t)y * w + xr] : 0.0f, br = xr < w ? py[(size_t)y * w + xr] : 0.0f;
                const float wd = taps[5 - d];
                s[0] += (al + ar) * wd;
                s[1] += (al * al + ar * ar) * wd;
                s[2] += (bl + br) * wd;
                s[3] += (bl * bl + br * br) * wd;
                s[4] += (al * bl + ar * br) * wd;
            }
            const float ac = px[(size_t)y * w + x], bc = py[(size_t)y * w + x], wc = taps[5];
            s[0] += ac * wc;
            s[1] += ac * ac * wc;
            s[2] += bc * wc;
            s[3] += bc * bc * wc;
            s[4] += ac * bc * wc;
            memcpy(tmp + ((size_t)y * w + x) * 5, s, sizeof(s));
        }
    for (int y = 0; y < h; y++)
        for (int x = 0; x < w; x++)
            for (int k = 0; k < 5; k++) {
                float s = 0.0f;
                for (int d = 1; d <= 5; d++) {
                    const float t = y - d >= 0 ? tmp[((size_t)(y - d) * w + x) * 5 + k] : 0.0f;
                    const float b = y + d < h ? tmp[((size_t)(y + d) * w + x) * 5 + k] : 0.0f;
                    s += (t + b) * taps[5 - d];
                }
                s += tmp[((size_t)y * w + x) * 5 + k] * taps[5];
                m5[((size_t)y * w + x) * 5 + k] = s;
            }
    free(tmp);
}

/* SSIM and its partials from the moments (lib.rs:192-209, 502-520). */
static float ssim_of(const float* o, float* dmu1, float* dsig1, float* dsig12) {
    const float mu1 = o[0], mu2 = o[2];
    const float mu1_sq = mu1 * mu1, mu2_sq = mu2 * mu2;
    const float sigma1_sq = fmaxf(0.0f, o[1] - mu1_sq);
    const float sigma2_sq = fmaxf(0.0f, o[3] - mu2_sq);
    const float sigma12 = o[4] - mu1 * mu2;
    const float a = mu1_sq + mu2_sq + kC1;
    const float b = sigma1_sq + sigma2_sq + kC2;
    const float c_top = 2.0f * mu1 * mu2 + kC1;
    const float d_top = 2.0f * sigma12 + kC2;
    const float inv_ab = 1.0f / (a * b);
    const float cd = c_top * d_top * inv_ab;
    const int clamped = cd < -1.0f || cd > 1.0f;
    *dmu1 = clamped ? 0.0f : 2.0f * mu2 * inv_ab * (d_top - c_top) - 2.0f * mu1 * cd * (1.0f / a - 1.0f / b);
    *dsig1 = clamped ? 0.0f : -cd / b;
    *dsig12 = clamped ? 0.0f : 2.0f * c_top * inv_ab;
    const float raw = (c_top * d_top) / (a * b);
    return fminf(fmaxf(raw, -1.0f), 1.0f);
}

/* image_loss forward (lib.rs:228-555): map[H, W, channels]. */
void or_image_loss_forward(const float* pred, uint32_t stride, uint32_t channels, const uint32_t* gt,
                           uint32_t w, uint32_t h, const bh_image_loss_config* cfg, float* map) {
    float taps[6];
    or_gauss_taps(taps);
    const size_t n = (size_t)w * h;
    float* px = (float*)malloc(n * sizeof(float));
    float* py = (float*)malloc(n * sizeof(float));
    float* m5 = (float*)malloc(n * 5 * sizeof(float));
    for (uint32_t c = 0; c < channels; c++) {
        if (c == 3) {
            for (size_t i = 0; i < n; i++) {
                float ga;
                (void)gt_eff(gt[i], 0, cfg, &ga);
                float v = fabsf(pred[i * stride + 3] - ga);
                if (cfg->mask) v = v * ga;
                map[i * channels + 3] = v;
            }
            continue;
        }
        float ga;
        for (size_t i = 0; i < n; i++) {
            px[i] = pred[i * stride + c];
            py[i] = gt_eff(gt[i], c, cfg, &ga);
        }
        if (cfg->ssim_weight != 0.0f) moments(px, py, m5, (int)w, (int)h, taps);
        for (size_t i = 0; i < n; i++) {
            float v;
            if (cfg->ssim_weight != 0.0f) {
                float a, b, d;
                const float ssim = ssim_of(m5 + i * 5, &a, &b, &d);
                v = cfg->l1_weight * fabsf(px[i] - py[i]) + cfg->ssim_weight * ssim;
            } else {
                v = cfg->l1_weight * fabsf(px[i] - py[i]);
            }
            if (cfg->mask) {
                (void)gt_eff(gt[i], c, cfg, &ga);
                v = v * ga;
            }
            map[i * channels + c] = v;
        }
    }
    free(px);
    free(py);
    free(m5);
}

/* image_loss backward (lib.rs:280-893): dl_dpred[H, W, stride], zeros in the
 * channels past `channels`. */
void or_image_loss_backward(const float* pred, uint32_t stride, uint32_t channels, const uint32_t* gt,
                            uint32_t w, uint32_t h, const bh_image_loss_config* cfg, const float* dl_dmap,
                            float* dl_dpred) {
    float taps[6];
    or_gauss_taps(taps);
    const size_t n = (size_t)w * h;
    for (size_t i = 0; i < n * stride; i++) dl_dpred[i] = 0.0f;
    float* px = (float*)malloc(n * sizeof(float));
    float* py = (float*)malloc(n * sizeof(float));
    float* m5 = (float*)malloc(n * 5 * sizeof(float));
    float* part = (float*)malloc(n * 3 * sizeof(float));
    float* blur = (float*)malloc(n * 3 * sizeof(float));
    float* tmp = (float*)malloc(n * 3 * sizeof(float));
    for (uint32_t c = 0; c < channels; c++) {
        float ga;
        if (c == 3) {
            for (size_t i = 0; i < n; i++) {
                (void)gt_eff(gt[i], 0, cfg, &ga);
                float chain = dl_dmap[i * channels + 3];
                if (cfg->mask) chain = chain * ga;
                dl_dpred[i * stride + 3] = sign1(pred[i * stride + 3] - ga) * chain;
            }
            continue;
        }
        for (size_t i = 0; i < n; i++) {
            px[i] = pred[i * stride + c];
            py[i] = gt_eff(gt[i], c, cfg, &ga);
        }
        if (cfg->ssim_weight == 0.0f) {
            for (size_t i = 0; i < n; i++) {
                (void)gt_eff(gt[i], c, cfg, &ga);
                float chain = dl_dmap[i * channels + c];
                if (cfg->mask) chain = chain * ga;
                dl_dpred[i * stride + c] = cfg->l1_weight * sign1(px[i] - py[i]) * chain;
            }
            continue;
        }
        moments(px, py, m5, (int)w, (int)h, taps);
        for (size_t i = 0; i < n; i++) {
            float dm, ds, dsc;
            (void)ssim_of(m5 + i * 5, &dm, &ds, &dsc);
            float chain = dl_dmap[i * channels + c];
            if (cfg->mask) {
                (void)gt_eff(gt[i], c, cfg, &ga);
                chain = chain * ga;
            }
            part[i * 3] = dm * chain;
            part[i * 3 + 1] = ds * chain;
            part[i * 3 + 2] = dsc * chain;
        }
        blur2d(part, blur, tmp, (int)w, (int)h, 3, taps);
        for (size_t i = 0; i < n; i++) {
            (void)gt_eff(gt[i], c, cfg, &ga);
            const float p1 = px[i];
            const float ssim_grad = blur[i * 3] + (2.0f * p1) * blur[i * 3 + 1] + py[i] * blur[i * 3 + 2];
            float chain = dl_dmap[i * channels + c];
            if (cfg->mask) chain = chain * ga;
            dl_dpred[i * stride + c] = cfg->ssim_weight * ssim_grad + cfg->l1_weight * sign1(p1 - py[i]) * chain;
        }
    }
    free(px);
    free(py);
    free(m5);
    free(part);
    free(blur);
    free(tmp);
}

/* AdamScaled::step (crates/brush-train/src/adam_scaled.rs:216-383) on a
 * [rows, row_len] parameter.  `time` counts steps including this one; on the
 * first step the moments are formed from the gradient alone. */
void or_adam_scaled_step(float* param, const float* grad, float* m1, float* m2, const float* scaling, uint32_t rows,
                         uint32_t row_len, uint32_t reduce, float lr, uint32_t time, const bh_adam_config* cfg) {
    const float b1 = cfg->beta_1, b2 = cfg->beta_2;
    const float f1 = 1.0f - b1, f2 = 1.0f - b2;
    float p1 = 1.0f, p2 = 1.0f;
    {  /* b^t by binary exponentiation */
        float base1 = b1, base2 = b2;
        uint32_t t = time;
        for (;;) {
            if (t & 1u) {
                p1 *= base1;
                p2 *= base2;
            }
            t >>= 1;
            if (t == 0) break;
            base1 *= base1;
            base2 *= base2;
        }
    }
    const float bc1 = 1.0f - p1, bc2 = 1.0f - p2;
    const int first = time == 1;
    const int red = reduce && row_len > 1;
    for (uint32_t r = 0; r < rows; r++) {
        float v2row = 0.0f;
        if (red) {
            float sum = 0.0f;
            for (uint32_t k = 0; k < row_len; k++) {
                const float g = grad[(size_t)r * row_len + k];
                sum += g * g;
            }
            const float mean = sum / (float)row_len;
            v2row = first ? mean * f2 : m2[r] * b2 + mean * f2;
            m2[r] = v2row;
        }
        for (uint32_t k = 0; k < row_len; k++) {
            const size_t e = (size_t)r * row_len + k;
            const float g = grad[e];
            float v2;
            if (red) {
                v2 = v2row;
            } else {
                const float g2 = g * g;
                v2 = first ? g2 * f2 : m2[e] * b2 + g2 * f2;
                m2[e] = v2;
            }
            const float v1 = first ? g * f1 : m1[e] * b1 + g * f1;
            m1[e] = v1;
            const float step = (v1 / bc1) / (sqrtf(v2 / bc2) + cfg->epsilon);
            const float delta = scaling ? step * (scaling[k] * lr) : step * lr;
            param[e] = param[e] - delta;
        }
    }
}
