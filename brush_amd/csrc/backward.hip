// backward.hip — rasterize backward and project backward for gfx950.
//
// rasterize_backward: one wave64 workgroup per 16x16 tile.  Lane j owns splat j
// of a 64-splat batch and walks the tile's 256 pixels in row-major order; at
// step i lane j handles pixel i - j, so pixel p is visited front to back by
// the batch's splats on consecutive steps and its transmittance / remaining
// colour state in LDS is always up to date (the diagonal replay of
// crates/brush-render-bwd/src/kernels/rasterize_backwards.rs:79-443, re-laid
// out for 64-wide waves: the reference batches 32 splats to match a 32-lane
// SIMD group).  The per-pixel upstream terms (dL/drgb, the alpha term
// (v_a - bg . v_rgb) T_final, final alpha) are computed once per pixel into
// LDS instead of per (splat, pixel) pair.  Each lane accumulates its splat's
// gradient for the whole tile in registers and adds it to v_combined with one
// hardware float atomic per lane per batch.
//
// project_backward: one thread per *global* id, so every dense output row is
// written exactly once (zeros for culled splats or splats without gradient)
// and no separate zero fill of the ~240 MB SH3 gradient is needed
// (crates/brush-render-bwd/src/kernels/project_backwards.rs:101-263 and
// render_bwd.rs:338-350 restated).
#include <hip/hip_runtime.h>

#include "bh_internal.h"
#include "bh_splat_math.h"

namespace bh {

template <bool SMOOTH, bool REFINE, bool DEPTH>
__global__ __launch_bounds__(64) void rasterize_backward_kernel(
    uint32_t img_w, uint32_t img_h, uint32_t tile_bw, float bg_r, float bg_g, float bg_b, uint32_t num_visible,
    const float* __restrict__ out_img, const float* __restrict__ projected, const uint32_t* __restrict__ cgids,
    const uint32_t* __restrict__ offsets, const float* __restrict__ v_output, float* __restrict__ v_combined) {
    constexpr uint32_t CH = DEPTH ? 5u : 4u;
    __shared__ float4 s_state[256];  // remaining r, g, b; transmittance
    __shared__ float4 s_vout[256];   // dL/dr, dL/dg, dL/db, (v_a - bg . v_rgb) * T_final
    __shared__ float s_final_a[256];
    __shared__ float s_state_d[DEPTH ? 256 : 1];
    __shared__ float s_vod[DEPTH ? 256 : 1];

    const uint32_t tile = blockIdx.x;
    const uint32_t ox = (tile % tile_bw) * 16u, oy = (tile / tile_bw) * 16u;
    const uint32_t lane = threadIdx.x;
    for (uint32_t p = lane; p < 256u; p += 64u) {
        const uint32_t px = ox + (p & 15u), py = oy + (p >> 4);
        if (px < img_w && py < img_h) {
            const size_t pix = (size_t)py * img_w + px;
            const float* o = out_img + pix * CH;
            const float* vo = v_output + pix * CH;
            const float final_a = o[3];
            const float t_final = 1.0f - final_a;
            s_state[p] = make_float4(o[0] - t_final * bg_r, o[1] - t_final * bg_g, o[2] - t_final * bg_b, 1.0f);
            const float vox = vo[0], voy = vo[1], voz = vo[2], va = vo[3];
            const float vow = (va - (bg_r * vox + bg_g * voy + bg_b * voz)) * t_final;
            s_vout[p] = make_float4(vox, voy, voz, vow);
            s_final_a[p] = final_a;
            if (DEPTH) {
                s_state_d[p] = o[4];
                s_vod[p] = vo[4];
            }
        } else {
            s_state[p] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            s_vout[p] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            s_final_a[p] = 0.0f;
            if (DEPTH) {
                s_state_d[p] = 0.0f;
                s_vod[p] = 0.0f;
            }
        }
    }
    const uint32_t lo = offsets[2 * tile], hi = offsets[2 * tile + 1];
    const float img_wf = (float)img_w, img_hf = (float)img_h;
    __syncthreads();

    for (uint32_t b = lo; b < hi; b += 64u) {
        const uint32_t idx = b + lane;
        const bool active = idx < hi;
        uint32_t c = 0;
        float s[10];
#pragma unroll
        for (int k = 0; k < 10; k++) s[k] = 0.0f;
        if (active) {
            c = min(cgids[idx], num_visible - 1u);
            const float2* row = reinterpret_cast<const float2*>(projected + (size_t)c * 10);
#pragma unroll
            for (int k = 0; k < 5; k++) {
                float2 q = row[k];
                s[2 * k] = q.x;
                s[2 * k + 1] = q.y;
            }
        }
        const S2 conic{s[2], s[3], s[4]};
        const float opac = s[5];
        const float cr = bh_maxf(s[6], 0.0f), cgc = bh_maxf(s[7], 0.0f), cb = bh_maxf(s[8], 0.0f);
        float g[11];
#pragma unroll
        for (int k = 0; k < 11; k++) g[k] = 0.0f;
        const uint32_t cnt = min(64u, hi - b);
        const uint32_t iters = cnt + 255u;
        for (uint32_t i = 0; i < iters; i++) {
            const int p = (int)i - (int)lane;
            if (active && p >= 0 && p < 256) {
                const float4 st = s_state[p];
                if (st.w > 1.0e-4f) {
                    const uint32_t px = ox + ((uint32_t)p & 15u), py = oy + ((uint32_t)p >> 4);
                    const float pcx = (float)px + 0.5f, pcy = (float)py + 0.5f;
                    const float dx = s[0] - pcx, dy = s[1] - pcy;
                    const float sigma = 0.5f * (conic.c00 * dx * dx + conic.c11 * dy * dy) + conic.c01 * dx * dy;
                    const float gaussian = bh_expf(-sigma);
                    const float alpha = bh_minf(0.999f, opac * gaussian);
                    const float w = SMOOTH ? cutoff_weight(alpha) : (alpha >= kCutMid ? 1.0f : 0.0f);
                    if (sigma >= 0.0f && w > 0.0f) {
                        const float ae = alpha * w;
                        const float next_t = st.w * (1.0f - ae);
                        if (next_t <= 1.0e-4f) {
                            s_state[p].w = 0.0f;
                        } else {
                            const float vis = ae * st.w;
                            const float4 vo = s_vout[p];
                            g[5] += s[6] >= 0.0f ? vis * vo.x : 0.0f;
                            g[6] += s[7] >= 0.0f ? vis * vo.y : 0.0f;
                            g[7] += s[8] >= 0.0f ? vis * vo.z : 0.0f;
                            const float ra = 1.0f / (1.0f - ae);
                            const float dot_rgb =
                                ((st.w * cr - st.x) * vo.x + (st.w * cgc - st.y) * vo.y + (st.w * cb - st.z) * vo.z) * ra;
                            const float nrx = st.x - vis * cr, nry = st.y - vis * cgc, nrz = st.z - vis * cb;
                            if (DEPTH) {
                                g[10] += vis * s_vod[p];
                                s_state_d[p] = s_state_d[p] - vis * s[9];
                            }
                            const float v_ae = dot_rgb + vo.w * ra;
                            const float dw = SMOOTH ? cutoff_weight_deriv(alpha) : 0.0f * alpha;
                            const float v_alpha = v_ae * (w + alpha * dw);
                            const float v_sigma = -alpha * v_alpha;
                            const float vxy_x = v_sigma * (conic.c00 * dx + conic.c01 * dy);
                            const float vxy_y = v_sigma * (conic.c01 * dx + conic.c11 * dy);
                            if (opac * gaussian <= 0.999f) {
                                g[2] += 0.5f * v_sigma * dx * dx;
                                g[3] += v_sigma * dx * dy;
                                g[4] += 0.5f * v_sigma * dy * dy;
                                g[0] += vxy_x;
                                g[1] += vxy_y;
                                g[8] += v_alpha * gaussian;
                                if (REFINE) {
                                    const float len = sqrtf(vxy_x * img_wf * vxy_x * img_wf + vxy_y * img_hf * vxy_y * img_hf);
                                    g[9] += len / bh_maxf(s_final_a[p], 1.0e-5f);
                                }
                            }
                            s_state[p] = make_float4(nrx, nry, nrz, next_t);
                        }
                    }
                }
            }
            __syncthreads();
        }
        if (active) {
            float* out = v_combined + (size_t)c * 11;
#pragma unroll
            for (int k = 0; k < 9; k++) unsafeAtomicAdd(out + k, g[k]);
            if (REFINE) unsafeAtomicAdd(out + 9, g[9]);
            if (DEPTH) unsafeAtomicAdd(out + 10, g[10]);
        }
    }
}

void launch_rasterize_backward(bh_ctx* ctx, uint32_t img_w, uint32_t img_h, uint32_t tile_bw, uint32_t tile_bh,
                               const float* bg, uint32_t num_visible, const float* out_img, const float* projected, const uint32_t* cgids,
                               const uint32_t* offsets, const float* v_output, uint32_t flags, float* v_combined) {
    const uint32_t num_tiles = tile_bw * tile_bh;
    if (num_tiles == 0 || num_visible == 0) return;
    const bool smooth = (flags & BH_FLAG_SMOOTH_CUTOFF) != 0;
    const bool refine = (flags & BH_FLAG_REFINE_WEIGHT) != 0;
    const bool depth = (flags & BH_FLAG_RENDER_DEPTH) != 0;
    KernelTimer t(ctx, "rasterize_backward");
#define BH_RB(S, R, D)                                                                                          \
    rasterize_backward_kernel<S, R, D><<<num_tiles, 64, 0, ctx->stream>>>(img_w, img_h, tile_bw, bg[0], bg[1], \
                                                                          bg[2], num_visible, out_img,          \
                                                                          projected, cgids, offsets, v_output,  \
                                                                          v_combined)
    if (smooth) {
        if (refine) {
            if (depth) BH_RB(true, true, true); else BH_RB(true, true, false);
        } else {
            if (depth) BH_RB(true, false, true); else BH_RB(true, false, false);
        }
    } else {
        if (refine) {
            if (depth) BH_RB(false, true, true); else BH_RB(false, true, false);
        } else {
            if (depth) BH_RB(false, false, true); else BH_RB(false, false, false);
        }
    }
#undef BH_RB
}

// ---- project backward ---------------------------------------------------------------

__global__ __launch_bounds__(256) void invert_permutation_kernel(const uint32_t* __restrict__ gfc,
                                                                  uint32_t num_visible, uint32_t n,
                                                                  uint32_t* __restrict__ cfg) {
    const uint32_t c = blockIdx.x * 256u + threadIdx.x;
    if (c < num_visible) {
        const uint32_t g = gfc[c];
        if (g < n) cfg[g] = c;
    }
}

void launch_invert_permutation(bh_ctx* ctx, const uint32_t* gfc, uint32_t num_visible, uint32_t n,
                               uint32_t* compact_from_global) {
    launch_fill_u32(ctx, compact_from_global, 0xFFFFFFFFu, n);
    if (num_visible == 0) return;
    KernelTimer t(ctx, "invert_permutation");
    invert_permutation_kernel<<<div_up(num_visible, 256), 256, 0, ctx->stream>>>(gfc, num_visible, n,
                                                                                    compact_from_global);
}

template <int NC>
__device__ __forceinline__ void store_row(float* __restrict__ dst, const float* v) {
    if ((3 * NC) % 4 == 0) {
        float4* d4 = reinterpret_cast<float4*>(dst);
#pragma unroll
        for (int i = 0; i < (3 * NC) / 4; i++) d4[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    } else {
#pragma unroll
        for (int i = 0; i < 3 * NC; i++) dst[i] = v[i];
    }
}

template <int DEG, bool MIP>
__global__ __launch_bounds__(256) void project_backward_kernel(
    bh_project_uniforms u, const float* __restrict__ transforms, const float* __restrict__ sh,
    const float* __restrict__ raw_opac, const uint32_t* __restrict__ cfg, uint32_t n,
    const float* __restrict__ v_combined, float* __restrict__ v_transforms, float* __restrict__ v_coeffs,
    float* __restrict__ v_raw_opac, float* __restrict__ v_refine) {
    constexpr int NC = (DEG + 1) * (DEG + 1);
    const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
    if (gid >= n) return;
    const uint32_t c = cfg[gid];
    float rg[11];
#pragma unroll
    for (int k = 0; k < 11; k++) rg[k] = 0.0f;
    bool any = false;
    if (c != 0xFFFFFFFFu) {
        const float* src = v_combined + (size_t)c * 11;
#pragma unroll
        for (int k = 0; k < 11; k++) {
            rg[k] = src[k];
            any = any || rg[k] != 0.0f;
        }
    }
    float2* vt = reinterpret_cast<float2*>(v_transforms + (size_t)gid * 10);
    float* vc_row = v_coeffs + (size_t)gid * (3 * NC);
    float vcoef[3 * NC];
    if (!any) {
#pragma unroll
        for (int k = 0; k < 5; k++) vt[k] = make_float2(0.0f, 0.0f);
#pragma unroll
        for (int k = 0; k < 3 * NC; k++) vcoef[k] = 0.0f;
        store_row<NC>(vc_row, vcoef);
        v_raw_opac[gid] = 0.0f;
        v_refine[gid] = 0.0f;
        return;
    }
    const float2* row = reinterpret_cast<const float2*>(transforms + (size_t)gid * 10);
    float t[10];
#pragma unroll
    for (int i = 0; i < 5; i++) {
        float2 p = row[i];
        t[2 * i] = p.x;
        t[2 * i + 1] = p.y;
    }
    const V3 mean = v3(t[0], t[1], t[2]);
    const V3 sc = v3(bh_expf(t[7]), bh_expf(t[8]), bh_expf(t[9]));
    const Q4 qu{t[3], t[4], t[5], t[6]};
    const Q4 q = qnormalize(qu);
    const V3 uw = mean - v3(u.camera_pos[0], u.camera_pos[1], u.camera_pos[2]);
    const float ulen = sqrtf(dot(uw, uw));
    const V3 v = uw * (1.0f / ulen);
    const V3 vcol = v3(rg[5], rg[6], rg[7]);
    {
        float basis[NC];
        sh_basis<DEG>(v, basis);
#pragma unroll
        for (int k = 0; k < NC; k++) {
            vcoef[3 * k] = vcol.x * basis[k];
            vcoef[3 * k + 1] = vcol.y * basis[k];
            vcoef[3 * k + 2] = vcol.z * basis[k];
        }
        store_row<NC>(vc_row, vcoef);
    }
    V3 v_mean_sh;
    {
        float coeffs[3 * NC];
        const float* srow = sh + (size_t)gid * (3 * NC);
        if ((3 * NC) % 4 == 0) {
            const float4* s4 = reinterpret_cast<const float4*>(srow);
#pragma unroll
            for (int i = 0; i < (3 * NC) / 4; i++) {
                float4 qq = s4[i];
                coeffs[4 * i] = qq.x;
                coeffs[4 * i + 1] = qq.y;
                coeffs[4 * i + 2] = qq.z;
                coeffs[4 * i + 3] = qq.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 3 * NC; i++) coeffs[i] = srow[i];
        }
        const V3 vv = sh_viewdir_vjp<DEG>(coeffs, v, vcol);
        const float vdot = dot(v, vv);
        v_mean_sh = (vv - v * vdot) * (1.0f / ulen);
    }
    const V3 mean_c = world_to_cam(u, mean);
    const M3 r = qmat(q);
    const M3 m = mul_diag(r, sc);
    const S2 raw_cov = calc_cov2d(u, sc, q, mean_c);
    float comp;
    const S2 cov = compensate_cov2d<MIP>(raw_cov, comp);
    const float sig = bh_sigmoidf(raw_opac[gid]);
    v_raw_opac[gid] = comp * rg[8] * sig * (1.0f - sig);
    const float rc = bh_is_finite(rg[9]) ? rg[9] : 0.0f;
    v_refine[gid] = bh_clampf(rc, 0.0f, 1.0e32f);
    const S2 conic_inv = inverse(cov);
    const S2 v_inv{rg[2], rg[3] * 0.5f, rg[4]};
    const S2 v_cov2d = inverse2x2_vjp(conic_inv, v_inv);
    const S3 covar = outer_self(m);
    const M3 vr = view_rot(u);
    const S3 cov_c = cong(covar, vr);
    const M23 J = jacobian(u, mean_c);
    V3 v_mean_c = projection_vjp(u, J, mean_c, cov_c, v_cov2d, v2(rg[0], rg[1]));
    v_mean_c = v3(v_mean_c.x, v_mean_c.y, v_mean_c.z + rg[10]);
    const S3 vcc = tcong(J, v_cov2d);
    const V3 v_mean = tmulv(vr, v_mean_c) + v_mean_sh;
    const M3 v_m = mul(scale(tcong(vcc, vr), 2.0f), m);
    const V3 v_scale =
        v3(dot(col0(r), col0(v_m)) * sc.x, dot(col1(r), col1(v_m)) * sc.y, dot(col2(r), col2(v_m)) * sc.z);
    const Q4 qg = quat_to_mat_vjp(q, mul_diag(v_m, sc));
    const Q4 vq = normalize_vjp(qu, qg);
    vt[0] = make_float2(v_mean.x, v_mean.y);
    vt[1] = make_float2(v_mean.z, vq.w);
    vt[2] = make_float2(vq.x, vq.y);
    vt[3] = make_float2(vq.z, v_scale.x);
    vt[4] = make_float2(v_scale.y, v_scale.z);
}

template <int DEG>
static void launch_pb(bh_ctx* ctx, bool mip, const bh_project_uniforms& u, const float* transforms, const float* sh,
                      const float* raw_opac, const uint32_t* cfg, uint32_t n, const float* v_combined,
                      float* v_transforms, float* v_coeffs, float* v_raw_opac, float* v_refine) {
    uint32_t blocks = div_up(n, 256);
    if (mip)
        project_backward_kernel<DEG, true><<<blocks, 256, 0, ctx->stream>>>(
            u, transforms, sh, raw_opac, cfg, n, v_combined, v_transforms, v_coeffs, v_raw_opac, v_refine);
    else
        project_backward_kernel<DEG, false><<<blocks, 256, 0, ctx->stream>>>(
            u, transforms, sh, raw_opac, cfg, n, v_combined, v_transforms, v_coeffs, v_raw_opac, v_refine);
}

void launch_project_backward(bh_ctx* ctx, const bh_project_uniforms& u, const float* transforms, const float* sh,
                             const float* raw_opac, const uint32_t* cfg, uint32_t n, uint32_t sh_degree, bool mip,
                             const float* v_combined, float* v_transforms, float* v_coeffs, float* v_raw_opac,
                             float* v_refine) {
    if (n == 0) return;
    KernelTimer t(ctx, "project_backward");
    switch (sh_degree) {
        case 0: launch_pb<0>(ctx, mip, u, transforms, sh, raw_opac, cfg, n, v_combined, v_transforms, v_coeffs, v_raw_opac, v_refine); break;
        case 1: launch_pb<1>(ctx, mip, u, transforms, sh, raw_opac, cfg, n, v_combined, v_transforms, v_coeffs, v_raw_opac, v_refine); break;
        case 2: launch_pb<2>(ctx, mip, u, transforms, sh, raw_opac, cfg, n, v_combined, v_transforms, v_coeffs, v_raw_opac, v_refine); break;
        case 3: launch_pb<3>(ctx, mip, u, transforms, sh, raw_opac, cfg, n, v_combined, v_transforms, v_coeffs, v_raw_opac, v_refine); break;
        default: launch_pb<4>(ctx, mip, u, transforms, sh, raw_opac, cfg, n, v_combined, v_transforms, v_coeffs, v_raw_opac, v_refine); break;
    }
}

}  // namespace bh
