/*
 * bh_oracle.h — CPU restatement of Brush's differentiable tile rasterizer.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the gfx950
 * kernels and the timed CPU baseline of bench.py.  Nothing in the product
 * (brush_amd/, include/) links it or calls it.
 *
 * Every function restates one piece of the reference in plain C11, in the
 * reference's own float operation order (left-to-right as written in the
 * CubeCL source, no contraction), so that integer outputs can be compared bit
 * for bit.  exp/log come from brush_amd/csrc/bh_math.h, which the kernels use
 * too; those two functions are pinned separately against float64 libm.
 *
 * Parity status per function (what pins each one is listed in the .c file
 * above the function):
 *   or_project_forward, or_project_visible, or_map_intersects,
 *   or_stable_sort, or_prefix_sum, or_tile_offsets, or_rasterize,
 *   or_rasterize_reference, or_rasterize_backward, or_project_backward,
 *   or_gauss_taps, or_image_loss_forward, or_image_loss_backward,
 *   or_adam_scaled_step: pinned (see tests/test_oracle.py and
 *   tests/test_oracle_train.py).
 */
#ifndef BH_ORACLE_H
#define BH_ORACLE_H

#include <stdint.h>
#include "../include/brush_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Number of OpenMP threads the parallel loops may use (1 = sequential). */
void or_set_threads(int n);
/* Element-wise bh_expf / bh_logf, for pinning them against libm. */
void or_expf(const float* in, float* out, uint64_t n);
void or_exp2_neg(const float* in, float* out, uint64_t n);
void or_div_by_recip(const float* num, const float* den, float* out, uint64_t n);
void or_power_log2(const float* c00, const float* c01, const float* c11, const float* dx, const float* dy,
                   float* out, uint64_t n);
void or_logf(const float* in, float* out, uint64_t n);
void or_atan2f(const float* y, const float* x, float* out, uint64_t n);
/* camera models on their own (test hooks): projection and depth cull,
 * Jacobian rows (du/dx du/dy du/dz dv/dx dv/dy dv/dz), projection VJP */
void or_camera_project(const bh_project_uniforms* u, const float* pts, uint64_t n, float* out, uint8_t* culled);
void or_camera_jacobian(const bh_project_uniforms* u, const float* pts, uint64_t n, float* out);
void or_camera_vjp(const bh_project_uniforms* u, const float* mean_c, const float* cov_c, const float* v_cov2d,
                   const float* v_mean2d, uint64_t n, float* out);
int or_get_max_threads(void);

/* tile_h: 16, or 8 for 16x8 tiles (BH_FLAG_TILE_16X8); u->tile_bh must match */
uint64_t or_project_forward(const bh_project_uniforms* u, const float* transforms,
                            const float* raw_opac, uint32_t n, uint32_t mip, uint32_t tile_h,
                            uint32_t* intersect_counts, float* max_radius, float* depths,
                            uint8_t* visible_mask);

void or_stable_sort(uint32_t* keys, uint32_t* vals, uint64_t n, uint32_t sorting_bits);

void or_prefix_sum(const uint32_t* in, uint32_t* out, uint64_t n);

void or_project_visible(const bh_project_uniforms* u, const float* transforms,
                        const float* sh_coeffs, const float* raw_opac,
                        const uint32_t* global_from_compact_gid, uint32_t num_visible,
                        uint32_t sh_degree, uint32_t mip, float* projected);

void or_map_intersects(uint32_t tile_bw, uint32_t tile_bh, uint32_t tile_h, const float* projected,
                       const uint32_t* cum_tiles_hit, uint32_t num_visible,
                       uint32_t* tile_id_from_isect, uint32_t* compact_gid_from_isect);

void or_tile_offsets(const uint32_t* tile_id_from_isect, uint64_t num_inter, uint32_t num_tiles,
                     uint32_t* tile_offsets);

void or_rasterize(uint32_t img_w, uint32_t img_h, uint32_t tile_bw, uint32_t tile_bh,
                  const float* background, const float* projected,
                  const uint32_t* compact_gid_from_isect,
                  const uint32_t* global_from_compact_gid, const uint32_t* tile_offsets_pre,
                  uint32_t flags, void* out_img, float* visible, uint32_t* tile_offsets_post);

void or_rasterize_reference(const float* projected, uint32_t num_splats, uint32_t img_w,
                            uint32_t img_h, const float* background, uint32_t smooth_cutoff,
                            float* out_rgba);

void or_rasterize_backward(uint32_t img_w, uint32_t img_h, uint32_t tile_bw, uint32_t tile_bh,
                           const float* background, const float* out_img,
                           const float* projected, const uint32_t* compact_gid_from_isect,
                           const uint32_t* tile_offsets, uint32_t num_visible,
                           const float* v_output, uint32_t flags, float* v_combined);

/* Test support for the gradient tolerance.  or_rasterize_backward_check is
 * or_rasterize_backward with additions:
 *   check: OR_CHECK_DROP_LAST_BATCH plants a mistake (the last batch of 64
 *     entries of every tile's list is skipped);
 *   v_abs [max(V,1),11] (may be NULL): per lane, the sum of its per-pixel
 *     terms' magnitudes (the 2D-mean lanes as |c00 v_sigma dx| + |c01 v_sigma
 *     dy| and the like): a sum in another order differs by a small multiple
 *     of the unit roundoff times this;
 *   v_sq [max(V,1),11] (used when v_abs is given): per lane, the sum of the
 *     squares of its per-pixel terms' rounding scales: the magnitudes each
 *     term is formed from (the colour gap |T c| + |S| with the rounding the
 *     remaining colour S has gathered along the walk, as a root sum of
 *     squares of the magnitudes it was rounded at, then |v_out| and the
 *     alpha, conic and offset factors).  Another f32 evaluation of the terms
 *     moves the lane by a small multiple of the unit roundoff times the root
 *     of this.
 * or_rasterize_backward_f64 evaluates the same backward in double (the same
 * decisions and the same f32 alpha). */
#define OR_CHECK_DROP_LAST_BATCH 1u
void or_rasterize_backward_check(uint32_t img_w, uint32_t img_h, uint32_t tile_bw, uint32_t tile_bh,
                                 const float* background, const float* out_img, const float* projected,
                                 const uint32_t* compact_gid_from_isect, const uint32_t* tile_offsets,
                                 uint32_t num_visible, const float* v_output, uint32_t flags, uint32_t check,
                                 float* v_combined, float* v_abs, float* v_sq);
void or_rasterize_backward_f64(uint32_t img_w, uint32_t img_h, uint32_t tile_bw, uint32_t tile_bh,
                               const float* background, const float* out_img, const float* projected,
                               const uint32_t* compact_gid_from_isect, const uint32_t* tile_offsets,
                               uint32_t num_visible, const float* v_output, uint32_t flags, float* v_combined);

void or_project_backward(const bh_project_uniforms* u, const float* transforms,
                         const float* sh_coeffs, const float* raw_opac,
                         const uint32_t* global_from_compact_gid, uint32_t num_visible,
                         uint32_t num_splats, uint32_t sh_degree, uint32_t mip,
                         const float* v_combined, float* v_transforms, float* v_coeffs,
                         float* v_raw_opac, float* v_refine);

/* bh_oracle_train.c: the image loss and the optimizer step. */
void or_gauss_taps(float* taps6);
void or_image_loss_forward(const float* pred, uint32_t stride, uint32_t channels, const uint32_t* gt,
                           uint32_t w, uint32_t h, const bh_image_loss_config* cfg, float* map);
void or_image_loss_backward(const float* pred, uint32_t stride, uint32_t channels, const uint32_t* gt,
                            uint32_t w, uint32_t h, const bh_image_loss_config* cfg, const float* dl_dmap,
                            float* dl_dpred);
void or_adam_scaled_step(float* param, const float* grad, float* m1, float* m2, const float* scaling,
                         uint32_t rows, uint32_t row_len, uint32_t reduce, float lr, uint32_t time,
                         const bh_adam_config* cfg);

#ifdef __cplusplus
}
#endif

#endif
