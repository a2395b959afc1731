/*
 * brush_hip.h — C ABI of the gfx950 differentiable tile rasterizer.
 *
 * This is the drop-in boundary for Brush's rasterizer path.  Each entry
 * point replaces one operation of the reference's Burn backend extension and
 * takes plain device pointers and sizes (no framework types), so a Rust
 * `-sys` crate, Python ctypes or C++ can bind it.  Device pointers are
 * ordinary HIP device allocations on the context's device; every call is
 * stream-ordered on the context's stream.
 *
 * Layouts are the reference's row-major contiguous layouts
 * (brush-render/src/render.rs:103-110):
 *   transforms      f32 [N,10]  means xyz | quat wxyz | log-scales xyz
 *                   (brush-render/src/gaussian_splats.rs:110-127)
 *   sh_coeffs       f32 [N,C,3] C = (degree+1)^2, coefficient-major, rgb inner
 *   raw_opacities   f32 [N]     logits
 *   projected       f32 [V,10]  x y | conic c00 c01 c11 | opacity | r g b | depth
 *                   (brush-render/src/kernels/helpers.rs:192-196)
 *   v_combined      f32 [V,11]  dx dy | dc00 dc01 dc11 | dr dg db | dalpha |
 *                   refine | ddepth
 *                   (brush-render-bwd/src/kernels/rasterize_backwards.rs:28-40)
 *   tile_offsets    u32 [TY,TX,2] [start, end) per 16x16 tile
 *   out_img         f32 [H,W,4] (or [H,W,5] with depth) when BH_FLAG_BWD_INFO,
 *                   otherwise u32 [H,W] packed r|g<<8|b<<16|a<<24
 *
 * Errors: every entry point returns a bh_status and never aborts.  The text
 * of the last error on a context is available from bh_last_error().
 * A context is externally synchronised: do not call into one context from two
 * threads at once.
 */
#ifndef BRUSH_HIP_H
#define BRUSH_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum bh_status {
    BH_OK = 0,
    BH_ERR_INVALID_ARG = 1, /* null pointer, zero image size, bad flag       */
    BH_ERR_SHAPE = 2,       /* sizes inconsistent with each other            */
    BH_ERR_OOM = 3,         /* device allocation failed                      */
    BH_ERR_DEVICE = 4,      /* a HIP runtime call failed                     */
    BH_ERR_INTERNAL = 5,    /* a kernel reported a broken invariant          */
    BH_ERR_NOT_FINITE = 6   /* non-finite value where the reference panics   */
} bh_status;

/* Render flags.  BWD_INFO and SMOOTH_CUTOFF together encode the reference's
 * RasterPass {Forward, Backward, BackwardSmoothCutoff}
 * (brush-render/src/gaussian_splats.rs:43-66); RENDER_DEPTH is
 * RasterizationMode::RgbaAndDepth (:24-40); MIP is SplatRenderMode::Mip. */
#define BH_FLAG_BWD_INFO 1u
#define BH_FLAG_SMOOTH_CUTOFF 2u
#define BH_FLAG_RENDER_DEPTH 4u
#define BH_FLAG_MIP 8u
/* Backward-only flag: accumulate the refine weight lane (v_combined[:,9]). */
#define BH_FLAG_REFINE_WEIGHT 16u
/* Rasterizer::Candidate (brush-render/src/gaussian_splats.rs:68-101): 16x8
 * tiles instead of 16x16 (tile grid ceil(W/16) x ceil(H/8)).  Pass it to the
 * forward and to every backward entry point of that forward. */
#define BH_FLAG_TILE_16X8 32u

#define BH_TILE_WIDTH 16u
#define BH_PROJECTED_LANES 10u
#define BH_COMPACT_GRAD_LANES 11u

/* Mirrors ProjectUniforms (brush-render/src/kernels/types.rs:53-83 and
 * brush-render/src/shaders.rs:19-67).  viewmat is the top 3 rows of the
 * world-to-camera matrix, column-major: column i is viewmat[3i..3i+2], column 3
 * is the translation.  Build it with the host helpers of the Python package
 * (camera.rs:63-119,200-254 restated). */
typedef struct bh_project_uniforms {
    float viewmat[12];
    float half_max_render_fov;
    float fx, fy, cx, cy;
    float lim_pos_x, lim_pos_y, lim_neg_x, lim_neg_y;
    float camera_pos[3];
    uint32_t img_w, img_h;
    uint32_t tile_bw, tile_bh;
    uint32_t sh_degree;
    uint32_t total_splats;
    uint32_t num_visible; /* filled in by the forward pass */
    /* CameraModel (brush-render/src/kernels/camera_model/mod.rs:34-41): one of
     * BH_CAMERA_* and its coefficients, in the order of the reference's
     * parameter structs: KB4 k1..k4; RT8 k1..k6, p1, p2; TPF k1..k4, p1, p2,
     * sx1, sy1 (kannala_brandt_4.rs:11-16, radial_tangential_8.rs:12-21,
     * thin_prism_fisheye.rs:23-30).  Unused entries are ignored. */
    uint32_t camera_model;
    float camera_params[8];
} bh_project_uniforms;

#define BH_CAMERA_PINHOLE 0u
#define BH_CAMERA_KB4 1u /* Kannala-Brandt 4 (equidistant fisheye) */
#define BH_CAMERA_RT8 2u /* radial-tangential with 6 radial + 2 tangential */
#define BH_CAMERA_TPF 3u /* thin-prism fisheye: KB4 + tangential + thin prism */

typedef struct bh_ctx bh_ctx;
typedef struct bh_fwd_state bh_fwd_state;

/* Device pointers and counts of one forward pass (RenderOutput and
 * RenderAuxInner, brush-render/src/render_aux.rs:17-68).  Buffers sized by a
 * count are allocated with max(count, 1) rows like the reference
 * (render.rs:337,373).  They stay valid until bh_fwd_state_release(). */
typedef struct bh_fwd_info {
    uint32_t num_splats;
    uint32_t num_visible;
    uint32_t num_intersections;
    uint32_t num_tiles;
    uint32_t tile_bw, tile_bh;
    uint32_t img_w, img_h;
    uint32_t sh_degree;
    uint32_t flags;
    bh_project_uniforms uniforms;      /* num_visible filled in              */
    const float* projected;            /* [V,10] in depth (compact) order    */
    const uint32_t* global_from_compact_gid; /* [V] depth-sorted global ids  */
    const float* depths;               /* [V] ascending view-space depths    */
    const uint32_t* intersect_counts;  /* [N] tiles hit per global id        */
    const uint32_t* cum_tiles_hit;     /* [V] inclusive scan, compact order  */
    const uint32_t* tile_id_from_isect;      /* [M] tile-sorted tile ids     */
    const uint32_t* compact_gid_from_isect;  /* [M] tile-sorted compact ids  */
    const uint32_t* tile_offsets_pre;  /* [TY,TX,2] before rasterize shrinks */
} bh_fwd_info;

/* Image loss configuration: brush-loss ImageLossConfig
 * (crates/brush-loss/src/lib.rs:927-941).  composite != 0 composites GT over
 * `background` (gt + (1 - gt.a) * bg); mask != 0 multiplies the loss map by
 * gt.a. */
typedef struct bh_image_loss_config {
    float l1_weight;
    float ssim_weight;
    uint32_t composite;
    float background[3];
    uint32_t mask;
} bh_image_loss_config;

/* AdamScaledConfig (crates/brush-train/src/adam_scaled.rs:57-69). */
typedef struct bh_adam_config {
    float beta_1;
    float beta_2;
    float epsilon;
} bh_adam_config;

/* ---- context ------------------------------------------------------------ */

/* Create a context on HIP device `device` with the null stream.
 * No counterpart in the reference (the reference's device is a Burn
 * WgpuDevice, brush-process/src/lib.rs:34-39). */
bh_status bh_ctx_create(int device, bh_ctx** out);
void bh_ctx_destroy(bh_ctx* ctx);
/* Use `hip_stream` (a hipStream_t) for all later work.  If it differs from the
 * current stream, the current stream is synchronised first so that cached
 * workspace is not reused across streams. */
bh_status bh_ctx_set_stream(bh_ctx* ctx, void* hip_stream);
const char* bh_last_error(const bh_ctx* ctx);
/* Kernel timing with HIP events on the context's stream (for benchmarking).
 * When enabled, every launch is bracketed by events and its duration is
 * accumulated per kernel name. */
bh_status bh_ctx_set_timing(bh_ctx* ctx, int enable);
/* Restricts timing to launches of the kernel called `name` (NULL or "" times
 * every kernel), so that a benchmark can time one kernel without bracketing the
 * others with events. */
bh_status bh_ctx_set_timing_filter(bh_ctx* ctx, const char* name);
typedef struct bh_kernel_timing {
    char name[48];
    uint32_t launches;
    double total_ms;
} bh_kernel_timing;
/* Synchronises the stream, then copies up to `max` entries. */
bh_status bh_ctx_read_timings(bh_ctx* ctx, bh_kernel_timing* out, int max, int* count);
bh_status bh_ctx_reset_timings(bh_ctx* ctx);
/* Debug modes (off by default; not for benchmarking).
 * BH_DEBUG_POISON: every workspace block the library hands out (pool blocks,
 *   forward-state buffers, the allocation-free sort's scratch) is first filled
 *   with 0xFF bytes (NaN as f32, 0xFFFFFFFF as u32), so a missed initialisation
 *   shows up in the results instead of reading zeros left by an earlier call;
 *   the reference noises its uninitialised test tensors the same way
 *   (crates/brush-cube/src/host.rs:52-65).
 * BH_DEBUG_VALIDATE: bh_render_forward returns BH_ERR_NOT_FINITE when a splat
 *   parameter is NaN or infinite, and bh_render_backward when a gradient it
 *   produced is, naming the array and the first index; the reference panics
 *   there under its debug validation (Splats::validate_values / bwd_validate,
 *   crates/brush-render/src/gaussian_splats.rs:322-415, validation.rs:6-84).
 *   Costs one pass over the inputs (outputs) and one host synchronisation.
 * BH_DEBUG_EXACT_SIZES: bh_render_forward waits for its counts (visible
 *   splats, intersections, depth-key range) before it queues the launches that
 *   depend on them, as the reference does (render.rs:309-329).  By default a
 *   forward after the first on a context queues those launches sized from the
 *   previous forward's counts (buffers for that many intersections, plus
 *   1/8), with the kernels reading the actual counts from device memory, and
 *   checks the counts only after queueing; when they do not fit it queues the
 *   exact launches again before it returns.  Both give identical results. */
#define BH_DEBUG_POISON 1u
#define BH_DEBUG_VALIDATE 2u
#define BH_DEBUG_EXACT_SIZES 4u
/* BH_DEBUG_KEEP_LANES: bh_render_backward keeps the per-splat gradient lanes
 *   it accumulated in the forward state (bh_fwd_state_backward_lanes) instead
 *   of returning them to the workspace pool, so a test can compare them with
 *   rasterize_bwd's v_combined lane by lane. */
#define BH_DEBUG_KEEP_LANES 8u
bh_status bh_ctx_set_debug(bh_ctx* ctx, uint32_t flags);
/* Bytes currently cached by the context's workspace pool. */
uint64_t bh_ctx_workspace_bytes(const bh_ctx* ctx);
/* Synchronises the stream, then frees every cached workspace block that no
 * forward state holds (the counterpart of a caching allocator's empty-cache
 * call; no counterpart in the reference, whose buffers belong to Burn's
 * allocator).  Later calls allocate again as needed. */
bh_status bh_ctx_release_workspace(bh_ctx* ctx);

/* ---- primitives ---------------------------------------------------------- */

/* Stable LSD radix argsort of u32 keys carrying u32 values, considering the
 * low `sorting_bits` (<= 32) bits.  Replaces brush-sort `radix_argsort`
 * (crates/brush-sort/src/lib.rs:16-129).  Outputs are caller allocated and
 * must not alias the inputs.  n == 0 is a no-op. */
bh_status bh_radix_argsort(bh_ctx* ctx, const uint32_t* keys_in, const uint32_t* vals_in,
                           uint32_t n, uint32_t sorting_bits, uint32_t* keys_out,
                           uint32_t* vals_out);

/* bh_radix_argsort without any allocation: no hipMalloc, hipFree or
 * allocating library call, for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid it).  It has no
 * counterpart in the reference.  Same arguments, results and errors as
 * bh_radix_argsort, for n <= BH_NOALLOC_SORT_MAX_KEYS (larger n returns
 * BH_ERR_INVALID_ARG).  The workspace is a fixed 48 MiB device array of the
 * library, one per GPU, held until the process ends; every call on one GPU
 * shares it, so calls that overlap on one GPU (from any context or stream)
 * race. */
#define BH_NOALLOC_SORT_MAX_KEYS 2097152u
bh_status bh_radix_argsort_noalloc(bh_ctx* ctx, const uint32_t* keys_in, const uint32_t* vals_in, uint32_t n,
                                   uint32_t sorting_bits, uint32_t* keys_out, uint32_t* vals_out);

/* Inclusive u32 prefix sum.  Replaces brush-prefix-sum `prefix_sum`
 * (crates/brush-prefix-sum/src/lib.rs:11-87).  out may alias in. */
bh_status bh_prefix_sum(bh_ctx* ctx, const uint32_t* in, uint32_t* out, uint32_t n);

/* [start, end) of each tile's run in tile-sorted ids; ids >= num_tiles are
 * sentinels and write nothing.  Replaces `get_tile_offsets`
 * (brush-render/src/get_tile_offset.rs:10-62) together with its zero fill
 * (brush-render/src/render.rs:396-400): every entry of tile_offsets[2*T] is
 * written. */
bh_status bh_get_tile_offsets(bh_ctx* ctx, const uint32_t* tile_id_from_isect,
                              uint32_t num_intersections, uint32_t num_tiles,
                              uint32_t* tile_offsets);

/* ---- forward ------------------------------------------------------------- */

/* Full forward render: project + cull, depth sort, scan, project visible
 * (SH -> RGB), map to intersections, tile sort, tile offsets, blend.
 * Replaces SplatRasterizerOps::render_with_rasterizer with the 16x16
 * rasterizer (brush-render/src/render.rs:78-543; trait at
 * brush-render/src/lib.rs:69-108).
 *
 * `u` supplies the camera part of ProjectUniforms; img_w/img_h must be > 0;
 * tile_bw/tile_bh, sh_degree, total_splats are recomputed from the sizes.
 * Caller-allocated outputs:
 *   out_img       BWD_INFO: f32 [H,W,4] ([H,W,5] with RENDER_DEPTH)
 *                 otherwise u32 [H,W] packed RGBA8
 *   visible       f32 [N] (BWD_INFO only, else may be NULL)
 *   max_radius    f32 [N]
 *   tile_offsets  u32 [TY,TX,2]; with BWD_INFO the end of each tile is shrunk to
 *                 one past the last splat that contributed (rasterize.rs:193-199)
 * One blocking 16-byte device-to-host read per call sizes the count-dependent
 * buffers (render.rs:308-330).  *state receives the forward state, which the
 * caller releases with bh_fwd_state_release(). */
bh_status bh_render_forward(bh_ctx* ctx, const bh_project_uniforms* u, const float background[3],
                            const float* transforms, const float* sh_coeffs,
                            const float* raw_opacities, uint32_t num_splats, uint32_t sh_degree,
                            uint32_t flags, void* out_img, float* visible, float* max_radius,
                            uint32_t* tile_offsets, bh_fwd_state** state);

bh_status bh_fwd_state_info(const bh_fwd_state* state, bh_fwd_info* out);
/* Debug: the per-splat gradient lanes f32 [N,11] (row = global id, lanes as
 * v_combined) that the state's latest bh_render_backward accumulated, when
 * that backward ran with BH_DEBUG_KEEP_LANES set; *lanes is NULL otherwise.
 * Valid until the state's next backward or its release.  No counterpart in
 * the reference (its v_combined is an ordinary tensor, rasterize_bwd's
 * output). */
bh_status bh_fwd_state_backward_lanes(const bh_fwd_state* state, const float** lanes);
/* Returns the state's buffers to the context pool (stream ordered). */
void bh_fwd_state_release(bh_fwd_state* state);

/* ---- backward ------------------------------------------------------------ */

/* Rasterize backward.  Replaces SplatBwdOps::rasterize_bwd /
 * rasterize_bwd_with_refine_weight (brush-render-bwd/src/burn_glue.rs:79-172,
 * impl render_bwd.rs:90-238).  Inputs are the forward's out_img (f32),
 * projected [V,10], tile-sorted compact_gid_from_isect, the post-rasterize
 * tile_offsets, and the upstream gradient v_output (same shape as out_img).
 * flags: BH_FLAG_SMOOTH_CUTOFF, BH_FLAG_REFINE_WEIGHT, BH_FLAG_RENDER_DEPTH.
 * v_combined [max(V,1),11] is caller allocated; it is fully overwritten. */
bh_status bh_rasterize_backward(bh_ctx* ctx, const float* out_img, const float* projected,
                                const uint32_t* compact_gid_from_isect,
                                const uint32_t* tile_offsets, uint32_t num_visible,
                                const float background[3], uint32_t img_w, uint32_t img_h,
                                const float* v_output, uint32_t flags, float* v_combined);

/* Both backward operations of one forward state in one call: the backward of
 * RenderBackwards (brush-render-bwd/src/burn_glue.rs:292-378), which runs
 * rasterize_bwd then project_bwd and keeps v_combined internal.  Here the
 * gradient lanes are accumulated per global id, so project backward reads
 * them in order.  `state` comes from a forward with BH_FLAG_BWD_INFO;
 * out_img and tile_offsets are that forward's outputs; flags:
 * BH_FLAG_SMOOTH_CUTOFF, BH_FLAG_REFINE_WEIGHT, BH_FLAG_RENDER_DEPTH
 * (BH_FLAG_MIP follows the forward).  Outputs as bh_project_backward.
 *
 * The call changes the state: the first backward of a state accumulates into
 * the [N,11] lane rows that the forward zeroed (held by the state until
 * then) and returns them to the context's workspace pool once its work is
 * queued; a later backward of the same state zeroes workspace rows of its
 * own.  Backwards of one state must therefore not overlap; since a state
 * belongs to one context, and calls on a context are externally
 * synchronised, this is the context's rule.
 *
 * Every entry of the four output arrays is written (zeros for splats without
 * a gradient), all of it on the context's stream. */
bh_status bh_render_backward(bh_ctx* ctx, const bh_fwd_state* state, const float* out_img,
                             const uint32_t* tile_offsets, const float background[3],
                             const float* transforms, const float* sh_coeffs,
                             const float* raw_opacities, const float* v_output, uint32_t flags,
                             float* v_transforms, float* v_coeffs, float* v_raw_opac, float* v_refine);

/* ---- training: image loss and optimizer ------------------------------------ */

/* Fused L1 + SSIM loss map.  Replaces LossOps::image_loss_forward
 * (crates/brush-loss/src/lib.rs:946-963; kernels lib.rs:228-555).
 * pred: f32 [H, W, pred_stride] of which the first `channels` (3 or 4) are
 * compared; gt_packed: u32 [H, W] RGBA8 (r in the low byte).  loss_map:
 * f32 [H, W, channels].  With channels == 4 the alpha channel of the map is
 * |pred.a - gt.a|.  ssim_weight == 0 selects the L1-only path. */
bh_status bh_image_loss_forward(bh_ctx* ctx, const float* pred, uint32_t pred_stride, uint32_t channels,
                                const uint32_t* gt_packed, uint32_t img_w, uint32_t img_h,
                                const bh_image_loss_config* cfg, float* loss_map);
/* VJP of bh_image_loss_forward.  Replaces LossOps::image_loss_backward
 * (lib.rs:952-957; kernels lib.rs:280-893).  dl_dmap: f32 [H, W, channels];
 * dl_dpred: f32 [H, W, pred_stride], every element written (zeros in the
 * channels past `channels`), so it can be fed to the rasterizer's backward
 * as the gradient of an RGBA render. */
bh_status bh_image_loss_backward(bh_ctx* ctx, const float* pred, uint32_t pred_stride, uint32_t channels,
                                 const uint32_t* gt_packed, uint32_t img_w, uint32_t img_h,
                                 const bh_image_loss_config* cfg, const float* dl_dmap, float* dl_dpred);
/* One AdamScaled step on a [rows, row_len] parameter, in place.  Replaces
 * AdamScaled::step (crates/brush-train/src/adam_scaled.rs:216-383).
 * moment_1 has the parameter's shape; moment_2 has it too, or [rows] when
 * reduce_moment_2 != 0 (mean of grad^2 over each row, the SH setting of
 * train.rs:966-990).  scaling: per-column factors [row_len] or NULL; the
 * decrement is step * (scaling[col] * lr).  time is the step count including
 * this step (1 on the first step, when the moments are initialised from the
 * gradient and their previous contents are ignored). */
bh_status bh_adam_scaled_step(bh_ctx* ctx, float* param, const float* grad, float* moment_1, float* moment_2,
                              const float* scaling, uint32_t rows, uint32_t row_len, uint32_t reduce_moment_2,
                              float lr, uint32_t time, const bh_adam_config* cfg);

/* Project backward.  Replaces SplatBwdOps::project_bwd
 * (brush-render-bwd/src/burn_glue.rs:79-172, impl render_bwd.rs:298-447,
 * kernel kernels/project_backwards.rs:101-263).  `u` is the forward's uniforms
 * with num_visible filled in (bh_fwd_info.uniforms).  flags: BH_FLAG_MIP.
 * Dense caller-allocated outputs, every element written:
 *   v_transforms f32 [N,10], v_coeffs f32 [N,C,3], v_raw_opac f32 [N],
 *   v_refine f32 [N]. */
bh_status bh_project_backward(bh_ctx* ctx, const bh_project_uniforms* u, const float* transforms,
                              const float* sh_coeffs, const float* raw_opacities,
                              const uint32_t* global_from_compact_gid, const float* v_combined,
                              uint32_t flags, float* v_transforms, float* v_coeffs,
                              float* v_raw_opac, float* v_refine);

/* ---- PLY rows (brush-serde) ------------------------------------------------ */

/* Scalar types of PLY properties (the header's char .. double). */
#define BH_PLY_I8 1u
#define BH_PLY_U8 2u
#define BH_PLY_I16 3u
#define BH_PLY_U16 4u
#define BH_PLY_I32 5u
#define BH_PLY_U32 6u
#define BH_PLY_F32 7u
#define BH_PLY_F64 8u
/* A column with no property in the file: the value is `konst`. */
#define BH_PLY_CONST 0u
/* Column ops: PLAIN converts the value to f32 (Rust `as f32`); COLOR is a
 * red/green/blue override: u8 / 255, u16 / 65535 or f32 as is
 * (ply_gaussian.rs:35-56), then rgb_to_sh, (c - 0.5) / SH_C0 (sh.rs:20-31). */
#define BH_PLY_OP_PLAIN 0u
#define BH_PLY_OP_COLOR 1u
/* flags */
#define BH_PLY_BIG_ENDIAN 1u

/* Where one output value comes from in a vertex row. */
typedef struct bh_ply_column {
    uint32_t offset; /* byte offset of the property in the row */
    uint16_t type;   /* BH_PLY_* scalar type, or BH_PLY_CONST */
    uint16_t op;     /* BH_PLY_OP_* */
    float konst;     /* value of a BH_PLY_CONST column */
} bh_ply_column;

/* Decode the rows of a standard PLY vertex element straight into the splat
 * layout.  Replaces the row visitor of parse_ply
 * (crates/brush-serde/src/import.rs:341-502) with SplatData::into_splats
 * (import.rs:76-91) fused in: the caller resolves the header into
 * 11 + 3 * num_coeffs columns, in output order
 *   x y z rot_0..3 scale_0..2 | opacity | sh[c][channel] for c < num_coeffs,
 * with the into_splats defaults as BH_PLY_CONST columns.
 * rows: device copy of the element's bytes (binary little- or big-endian per
 * flags; an ASCII file is first converted by the host), 4-byte aligned,
 * rows_bytes >= num_rows * row_bytes.  Row k * subsample becomes splat k for
 * k < ceil(num_rows / subsample); num_coeffs is 1, 4, 9, 16 or 25; rows are
 * at most 32 KiB.  Outputs (device, every element written):
 * transforms f32 [n,10], sh_coeffs f32 [n,num_coeffs,3], raw_opac f32 [n]. */
bh_status bh_ply_decode_rows(bh_ctx* ctx, const uint8_t* rows, uint64_t rows_bytes, uint32_t row_bytes,
                             uint64_t num_rows, uint32_t subsample, uint32_t flags,
                             const bh_ply_column* columns, uint32_t num_coeffs, float* transforms,
                             float* sh_coeffs, float* raw_opac);

/* The SuperSplat compressed layout (import.rs:504-720, quant.rs:1-71). */
typedef struct bh_ply_compressed_layout {
    uint32_t vertex_row_bytes;
    uint32_t position_offset; /* byte offsets of the four packed u32 words */
    uint32_t scale_offset;
    uint32_t rotation_offset;
    uint32_t color_offset;
    uint32_t sh_row_bytes;    /* bytes of one `sh` row; 0 without an sh element */
    uint32_t sh_rest_count;   /* 0, 9, 24, 45 or 72 u8 properties */
    uint16_t sh_offsets[72];  /* byte offset of f_rest_k in an sh row */
} bh_ply_compressed_layout;

/* Decode a compressed PLY.  Replaces parse_compressed_ply
 * (import.rs:504-720).  chunks: device f32 [num_chunks, 18] holding each
 * chunk row's min_x max_x min_y max_y min_z max_z min_scale_x max_scale_x
 * min_scale_y max_scale_y min_scale_z max_scale_z min_r max_r min_g max_g
 * min_b max_b; num_chunks >= ceil(num_rows / 256).  vertex_rows / sh_rows:
 * device copies of the vertex and sh elements (sh_rows may be NULL when
 * layout->sh_row_bytes is 0), 4-byte aligned.  Outputs as bh_ply_decode_rows
 * with num_coeffs = 1 + sh_rest_count / 3. */
bh_status bh_ply_decode_compressed(bh_ctx* ctx, const float* chunks, uint64_t num_chunks,
                                   const uint8_t* vertex_rows, uint64_t vertex_bytes, const uint8_t* sh_rows,
                                   uint64_t sh_bytes, uint64_t num_rows, uint32_t subsample, uint32_t flags,
                                   const bh_ply_compressed_layout* layout, float* transforms, float* sh_coeffs,
                                   float* raw_opac);

/* Encode splats as the rows of an exported PLY.  Replaces read_splat_data
 * (crates/brush-serde/src/export.rs:83-178): per splat, 11 + 3 * num_coeffs
 * f32 values x y z scale_0..2 opacity rot_0..3 f_dc_0..2 f_rest_*, the
 * quaternion divided by max(|q|, 1e-12) and the rest coefficients
 * channel-major.  rows: device f32 [n, 11 + 3 * num_coeffs] (little-endian,
 * ready to follow the header). */
bh_status bh_ply_encode_rows(bh_ctx* ctx, const float* transforms, const float* sh_coeffs,
                             const float* raw_opac, uint64_t n, uint32_t num_coeffs, float* rows);

/* ---- host/device copies (plumbing for bindings without a tensor library) */
bh_status bh_copy_to_host(bh_ctx* ctx, void* dst_host, const void* src_device, uint64_t bytes);
bh_status bh_copy_to_device(bh_ctx* ctx, void* dst_device, const void* src_host, uint64_t bytes);
/* Stream-ordered device-to-device copy (does not synchronise). */
bh_status bh_copy_device(bh_ctx* ctx, void* dst_device, const void* src_device, uint64_t bytes);
bh_status bh_device_alloc(bh_ctx* ctx, void** out, uint64_t bytes);
bh_status bh_device_free(bh_ctx* ctx, void* ptr);
bh_status bh_synchronize(bh_ctx* ctx);

#ifdef __cplusplus
}
#endif

#endif /* BRUSH_HIP_H */
