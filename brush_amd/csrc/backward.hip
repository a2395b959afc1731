// backward.hip — rasterize backward and project backward for gfx950.
//
// rasterize_backward: one single-wave workgroup per 8x8 pixel block of a
// 16x16 tile, one pixel per lane.  Every pixel replays the tile's splats front
// to back with the same per-pair arithmetic as the reference's replay
// (crates/brush-render-bwd/src/kernels/rasterize_backwards.rs:79-443, where
// instead a 32-lane workgroup owns 32 splats and walks the pixels on a
// diagonal); the transmittance / remaining-colour state never leaves the
// lane's registers.  Each wave stages the tile's splats in LDS in batches of
// 64 and keeps those that may touch its block (a ballot of a conservative
// rectangle test), so the four blocks of a tile run independently, without
// workgroup barriers, and a block whose 64 pixels have all saturated stops.
// For a splat with any contributing pixel the wave sums its 9-11 gradient
// lanes over all 64 pixels with a transposed reduction (permlane32 and
// permlane16 swaps fold four lanes into one register, then four DPP row
// steps), which leaves up to four different gradient lanes in lanes 15, 31,
// 47 and 63, so one float-atomic instruction adds four of them.
//
// project_backward: one thread per *global* id, so every dense output row is
// written exactly once (zeros for culled splats or splats without gradient)
// and no separate zero fill of the ~240 MB SH3 gradient is needed
// (crates/brush-render-bwd/src/kernels/project_backwards.rs:101-263 and
// render_bwd.rs:338-350 restated).
#include <hip/hip_runtime.h>

#include <type_traits>

#include "bh_internal.h"
#include "bh_splat_math.h"
#include "bh_splat_record.h"
#include "bh_tile_walk.h"

// Candidates staged per batch by the recorded backward (32 or 64).  32
// keeps its LDS at 9 KB (17 workgroups per CU) with three summing slots.
#ifndef BH_BWD_BATCH
#define BH_BWD_BATCH 32
#endif

namespace bh {

// Sum of x over each 16-lane row of the wave, left in the row's last lane
// (inclusive Hillis-Steele steps as DPP adds).
template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
    return x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float row_sum_last_lane(float x) {
    x = dpp_add<0x111>(x);  // row_shr:1
    x = dpp_add<0x112>(x);  // row_shr:2
    x = dpp_add<0x114>(x);  // row_shr:4
    x = dpp_add<0x118>(x);  // row_shr:8
    return x;
}

// Transposed wave reduction.  psum32(a, b): rows 0-1 (lanes 0-31) hold a
// summed over lanes i and i + 32, rows 2-3 hold b likewise.  psum16(p, q) of
// two such values: row 0 holds p's rows 0+1, row 1 q's rows 0+1, row 2 p's
// rows 2+3 and row 3 q's rows 2+3.  Two levels fold four values into one
// register with one swap and one add per pair.
__device__ __forceinline__ float psum32(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float psum16(float p, float q) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(p), __float_as_uint(q), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

constexpr int kNG = 11;

// One workgroup (a single wave) per 8x8 pixel block of a 16x16 tile.  The
// dispatcher deals workgroups to the eight XCDs in turn, so the four blocks of
// a tile are given ids that agree modulo 8 and share an L2.
template <int TH>
__device__ __forceinline__ void block_of_workgroup(uint32_t g, uint32_t& tile, uint32_t& blk) {
    constexpr uint32_t BPT = 2u * (uint32_t)TH / 8u;
    const uint32_t slot = g >> 3;
    tile = ((slot / BPT) << 3) | (g & 7u);
    blk = slot % BPT;
}

template <bool SMOOTH, bool REFINE, bool DEPTH, int TH>
__global__ __launch_bounds__(64) void rasterize_backward_kernel(
    uint32_t img_w, uint32_t img_h, uint32_t tile_bw, uint32_t num_tiles, float bg_r, float bg_g, float bg_b,
    uint32_t num_visible, const float* __restrict__ out_img, const float* __restrict__ projected,
    const uint32_t* __restrict__ cgids, const uint32_t* __restrict__ offsets, const float* __restrict__ v_output,
    const uint32_t* __restrict__ row_of, const uint32_t* __restrict__ order, float* __restrict__ v_combined) {
    constexpr uint32_t CH = DEPTH ? 5u : 4u;
    __shared__ float4 s_xyco[64];  // x, y, conic c00, c01
    __shared__ float4 s_crgb[64];  // conic c11, opacity, r, g (staged_colour)
    __shared__ float4 s_bd[64];    // b (staged_colour), depth, sigma cutoff
    __shared__ uint32_t s_cid[64];

    uint32_t tile, blk;
    block_of_workgroup<TH>(blockIdx.x, tile, blk);
    if (tile >= num_tiles) return;
    if (order) tile = order[tile];
    const uint32_t lane = threadIdx.x;
    const uint32_t ox = (tile % tile_bw) * 16u + (blk & 1u) * 8u;
    const uint32_t oy = (tile / tile_bw) * (uint32_t)TH + (blk >> 1) * 8u;
    const uint32_t px = ox + (lane & 7u), py = oy + (lane >> 3);
    const bool inside = px < img_w && py < img_h;
    const float pcx = (float)px + 0.5f, pcy = (float)py + 0.5f;

    // Pixel state of the front-to-back replay (rasterize_backwards.rs:193-250):
    // remaining colour (final minus background pre-roll) and transmittance.
    float sx = 0.0f, sy = 0.0f, sz = 0.0f, sw = 0.0f, sd = 0.0f;
    float vox = 0.0f, voy = 0.0f, voz = 0.0f, vow = 0.0f, vod = 0.0f, final_a = 0.0f;
    if (inside) {
        const size_t pix = (size_t)py * img_w + px;
        const float* o = out_img + pix * CH;
        const float* vo = v_output + pix * CH;
        final_a = o[3];
        const float t_final = 1.0f - final_a;
        sx = o[0] - t_final * bg_r;
        sy = o[1] - t_final * bg_g;
        sz = o[2] - t_final * bg_b;
        sw = 1.0f;
        vox = vo[0];
        voy = vo[1];
        voz = vo[2];
        vow = (vo[3] - (bg_r * vox + bg_g * voy + bg_b * voz)) * t_final;
        if (DEPTH) {
            sd = o[4];
            vod = vo[4];
        }
    }
    const uint32_t lo = offsets[2 * tile], hi = offsets[2 * tile + 1];
    // Work is concentrated in few tiles (at config 1, 28 % of the tiles hold
    // splats; the heaviest replays ~480, the mean ~53), so the kernel ends
    // with the long blocks sharing their SIMDs.  A block's wave priority
    // rises with its tile's splat count, so the SIMD issues long blocks first.
    const uint32_t len = hi - lo;
    if (len >= 256u)
        __builtin_amdgcn_s_setprio(3);
    else if (len >= 128u)
        __builtin_amdgcn_s_setprio(2);
    else if (len >= 64u)
        __builtin_amdgcn_s_setprio(1);
    const float img_wf = (float)img_w, img_hf = (float)img_h;
    const float inv_final_a = __builtin_amdgcn_rcpf(bh_maxf(final_a, 1.0e-5f));
    const float bx0 = (float)ox + 0.5f, by0 = (float)oy + 0.5f;
    bool wave_live = __ballot(sw > 1.0e-4f) != 0ull;

    for (uint32_t b = lo; wave_live && b < hi; b += 64u) {
        const uint32_t cnt = min(64u, hi - b);
        bool touch = false;
        if (lane < cnt) {
            const uint32_t c = min(cgids[b + lane], num_visible - 1u);
            const float2* prow = reinterpret_cast<const float2*>(projected + (size_t)c * 10);
            const float2 r0 = prow[0], r1 = prow[1], r2 = prow[2], r3 = prow[3], r4 = prow[4];
            const float cut = sigma_cutoff<SMOOTH>(r2.y);
            s_xyco[lane] = make_float4(r0.x, r0.y, r1.x, r1.y);
            s_crgb[lane] = make_float4(r2.x, r2.y, staged_colour(r3.x), staged_colour(r3.y));
            // the cutoff on the power in base 2 (power log2(e); the cutoff's
            // margin of 1e-3 covers the rounding)
            s_bd[lane] = make_float4(staged_colour(r4.x), r4.y, kLog2e * cut, 0.0f);
            s_cid[lane] = row_of ? row_of[c] : c;
            touch = may_touch_rect(r0.x, r0.y, S2{r1.x, r1.y, r2.x}, cut, bx0, by0, bx0 + 7.0f, by0 + 7.0f);
        }
        // splats of the batch that may touch this block, in order
        uint64_t todo = __ballot(touch);
        wave_lds_fence();
        while (todo) {
            const uint32_t j = (uint32_t)__builtin_ctzll(todo);
            todo &= todo - 1ull;
            const float4 xc = s_xyco[j];
            const float4 cr4 = s_crgb[j];
            const float4 bd = s_bd[j];
            const S2 conic{xc.z, xc.w, cr4.x};
            const float opac = cr4.y;
            const float dx = xc.x - pcx, dy = xc.y - pcy;
            // the forward's Gaussian (bh_math.h: the power in base 2)
            float ka, kb, kc;
            bh_conic_log2(conic.c00, conic.c01, conic.c11, &ka, &kb, &kc);
            const float power = bh_power_log2(ka, kb, kc, dx, dy);
            const bool maybe = sw > 1.0e-4f && power >= 0.0f && !(power > bd.z);
            if (__ballot(maybe) == 0ull) continue;
            // lanes outside `maybe` compute values that the selects below discard
            const float gaussian = bh_exp2_neg(-power);
            const float alpha = bh_minf(0.999f, opac * gaussian);
            const float w = SMOOTH ? cutoff_weight(alpha) : (alpha >= kCutMid ? 1.0f : 0.0f);
            const bool pass = maybe && w > 0.0f;
            const float ae = SMOOTH ? alpha * w : (alpha >= kCutMid ? alpha : 0.0f);
            const float next_t = sw * (1.0f - ae);
            const bool saturate = pass && next_t <= 1.0e-4f;
            const bool contrib = pass && !saturate;
            if (saturate) sw = 0.0f;
            if (__ballot(contrib) == 0ull) {
                wave_live = __ballot(sw > 1.0e-4f) != 0ull;
                if (!wave_live) break;
                continue;
            }
            float g[12];
            {
#pragma clang fp contract(fast)
                // Gradient-only arithmetic and the remaining-colour state, which
                // feeds only gradients: products and sums fuse into FMAs here.
                // The replay's decisions above (alpha, transmittance, saturation)
                // stay uncontracted, bit for bit the forward's.
                // staged colours: max(c, 0) in value, the c >= 0 gate in the sign bit
                const float cr = cr4.z, cgc = cr4.w, cb = bd.x;
                const float vis = ae * sw;
                g[5] = contrib && colour_gate(cr) ? vis * vox : 0.0f;
                g[6] = contrib && colour_gate(cgc) ? vis * voy : 0.0f;
                g[7] = contrib && colour_gate(cb) ? vis * voz : 0.0f;
                // gradient-only quantities: hardware reciprocal / sqrt (1 ulp)
                const float ra = __builtin_amdgcn_rcpf(1.0f - ae);
                const float dot_rgb = ((sw * cr - sx) * vox + (sw * cgc - sy) * voy + (sw * cb - sz) * voz) * ra;
                const float v_ae = dot_rgb + vow * ra;
                // with the hard cutoff the weight is a step and its derivative 0.
                // The position, conic, opacity and refine lanes are gated on
                // contributing and unclamped (o G <= 0.999) pairs.  Lanes outside
                // `maybe` may hold any alpha and gaussian: a sigma far below zero
                // (rounding on a nearly singular conic) overflows the exponential's
                // range reduction into inf or a negative value.  So the selects sit
                // on v_sigma and on the opacity lane; a zero v_sigma then zeroes the
                // position, conic and refine lanes (up to the sign of a zero), whose
                // other factors dx, dy and the conic (|c| <= 10: every 2D covariance
                // carries a blur of at least 0.1 on its diagonal) are finite.
                const bool unclamped = opac * gaussian <= 0.999f;
                const bool gate = contrib && unclamped;
                const float v_alpha = SMOOTH ? v_ae * (w + alpha * cutoff_weight_deriv(alpha)) : v_ae * w;
                const float v_sigma = gate ? -alpha * v_alpha : 0.0f;
                const float vxy_x = v_sigma * (conic.c00 * dx + conic.c01 * dy);
                const float vxy_y = v_sigma * (conic.c01 * dx + conic.c11 * dy);
                g[2] = 0.5f * v_sigma * dx * dx;
                g[3] = v_sigma * dx * dy;
                g[4] = 0.5f * v_sigma * dy * dy;
                g[0] = vxy_x;
                g[1] = vxy_y;
                g[8] = gate ? v_alpha * gaussian : 0.0f;
                g[9] = REFINE ? __builtin_amdgcn_sqrtf(vxy_x * img_wf * vxy_x * img_wf + vxy_y * img_hf * vxy_y * img_hf) *
                                    inv_final_a
                              : 0.0f;
                g[10] = DEPTH && contrib ? vis * vod : 0.0f;
                g[11] = 0.0f;
                if (contrib) {
                    sx = sx - vis * cr;
                    sy = sy - vis * cgc;
                    sz = sz - vis * cb;
                    if (DEPTH) sd = sd - vis * bd.y;
                }
            }
            if (contrib) sw = next_t;
            // whole-wave sums: rows of q0 hold lanes 0, 2, 1, 3; of q1 lanes 4, 6,
            // 5, 7; of q2 lanes 8, 10, 9, 11 (8, 8, 9, 9 without depth, of which
            // one lane each is added: two lanes of one atomic instruction on one
            // address measured 124 us per frame slower)
            const float q0 = row_sum_last_lane(psum16(psum32(g[0], g[1]), psum32(g[2], g[3])));
            const float q1 = row_sum_last_lane(psum16(psum32(g[4], g[5]), psum32(g[6], g[7])));
            const float p4 = psum32(g[8], g[9]);
            const float q2 = row_sum_last_lane(DEPTH ? psum16(p4, psum32(g[10], g[11])) : psum16(p4, p4));
            // the splat's gradient row: wave-uniform, so its address is scalar
            const uint32_t cid = __builtin_amdgcn_readfirstlane(s_cid[j]);
            float* dst = v_combined + (size_t)cid * kNG;
            // one atomic instruction for all three sums: q1's and q2's row totals
            // move from lane 15 of each row to lanes 14 and 13 (DPP row_shl),
            // so lanes 13-15 of a row add to three distinct words of the row
            const float q1s = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(q1), 0x101, 0xF, 0xF, true));
            const float q2s = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(q2), 0x102, 0xF, 0xF, true));
            const uint32_t r = lane & 15u;
            if (r >= 13u) {
                const uint32_t row = lane >> 4;
                const uint32_t k = (row & 1u) * 2u + (row >> 1);
                const bool want = DEPTH ? (k == 0u || (k == 1u && REFINE) || k == 2u) : (k == 0u || (row == 2u && REFINE));
                const uint32_t off = r == 15u ? k : r == 14u ? 4u + k : (DEPTH ? 8u + k : 8u + (row >> 1));
                const float val = r == 15u ? q0 : r == 14u ? q1s : q2s;
                if (r != 13u || want) unsafeAtomicAdd(dst + off, val);
            }
            wave_live = __ballot(sw > 1.0e-4f) != 0ull;
            if (!wave_live) break;
        }
        wave_lds_fence();
    }
}

void launch_rasterize_backward(bh_ctx* ctx, uint32_t img_w, uint32_t img_h, uint32_t tile_bw, uint32_t tile_bh,
                               const float* bg, uint32_t num_visible, const float* out_img, const float* projected, const uint32_t* cgids,
                               const uint32_t* offsets, const float* v_output, uint32_t flags,
                               const uint32_t* row_of, const uint32_t* order, float* v_combined) {
    const uint32_t num_tiles = tile_bw * tile_bh;
    if (num_tiles == 0 || num_visible == 0) return;
    const bool smooth = (flags & BH_FLAG_SMOOTH_CUTOFF) != 0;
    const bool refine = (flags & BH_FLAG_REFINE_WEIGHT) != 0;
    const bool depth = (flags & BH_FLAG_RENDER_DEPTH) != 0;
    const bool fine = (flags & BH_FLAG_TILE_16X8) != 0;
    const uint32_t groups = div_up(num_tiles, 8) * (fine ? 16u : 32u);
    KernelTimer t(ctx, "rasterize_backward");
#define BH_RB_T(S, R, D, T)                                                                                      \
    launch(ctx, rasterize_backward_kernel<S, R, D, T>, dim3(groups), dim3(64), 0u, img_w, img_h, tile_bw, num_tiles,   \
           bg[0], bg[1], bg[2], num_visible, out_img, projected, cgids, offsets, v_output, row_of, order, v_combined)
#define BH_RB(S, R, D) \
    do {               \
        if (fine)      \
            BH_RB_T(S, R, D, 8); \
        else           \
            BH_RB_T(S, R, D, 16); \
    } while (0)
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
#undef BH_RB_T
#undef BH_RB
}

// ---- fused rasterize backward from the forward's record ----------------------------

// The fused backward (bh_render_backward) reads the pairs the forward recorded
// (bh_splat_record.h) instead of replaying the forward's decisions: per 8x8
// block it visits only splats some pixel blended, and a pixel takes part only
// where its own bit is set, so no cutoff test is evaluated.  The per-pair
// arithmetic is the reference's (rasterize_backwards.rs:308-441), rearranged
// so that every factor that is constant over a splat is applied once, after
// the sum over the block's pixels, instead of once per pixel:
//   * alpha and transmittance exactly as the forward computed them (the
//     power in base 2 from the same scaled conic, the same exponential, no
//     contraction): the remaining colour below is the forward's final colour
//     minus these contributions, and deep in a stack it is a small difference
//     of nearly equal numbers, which an alpha off by an ulp would make
//     inconsistent (with the hardware exp2, a few ulp from the forward's
//     Gaussian, config 2's clustered scene put a scale gradient at three
//     times its tolerance);
//   * the remaining colour S enters the gradient only through the dot product
//     S . v_out, so a pixel carries that one number (D = S . v_out, updated as
//     D -= vis (c . v_out)) instead of the three channels of S;
//   * the 2D-mean gradient v_sigma (C d) is linear in the conic, so the block
//     sums v_sigma dx and v_sigma dy and the conic multiplies the two sums;
//     the conic lanes sum v_sigma dx dx, dx dy, dy dy and take their factor
//     0.5 after the sum; the colour lanes sum vis v_out and take the colour
//     gates (v_rgb only where c >= 0) after the sum;
//   * the refine weight |(W vx, H vy)| / A is not linear and stays per pixel.
// The gradient-only products use FMA contraction.
//
// A splat's K gradient sums are formed through LDS: every lane writes its K
// values into rows of 64 (one row per sum) of a slot, and once three splats
// are queued (two where K = 11: the rows of three slots must fit the wave's
// 32 row pairs), two lanes per row sum its halves (a float4 loop) and one
// lane per row applies the splat's factor and adds the total to the splat's
// gradient row in HBM: about one VALU add per value and one atomic
// instruction per three splats.  A slot's rows start at an even row, so its
// two mean rows lie in one lane quad and a quad permute brings each the
// other's total.
template <bool SMOOTH, bool REFINE, bool DEPTH, int TH>
__global__ __launch_bounds__(64) void rasterize_backward_recorded_kernel(
    uint32_t img_w, uint32_t img_h, uint32_t tile_bw, uint32_t num_tiles, float bg_r, float bg_g, float bg_b,
    uint32_t num_visible, const float* __restrict__ out_img, const float* __restrict__ projected,
    const uint32_t* __restrict__ cgids, const uint32_t* __restrict__ off_pre, SplatRecord rec,
    const float* __restrict__ v_output, const uint32_t* __restrict__ row_of, const uint32_t* __restrict__ order,
    float* __restrict__ v_rows, FillRanges fill, uint32_t fill_slots, uint32_t all_slots) {
    constexpr uint32_t CH = DEPTH ? 5u : 4u;
    constexpr uint32_t BPT = 2u * (uint32_t)TH / 8u;
    // sums per splat: v_sigma dx, v_sigma dy, v_sigma dx dx, v_sigma dx dy,
    // v_sigma dy dy, vis v_r, vis v_g, vis v_b, the opacity lane, (refine), (depth)
    constexpr int K = 9 + (REFINE ? 1 : 0) + (DEPTH ? 1 : 0);
    constexpr int KP = (K + 1) & ~1;  // rows per slot (even)
    // slots summed per flush: three where their rows fit the 32 row pairs of
    // a wave (K <= 10), else two
    constexpr int NS = 3 * KP <= 32 ? 3 : 2;
    constexpr int R = NS * KP;  // rows in use
    static_assert(R <= 32, "flush geometry: at most 32 rows, two lanes each");
    // the conic from its scaled form (bh_conic_log2): c00 = 2 ln2 a,
    // c01 = ln2 b, c11 = 2 ln2 c
    constexpr float kLn2 = 0.69314718055994530942f;
    constexpr float kTwoLn2 = 1.38629436111989061883f;
    // the batch's candidates (a batch of BATCH candidates; a smaller batch
    // takes less LDS, so more blocks fit a CU)
    constexpr uint32_t BATCH = BH_BWD_BATCH;
    static_assert(BATCH == 32 || BATCH == 64, "batch of 32 or 64 candidates");
    __shared__ float4 s_geo[BATCH];   // x, y, scaled conic a, b (bh_conic_log2)
    __shared__ float4 s_op[BATCH];    // scaled conic c, opacity, max(r, 0), max(g, 0)
    // max(b, 0) (bits), colour gates (bit c where channel c >= 0), gradient
    // row (global id): the candidate's three 16-byte records share one
    // address
    __shared__ uint4 s_aux[BATCH];
    // R rows of 64 floats, lane l's value in column l (conflict-free
    // stores); the summing lanes' reads are spread over the banks by their
    // order (below)
    constexpr int RS = 64;  // row stride in floats
    __shared__ float4 s_red4[R * RS / 4];
    float* s_red = reinterpret_cast<float*>(s_red4);

    // fill_slots of the all_slots slots of 8 workgroups (one per XCD) zero
    // the fill ranges, spread evenly among the blend's: slot s is a fill
    // slot where floor((s + 1) F / T) > floor(s F / T), the fill slot
    // floor(s F / T), else blend slot s - floor(s F / T)
    uint32_t g = blockIdx.x;
    if (fill_slots) {
        const uint32_t s = g >> 3;
        const uint32_t f0 = (uint32_t)((uint64_t)s * fill_slots / all_slots);
        const uint32_t f1 = (uint32_t)((uint64_t)(s + 1u) * fill_slots / all_slots);
        if (f1 > f0) {
            fill_ranges_strided<true>(fill, (uint64_t)(f0 * 8u + (g & 7u)) * 64u + threadIdx.x,
                                      (uint64_t)fill_slots * 512u);
            return;
        }
        g = ((s - f0) << 3) | (g & 7u);
    }
    uint32_t tile, blk;
    block_of_workgroup<TH>(g, tile, blk);
    if (tile >= num_tiles) return;
    if (order)
        tile = order[tile];
    else if (rec.order.list) {
        // the order the forward blend recorded (tiles some pixel blended)
        tile = ordered_tile(tile, rec.order.count, rec.order.list, num_tiles);
        if (tile >= num_tiles) return;
    }
    const uint32_t lo = off_pre[2 * tile], hi = off_pre[2 * tile + 1];
    const uint32_t end = rec.block_end[tile * BPT + blk];
    if (end <= lo) return;
    const uint32_t lane = threadIdx.x;
    const uint32_t ox = (tile % tile_bw) * 16u + (blk & 1u) * 8u;
    const uint32_t oy = (tile / tile_bw) * (uint32_t)TH + (blk >> 1) * 8u;
    const uint32_t px = ox + (lane & 7u), py = oy + (lane >> 3);
    const bool inside = px < img_w && py < img_h;
    const float pcx = (float)px + 0.5f, pcy = (float)py + 0.5f;

    // transmittance and D = (final colour minus background pre-roll) . v_out
    // (rasterize_backwards.rs:193-250)
    float sw = 0.0f, dsum = 0.0f;
    float vox = 0.0f, voy = 0.0f, voz = 0.0f, vow = 0.0f, vod = 0.0f, final_a = 0.0f;
    if (inside) {
        const size_t pix = (size_t)py * img_w + px;
        const float* o = out_img + pix * CH;
        const float* vo = v_output + pix * CH;
        final_a = o[3];
        const float t_final = 1.0f - final_a;
        const float sx = o[0] - t_final * bg_r;
        const float sy = o[1] - t_final * bg_g;
        const float sz = o[2] - t_final * bg_b;
        sw = 1.0f;
        vox = vo[0];
        voy = vo[1];
        voz = vo[2];
        vow = (vo[3] - (bg_r * vox + bg_g * voy + bg_b * voz)) * t_final;
        if (DEPTH) vod = vo[4];
        dsum = sx * vox + sy * voy + sz * voz;
    }
    // long blocks first (work sits in few tiles; see the replay kernel above)
    const uint32_t len = end - lo;
    if (len >= 256u)
        __builtin_amdgcn_s_setprio(3);
    else if (len >= 128u)
        __builtin_amdgcn_s_setprio(2);
    else if (len >= 64u)
        __builtin_amdgcn_s_setprio(1);
    const float wf = (float)img_w, hf = (float)img_h;
    // the refine weight |(W vx, H vy)| / A with (vx, vy) = v_sigma ln2 (gx, gy)
    const float refine_scale = kLn2 * __builtin_amdgcn_rcpf(bh_maxf(final_a, 1.0e-5f));
    const size_t rbase = record_base<BPT>(blk, lo, hi) - lo;
    // where this lane's value goes in a row; the row and half a summing lane
    // sums, and what multiplies its total: its own total times c00 (a slot's
    // v_sigma dx row), c11 (its v_sigma dy row), 0.5 (the dx dx and dy dy
    // rows), the colour gate (a colour row) or 1, plus the quad partner row's
    // total times c01 (the two mean rows)
    // byte offsets of this lane's column in rows 0, 4 and 8 of each slot: a
    // row store's offset from them fits the 8-bit dword offsets of paired
    // LDS stores (rows 64 floats apart); kept in registers (opaque to the
    // compiler, which would otherwise rebuild them with an add per store pair)
    uint32_t wbase[NS][3];
#pragma unroll
    for (int sl = 0; sl < NS; ++sl)
#pragma unroll
        for (int gr = 0; gr < 3; ++gr) {
            wbase[sl][gr] = ((uint32_t)(sl * KP + 4 * gr) * RS + lane) * 4u;
            __asm__ volatile("" : "+v"(wbase[sl][gr]));
        }
    const uint32_t frow = lane >> 1, fq = lane & 1u;
    const uint32_t fslot = frow / (uint32_t)KP, fk = frow % (uint32_t)KP;
    // the byte offsets of the eight float4 groups of its row's half a summing
    // lane reads, group 8 h + ((q + r + 4 h) mod 8) at step q (row r, half
    // h): the 16 lanes of a read phase (8 rows, both halves) read 16
    // distinct groups of four banks, the 8 of a narrower phase (4 rows)
    // groups distinct modulo 8 (in registers, computed once; the lanes past
    // the R rows read row R - 1 and discard it)
    uint32_t faddr[8];
    const uint32_t frow_c = min(frow, (uint32_t)R - 1u);
#pragma unroll
    for (uint32_t q = 0; q < 8u; ++q) {
        faddr[q] = (frow_c * (uint32_t)RS + 4u * (8u * fq + ((q + frow_c + 4u * fq) & 7u))) * 4u;
        __asm__ volatile("" : "+v"(faddr[q]));
    }
    // the factors as weights of the staged a, c, b and a constant (exact
    // products by 0: a splat's conic is finite)
    const float f00 = fk == 0u ? kTwoLn2 : 0.0f, f11 = fk == 1u ? kTwoLn2 : 0.0f;
    const float f01 = fk < 2u ? kLn2 : 0.0f;
    const uint32_t fgate = fk >= 5u && fk <= 7u ? 1u << (fk - 5u) : 0u;
    const float fconst = fk < 2u || fgate ? 0.0f : ((fk == 2u || fk == 4u) ? 0.5f : 1.0f);
    const uint32_t fdst = fk < 9u ? fk : (fk == 9u && REFINE ? 9u : 10u);
    const bool fwriter = fq == 0u;

    // Sums the queued slots' rows, applies each splat's factors and adds the
    // totals to the splats' gradient rows.  A slot holds the candidate index
    // of its splat in the current batch (the staging arrays outlive the
    // slot: pending slots are flushed before the next batch is staged).
    uint32_t slot_js = 0;  // queued candidate indices: slot s in bits 6 s to 6 s + 5
    auto flush = [&](uint32_t nslots) {
        wave_lds_fence();
        const bool active = fslot < nslots && fk < (uint32_t)K;
        // every lane reads its slot's splat (a valid candidate index either way)
        const uint32_t js = (slot_js >> (6u * fslot)) & 63u;
        const float4 geo = s_geo[js];
        const float c11 = s_op[js].x;
        const uint4 aux = s_aux[js];
        // all eight reads of the row half in flight before the first add
        // (every lane reads; an inactive lane's sum is discarded)
        float4 rv[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
            rv[q] = *reinterpret_cast<const float4*>(reinterpret_cast<const char*>(s_red4) + faddr[q]);
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t gates = aux.y, row = aux.z;
        float acc = (rv[0].x + rv[0].y) + (rv[0].z + rv[0].w);
#pragma unroll
        for (int q = 1; q < 8; ++q) acc += (rv[q].x + rv[q].y) + (rv[q].z + rv[q].w);
        acc = active ? acc : 0.0f;
        acc = dpp_add<0xB1>(acc);  // quad_perm [1, 0, 3, 2]: the row's two halves
        // quad_perm [2, 3, 0, 1]: the other row of the lane quad (a slot's
        // v_sigma dx row for its v_sigma dy row and back)
        const float other = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0x4E, 0xF, 0xF, true));
        const float fg = (gates & fgate) ? 1.0f : 0.0f;
        const float fself = f00 * geo.z + (f11 * c11 + (fconst + fg));
        const float v = fself * acc + (f01 * geo.w) * other;
        if (active && fwriter && v != 0.0f) unsafeAtomicAdd(v_rows + (size_t)row * kNG + fdst, v);
        wave_lds_fence();
    };

    // lane j of a batch: the pixels that blended candidate b + j, and its id.
    // Every load below is unconditional (indices clamped into the block's
    // range), so the compiler's wait counts are exact: a batch's ids are read
    // right after the previous batch's rows and arrive while it is evaluated.
    const uint32_t last = end - 1u;
    const uint32_t bl = lane & (BATCH - 1u);  // lanes >= BATCH repeat a load and stage nothing
    uint2 mask_n = rec.masks[rbase + min(lo + bl, last)];
    uint32_t cid_n = cgids[min(lo + bl, last)];
    for (uint32_t b = lo; b < end; b += BATCH) {
        const uint2 mask = lane < BATCH && b + lane <= last ? mask_n : make_uint2(0u, 0u);
        const uint32_t c = min(cid_n, num_visible - 1u);
        const float2* prow = reinterpret_cast<const float2*>(projected + (size_t)c * 10);
        const float2 r0 = prow[0], r1 = prow[1], r2 = prow[2], r3 = prow[3], r4 = prow[4];
        const uint32_t grow = row_of[c];
        // keep the issue order: these rows, then the next batch's ids, then
        // their uses (the wait for the rows must not cover the ids)
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t bn = min(b + BATCH + bl, last);
        mask_n = rec.masks[rbase + bn];
        cid_n = cgids[bn];
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        const bool any = (mask.x | mask.y) != 0u;
        // every lane stages (a candidate without pixels is never read; lanes
        // bl and bl + 32 of a 32-candidate batch store the same values), so
        // the row loads stay ahead of the barrier above
        float ka, kb, kc;
        bh_conic_log2(r1.x, r1.y, r2.x, &ka, &kb, &kc);
        s_geo[bl] = make_float4(r0.x, r0.y, ka, kb);
        s_op[bl] = make_float4(kc, r2.y, bh_maxf(r3.x, 0.0f), bh_maxf(r3.y, 0.0f));
        s_aux[bl] = make_uint4(__float_as_uint(bh_maxf(r4.x, 0.0f)),
                               (r3.x >= 0.0f ? 1u : 0u) | (r3.y >= 0.0f ? 2u : 0u) | (r4.x >= 0.0f ? 4u : 0u), grow, 0u);
        uint64_t todo = __builtin_amdgcn_ballot_w64(any);
        wave_lds_fence();
        // One candidate: its gradient values into slot SLOT.  The loop below
        // reads the next candidate's parameters while the current one is
        // evaluated, two register sets in turn, and sums the slots once all
        // NS are filled.
        auto eval_one = [&](auto slot, uint32_t j, const float4& geo, const float4& op, float cb) {
            constexpr uint32_t SLOT = decltype(slot)::value;
            // candidate j's mask, read into scalar registers, is the lane condition
            // (readlane returns a signed int: widen through uint32_t, never by
            // sign extension)
            const uint64_t mj = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(mask.y, j) << 32) |
                                (uint64_t)(uint32_t)__builtin_amdgcn_readlane(mask.x, j);
            const bool contrib = __builtin_amdgcn_inverse_ballot_w64(mj);
            const float ka = geo.z, kb = geo.w, kc = op.x, opac = op.y;
            const float cr = op.z, cg = op.w;
            // d = mean - pixel centre; the forward's power and Gaussian, bit
            // for bit
            const float dx = geo.x - pcx, dy = geo.y - pcy;
            const float gauss = bh_exp2_neg(-bh_power_log2(ka, kb, kc, dx, dy));
            const float og = opac * gauss;
            const float alpha = bh_minf(0.999f, og);
            float w = 1.0f, ae = alpha;
            if (SMOOTH) {
                w = cutoff_weight(alpha);
                ae = alpha * w;
            }
            ae = contrib ? ae : 0.0f;
            const float vis = ae * sw;
            const float one_minus = 1.0f - ae;
            // position, conic, opacity and refine lanes: contributing and
            // unclamped pairs (o G <= 0.999); the selects sit on v_sigma and on
            // the opacity lane, so other lanes' values never reach a sum
            const bool gate = contrib && og <= 0.999f;
            float g[K];
            {
#pragma clang fp contract(fast)
                // gradient-only arithmetic: products and sums fuse into FMAs
                const float ra = __builtin_amdgcn_rcpf(one_minus);
                const float cv = cr * vox + cg * voy + cb * voz;
                // ((T c - S) . v_out + v_ow) / (1 - alpha)
                const float v_ae = (sw * cv - dsum + vow) * ra;
                const float v_alpha = SMOOTH ? v_ae * (w + alpha * cutoff_weight_deriv(alpha)) : v_ae;
                const float v_sigma = gate ? -alpha * v_alpha : 0.0f;
                const float t = v_sigma * dx, u = v_sigma * dy;
                g[0] = t;
                g[1] = u;
                g[2] = t * dx;
                g[3] = t * dy;
                g[4] = u * dy;
                g[5] = vis * vox;
                g[6] = vis * voy;
                g[7] = vis * voz;
                g[8] = gate ? v_alpha * gauss : 0.0f;
                if constexpr (REFINE) {
                    // (vx, vy) = v_sigma C d = v_sigma ln2 (gx, gy) with
                    // gx = 2 a dx + b dy = q + a dx (q = a dx + b dy of the
                    // power) and gy = b dx + 2 c dy
                    const float q = bh_fmaf(ka, dx, kb * dy);
                    const float cdy = kc * dy;
                    const float gx = bh_fmaf(ka, dx, q), gy = bh_fmaf(kb, dx, cdy + cdy);
                    const float ax = wf * gx, ay = hf * gy;
                    g[9] = (__builtin_fabsf(v_sigma) * refine_scale) * __builtin_amdgcn_sqrtf(ax * ax + ay * ay);
                }
                if constexpr (DEPTH) g[K - 1] = vis * vod;
                // the reference's state update (rasterize_backwards.rs:356-358,
                // 432-435) as D -= vis (c . v_out)
                dsum = dsum - vis * cv;
            }
            sw = sw * one_minus;
#pragma unroll
            for (int k = 0; k < K; ++k)
                *reinterpret_cast<float*>(reinterpret_cast<char*>(s_red) + wbase[SLOT][k >> 2] + (k & 3) * RS * 4) = g[k];
            if (SLOT == 0u)
                slot_js = j;
            else
                slot_js |= j << (6u * SLOT);
        };
        using Slot0 = std::integral_constant<uint32_t, 0u>;
        using Slot1 = std::integral_constant<uint32_t, 1u>;
        using Slot2 = std::integral_constant<uint32_t, 2u>;
        // reads the next candidate of the batch into a register set; false
        // (and the set untouched) when none is left
        auto next = [&](uint32_t& j, float4& geo, float4& op, float& cb) -> bool {
            if (todo == 0ull) return false;
            j = (uint32_t)__builtin_ctzll(todo);
            todo &= todo - 1ull;
            geo = s_geo[j];
            op = s_op[j];
            cb = __uint_as_float(s_aux[j].x);
            return true;
        };
        uint32_t pend = 0u;  // slots filled since the last flush
        uint32_t ja = 0u, jb = 0u;
        float4 geoa, opa, geob, opb;
        float cba = 0.0f, cbb = 0.0f;
        if (next(ja, geoa, opa, cba)) {
            if constexpr (NS == 2) {
                while (true) {
                    const bool hb = next(jb, geob, opb, cbb);
                    eval_one(Slot0{}, ja, geoa, opa, cba);
                    if (!hb) { pend = 1u; break; }
                    const bool ha = next(ja, geoa, opa, cba);
                    eval_one(Slot1{}, jb, geob, opb, cbb);
                    flush(2u);
                    if (!ha) break;
                }
            } else {
                // slots 0, 1, 2 from sets a, b, a, then b, a, b
                while (true) {
                    bool hb = next(jb, geob, opb, cbb);
                    eval_one(Slot0{}, ja, geoa, opa, cba);
                    if (!hb) { pend = 1u; break; }
                    bool ha = next(ja, geoa, opa, cba);
                    eval_one(Slot1{}, jb, geob, opb, cbb);
                    if (!ha) { pend = 2u; break; }
                    hb = next(jb, geob, opb, cbb);
                    eval_one(Slot2{}, ja, geoa, opa, cba);
                    flush(3u);
                    if (!hb) break;
                    ha = next(ja, geoa, opa, cba);
                    eval_one(Slot0{}, jb, geob, opb, cbb);
                    if (!ha) { pend = 1u; break; }
                    hb = next(jb, geob, opb, cbb);
                    eval_one(Slot1{}, ja, geoa, opa, cba);
                    if (!hb) { pend = 2u; break; }
                    ha = next(ja, geoa, opa, cba);
                    eval_one(Slot2{}, jb, geob, opb, cbb);
                    flush(3u);
                    if (!ha) break;
                }
            }
        }
        // sum the rest before the next batch overwrites the staging arrays
        // the slots refer to
        if (pend) flush(pend);
        wave_lds_fence();
    }
}


template <bool S, bool R, bool D, int T>
static void launch_recorded_t(bh_ctx* ctx, uint32_t groups, uint32_t img_w, uint32_t img_h, uint32_t tile_bw,
                              uint32_t num_tiles, const float* bg, uint32_t num_visible, const float* out_img,
                              const float* projected, const uint32_t* cgids, const uint32_t* off_pre,
                              const SplatRecord& rec, const float* v_output, const uint32_t* row_of,
                              const uint32_t* order, float* v_rows, const FillRanges& fill, uint32_t fill_slots) {
    const uint32_t all_slots = groups / 8u + fill_slots;
    launch(ctx, rasterize_backward_recorded_kernel<S, R, D, T>, dim3(all_slots * 8u), dim3(64), 0u, img_w, img_h,
           tile_bw, num_tiles, bg[0], bg[1], bg[2], num_visible, out_img, projected, cgids, off_pre, rec, v_output,
           row_of, order, v_rows, fill, fill_slots, all_slots);
}

// 16-byte stores per lane of a workgroup that zeroes the fill ranges inside the
// rasterize backward (about 64 KiB a workgroup)
#ifndef BH_FUSED_FILL_ITERS
#define BH_FUSED_FILL_ITERS 64
#endif
constexpr uint64_t kFusedFillIters = BH_FUSED_FILL_ITERS;

bool launch_rasterize_backward_recorded(bh_ctx* ctx, uint32_t img_w, uint32_t img_h, uint32_t tile_bw,
                                        uint32_t tile_bh, const float* bg, uint32_t num_visible, const float* out_img,
                                        const float* projected, const uint32_t* cgids, const uint32_t* off_pre,
                                        const SplatRecord& rec, const float* v_output, uint32_t flags,
                                        const uint32_t* row_of, const uint32_t* order, float* v_rows,
                                        const FillRange* zero, int zero_k) {
    const uint32_t num_tiles = tile_bw * tile_bh;
    if (num_tiles == 0 || num_visible == 0 || !rec.masks) return false;
    FillRanges fill{};
    uint64_t quads = 0;
    const bool fits = zero_k <= kMaxFillRanges;  // else the caller zeroes them
    for (int j = 0; fits && j < zero_k; j++) {
        if (zero[j].count == 0 || !zero[j].p) continue;
        fill.r[fill.k++] = zero[j];
        quads += div_up(zero[j].count, (uint64_t)4);
    }
    // a fill workgroup stores about kFusedFillIters 16-byte words per lane
    const uint32_t fill_slots =
        (uint32_t)std::min<uint64_t>(div_up(quads, (uint64_t)512 * kFusedFillIters), 1u << 20);
    const bool smooth = (flags & BH_FLAG_SMOOTH_CUTOFF) != 0;
    const bool refine = (flags & BH_FLAG_REFINE_WEIGHT) != 0;
    const bool depth = (flags & BH_FLAG_RENDER_DEPTH) != 0;
    const bool fine = (flags & BH_FLAG_TILE_16X8) != 0;
    const uint32_t groups = div_up(num_tiles, 8) * (fine ? 16u : 32u);
    KernelTimer t(ctx, "rasterize_backward");
#define BH_RBR_T(S, R, D, T)                                                                                      \
    launch_recorded_t<S, R, D, T>(ctx, groups, img_w, img_h, tile_bw, num_tiles, bg, num_visible, out_img,       \
                                  projected, cgids, off_pre, rec, v_output, row_of, order, v_rows, fill, fill_slots)
#define BH_RBR(S, R, D)              \
    do {                             \
        if (fine)                    \
            BH_RBR_T(S, R, D, 8);    \
        else                         \
            BH_RBR_T(S, R, D, 16);   \
    } while (0)
    if (smooth) {
        if (refine) {
            if (depth) BH_RBR(true, true, true); else BH_RBR(true, true, false);
        } else {
            if (depth) BH_RBR(true, false, true); else BH_RBR(true, false, false);
        }
    } else {
        if (refine) {
            if (depth) BH_RBR(false, true, true); else BH_RBR(false, true, false);
        } else {
            if (depth) BH_RBR(false, false, true); else BH_RBR(false, false, false);
        }
    }
#undef BH_RBR
#undef BH_RBR_T
    return fits;
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
    launch(ctx, invert_permutation_kernel, dim3(div_up(num_visible, 256)), dim3(256), 0u, gfc, num_visible, n,
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

// The projection VJP of one splat with gradient lanes rg, written to its dense
// rows (project_backwards.rs:101-263).
template <int DEG, bool MIP, int CAM>
__device__ void project_backward_one(const bh_project_uniforms& u, const float* __restrict__ transforms,
                                     const float* __restrict__ sh, const float* __restrict__ raw_opac, uint32_t gid,
                                     const float* rg, float* __restrict__ v_transforms, float* __restrict__ v_coeffs,
                                     float* __restrict__ v_raw_opac, float* __restrict__ v_refine) {
    constexpr int NC = (DEG + 1) * (DEG + 1);
    float2* vt = reinterpret_cast<float2*>(v_transforms + (size_t)gid * 10);
    float* vc_row = v_coeffs + (size_t)gid * (3 * NC);
    float vcoef[3 * NC];
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
    const S2 raw_cov = calc_cov2d<CAM>(u, sc, q, mean_c);
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
    const M23 J = jacobian<CAM>(u, mean_c);
    V3 v_mean_c = projection_vjp<CAM>(u, J, mean_c, cov_c, v_cov2d, v2(rg[0], rg[1]));
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

// Zero-fills floats [begin, end) of p with the block's threads, 16 bytes per
// store where p + begin is 16-byte aligned.
__device__ __forceinline__ void block_zero(float* __restrict__ p, size_t begin, size_t end) {
    float* q = p + begin;
    const size_t count = end - begin;
    size_t head = 0;
    if ((reinterpret_cast<uintptr_t>(q) & 15u) == 0u) {
        float4* q4 = reinterpret_cast<float4*>(q);
        head = count / 4u * 4u;
        for (size_t i = threadIdx.x; i < count / 4u; i += blockDim.x) q4[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    for (size_t i = head + threadIdx.x; i < count; i += blockDim.x) q[i] = 0.0f;
}

// Each block owns PB_SPLATS consecutive global ids.  It reads their gradient
// lanes and compacts the ids that have gradient into an LDS list, zero-fills
// its dense output rows with contiguous stores (rows without gradient --
// culled splats, splats behind saturated pixels -- are most rows), and then
// runs the VJP over the list with every lane busy, overwriting those rows.
// One block covers four times the ids one pass of its threads reads, so the
// VJP's latency (its rows' loads, then a dependent chain) is paid once per
// 1024 ids and ~1000 blocks are all resident at once.  cfg == nullptr:
// v_combined holds one row per global id (the fused backward), else
// v_combined[cfg[gid]].
constexpr uint32_t PB_SPLATS = 1024u;

template <int DEG, bool MIP, int CAM>
__global__ __launch_bounds__(256) void project_backward_kernel(
    bh_project_uniforms u, const float* __restrict__ transforms, const float* __restrict__ sh,
    const float* __restrict__ raw_opac, const uint32_t* __restrict__ cfg, uint32_t n,
    const float* __restrict__ v_combined, float* __restrict__ v_transforms, float* __restrict__ v_coeffs,
    float* __restrict__ v_raw_opac, float* __restrict__ v_refine, bool zeroed) {
    constexpr int NC = (DEG + 1) * (DEG + 1);
    constexpr uint32_t PASSES = PB_SPLATS / 256u;
    __shared__ uint32_t s_gid[PB_SPLATS];
    __shared__ uint32_t s_row[PB_SPLATS];
    __shared__ uint32_t s_count[PASSES][4];
    const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
    const size_t g0 = (size_t)blockIdx.x * PB_SPLATS, g1 = min<size_t>(g0 + PB_SPLATS, n);
    // every pass's lanes read first (the loads of all passes in flight
    // together), then the ballots
    uint32_t cs[PASSES];
    bool any[PASSES];
#pragma unroll
    for (uint32_t p = 0; p < PASSES; ++p) {
        const size_t gid = g0 + p * 256u + t;
        cs[p] = gid < n ? (cfg ? cfg[gid] : (uint32_t)gid) : 0xFFFFFFFFu;
    }
    // every lane of every pass loaded unconditionally (an id without a row
    // reads row 0 and is discarded), then tested with one OR: a short-circuit
    // test makes each load wait for the one before it, eleven memory round
    // trips per pass for a splat without gradient (most of them)
#pragma unroll
    for (uint32_t p = 0; p < PASSES; ++p) {
        const bool have = cs[p] != 0xFFFFFFFFu;
        const float* src = v_combined + (size_t)(have ? cs[p] : 0u) * 11;
        uint32_t bits = 0u;
#pragma unroll
        for (int k = 0; k < 11; k++) bits |= __float_as_uint(src[k]) << 1;  // any lane other than +-0 (NaN counts)
        any[p] = have && bits != 0u;
    }
    uint64_t masks[PASSES];
#pragma unroll
    for (uint32_t p = 0; p < PASSES; ++p) {
        masks[p] = __ballot(any[p]);
        if (lane == 0) s_count[p][wave] = (uint32_t)__popcll(masks[p]);
    }
    if (!zeroed) {  // (uniform) else the caller zeroed the rows
        block_zero(v_transforms, g0 * 10u, g1 * 10u);
        block_zero(v_coeffs, g0 * (3u * NC), g1 * (3u * NC));
        block_zero(v_raw_opac, g0, g1);
        block_zero(v_refine, g0, g1);
    }
    __syncthreads();
    // compact the ids with gradient: list order = pass, wave, lane
    uint32_t base = 0;
#pragma unroll
    for (uint32_t p = 0; p < PASSES; ++p) {
        uint32_t before = base;
#pragma unroll
        for (uint32_t w = 0; w < 4u; w++) {
            before += w < wave ? s_count[p][w] : 0u;
            base += s_count[p][w];
        }
        if (any[p]) {
            const uint32_t slot = before + lanes_below(masks[p]);
            s_gid[slot] = (uint32_t)(g0 + p * 256u + t);
            s_row[slot] = cs[p];
        }
    }
    const uint32_t total = base;
    // the zero-fill's stores precede the list's stores to the same rows
    // (the barrier's workgroup release), and the list is complete
    __syncthreads();
    for (uint32_t i = t; i < total; i += 256u) {
        const uint32_t g = s_gid[i];
        const float* src = v_combined + (size_t)s_row[i] * 11;
        float rg[11];
#pragma unroll
        for (int k = 0; k < 11; k++) rg[k] = src[k];
        project_backward_one<DEG, MIP, CAM>(u, transforms, sh, raw_opac, g, rg, v_transforms, v_coeffs,
                                            v_raw_opac, v_refine);
    }
}

template <int DEG, bool MIP>
static void launch_pb_cam(bh_ctx* ctx, const bh_project_uniforms& u, const float* transforms, const float* sh,
                          const float* raw_opac, const uint32_t* cfg, uint32_t n, const float* v_combined,
                          float* v_transforms, float* v_coeffs, float* v_raw_opac, float* v_refine, bool zeroed) {
    const uint32_t blocks = div_up(n, PB_SPLATS);
#define BH_PB(C)                                                                                                  \
    launch(ctx, project_backward_kernel<DEG, MIP, C>, dim3(blocks), dim3(256), 0u, u, transforms, sh, raw_opac, cfg,   \
           n, v_combined, v_transforms, v_coeffs, v_raw_opac, v_refine, zeroed)
    switch (u.camera_model) {
        case kCamKB4: BH_PB(kCamKB4); break;
        case kCamRT8: BH_PB(kCamRT8); break;
        case kCamTPF: BH_PB(kCamTPF); break;
        default: BH_PB(kCamPinhole); break;
    }
#undef BH_PB
}
template <int DEG>
static void launch_pb(bh_ctx* ctx, bool mip, const bh_project_uniforms& u, const float* transforms, const float* sh,
                      const float* raw_opac, const uint32_t* cfg, uint32_t n, const float* v_combined,
                      float* v_transforms, float* v_coeffs, float* v_raw_opac, float* v_refine, bool zeroed) {
    if (mip)
        launch_pb_cam<DEG, true>(ctx, u, transforms, sh, raw_opac, cfg, n, v_combined, v_transforms, v_coeffs,
                                 v_raw_opac, v_refine, zeroed);
    else
        launch_pb_cam<DEG, false>(ctx, u, transforms, sh, raw_opac, cfg, n, v_combined, v_transforms, v_coeffs,
                                  v_raw_opac, v_refine, zeroed);
}
void launch_project_backward(bh_ctx* ctx, const bh_project_uniforms& u, const float* transforms, const float* sh,
                             const float* raw_opac, const uint32_t* cfg, uint32_t n, uint32_t sh_degree, bool mip,
                             const float* v_combined, float* v_transforms, float* v_coeffs, float* v_raw_opac,
                             float* v_refine, bool zeroed) {
    if (n == 0) return;
    KernelTimer t(ctx, "project_backward");
#define BH_PBD(D) \
    launch_pb<D>(ctx, mip, u, transforms, sh, raw_opac, cfg, n, v_combined, v_transforms, v_coeffs, v_raw_opac, v_refine, zeroed)
    switch (sh_degree) {
        case 0: BH_PBD(0); break;
        case 1: BH_PBD(1); break;
        case 2: BH_PBD(2); break;
        case 3: BH_PBD(3); break;
        default: BH_PBD(4); break;
    }
#undef BH_PBD
}

}  // namespace bh
