// bh_tile_walk.h — wave-cooperative walk over the tile bounding boxes of 64 splats.
//
// The reference tests a splat's bounding-box tiles in a loop run by the
// splat's own thread (project_forward.rs:105-118, map_gaussians.rs:56-79), so
// a wave waits for its largest splat while most lanes idle.  Here a wave
// flattens the (splat, bbox tile) items of its 64 splats into one list, in
// splat order and, within a splat, in the reference's row-major tile order,
// and tests 64 items per step.  Per step, every lane finds the splat that owns
// its item (a scatter of segment starts into LDS and a max-scan), fetches that
// splat's record from LDS and evaluates the same tile predicate.  The lane
// holding a splat's last item records the wave's running count of passing
// items through it, and a splat's hits are the difference of two such
// prefixes.  Passing items come out in exactly the order the per-splat loops
// would emit them, so the map kernel writes them contiguously.
#pragma once

#include "bh_splat_math.h"
#include "bh_wave.h"

namespace bh {

// One splat's walk record in LDS (64 bytes, four reads).
struct WalkRec {
    float4 a;  // mean x, mean y, conic c00, conic c01
    float4 b;  // conic c11, power threshold, 1 / bbox width, end item index (bits)
    uint4 c;   // bbox min_x, bbox min_y, bbox width, first item index
    float4 d;  // the predicate's divisors' reciprocals 1 / (16^2 c00), 1 / (TH^2 c11)
};

// RN(num / den) from y = RN(1 / den) for den > 0 and num < den (quotient
// below 1, so nothing overflows): q0 = RN(num y) is within an ulp of the
// quotient, the residual num - den q0 is exact in one fma, and RN(q0 + r y)
// is the correctly rounded quotient (Markstein's theorem for a correctly
// rounded reciprocal and a faithful first quotient; the quotient's
// correctly rounded value is what the reference's division gives).  Below the
// normal range the result can differ from the division in the last place of
// a subnormal, which the predicate then adds to a tile edge that absorbs it.
__device__ __forceinline__ float div_by_recip(float num, float den, float y) {
    const float q0 = num * y;
    const float r = __builtin_fmaf(-den, q0, num);
    return __builtin_fmaf(r, y, q0);
}

// Orders this wave's LDS writes before its later LDS reads as seen by the
// compiler: without it, a lane's read of a slot it wrote itself may be
// forwarded from its own store even when another lane of the wave overwrote
// the slot in between.  Wavefront scope: no instruction is emitted.
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// The power will_contribute (bh_splat_math.h) compares with the threshold,
// evaluated without branches: both edge quotients and the power at the
// clamped edge point are computed for every lane and the predicate's selects
// pick them, so `power <= pt` is the predicate's decision bit for bit (a splat
// whose mean lies in the tile gets -1, which passes).  Tile widths 16 and TH
// are exact differences of the tile's float edges for tile columns < 2^20.
template <int TH>
__device__ __forceinline__ float tile_power(uint32_t tx, uint32_t ty, V2 m, const S2& c, float rx, float ry) {
    const float min_x = (float)(tx * 16u), min_y = (float)(ty * (uint32_t)TH);
    const float max_x = min_x + 16.0f, max_y = min_y + (float)TH;
    const bool x_left = m.x < min_x, x_right = m.x > max_x;
    const bool in_x = !(x_left || x_right);
    const bool y_above = m.y < min_y, y_below = m.y > max_y;
    const bool in_y = !(y_above || y_below);
    const float corner_x = x_left ? min_x : max_x;
    const float corner_y = y_above ? min_y : max_y;
    const float dxf = x_left ? 16.0f : -16.0f;
    const float dyf = y_above ? (float)TH : -(float)TH;
    const float diff_x = m.x - corner_x;
    const float diff_y = m.y - corner_y;
    // the reference's quotients (dxf c00 dx + dxf c01 dy) / (dxf c00 dxf),
    // their divisors 16^2 c00 and TH^2 c11 for either sign of dxf, dyf; a
    // quotient at or above 1 clamps to 1 either way
    const float nx = dxf * c.c00 * diff_x + dxf * c.c01 * diff_y, dnx = dxf * c.c00 * dxf;
    const float ny = dyf * c.c01 * diff_x + dyf * c.c11 * diff_y, dny = dyf * c.c11 * dyf;
    const float qx = nx >= dnx ? 1.0f : bh_maxf(div_by_recip(nx, dnx, rx), 0.0f);
    const float qy = ny >= dny ? 1.0f : bh_maxf(div_by_recip(ny, dny, ry), 0.0f);
    const float tt_x = in_y ? 0.0f : qx;
    const float tt_y = in_x ? 0.0f : qy;
    const float px = corner_x + tt_x * dxf;
    const float py = corner_y + tt_y * dyf;
    const float power = calc_sigma(px, py, c, m.x, m.y);
    return (in_x && in_y) ? -1.0f : power;
}

// Items (bbox tiles) of a splat whose box is bb; zero for an empty box.
__device__ __forceinline__ uint32_t bbox_items(const TileBox& bb) {
    return (bb.max_x > bb.min_x && bb.max_y > bb.min_y) ? (bb.max_x - bb.min_x) * (bb.max_y - bb.min_y) : 0u;
}

// Cooperative walk of one wave over 16 x TH tiles.  Every lane of the wave must call it (it uses
// wave-wide DPP and ballots).  `items` is this lane's bbox tile count (0 for a
// culled or absent splat); m, conic, pt, bb describe its splat.  `rec`,
// `owner_slot` and `ends` are this wave's 64-entry LDS arrays.
//
// Returns the number of passing tiles of this lane's splat.  With WRITE, the
// passing items are stored at out_base + (passing items before it in walk
// order): tile id tx + ty * tile_bw into tile_ids (as TileT) and id_base +
// owner lane into ids, skipping positions >= out_end.
template <bool WRITE, int TH, typename TileT>
__device__ uint32_t wave_tile_walk(uint32_t lane, uint32_t items, V2 m, const S2& conic, float pt,
                                   const TileBox& bb, WalkRec* rec, uint32_t* owner_slot, uint32_t* ends,
                                   uint32_t tile_bw, uint32_t out_base, uint32_t out_end, uint32_t id_base,
                                   TileT* __restrict__ tile_ids, uint32_t* __restrict__ ids) {
    const uint32_t incl = wave_incl_add_u32(items);
    const uint32_t start = incl - items;
    const uint32_t total = __builtin_amdgcn_readlane(incl, 63);
    const uint32_t bw = bb.max_x - bb.min_x;
    rec[lane].a = make_float4(m.x, m.y, conic.c00, conic.c01);
    rec[lane].b = make_float4(conic.c11, pt, items ? 1.0f / (float)bw : 0.0f, __uint_as_float(incl));
    rec[lane].c = make_uint4(bb.min_x, bb.min_y, bw, start);
    rec[lane].d = make_float4(items ? 1.0f / (256.0f * conic.c00) : 0.0f,
                              items ? 1.0f / ((float)(TH * TH) * conic.c11) : 0.0f, 0.0f, 0.0f);
    ends[lane] = 0u;
    wave_lds_fence();
    uint32_t written = 0;  // passing items of earlier steps (wave uniform)
    for (uint32_t base = 0; base < total; base += 64u) {
        // owner of item base + lane: the splat with the largest start <= item
        owner_slot[lane] = 0u;
        const bool in_window = items != 0u && start < base + 64u && incl > base;
        if (in_window) owner_slot[start > base ? start - base : 0u] = lane + 1u;
        wave_lds_fence();
        const uint32_t owner = wave_incl_max_u32(owner_slot[lane]) - 1u;
        const uint32_t item = base + lane;
        const bool valid = item < total;
        const WalkRec r = rec[owner & 63u];
        // the owner's item prefix, read with the rest of its record (left to
        // itself the compiler reads it again inside the branch below: one
        // more LDS round trip per step)
        uint32_t r_incl = __float_as_uint(r.b.w);
        __asm__ volatile("" : "+v"(r_incl));
        const uint32_t local = item - r.c.w;
        // row = local / width, exactly, through the float reciprocal: with
        // w = width and 1/w rounded, (local + 0.5) / w lies at least 0.5 / w
        // from an integer and the two roundings move it by less than
        // (row + 1) 2^-23, below 0.5 / w while (row + 1) w < 2^22 (a box
        // holds at most tile_bw * tile_bh < 2^21 tiles: bh_render_forward
        // rejects larger images)
        const uint32_t row = (uint32_t)(((float)local + 0.5f) * r.b.z);
        const uint32_t col = local - __umul24(row, r.c.z);  // both factors and the product < 2^21
        const uint32_t tx = r.c.x + col, ty = r.c.y + row;
        // will_contribute as one comparison; the lane conditions stay wave masks
        const float power = tile_power<TH>(tx, ty, v2(r.a.x, r.a.y), S2{r.a.z, r.a.w, r.b.x}, r.d.x, r.d.y);
        const uint64_t pmask = __builtin_amdgcn_ballot_w64(power <= r.b.y) & __builtin_amdgcn_ballot_w64(valid);
        const bool pass = __builtin_amdgcn_inverse_ballot_w64(pmask);
        // the wave's passing items up to and including this one, kept at a
        // splat's last item
        const uint32_t below = lanes_below(pmask);
        if (valid && item + 1u == r_incl) ends[owner & 63u] = written + below + (pass ? 1u : 0u);
        if (WRITE && pass) {
            const uint32_t pos = out_base + written + below;
            if (pos < out_end) {
                tile_ids[pos] = (TileT)(tx + __umul24(ty, tile_bw));  // a tile id < 2^21
                ids[pos] = id_base + owner;
            }
        }
        written += (uint32_t)__popcll(pmask);
        wave_lds_fence();
    }
    // a splat without items takes the prefix of the splats before it
    const uint32_t through = wave_incl_max_u32(ends[lane]);
    owner_slot[lane] = through;
    wave_lds_fence();
    const uint32_t before = lane ? owner_slot[lane - 1u] : 0u;
    return through - before;
}

}  // namespace bh
