// raster.hip — tile offsets and the forward front-to-back blend for gfx950.
//
//   tile_offsets  [start, end) of each tile's run in the tile-sorted list
//                 (crates/brush-render/src/get_tile_offset.rs:10-62)
//   rasterize     one single-wave workgroup per 8x8 pixel block of a 16x16
//                 tile, one pixel per lane; each wave stages the tile's splats
//                 in LDS in batches of 64, keeps those that may touch its block
//                 (ballot of a conservative rectangle test) and stops when its
//                 64 pixels have saturated
//                 (crates/brush-render/src/kernels/rasterize.rs:24-200).
//
// With BWD_INFO the kernel also marks contributing splats visible — once per
// (splat, block) through a ballot instead of once per pixel — and shrinks each
// tile's end to one past the last splat any pixel consumed (an atomic max over
// the tile's four blocks).  It also records which pairs contributed, for the
// fused backward (bh_splat_record.h): per block and candidate, the 64-bit mask
// of the block's pixels that blended it (the ballot of the blend decision,
// moved into the candidate's lane), and per block the end of the candidates its
// pixels consumed.
#include <hip/hip_runtime.h>

#include "bh_internal.h"
#include "bh_splat_math.h"
#include "bh_splat_record.h"
#include "bh_tile_walk.h"

namespace bh {

// Four consecutive ids per thread (one 16-byte load when the quad lies in
// range and `ids` is 16-byte aligned), each compared with its predecessor:
// a change of id at i ends the previous tile's run and starts the next one.
__global__ __launch_bounds__(256) void tile_offsets_kernel(const uint32_t* __restrict__ ids, uint32_t m,
                                                            uint32_t num_tiles, uint32_t* __restrict__ off,
                                                            const uint32_t* __restrict__ dev_m) {
    if (dev_m) m = min(m, *dev_m);
    const uint32_t i0 = (blockIdx.x * 256u + threadIdx.x) * 4u;
    if (i0 >= m) return;
    uint32_t v[4];
    if (i0 + 4u <= m && (reinterpret_cast<uintptr_t>(ids) & 15u) == 0u) {
        const uint4 q = reinterpret_cast<const uint4*>(ids)[i0 / 4u];
        v[0] = q.x, v[1] = q.y, v[2] = q.z, v[3] = q.w;
    } else {
#pragma unroll
        for (uint32_t k = 0; k < 4u; k++) v[k] = i0 + k < m ? ids[i0 + k] : 0u;
    }
    uint32_t prev = i0 > 0 ? ids[i0 - 1] : 0u;
#pragma unroll
    for (uint32_t k = 0; k < 4u; k++) {
        const uint32_t i = i0 + k;
        if (i >= m) break;
        const uint32_t tid = v[k];
        if (i == 0) {
            if (tid < num_tiles) off[2 * tid] = 0;
        } else if (tid != prev) {
            if (prev < num_tiles) off[2 * prev + 1] = i;
            if (tid < num_tiles) off[2 * tid] = i;
        }
        if (i == m - 1 && tid < num_tiles) off[2 * tid + 1] = i + 1;
        prev = tid;
    }
}

void launch_tile_offsets(bh_ctx* ctx, const uint32_t* tile_ids, uint32_t m, uint32_t num_tiles,
                         uint32_t* offsets, bool zeroed, const uint32_t* dev_m) {
    if (!zeroed) launch_fill_u32(ctx, offsets, 0u, (uint64_t)num_tiles * 2);
    if (m == 0) return;
    KernelTimer t(ctx, "tile_offsets");
    launch(ctx, tile_offsets_kernel, dim3(div_up(div_up(m, 4), 256)), dim3(256), 0u, tile_ids, m, num_tiles, offsets,
           dev_m);
}

// v_writelane_b32: writes the wave-uniform `value` into lane `lane` of `old`,
// the other lanes keep theirs.  This compiler exposes no builtin for it, so the
// declaration binds to the LLVM intrinsic, which also places the lane select
// where the constant bus allows.
extern "C" __device__ int bh_llvm_writelane(int value, int lane, int old) __asm("llvm.amdgcn.writelane.i32");
__device__ __forceinline__ uint32_t write_lane(uint32_t old, uint32_t value, uint32_t lane) {
    return (uint32_t)bh_llvm_writelane((int)value, (int)lane, (int)old);
}

// One workgroup (a single wave) per 8x8 pixel block of a 16 x TH tile; the
// 2 * TH / 8 blocks of a tile get workgroup ids that agree modulo 8, which the
// dispatcher places on one XCD (shared L2 for the tile's splat rows).
template <int TH>
__device__ __forceinline__ void raster_block_of_workgroup(uint32_t g, uint32_t& tile, uint32_t& blk) {
    constexpr uint32_t BPT = 2u * (uint32_t)TH / 8u;
    const uint32_t slot = g >> 3;
    tile = ((slot / BPT) << 3) | (g & 7u);
    blk = slot % BPT;
}

// Dispatch order of the tiles: by descending splat count, in buckets of a
// quarter octave (exact order inside a bucket is not needed), so the longest
// blocks start first.  One workgroup; order[i] is the i-th tile to dispatch.
__device__ __forceinline__ uint32_t tile_bucket(uint2 off) {
    const uint32_t lo = off.x, hi = off.y;
    const uint32_t c = hi > lo ? hi - lo : 0u;
    uint32_t b = c;
    if (c >= 4u) {
        const uint32_t msb = 31u - (uint32_t)__builtin_clz(c);
        b = msb * 4u + ((c >> (msb - 2u)) & 3u);
    }
    return 127u - min(b, 127u);
}
__device__ __forceinline__ uint32_t tile_load_bucket(const uint32_t* __restrict__ offsets, uint32_t t) {
    return tile_bucket(make_uint2(offsets[2 * t], offsets[2 * t + 1]));
}

// Adds one to s[b] for each lane of the (fully active) wave whose b is a
// bucket (b <= 127) and returns the lane's previous count.  Empty tiles, most
// of the image, all fall in bucket 127: the wave adds those in one atomic from
// its first such lane and hands out consecutive slots, since same-address
// atomics of one instruction serialise in LDS.
__device__ __forceinline__ uint32_t bucket_add(uint32_t* s, uint32_t b) {
    const uint64_t e = __ballot(b == 127u);
    const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(e >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)e, 0u));
    uint32_t r = 0u;
    if (b < 127u)
        r = atomicAdd(&s[b], 1u);
    else if (b == 127u && rank == 0u)
        r = atomicAdd(&s[127], (uint32_t)__popcll(e));
    const int leader = e ? __ffsll((unsigned long long)e) - 1 : 0;
    const uint32_t base = (uint32_t)__shfl((int)r, leader, 64);
    return b == 127u ? base + rank : r;
}

// Every lane of the workgroup runs each call (the loops below have uniform
// trip counts), so the wave-wide ballot and shuffle in bucket_add see all 64
// lanes.  The first 16 x 1024 tiles' buckets stay in registers between the
// count and the scatter, and their loads are all issued before the first
// atomic: the two passes cost one memory round trip, not one per tile.
__device__ __forceinline__ void tile_order_block(const uint32_t* __restrict__ offsets, uint32_t num_tiles,
                                                 uint32_t* __restrict__ order) {
    constexpr uint32_t K = 16u;
    constexpr uint32_t NONE = 0xFFFFFFFFu;
    __shared__ uint32_t s_cur[128];
    const uint32_t t = threadIdx.x;
    if (t < 128u) s_cur[t] = 0u;
    // every load issued before the first wait: unconditional, at indices
    // clamped into the tiles (a load behind `i < num_tiles` is a branch of its
    // own with its own wait, one memory round trip per k)
    uint2 off[K];
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) {
        const uint32_t i = min(k * 1024u + t, num_tiles - 1u);
        off[k] = make_uint2(offsets[2 * i], offsets[2 * i + 1]);
    }
    uint32_t bk[K];
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) bk[k] = k * 1024u + t < num_tiles ? tile_bucket(off[k]) : NONE;
    __syncthreads();
#pragma unroll
    for (uint32_t k = 0; k < K; ++k)
        if (k * 1024u < num_tiles) bucket_add(s_cur, bk[k]);
    for (uint32_t b0 = K * 1024u; b0 < num_tiles; b0 += 1024u) {
        const uint32_t i = b0 + t;
        bucket_add(s_cur, i < num_tiles ? tile_load_bucket(offsets, i) : NONE);
    }
    __syncthreads();
    if (t < 64u) {
        // exclusive scan of the 128 bucket sizes, two per lane
        const uint32_t a = s_cur[2u * t], b = s_cur[2u * t + 1u];
        uint32_t x = a + b;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t y = __shfl_up(x, o, 64);
            if ((int)t >= o) x += y;
        }
        const uint32_t excl = x - a - b;
        s_cur[2u * t] = excl;
        s_cur[2u * t + 1u] = excl + a;
    }
    __syncthreads();
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) {
        if (k * 1024u < num_tiles) {
            const uint32_t pos = bucket_add(s_cur, bk[k]);
            if (bk[k] != NONE) order[pos] = k * 1024u + t;
        }
    }
    for (uint32_t b0 = K * 1024u; b0 < num_tiles; b0 += 1024u) {
        const uint32_t i = b0 + t;
        const uint32_t b = i < num_tiles ? tile_load_bucket(offsets, i) : NONE;
        const uint32_t pos = bucket_add(s_cur, b);
        if (b != NONE) order[pos] = i;
    }
}

__global__ __launch_bounds__(1024) void tile_order_kernel(const uint32_t* __restrict__ offsets, uint32_t num_tiles,
                                                          uint32_t* __restrict__ order) {
    tile_order_block(offsets, num_tiles, order);
}

// The tile order in the first workgroup (dispatched first, so it starts at
// once) while the others zero p[0, words): the backward's gradient rows and
// its order are independent, and the order's single workgroup (~12 us of
// latency) runs beside the fill.
__global__ __launch_bounds__(1024) void zero_and_tile_order_kernel(uint32_t* __restrict__ p, uint64_t words,
                                                                   const uint32_t* __restrict__ offsets,
                                                                   uint32_t num_tiles, uint32_t* __restrict__ order) {
    if (blockIdx.x == 0u) {
        tile_order_block(offsets, num_tiles, order);
        return;
    }
    const uint64_t b = blockIdx.x - 1u;
    const uint64_t stride = (uint64_t)(gridDim.x - 1u) * 1024u;
    const uint64_t quads = words / 4u;
    uint4* q = reinterpret_cast<uint4*>(p);
    for (uint64_t i = b * 1024u + threadIdx.x; i < quads; i += stride) q[i] = make_uint4(0u, 0u, 0u, 0u);
    for (uint64_t i = quads * 4u + b * 1024u + threadIdx.x; i < words; i += stride) p[i] = 0u;
}

void launch_tile_order(bh_ctx* ctx, const uint32_t* offsets, uint32_t num_tiles, uint32_t* order) {
    if (num_tiles == 0) return;
    KernelTimer t(ctx, "tile_order");
    launch(ctx, tile_order_kernel, dim3(1), dim3(1024), 0u, offsets, num_tiles, order);
}

void launch_zero_and_tile_order(bh_ctx* ctx, uint32_t* p, uint64_t words, const uint32_t* offsets,
                                uint32_t num_tiles, uint32_t* order) {
    if (num_tiles == 0) {
        launch_fill_u32(ctx, p, 0u, words);
        return;
    }
    KernelTimer t(ctx, "zero_and_tile_order");
    const uint32_t fill_blocks = (uint32_t)std::min<uint64_t>((words / 4u + 1023u) / 1024u + 1u, 1024u);
    launch(ctx, zero_and_tile_order_kernel, dim3(fill_blocks + 1u), dim3(1024), 0u, p, words, offsets, num_tiles,
           order);
}

constexpr uint32_t kFillQuadsPerLane = 16;

template <bool BWD_INFO, bool SMOOTH, bool DEPTH, int TH>
__global__ __launch_bounds__(64) void rasterize_kernel(uint32_t img_w, uint32_t img_h, uint32_t tile_bw,
                                                        uint32_t num_tiles, float bg_r, float bg_g, float bg_b,
                                                        uint32_t num_visible, const float* __restrict__ projected,
                                                        const uint32_t* __restrict__ cgids,
                                                        const uint32_t* __restrict__ gfc,
                                                        const uint32_t* __restrict__ off_pre,
                                                        const uint32_t* __restrict__ order,
                                                        void* __restrict__ out_img, float* __restrict__ visible,
                                                        uint32_t* __restrict__ off_post, SplatRecord rec,
                                                        uint32_t* __restrict__ fill, uint64_t fill_words,
                                                        uint32_t blend_groups) {
    // the conic scaled for the power in base 2 (bh_conic_log2: a, b, c)
    __shared__ float4 s_xyco[64];  // x, y, a, b
    __shared__ float4 s_c11a[64];  // c, opacity, cutoff on the power in base 2
    __shared__ float4 s_rgbd[64];  // r, g, b (staged_colour), depth

    if (BWD_INFO && blockIdx.x >= blend_groups) {
        // the backward's gradient rows: 16 KB per trailing workgroup, which
        // the dispatcher starts as the blend's blocks drain
        const uint64_t q0 = (uint64_t)(blockIdx.x - blend_groups) * (64u * kFillQuadsPerLane);
        uint4* q = reinterpret_cast<uint4*>(fill);
        const uint64_t quads = fill_words / 4u;
#pragma unroll
        for (uint32_t k = 0; k < kFillQuadsPerLane; k++) {
            const uint64_t i = q0 + k * 64u + threadIdx.x;
            if (i < quads) q[i] = make_uint4(0u, 0u, 0u, 0u);
        }
        if (q0 == 0u && threadIdx.x < fill_words % 4u) fill[quads * 4u + threadIdx.x] = 0u;
        return;
    }
    uint32_t tile, blk;
    raster_block_of_workgroup<TH>(blockIdx.x, tile, blk);
    if (tile >= num_tiles) return;
    if (order) tile = order[tile];
    const uint32_t lane = threadIdx.x;
    const uint32_t ox = (tile % tile_bw) * 16u + (blk & 1u) * 8u;
    const uint32_t oy = (tile / tile_bw) * (uint32_t)TH + (blk >> 1) * 8u;
    const uint32_t px = ox + (lane & 7u), py = oy + (lane >> 3);
    const bool inside = px < img_w && py < img_h;
    const uint32_t lo = off_pre[2 * tile], hi = off_pre[2 * tile + 1];
    // Long blocks first: the wave priority rises with the tile's candidate
    // count (work is concentrated in few tiles; see the backward kernel).
    const uint32_t len = hi - lo;
    if (len >= 6144u)
        __builtin_amdgcn_s_setprio(3);
    else if (len >= 3072u)
        __builtin_amdgcn_s_setprio(2);
    else if (len >= 1024u)
        __builtin_amdgcn_s_setprio(1);
    const float pcx = (float)px + 0.5f, pcy = (float)py + 0.5f;
    const float bx0 = (float)ox + 0.5f, by0 = (float)oy + 0.5f;
    float t_acc = 1.0f, pr = 0.0f, pg = 0.0f, pb = 0.0f, pd = 0.0f;
    // pixels whose transmittance has saturated (or that lie outside the image)
    uint64_t done_m = __builtin_amdgcn_ballot_w64(!inside);
    uint32_t last = lo;
    // a forward with BWD_INFO always records its pairs (the launcher passes
    // the record buffers whenever there are intersections)
    constexpr uint32_t BPT = 2u * (uint32_t)TH / 8u;
    constexpr bool record = BWD_INFO;
    const size_t rbase = record ? record_base<BPT>(blk, lo, hi) : 0;

    // A batch's global accesses are ordered so that a wait never covers a
    // later one: its candidate ids were read before the previous batch was
    // blended; its rows (and, with BWD_INFO, the splats' global ids) are read
    // first, then the previous batch's record and visibility stores go out,
    // then the next batch's ids are read, so they arrive while this batch is
    // blended.  The reads are unconditional, at indices clamped into the
    // tile's run.
    const uint32_t lastc = hi - 1u;
    uint32_t cid_n = 0u;
    if (hi > lo) cid_n = cgids[min(lo + lane, lastc)];
    // the previous batch's stores, deferred
    bool pend_vis = false, pend_mask = false;
    uint32_t pend_gid = 0u;
    size_t pend_at = 0;
    uint32_t mask_lo = 0u, mask_hi = 0u;  // pixels that blended this lane's candidate
    for (uint32_t batch = lo; batch < hi; batch += 64u) {
        if (done_m == ~0ull) break;
        // a block still blending after 256 candidates is one of the long ones
        // whatever its candidate count said: top priority from here on
        if (batch - lo == 256u) __builtin_amdgcn_s_setprio(3);
        const uint32_t cnt = min(64u, hi - batch);
        const uint32_t my_c = min(cid_n, num_visible - 1u);
        const float2* row = reinterpret_cast<const float2*>(projected + (size_t)my_c * 10);
        const float2 a = row[0], b = row[1], cc = row[2], d = row[3], e = row[4];
        const uint32_t my_gid = BWD_INFO ? gfc[my_c] : 0u;
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        if (BWD_INFO && pend_vis) visible[pend_gid] = 1.0f;
        if (record && pend_mask) rec.masks[pend_at] = make_uint2(mask_lo, mask_hi);
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        cid_n = cgids[min(batch + 64u + lane, lastc)];
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        const float cut = sigma_cutoff<SMOOTH>(cc.y);
        float ka, kb, kc;
        bh_conic_log2(b.x, b.y, cc.x, &ka, &kb, &kc);
        s_xyco[lane] = make_float4(a.x, a.y, ka, kb);
        // the cutoff's margin of 1e-3 covers the rounding of the scaled power
        s_c11a[lane] = make_float4(kc, cc.y, kLog2e * cut, 0.0f);
        s_rgbd[lane] = make_float4(staged_colour(d.x), staged_colour(d.y), staged_colour(e.x), e.y);
        const bool touch = lane < cnt && may_touch_rect(a.x, a.y, S2{b.x, b.y, cc.x}, cut, bx0, by0, bx0 + 7.0f,
                                                        by0 + 7.0f);
        // splats of the batch that may touch this block, in order
        uint64_t todo = __builtin_amdgcn_ballot_w64(touch);
        mask_lo = 0u;
        mask_hi = 0u;
        wave_lds_fence();
        // One candidate front to back; true once every pixel of the block is
        // done.  The loop below reads the next candidate's parameters while
        // the current one is evaluated, two register sets in turn.
        auto blend_one = [&](uint32_t j, const float4& xc, const float4& ca, const float4& col) -> bool {
            // the power sigma log2(e) of the pixel (bh_math.h)
            const float power = bh_power_log2(xc.z, xc.w, ca.x, xc.x - pcx, xc.y - pcy);
            // lane conditions are kept as wave masks (scalar registers), each
            // the ballot of a single comparison
            const uint64_t maybe_m = __builtin_amdgcn_ballot_w64(power >= 0.0f) &
                                     __builtin_amdgcn_ballot_w64(!(power > ca.z)) & ~done_m;
            if (maybe_m == 0ull) return done_m == ~0ull;
            // Branch-free from here: lanes outside `maybe` compute values the
            // selects discard.
            const float alpha = bh_minf(0.999f, ca.y * bh_exp2_neg(-power));
            // the hard cutoff's weight is a step: alpha * w is a select
            const float w = SMOOTH ? cutoff_weight(alpha) : (alpha >= kCutMid ? 1.0f : 0.0f);
            // with the hard cutoff alpha * w is alpha wherever it is used: the
            // lanes below the cutoff are outside `pass`, so their next_t and
            // vis never reach a mask, a sum or the transmittance
            const float ae = SMOOTH ? alpha * w : alpha;
            const float next_t = t_acc * (1.0f - ae);
            const uint64_t pass_m = maybe_m & __builtin_amdgcn_ballot_w64(w > 0.0f);
            const uint64_t sat_m = __builtin_amdgcn_ballot_w64(next_t <= 1.0e-4f) & pass_m;
            const uint64_t blended = pass_m & ~sat_m;
            const bool contrib = __builtin_amdgcn_inverse_ballot_w64(blended);
            done_m |= sat_m;
            // unconditional (a candidate past the pre-test nearly always
            // blends some pixel): vis is zero outside `contrib`, and adding
            // col * 0 (a signed zero; colours are finite) leaves a sum that is
            // >= +0 unchanged; an empty ballot written into lane j leaves its
            // record empty
            const float vis = contrib ? ae * t_acc : 0.0f;
            // the accumulation as one fma per channel, as the restatement
            // evaluates it
            pr = __builtin_fmaf(col.x, vis, pr);
            pg = __builtin_fmaf(col.y, vis, pg);
            pb = __builtin_fmaf(col.z, vis, pb);
            if (DEPTH) pd = __builtin_fmaf(col.w, vis, pd);
            t_acc = contrib ? next_t : t_acc;
            if (record) {
                // the ballot (scalar) goes into candidate j's lane
                mask_lo = write_lane(mask_lo, (uint32_t)blended, j);
                mask_hi = write_lane(mask_hi, (uint32_t)(blended >> 32), j);
            }
            return done_m == ~0ull;
        };
        if (todo) {
            uint32_t ja = (uint32_t)__builtin_ctzll(todo);
            todo &= todo - 1ull;
            float4 xa = s_xyco[ja], caa = s_c11a[ja], cola = s_rgbd[ja];
            while (true) {
                // the next candidate's parameters, read unconditionally (slot
                // 0 when the list is empty: read, never blended)
                const bool has_b = todo != 0ull;
                const uint32_t jb = has_b ? (uint32_t)__builtin_ctzll(todo) : 0u;
                todo &= ~(1ull << jb);
                const float4 xb = s_xyco[jb], cab = s_c11a[jb], colb = s_rgbd[jb];
                // the wave's done test once per two candidates: after a, b's
                // masks exclude the done pixels anyway
                blend_one(ja, xa, caa, cola);
                if (!has_b) break;
                const bool has_a = todo != 0ull;
                ja = has_a ? (uint32_t)__builtin_ctzll(todo) : 0u;
                todo &= ~(1ull << ja);
                xa = s_xyco[ja];
                caa = s_c11a[ja];
                cola = s_rgbd[ja];
                if (blend_one(jb, xb, cab, colb) || !has_a) break;
            }
        }
        if (BWD_INFO) {
            // the splats some pixel of the block blended (lane j: candidate
            // batch + j) and the block's last one (the tile end is the
            // maximum over its pixels, the same for every lane)
            const uint64_t used = __builtin_amdgcn_ballot_w64((mask_lo | mask_hi) != 0u);
            if (used) last = batch + 64u - (uint32_t)__builtin_clzll(used);
            pend_vis = (used >> lane) & 1ull;
        }
        pend_gid = my_gid;
        pend_mask = record && lane < cnt;
        pend_at = rbase + (batch - lo) + lane;
        wave_lds_fence();
    }
    if (BWD_INFO && pend_vis) visible[pend_gid] = 1.0f;
    if (record && pend_mask) rec.masks[pend_at] = make_uint2(mask_lo, mask_hi);

    if (inside) {
        const float fr = pr + t_acc * bg_r, fg = pg + t_acc * bg_g, fb = pb + t_acc * bg_b;
        const float fa = 1.0f - t_acc;
        const size_t pix = (size_t)py * img_w + px;
        if (BWD_INFO) {
            if (DEPTH) {
                float* o = (float*)out_img + pix * 5;
                o[0] = fr;
                o[1] = fg;
                o[2] = fb;
                o[3] = fa;
                o[4] = pd;
            } else {
                reinterpret_cast<float4*>(out_img)[pix] = make_float4(fr, fg, fb, fa);
            }
        } else {
            const uint32_t ur = (uint32_t)bh_clampf(fr * 255.0f, 0.0f, 255.0f);
            const uint32_t ug = (uint32_t)bh_clampf(fg * 255.0f, 0.0f, 255.0f);
            const uint32_t ub = (uint32_t)bh_clampf(fb * 255.0f, 0.0f, 255.0f);
            const uint32_t ua = (uint32_t)bh_clampf(fa * 255.0f, 0.0f, 255.0f);
            reinterpret_cast<uint32_t*>(out_img)[pix] = ur | (ug << 8) | (ub << 16) | (ua << 24);
        }
    }
    // post-raster tile end: one past the last splat any pixel of the tile
    // blended (the caller zero-filled off_post; every block of the tile adds
    // its own maximum)
    if (BWD_INFO) {
        const uint32_t m = last;  // wave-uniform: one past the block's last blended candidate
        if (lane == 0) atomicMax(&off_post[2 * tile + 1], m);
        if (record && lane == 0) rec.block_end[tile * BPT + blk] = m;
        if (record && lane == 0 && rec.order.list) {
            // the backward's order (bh_splat_record.h): the tile's last block
            // appends it under its longest block's bucket
            const unsigned long long add = (1ull << 32) | ((unsigned long long)order_bucket(m - lo) << (8u * blk));
            const unsigned long long w = atomicAdd(&rec.order.word[tile], add) + add;
            if ((uint32_t)(w >> 32) == BPT) {
                uint32_t b = kOrderBuckets - 1u;
#pragma unroll
                for (uint32_t k = 0; k < BPT; ++k) b = min(b, (uint32_t)(w >> (8u * k)) & 0xFFu);
                if (b != kOrderBuckets - 1u) order_append(rec.order, b, tile, num_tiles);
            }
        }
    }
    if (lane == 0 && blk == 0) {
        off_post[2 * tile] = lo;
        if (!BWD_INFO) off_post[2 * tile + 1] = hi;
    }
}

void launch_rasterize(bh_ctx* ctx, uint32_t img_w, uint32_t img_h, uint32_t tile_bw, uint32_t tile_bh,
                      const float* bg, uint32_t num_visible, const float* projected, const uint32_t* cgids, const uint32_t* gfc,
                      const uint32_t* off_pre, const uint32_t* order, uint32_t flags, void* out_img, float* visible,
                      uint32_t* off_post, bool off_post_zeroed, SplatRecord rec, uint32_t* fill,
                      uint64_t fill_words) {
    const uint32_t num_tiles = tile_bw * tile_bh;
    if (num_tiles == 0) return;
    const bool bwd = (flags & BH_FLAG_BWD_INFO) != 0;
    const bool smooth = (flags & BH_FLAG_SMOOTH_CUTOFF) != 0;
    const bool depth = bwd && (flags & BH_FLAG_RENDER_DEPTH) != 0;
    const uint32_t nv = num_visible > 0 ? num_visible : 1u;
    // a BWD_INFO blend writes its record (block ends always, masks with
    // intersections): never launch it without the buffers
    if (bwd && (!rec.masks || !rec.block_end)) return;
    if (bwd && !off_post_zeroed) launch_fill_u32(ctx, off_post, 0u, (uint64_t)num_tiles * 2);
    const bool fine = (flags & BH_FLAG_TILE_16X8) != 0;
    // 8 tiles per group of workgroup ids, 4 (16x16) or 2 (16x8) blocks per tile
    const uint32_t groups = div_up(num_tiles, 8) * (fine ? 16u : 32u);
    // trailing zero-fill workgroups (BWD_INFO only)
    if (!bwd || !fill) fill_words = 0;
    const uint32_t fill_groups = (uint32_t)div_up(div_up(fill_words, 4u), 64u * kFillQuadsPerLane);
    KernelTimer t(ctx, "rasterize");
#define BH_RASTER_T(B, S, D, T)                                                                                    \
    launch(ctx, rasterize_kernel<B, S, D, T>, dim3(groups + fill_groups), dim3(64), 0u, img_w, img_h, tile_bw,         \
           num_tiles, bg[0], bg[1], bg[2], nv, projected, cgids, gfc, off_pre, order, out_img, visible, off_post, rec, \
           fill, fill_words, groups)
#define BH_RASTER(B, S, D) \
    do {                   \
        if (fine)          \
            BH_RASTER_T(B, S, D, 8); \
        else               \
            BH_RASTER_T(B, S, D, 16); \
    } while (0)
    if (!bwd) {
        if (smooth) BH_RASTER(false, true, false); else BH_RASTER(false, false, false);
    } else if (depth) {
        if (smooth) BH_RASTER(true, true, true); else BH_RASTER(true, false, true);
    } else {
        if (smooth) BH_RASTER(true, true, false); else BH_RASTER(true, false, false);
    }
#undef BH_RASTER
#undef BH_RASTER_T
}

}  // namespace bh
