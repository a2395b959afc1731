// project.hip — per-splat projection kernels for gfx950.
//
//   project_forward   cull, 2D covariance and conic, power threshold, extent,
//                     contributing-tile count, max radius, depth key
//                     (crates/brush-render/src/kernels/project_forward.rs:20-144)
//   project_visible   depth-ordered projected rows with SH -> RGB
//                     (crates/brush-render/src/kernels/project_visible.rs:22-89):
//                     project_forward computes each visible splat's row in
//                     global-id order, project_gather_kernel orders them
//   map_intersects    (tile id, compact id) pairs for every contributing tile
//                     (crates/brush-render/src/kernels/map_gaussians.rs:14-92)
//
// Differences in organisation from the reference: project_forward does not
// compact visible splats with an atomic slot counter (whose order depends on
// scheduling); it writes a depth key per global id (all ones when culled) and
// the depth sort over all ids yields the compact order, with equal depths in
// global-id order.  Counters are aggregated per wave before the atomics.
#include <hip/hip_runtime.h>

#include "bh_internal.h"
#include "bh_splat_math.h"
#include "bh_tile_walk.h"

namespace bh {

// The cull part of project_forward_kernel (project_forward.rs:20-118): returns
// false if the splat is culled, else its screen mean, conic, power threshold
// and tile box.  The tile count is done by the wave-cooperative walk.
struct Projected {
    V2 m;
    S2 conic;
    float pt;
    TileBox bb;
    float radius;
    float depth;
    float opac;
};

template <bool MIP, int CAM, int TH>
__device__ bool project_cull(const bh_project_uniforms& u, const float* t, float raw_opac, Projected& o) {
    V3 mean_c = world_to_cam(u, v3(t[0], t[1], t[2]));
    if (!(finite3(mean_c) && mean_c.z <= 1.0e10f)) return false;
    if (depth_culled<CAM>(u, mean_c)) return false;
    V3 sc = v3(bh_expf(t[7]), bh_expf(t[8]), bh_expf(t[9]));
    if (!finite3(sc)) return false;
    Q4 qu{t[3], t[4], t[5], t[6]};
    float qn = qdot(qu, qu);
    if (!(qn >= 1.0e-6f && bh_is_finite(qn))) return false;
    if (!bh_is_finite(raw_opac)) return false;
    Q4 q = qnormalize(qu);
    S2 raw_cov = calc_cov2d<CAM>(u, sc, q, mean_c);
    float comp;
    S2 cov = compensate_cov2d<MIP>(raw_cov, comp);
    float opac = bh_sigmoidf(raw_opac) * comp;
    if (!finite2(cov)) return false;
    V2 m = project_point<CAM>(u, mean_c);
    if (!(opac >= 1.0f / 255.0f)) return false;
    float pt = bh_logf(opac * 255.0f);
    S2 conic = inverse(cov);
    V2 e = bbox_extent(conic, pt);
    if (!(e.x >= 0.0f && e.y >= 0.0f)) return false;
    float wf = (float)u.img_w, hf = (float)u.img_h;
    bool on_screen = m.x + e.x > 0.0f && m.x - e.x < wf && m.y + e.y > 0.0f && m.y - e.y < hf;
    if (!on_screen) return false;
    o.m = m;
    o.conic = conic;
    o.pt = pt;
    o.bb = tile_bbox<TH>(m, e, u.tile_bw, u.tile_bh);
    o.radius = bh_maxf(e.x / wf, e.y / hf);
    o.depth = mean_c.z;
    o.opac = opac;
    return true;
}

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = min(v, (uint32_t)__shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor(v, o, 64));
    return v;
}

template <int NC>
__device__ __forceinline__ void load_sh_row(const float* __restrict__ sh, uint32_t gid, float* c) {
    const float* row = sh + (size_t)gid * (3 * NC);
    if ((3 * NC) % 4 == 0) {
        const float4* r4 = reinterpret_cast<const float4*>(row);
#pragma unroll
        for (int i = 0; i < (3 * NC) / 4; i++) {
            float4 q = r4[i];
            c[4 * i] = q.x;
            c[4 * i + 1] = q.y;
            c[4 * i + 2] = q.z;
            c[4 * i + 3] = q.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 3 * NC; i++) c[i] = row[i];
    }
}

// A visible splat's projected row (project_visible.rs:22-89) in its global-id
// slot: 12 floats, x y c00 c01 | c11 opac r g | b depth pt -, pt being the
// tile predicate's power threshold ln(255 opac) for the map's walk.  Slots are packed
// (48 bytes): a wave's stores cover whole lines, where 48 bytes of a 64-byte
// slot cost partial-line writes.
// project_forward reads the parameters and SH rows in global-id order
// (coalesced), so the depth-ordered rows cost one aligned 64-byte gather each
// (in map_intersects) instead of three scattered parameter reads.  The SH row
// is loaded before the tile walk and used after it, so the walk hides the
// load latency.
template <int DEG>
__device__ __forceinline__ void write_row_from_coeffs(const bh_project_uniforms& u, const float* coeffs, uint32_t gid,
                                                      V3 mean, const Projected& p, float4* __restrict__ rows) {
    V3 v = mean - v3(u.camera_pos[0], u.camera_pos[1], u.camera_pos[2]);
    v = v * (1.0f / sqrtf(dot(v, v)));
    V3 raw = sh_to_color<DEG>(coeffs, v);
    const float cr = raw.x + 0.5f, cg = raw.y + 0.5f, cb = raw.z + 0.5f;
    const float r = bh_clampf(bh_is_finite(cr) ? cr : 0.0f, -100.0f, 100.0f);
    const float g = bh_clampf(bh_is_finite(cg) ? cg : 0.0f, -100.0f, 100.0f);
    const float b = bh_clampf(bh_is_finite(cb) ? cb : 0.0f, -100.0f, 100.0f);
    float4* dst = rows + (size_t)gid * 3;
    dst[0] = make_float4(p.m.x, p.m.y, p.conic.c00, p.conic.c01);
    dst[1] = make_float4(p.conic.c11, p.opac, r, g);
    dst[2] = make_float4(b, p.depth, p.pt, 0.0f);
}

template <bool MIP, int CAM, int TH, int DEG>
__global__ __launch_bounds__(256, DEG >= 4 ? 4 : 5) void project_forward_kernel(bh_project_uniforms u,
                                                               const float* __restrict__ transforms,
                                                               const float* __restrict__ raw_opac,
                                                               const float* __restrict__ sh, uint32_t n,
                                                               uint32_t* __restrict__ counts,
                                                               float* __restrict__ max_radius,
                                                               uint32_t* __restrict__ depth_keys,
                                                               float4* __restrict__ rows,
                                                               uint32_t* __restrict__ partials, ZeroRanges zero) {
    __shared__ uint32_t s_vis[4], s_kmin[4], s_kmax[4];
    __shared__ unsigned long long s_hits[4];
    __shared__ WalkRec s_rec[4][64];
    __shared__ uint32_t s_slot[4][64], s_count[4][64];
    const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    bool vis = false;
    V3 mean = v3(0.0f, 0.0f, 0.0f);
    Projected p{v2(0.0f, 0.0f), S2{0.0f, 0.0f, 0.0f}, 0.0f, TileBox{0u, 0u, 0u, 0u}, 0.0f, 0.0f, 0.0f};
    if (gid < n) {
        const float2* row = reinterpret_cast<const float2*>(transforms + (size_t)gid * 10);
        float t[10];
#pragma unroll
        for (int i = 0; i < 5; i++) {
            float2 q = row[i];
            t[2 * i] = q.x;
            t[2 * i + 1] = q.y;
        }
        // the cull fills q only for a splat it keeps: its early exits then
        // carry no copies of p's zeros
        Projected q;
        vis = project_cull<MIP, CAM, TH>(u, t, raw_opac[gid], q);
        if (vis) p = q;
        mean = v3(t[0], t[1], t[2]);
    }
    // Every parameter load has landed here (vmcnt(0); they have long since,
    // but a cull that exits early leaves some unread).  Without it, the merge
    // after the conditional SH loads below makes the compiler's first reuse of
    // such a register wait for all outstanding loads, the SH row included, and
    // the tile walk would no longer hide the row's latency.
    __builtin_amdgcn_s_waitcnt(0x0F70);
    constexpr int NC = (DEG + 1) * (DEG + 1);
    float coeffs[3 * NC];
    if (vis) load_sh_row<NC>(sh, gid, coeffs);
    // count_contributing_tiles (project_forward.rs:120-128) for the whole wave
    const uint32_t hits = wave_tile_walk<false, TH, uint32_t>(lane, vis ? bbox_items(p.bb) : 0u, p.m, p.conic, p.pt, p.bb,
                                                s_rec[wave], s_slot[wave], s_count[wave], u.tile_bw, 0u, 0u, 0u,
                                                nullptr, nullptr);
    if (gid < n) {
        counts[gid] = vis ? hits : 0u;
        max_radius[gid] = vis ? p.radius : 0.0f;
        depth_keys[gid] = vis ? bh_as_uint(p.depth) : 0xFFFFFFFFu;
    }
    if (vis) write_row_from_coeffs<DEG>(u, coeffs, gid, mean, p, rows);
    // per-block totals (no same-address atomics): wave shuffles, then LDS
    uint64_t vmask = __ballot(vis);
    uint64_t hsum = wave_sum_u64(vis ? (uint64_t)hits : 0ull);
    uint32_t kmin = wave_min_u32(vis ? bh_as_uint(p.depth) : 0xFFFFFFFFu);
    uint32_t kmax = wave_max_u32(vis ? bh_as_uint(p.depth) : 0u);
    if (lane == 0) {
        s_vis[wave] = (uint32_t)__popcll(vmask);
        s_hits[wave] = hsum;
        s_kmin[wave] = kmin;
        s_kmax[wave] = kmax;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t v = 0, mn = 0xFFFFFFFFu, mx = 0u;
        unsigned long long h = 0;
        for (int w = 0; w < 4; w++) {
            v += s_vis[w];
            h += s_hits[w];
            mn = min(mn, s_kmin[w]);
            mx = max(mx, s_kmax[w]);
        }
        uint32_t* out = partials + (size_t)blockIdx.x * 8;
        out[0] = v;
        out[1] = (uint32_t)h;
        out[2] = (uint32_t)(h >> 32);
        out[3] = mn;
        out[4] = mx;
    }
    // the forward's zero-fills (visible mask, sort scratch, tile offsets),
    // last, when the splat's registers are free
#pragma unroll
    for (int j = 0; j < 4; j++)
        for (uint64_t i = gid; i < zero.count[j]; i += (uint64_t)gridDim.x * 256u) zero.p[j][i] = 0u;
}

// Folds the per-block totals of project_forward into the context counters
// ([0] visible, [2..3] intersections, [4] min depth key, [5] max depth key),
// and writes what launches sized before the host reads them take from there:
// [6] the depth sort's key cap (max - min + 1) and [7] the intersection
// count when it fits `isect_cap` (else 0).  The same eight words also go to
// `host` (mapped, coherent pinned host memory, or null), followed, after a
// system-scope fence, by `generation` in host[8]: the host polls that word,
// so neither a copy nor an event marker runs between the reduction and the
// host's read.
__global__ __launch_bounds__(1024) void project_reduce_kernel(const uint32_t* __restrict__ partials,
                                                              uint32_t num_blocks, uint32_t isect_cap,
                                                              uint32_t* __restrict__ counters,
                                                              uint32_t* __restrict__ host, uint32_t generation) {
    __shared__ uint32_t s_v[16], s_mn[16], s_mx[16];
    __shared__ unsigned long long s_h[16];
    uint32_t v = 0, mn = 0xFFFFFFFFu, mx = 0u;
    unsigned long long h = 0;
    for (uint32_t i = threadIdx.x; i < num_blocks; i += 1024u) {
        const uint32_t* p = partials + (size_t)i * 8;
        v += p[0];
        h += (unsigned long long)p[1] | ((unsigned long long)p[2] << 32);
        mn = min(mn, p[3]);
        mx = max(mx, p[4]);
    }
    v = (uint32_t)wave_sum_u64(v);
    h = wave_sum_u64(h);
    mn = wave_min_u32(mn);
    mx = wave_max_u32(mx);
    const uint32_t wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        s_v[wave] = v;
        s_h[wave] = h;
        s_mn[wave] = mn;
        s_mx[wave] = mx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; w++) {
            v += s_v[w];
            h += s_h[w];
            mn = min(mn, s_mn[w]);
            mx = max(mx, s_mx[w]);
        }
        const uint32_t c[8] = {v, 0u /* no device error */, (uint32_t)h, (uint32_t)(h >> 32), mn, mx, mx - mn + 1u,
                               h <= (unsigned long long)isect_cap ? (uint32_t)h : 0u};
        reinterpret_cast<uint4*>(counters)[0] = make_uint4(c[0], c[1], c[2], c[3]);
        reinterpret_cast<uint4*>(counters)[1] = make_uint4(c[4], c[5], c[6], c[7]);
        if (host) {
            reinterpret_cast<uint4*>(host)[0] = make_uint4(c[0], c[1], c[2], c[3]);
            reinterpret_cast<uint4*>(host)[1] = make_uint4(c[4], c[5], c[6], c[7]);
            __threadfence_system();
            __hip_atomic_store(host + 8, generation, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

size_t project_partials_bytes(uint32_t n) { return (size_t)div_up(n, 256) * 8 * sizeof(uint32_t); }

template <bool MIP, int TH, int DEG>
static void launch_pf(bh_ctx* ctx, uint32_t blocks, const bh_project_uniforms& u, const float* transforms,
                      const float* raw_opac, const float* sh, uint32_t n, uint32_t* intersect_counts,
                      float* max_radius, uint32_t* depth_keys, float4* rows, uint32_t* partials,
                      const ZeroRanges& zero) {
#define BH_PF(C)                                                                                              \
    launch(ctx, project_forward_kernel<MIP, C, TH, DEG>, dim3(blocks), dim3(256), 0u, u, transforms, raw_opac, sh, \
           n, intersect_counts, max_radius, depth_keys, rows, partials, zero)
    switch (u.camera_model) {
        case kCamKB4: BH_PF(kCamKB4); break;
        case kCamRT8: BH_PF(kCamRT8); break;
        case kCamTPF: BH_PF(kCamTPF); break;
        default: BH_PF(kCamPinhole); break;
    }
#undef BH_PF
}

template <int DEG>
static void launch_pf_deg(bh_ctx* ctx, uint32_t blocks, const bh_project_uniforms& u, const float* transforms,
                          const float* raw_opac, const float* sh, uint32_t n, bool mip, uint32_t tile_h,
                          uint32_t* intersect_counts, float* max_radius, uint32_t* depth_keys, float4* rows,
                          uint32_t* partials, const ZeroRanges& zero) {
#define BH_PFM(M, T)                                                                                               \
    launch_pf<M, T, DEG>(ctx, blocks, u, transforms, raw_opac, sh, n, intersect_counts, max_radius, depth_keys, rows, \
                         partials, zero)
    if (tile_h == 8) {
        if (mip) BH_PFM(true, 8); else BH_PFM(false, 8);
    } else {
        if (mip) BH_PFM(true, 16); else BH_PFM(false, 16);
    }
#undef BH_PFM
}

void launch_project_forward(bh_ctx* ctx, const bh_project_uniforms& u, const float* transforms,
                            const float* raw_opac, const float* sh, uint32_t sh_degree, uint32_t n, bool mip,
                            uint32_t tile_h, uint32_t* intersect_counts, float* max_radius, uint32_t* depth_keys,
                            float* rows, uint32_t* partials, uint32_t* counters, uint32_t isect_cap,
                            const ZeroRanges& zero, uint32_t* host_counters, uint32_t generation) {
    if (n == 0) return;
    uint32_t blocks = div_up(n, 256);
    {
        KernelTimer t(ctx, "project_forward");
        float4* r4 = reinterpret_cast<float4*>(rows);
#define BH_PFD(D) \
    launch_pf_deg<D>(ctx, blocks, u, transforms, raw_opac, sh, n, mip, tile_h, intersect_counts, max_radius, depth_keys, \
                     r4, partials, zero)
        switch (sh_degree) {
            case 0: BH_PFD(0); break;
            case 1: BH_PFD(1); break;
            case 2: BH_PFD(2); break;
            case 3: BH_PFD(3); break;
            default: BH_PFD(4); break;
        }
#undef BH_PFD
    }
    KernelTimer t(ctx, "project_reduce");
    launch(ctx, project_reduce_kernel, dim3(1), dim3(1024), 0u, partials, blocks, isect_cap, counters, host_counters,
           generation);
}

// ---- project_visible ------------------------------------------------------------

// The depth-ordered projected rows and depths: compact id c takes the row
// project_forward wrote in the slot of global id gfc[c].  map_intersects does
// this itself; this kernel serves forwards with visible splats but no
// intersections.
__global__ __launch_bounds__(256) void project_gather_kernel(const float4* __restrict__ rows,
                                                              const uint32_t* __restrict__ gfc, uint32_t num_visible,
                                                              uint32_t num_splats, float* __restrict__ projected,
                                                              float* __restrict__ depths) {
    const uint32_t c = blockIdx.x * 256u + threadIdx.x;
    if (c >= num_visible) return;
    const uint32_t gid = min(gfc[c], num_splats - 1u);
    const float4* r = rows + (size_t)gid * 3;
    const float4 a = r[0], b = r[1], d = r[2];
    float2* dst = reinterpret_cast<float2*>(projected + (size_t)c * 10);
    dst[0] = make_float2(a.x, a.y);
    dst[1] = make_float2(a.z, a.w);
    dst[2] = make_float2(b.x, b.y);
    dst[3] = make_float2(b.z, b.w);
    dst[4] = make_float2(d.x, d.y);
    depths[c] = d.y;
}

void launch_project_visible(bh_ctx* ctx, const float* rows, const uint32_t* gfc, uint32_t num_visible,
                            uint32_t num_splats, float* projected, float* depths) {
    if (num_visible == 0) return;
    KernelTimer t(ctx, "project_visible");
    launch(ctx, project_gather_kernel, dim3(div_up(num_visible, 256)), dim3(256), 0u,
           reinterpret_cast<const float4*>(rows), gfc, num_visible, num_splats, projected, depths);
}

// ---- map_intersects ----------------------------------------------------------------

// Each lane takes its splat's row from the global-id slot project_forward
// filled (gfc[c]), stores it as compact row c of `projected` (with its
// depth), and walks its tiles with it.  With `dev` (the context counters),
// num_visible is a capacity and the visible count is dev[0]; the
// intersections are written only when their count fits the output
// (dev[7] == dev[2..3], set by project_reduce), so every store stays inside
// buffers sized for the capacity.
template <int TH, typename TileT>
__global__ __launch_bounds__(256) void map_intersects_kernel(uint32_t tile_bw, uint32_t tile_bh,
                                                              const float4* __restrict__ rows,
                                                              const uint32_t* __restrict__ gfc, uint32_t num_splats,
                                                              const uint32_t* __restrict__ cum, uint32_t num_visible,
                                                              float* __restrict__ projected,
                                                              float* __restrict__ depths,
                                                              TileT* __restrict__ tile_ids,
                                                              uint32_t* __restrict__ cgids,
                                                              uint32_t* __restrict__ zero, uint32_t zero_words,
                                                              const uint32_t* __restrict__ dev, uint32_t m_cap) {
    __shared__ WalkRec s_rec[4][64];
    __shared__ uint32_t s_slot[4][64], s_count[4][64];
    const uint32_t c = blockIdx.x * 256u + threadIdx.x;
    // the tile sort's zeroed scratch, cleared here instead of by a launch of its own
    for (uint32_t i = c; i < zero_words; i += gridDim.x * 256u) zero[i] = 0u;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    bool emit = true;
    if (dev) {
        num_visible = min(num_visible, dev[0]);
        emit = dev[3] == 0u && dev[7] == dev[2];
    }
    const uint32_t c0 = c - lane;  // first compact id of this wave
    if (c0 >= num_visible) return;  // the whole wave is past the end
    const bool active = c < num_visible;
    V2 m = v2(0.0f, 0.0f);
    S2 conic{0.0f, 0.0f, 0.0f};
    float pt = 0.0f;
    TileBox bb{0u, 0u, 0u, 0u};
    uint32_t base = 0, budget = 0;
    if (active) {
        const float4* r = rows + (size_t)min(gfc[c], num_splats - 1u) * 3;
        const float4 a = r[0], b = r[1], d = r[2];
        float2* dst = reinterpret_cast<float2*>(projected + (size_t)c * 10);
        dst[0] = make_float2(a.x, a.y);
        dst[1] = make_float2(a.z, a.w);
        dst[2] = make_float2(b.x, b.y);
        dst[3] = make_float2(b.z, b.w);
        dst[4] = make_float2(d.x, d.y);
        depths[c] = d.y;
        if (!emit) return;
        m = v2(a.x, a.y);
        conic = S2{a.z, a.w, b.x};
        pt = d.z;  // bh_logf(b.y * 255), as the counting walk used it
        bb = tile_bbox<TH>(m, bbox_extent(conic, pt), tile_bw, tile_bh);
        base = c == 0 ? 0u : cum[c - 1];
        budget = cum[c] - base;
    }
    if (!emit) return;  // uniform over the grid
    // The wave's splats own the contiguous output range [cum[c0 - 1], cum[last]);
    // the walk emits their tiles in that order.
    const uint32_t last = min(c0 + 63u, num_visible - 1u);
    const uint32_t out_base = c0 == 0 ? 0u : cum[c0 - 1];
    // no store lands past the pair buffers (m_cap pairs), whatever cum holds
    const uint32_t out_end = min(cum[last], m_cap);
    const uint32_t hits = wave_tile_walk<true, TH, TileT>(lane, active ? bbox_items(bb) : 0u, m, conic, pt, bb, s_rec[wave],
                                               s_slot[wave], s_count[wave], tile_bw, out_base, out_end, c0, tile_ids,
                                               cgids);
    if (__ballot(active && hits != budget) == 0ull) return;
    // A recount that disagrees with the forward counts (it cannot for identical
    // rows) falls back to the reference's per-splat loop, which clamps to the
    // budget and pads with the sentinel tile (map_gaussians.rs:56-91), and
    // rewrites the wave's whole output range.
    __threadfence();
    if (!active) return;
    uint32_t k = 0;
    budget = base < m_cap ? min(budget, m_cap - base) : 0u;
    for (uint32_t ty = bb.min_y; ty < bb.max_y && k < budget; ty++)
        for (uint32_t tx = bb.min_x; tx < bb.max_x && k < budget; tx++)
            if (will_contribute<TH>(tx, ty, m, conic, pt)) {
                tile_ids[base + k] = (TileT)(tx + ty * tile_bw);
                cgids[base + k] = c;
                k++;
            }
    for (; k < budget; k++) {
        tile_ids[base + k] = (TileT)(tile_bw * tile_bh);
        cgids[base + k] = c;
    }
}

void launch_map_intersects(bh_ctx* ctx, uint32_t tile_bw, uint32_t tile_bh, uint32_t tile_h, const float* rows,
                           const uint32_t* gfc, uint32_t num_splats, const uint32_t* cum, uint32_t num_visible,
                           float* projected, float* depths, void* tile_ids, bool tile_ids16, uint32_t* cgids,
                           uint32_t* zero, uint32_t zero_words, const uint32_t* dev, uint32_t m_cap) {
    if (num_visible == 0) return;
    KernelTimer t(ctx, "map_intersects");
    const uint32_t blocks = div_up(num_visible, 256);
    const float4* r4 = reinterpret_cast<const float4*>(rows);
#define BH_MAP(TH, T)                                                                                           \
    launch(ctx, map_intersects_kernel<TH, T>, dim3(blocks), dim3(256), 0u, tile_bw, tile_bh, r4, gfc, num_splats, \
           cum, num_visible, projected, depths, (T*)tile_ids, cgids, zero, zero_words, dev, m_cap)
    if (tile_h == 8) {
        if (tile_ids16) BH_MAP(8, uint16_t); else BH_MAP(8, uint32_t);
    } else {
        if (tile_ids16) BH_MAP(16, uint16_t); else BH_MAP(16, uint32_t);
    }
#undef BH_MAP
}

}  // namespace bh
