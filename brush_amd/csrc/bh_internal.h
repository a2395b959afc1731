// bh_internal.h — context, workspace pool and launch helpers shared by the
// C-ABI implementation and the kernel translation units.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <map>
#include <string>
#include <vector>

#include "../../include/brush_hip.h"
#include "bh_splat_record.h"

namespace bh {

// Stream-ordered caching pool.  Every allocation is used on the context's
// single stream, so a block returned to the pool can be handed out again
// immediately: later kernels on the stream are ordered after earlier users.
struct Pool {
    struct Block {
        void* ptr;
        size_t bytes;
    };
    std::vector<Block> free_blocks;
    std::map<void*, size_t> live;
    size_t cached_bytes = 0;

    hipError_t alloc(void** out, size_t bytes);
    void release(void* ptr);
    void trim();  // hipFree everything in the free list
};

// A named host-side range around the launches of one stage of the path,
// named as the reference's tracing spans name them (render.rs:187-459,
// render_bwd.rs:106-366), so a profile of this library lines up with one of
// the reference.  rocprofv3 --marker-trace records them; without a tool
// attached a range costs two calls that return at once.
struct StageRange {
    explicit StageRange(const char* name);
    ~StageRange();
    StageRange(const StageRange&) = delete;
    StageRange& operator=(const StageRange&) = delete;
};

struct KernelTimer;

struct Timing {
    std::string name;
    hipEvent_t start, stop;
};

struct TimingTotal {
    uint32_t launches = 0;
    double total_ms = 0.0;
};

// loss.hip
void launch_image_loss_forward(bh_ctx* ctx, const float* pred, uint32_t stride, uint32_t channels,
                               const uint32_t* gt, uint32_t w, uint32_t h, const bh_image_loss_config& cfg,
                               float* map);
void launch_image_loss_backward(bh_ctx* ctx, const float* pred, uint32_t stride, uint32_t channels,
                                const uint32_t* gt, uint32_t w, uint32_t h, const bh_image_loss_config& cfg,
                                const float* dl_dmap, float* dl_dpred);

// adam.hip
bh_status launch_adam_step(bh_ctx* ctx, float* param, const float* grad, float* m1, float* m2,
                           const float* scaling, uint32_t rows, uint32_t row_len, bool reduce, float lr,
                           uint32_t time, const bh_adam_config& cfg);

// ply.hip
bh_status launch_ply_decode_rows(bh_ctx* ctx, const uint8_t* rows, uint64_t rows_bytes, uint32_t row_bytes,
                                 uint64_t n_out, uint32_t subsample, uint32_t flags, const bh_ply_column* columns,
                                 uint32_t num_coeffs, float* transforms, float* sh, float* opac);
bh_status launch_ply_decode_compressed(bh_ctx* ctx, const float* chunks, const uint8_t* vrows, const uint8_t* srows,
                                       uint64_t n_out, uint32_t subsample, uint32_t flags,
                                       const bh_ply_compressed_layout& layout, float* transforms, float* sh,
                                       float* opac);
bh_status launch_ply_encode_rows(bh_ctx* ctx, const float* transforms, const float* sh, const float* opac, uint64_t n,
                                 uint32_t num_coeffs, float* rows);

}  // namespace bh

struct bh_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string last_error;
    bh::Pool pool;
    bool timing = false;
    std::string timing_filter;  // empty: time every kernel
    std::vector<bh::Timing> pending;
    std::vector<hipEvent_t> event_cache;
    std::vector<std::pair<std::string, bh::TimingTotal>> totals;
    bh::KernelTimer* timer = nullptr;  // the timer whose scope is open (bh::launch binds its events)
    // small device scratch: [0] num_visible, [1] error flags,
    // [2..3] num_intersections (u64), [4] min depth key, [5] max depth key,
    // [6] depth key cap, [7] intersections when they fit the planned capacity
    uint32_t* d_counters = nullptr;
    // pinned, mapped host copy of the eight counters; word 8 is the
    // generation of the reduction that wrote them, stored after them
    uint32_t* h_counters = nullptr;
    uint32_t* h_counters_dev = nullptr;  // h_counters as the device addresses it
    uint32_t count_generation = 0;       // of the last reduction queued
    // The forward's plan for the launches that depend on its counts, taken
    // from the previous forward on this context: the depth key width and the
    // intersection capacity (valid once a forward with splats has run).
    bool plan_valid = false;
    uint32_t plan_key_bits = 32;
    uint32_t plan_isect_cap = 0;
    // device address of the allocation-free entry point's fixed scratch on
    // this context's device (null when it could not be located)
    void* noalloc_scratch = nullptr;
    // BH_DEBUG_* flags (bh_ctx_set_debug)
    uint32_t debug = 0;
};

namespace bh {

constexpr uint32_t kErrOverflow = 2u;  // a count exceeded its field

// Scoped timing of one kernel launch on the context's stream.  The timer
// takes two events from the context and `launch` binds them to the kernel's
// own dispatch: hipExtLaunchKernel sets them from the kernel's start and end
// timestamps, so a timed kernel has no marker packets around it (a marker
// between two kernels left the GPU idle for ~5 us).  A launch binds the
// innermost open timer, and a timer binds only the first launch in its scope.
struct KernelTimer {
    bh_ctx* ctx;
    const char* name;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    bool bound = false;
    KernelTimer* outer = nullptr;
    KernelTimer(bh_ctx* c, const char* n);
    ~KernelTimer();
    KernelTimer(const KernelTimer&) = delete;
    KernelTimer& operator=(const KernelTimer&) = delete;
};

// Every kernel of the library is launched through here, on the context's
// stream, so that an open KernelTimer times it.
template <typename F, typename... Args>
inline void launch(bh_ctx* ctx, F kernel, dim3 grid, dim3 block, uint32_t lds, Args... args) {
    hipEvent_t e0 = nullptr, e1 = nullptr;
    KernelTimer* t = ctx->timer;
    if (t && t->e0 && t->e1 && !t->bound) {
        e0 = t->e0;
        e1 = t->e1;
        t->bound = true;
    }
    hipExtLaunchKernelGGL(kernel, grid, block, lds, ctx->stream, e0, e1, 0u, args...);
}

bh_status set_error(bh_ctx* ctx, bh_status st, const std::string& msg);
bh_status check_launch(bh_ctx* ctx, const char* what);

inline uint32_t div_up(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

// ---- kernel launchers implemented in the .hip translation units ----------------

// fill.hip
void launch_fill_u32(bh_ctx* ctx, uint32_t* p, uint32_t value, uint64_t count);
// Several fills in one launch (at most kMaxFillRanges; empty ranges allowed).
struct FillRange {
    uint32_t* p;
    uint32_t value;
    uint64_t count;
};
constexpr int kMaxFillRanges = 8;
struct FillRanges {
    FillRange r[kMaxFillRanges];
    int k;
};
// Thread `tid` of `stride` threads fills its share of every range in turn (the
// range index is uniform): single words up to each range's first 16-byte
// boundary and after its last, 16-byte stores between (non-temporal with NT:
// streamed past the caches other kernels are using).
template <bool NT>
__device__ __forceinline__ void fill_ranges_strided(const FillRanges& ranges, uint64_t tid, uint64_t stride) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    for (int j = 0; j < ranges.k; j++) {
        uint32_t* p = ranges.r[j].p;
        const uint32_t value = ranges.r[j].value;
        const uint64_t count = ranges.r[j].count;
        const uint64_t head = min<uint64_t>(count, ((16u - (reinterpret_cast<uintptr_t>(p) & 15u)) & 15u) / 4u);
        if (tid < head) p[tid] = value;
        const uint64_t quads = (count - head) / 4u;
        u32x4* q = reinterpret_cast<u32x4*>(p + head);
        const u32x4 v4 = {value, value, value, value};
        for (uint64_t i = tid; i < quads; i += stride) {
            if (NT)
                __builtin_nontemporal_store(v4, q + i);
            else
                q[i] = v4;
        }
        for (uint64_t i = head + quads * 4u + tid; i < count; i += stride) p[i] = value;
    }
}
void launch_fill_multi(bh_ctx* ctx, const FillRange* ranges, int k);
// Ranges a kernel zeroes beside its own work (a grid-stride loop per range;
// unused ranges have count 0), in place of a fill launch of their own.
struct ZeroRanges {
    uint32_t* p[4];
    uint64_t count[4];
};
// Debug validation: first[j] (u64, ~0 when none) = the index of the first NaN
// or infinity in float array j; first holds kMaxFiniteArrays entries.
constexpr int kMaxFiniteArrays = 4;
struct FiniteArrays {
    const float* p[kMaxFiniteArrays];
    uint64_t n[kMaxFiniteArrays];
    int k;
};
void launch_first_non_finite(bh_ctx* ctx, const FiniteArrays& a, unsigned long long* first);

// sort.hip
size_t radix_sort_scratch_bytes(uint32_t n, uint32_t key_bits);
// Sort inputs the kernels read from device memory instead of the host
// arguments (null: the host argument).  With `n`, the host n is a capacity
// that sizes the grid and the scratch, and the sort covers the first
// min(n, *dev.n) pairs; with key_sub / key_cap, the first pass's key
// transform takes its two constants from there.
struct SortDevice {
    const uint32_t* n = nullptr;
    const uint32_t* key_sub = nullptr;
    const uint32_t* key_cap = nullptr;
    // with drop_capped: the pairs left after the first pass (a capacity's
    // actual count; the host value is n_rest)
    const uint32_t* n_rest = nullptr;
    // the first pass drops every pair whose transformed key equals key_cap
    // (the depth sort's culled splats), so later passes sort n_rest pairs
    bool drop_capped = false;
    uint32_t n_rest_host = 0;
    // the first pass's upsweep also adds weight[index] of each counted key to
    // wsum[block][digit] (depth_sort_buckets: a digit's sum of tile counts)
    const uint32_t* weight = nullptr;
    uint32_t* wsum = nullptr;
};
// Stable sort of (key', value) pairs by the low key_bits bits of
// key' = min(key - key_sub, key_cap), in ceil(key_bits / 8) passes of equal
// digit width.  vals_in == nullptr means vals = index.  The transformed keys
// are what the sort emits.  tmp_* are n-element buffers.
// The first radix_sort_zeroed_words(n, key_bits) words of `scratch` must be
// zero when the sort starts; with scratch_zeroed the caller has done that
// (it may size the fill for 32 key bits, which covers any key_bits).
size_t radix_sort_zeroed_words(uint32_t n, uint32_t key_bits);
// With gather_out, the last pass also writes gather_out[i] =
// gather_src[vals_out[i]] (an n-element buffer).
bh_status radix_sort_pairs(bh_ctx* ctx, const uint32_t* keys_in, const uint32_t* vals_in, uint32_t n,
                           uint32_t key_bits, uint32_t key_sub, uint32_t key_cap, uint32_t* keys_out,
                           uint32_t* vals_out, uint32_t* tmp_keys, uint32_t* tmp_vals, void* scratch,
                           const char* tag = "radix", bool scratch_zeroed = false,
                           const uint32_t* gather_src = nullptr, uint32_t* gather_out = nullptr,
                           const SortDevice& dev = SortDevice{});
// The same over 16-bit keys (key_bits <= 16, no key transform): keys_in and
// tmp_keys hold uint16_t, the sorted keys land in keys_out as uint32_t.
bh_status radix_sort_pairs_k16(bh_ctx* ctx, const uint16_t* keys_in, const uint32_t* vals_in, uint32_t n,
                               uint32_t key_bits, uint32_t* keys_out, uint32_t* vals_out, uint16_t* tmp_keys,
                               uint32_t* tmp_vals, void* scratch, const char* tag = "radix",
                               bool scratch_zeroed = false, const SortDevice& dev = SortDevice{});
// Stable sort of (key', index) pairs as radix_sort_pairs sorts them (key' =
// min(key - key_sub, key_cap), the first pass's drop of capped keys, the
// sorted indices to vals_out), for any key width: one pass by the top 8 bits
// of key_cap's range, then every bucket sorted by one workgroup (in LDS up to
// 16384 pairs), which also writes cum[i] = the inclusive prefix sum of
// weight[vals_out[.]] through i (the forward's tile counts in depth order).
// keys_tmp, tmp_keys and tmp_vals are n-element buffers; the scratch is
// radix_sort_scratch_bytes(n, 32), its first depth_sort_buckets_zeroed_words(n)
// words zero (or zeroed here unless scratch_zeroed; at most
// radix_sort_zeroed_words(n, 32)).
bh_status depth_sort_buckets(bh_ctx* ctx, const uint32_t* keys_in, uint32_t n, uint32_t key_sub, uint32_t key_cap,
                             uint32_t* keys_tmp, uint32_t* vals_out, uint32_t* tmp_keys, uint32_t* tmp_vals,
                             void* scratch, bool scratch_zeroed, const uint32_t* weight, uint32_t* cum,
                             const SortDevice& dev);
size_t depth_sort_buckets_zeroed_words(uint32_t n);
// out[i] = in[i] & mask
void launch_mask_u32(bh_ctx* ctx, const uint32_t* in, uint32_t mask, uint32_t n, uint32_t* out);
// keys_out[i] = keys_in[perm[i]], vals_out[i] = vals_in[perm[i]]
void launch_gather_pairs(bh_ctx* ctx, const uint32_t* keys_in, const uint32_t* vals_in, const uint32_t* perm,
                         uint32_t n, uint32_t* keys_out, uint32_t* vals_out);
size_t scan_scratch_bytes(uint32_t n);
// Inclusive scan of in[0, n); out may alias in.  With dev_n, n is a capacity
// and the scan covers in[0, min(n, *dev_n)).
bh_status inclusive_scan(bh_ctx* ctx, const uint32_t* in, uint32_t* out, uint32_t n, void* scratch,
                         const uint32_t* dev_n = nullptr);

// project.hip
size_t project_partials_bytes(uint32_t n);
// Also writes each visible splat's projected row into rows [n, 16] (its
// global-id slot), for launch_project_visible to order by depth.  With
// host_counters (device address of mapped host memory), the reduction also
// stores the eight counters there and then `generation` in word 8.
void launch_project_forward(bh_ctx* ctx, const bh_project_uniforms& u, const float* transforms,
                            const float* raw_opac, const float* sh, uint32_t sh_degree, uint32_t n, bool mip,
                            uint32_t tile_h, uint32_t* intersect_counts, float* max_radius, uint32_t* depth_keys,
                            float* rows, uint32_t* partials, uint32_t* counters, uint32_t isect_cap = 0,
                            const ZeroRanges& zero = ZeroRanges{}, uint32_t* host_counters = nullptr,
                            uint32_t generation = 0);
void launch_project_visible(bh_ctx* ctx, const float* rows, const uint32_t* gfc, uint32_t num_visible,
                            uint32_t num_splats, float* projected, float* depths);
// Also writes compact rows `projected` [V,10] and `depths` [V] from the
// global-id rows of launch_project_forward, and zeroes zero[0, zero_words)
// (the tile sort's scratch).  With dev (the context counters after
// project_forward), num_visible is a capacity: the kernel reads the visible
// count from dev[0] and writes intersections only when they fit the buffers.
// The tile ids are written as uint16_t when tile_ids16 is set (fewer than
// 2^16 tiles, the sentinel included), else as uint32_t.  m_cap is the pair
// buffers' size: no pair is stored at or past it.
void launch_map_intersects(bh_ctx* ctx, uint32_t tile_bw, uint32_t tile_bh, uint32_t tile_h, const float* rows,
                           const uint32_t* gfc, uint32_t num_splats, const uint32_t* cum, uint32_t num_visible,
                           float* projected, float* depths, void* tile_ids, bool tile_ids16, uint32_t* cgids,
                           uint32_t* zero, uint32_t zero_words, const uint32_t* dev, uint32_t m_cap);

// raster.hip
// With dev_m, m is a capacity and the ids are tile_ids[0, min(m, *dev_m)).
void launch_tile_offsets(bh_ctx* ctx, const uint32_t* tile_ids, uint32_t m, uint32_t num_tiles,
                         uint32_t* offsets, bool zeroed = false, const uint32_t* dev_m = nullptr);
// order[num_tiles]: the tiles by descending load (launch_tile_order), or
// nullptr for tile-id order.
void launch_tile_order(bh_ctx* ctx, const uint32_t* offsets, uint32_t num_tiles, uint32_t* order);
// p[0, words) = 0 (p 16-byte aligned) and the tile order, in one launch.
void launch_zero_and_tile_order(bh_ctx* ctx, uint32_t* p, uint64_t words, const uint32_t* offsets,
                                uint32_t num_tiles, uint32_t* order);
// With BWD_INFO and rec.masks set, the blend also records its contributing
// pairs for the fused backward (bh_splat_record.h), and with rec.order.list
// the backward's dispatch order.  With BWD_INFO, workgroups after the blend's
// zero fill[0, fill_words) (16-byte aligned) in its tail.
void launch_rasterize(bh_ctx* ctx, uint32_t img_w, uint32_t img_h, uint32_t tile_bw, uint32_t tile_bh,
                      const float* bg, uint32_t num_visible, const float* projected, const uint32_t* cgids,
                      const uint32_t* gfc, const uint32_t* off_pre, const uint32_t* order, uint32_t flags,
                      void* out_img, float* visible, uint32_t* off_post, bool off_post_zeroed = false,
                      SplatRecord rec = SplatRecord{}, uint32_t* fill = nullptr, uint64_t fill_words = 0);

// backward.hip
void launch_rasterize_backward(bh_ctx* ctx, uint32_t img_w, uint32_t img_h, uint32_t tile_bw, uint32_t tile_bh,
                               const float* bg, uint32_t num_visible, const float* out_img, const float* projected,
                               const uint32_t* cgids, const uint32_t* offsets, const float* v_output,
                               uint32_t flags, const uint32_t* row_of, const uint32_t* order, float* v_combined);
// The fused backward's rasterize step from the forward's record; v_rows is
// indexed by row_of[compact id] (the global id).  Workgroups of the same
// launch, spread among the blend's, zero the zero_k ranges of `zero` (the
// blend neither reads nor writes them); returns whether they were zeroed
// (false when nothing was launched or more than kMaxFillRanges were given).
bool launch_rasterize_backward_recorded(bh_ctx* ctx, uint32_t img_w, uint32_t img_h, uint32_t tile_bw,
                                        uint32_t tile_bh, const float* bg, uint32_t num_visible, const float* out_img,
                                        const float* projected, const uint32_t* cgids, const uint32_t* off_pre,
                                        const SplatRecord& rec, const float* v_output, uint32_t flags,
                                        const uint32_t* row_of, const uint32_t* order, float* v_rows,
                                        const FillRange* zero = nullptr, int zero_k = 0);
void launch_invert_permutation(bh_ctx* ctx, const uint32_t* gfc, uint32_t num_visible, uint32_t n,
                               uint32_t* compact_from_global);
// compact_from_global == nullptr: v_combined is indexed by global id.  With
// zeroed the four gradient arrays are already zero (the splats without a
// gradient are skipped instead of zero-filled).
void launch_project_backward(bh_ctx* ctx, const bh_project_uniforms& u, const float* transforms, const float* sh,
                             const float* raw_opac, const uint32_t* compact_from_global, uint32_t n,
                             uint32_t sh_degree, bool mip, const float* v_combined, float* v_transforms,
                             float* v_coeffs, float* v_raw_opac, float* v_refine, bool zeroed = false);

}  // namespace bh
