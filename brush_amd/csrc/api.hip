// api.hip — C ABI of the gfx950 rasterizer (include/brush_hip.h).
//
// Host orchestration of the forward pass (crates/brush-render/src/render.rs:78-543
// restated) and of the two backward operations
// (crates/brush-render-bwd/src/render_bwd.rs:90-447 restated).  All work is
// queued on the context's stream; the forward reads back one 24-byte block of
// counters (visible count, intersection count, depth-key range, error flags).
#include <hip/hip_runtime.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <mutex>
#include <new>
#include <string>

#include <rocprofiler-sdk-roctx/roctx.h>

#include "bh_internal.h"

struct bh_fwd_state {
    bh_ctx* ctx;
    bh_fwd_info info;
    std::vector<void*> buffers;
    // the blend's record of contributing pairs (forward with BWD_INFO and
    // intersections), read by bh_render_backward
    bh::SplatRecord record;
    // gradient rows [N, 11] the forward zeroed for the backward (beside its
    // tile-order launch, which leaves the rest of the GPU idle); the first
    // backward takes them, a later one zeroes its own
    float* bwd_rows = nullptr;
    bool bwd_rows_clean = false;
    // BH_DEBUG_KEEP_LANES: the gradient lanes the latest backward accumulated
    float* kept_lanes = nullptr;

    // returns one of the state's buffers to the pool (stream ordered: later
    // users of the block run after the work already queued on it)
    void drop(void* p) {
        if (!p) return;
        auto it = std::find(buffers.begin(), buffers.end(), p);
        if (it == buffers.end()) return;
        buffers.erase(it);
        ctx->pool.release(p);
    }
};

namespace bh {

static const size_t kAlign = 256;

// Requests above 1 MiB are rounded up to a size class of 1/8 of their power
// of two (at most 12.5 % over), and a request that misses the cache allocates
// a block with 25 % headroom (the cache serves requests down to half a
// block's size), so a buffer whose size creeps up from call to call (the
// intersection count of a scene that is being trained, the per-splat arrays of
// a scene that densifies) keeps reusing one block instead of missing the cache
// and allocating every call.
static size_t size_class(size_t bytes) {
    bytes = std::max<size_t>(kAlign, (bytes + kAlign - 1) / kAlign * kAlign);
    if (bytes <= ((size_t)1 << 20)) return bytes;
    size_t top = (size_t)1 << (63 - __builtin_clzll((unsigned long long)bytes));
    const size_t step = top / 8;
    return (bytes + step - 1) / step * step;
}

hipError_t Pool::alloc(void** out, size_t bytes) {
    bytes = size_class(bytes);
    size_t best = (size_t)-1;
    for (size_t i = 0; i < free_blocks.size(); i++) {
        const Block& b = free_blocks[i];
        if (b.bytes >= bytes && b.bytes <= 2 * bytes + (1u << 20) &&
            (best == (size_t)-1 || b.bytes < free_blocks[best].bytes))
            best = i;
    }
    if (best != (size_t)-1) {
        Block b = free_blocks[best];
        free_blocks.erase(free_blocks.begin() + best);
        cached_bytes -= b.bytes;
        live[b.ptr] = b.bytes;
        *out = b.ptr;
        return hipSuccess;
    }
    void* p = nullptr;
    size_t got = size_class(bytes + bytes / 4);
    hipError_t e = hipMalloc(&p, got);
    if (e != hipSuccess) {
        // drop the cache and try once more, then without headroom
        (void)hipGetLastError();
        trim();
        e = hipMalloc(&p, got);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            got = bytes;
            e = hipMalloc(&p, got);
            if (e != hipSuccess) return e;
        }
    }
    live[p] = got;
    *out = p;
    return hipSuccess;
}

void Pool::release(void* ptr) {
    if (!ptr) return;
    auto it = live.find(ptr);
    if (it == live.end()) return;
    free_blocks.push_back(Block{ptr, it->second});
    cached_bytes += it->second;
    live.erase(it);
}

void Pool::trim() {
    for (auto& b : free_blocks) (void)hipFree(b.ptr);
    free_blocks.clear();
    cached_bytes = 0;
}

StageRange::StageRange(const char* name) { roctxRangePushA(name); }
StageRange::~StageRange() { roctxRangePop(); }

KernelTimer::KernelTimer(bh_ctx* c, const char* n) : ctx(c), name(n), outer(c->timer) {
    ctx->timer = this;
    if (!ctx->timing) return;
    if (!ctx->timing_filter.empty() && ctx->timing_filter != n) return;
    auto get = [&]() {
        hipEvent_t e = nullptr;
        if (!ctx->event_cache.empty()) {
            e = ctx->event_cache.back();
            ctx->event_cache.pop_back();
        } else if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) {
            // timing-only events: no system-scope fence (cache writeback and
            // invalidate) that would slow the kernels after the timed one
            e = nullptr;
        }
        return e;
    };
    e0 = get();
    e1 = get();
}

KernelTimer::~KernelTimer() {
    ctx->timer = outer;
    if (bound) {
        ctx->pending.push_back(Timing{name, e0, e1});
        return;
    }
    if (e0) ctx->event_cache.push_back(e0);
    if (e1) ctx->event_cache.push_back(e1);
}

bh_status set_error(bh_ctx* ctx, bh_status st, const std::string& msg) {
    if (ctx) ctx->last_error = msg;
    return st;
}

bh_status check_launch(bh_ctx* ctx, const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(ctx, BH_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
    return BH_OK;
}

static bh_status hip_check(bh_ctx* ctx, hipError_t e, const char* what) {
    if (e == hipSuccess) return BH_OK;
    (void)hipGetLastError();
    return set_error(ctx, e == hipErrorOutOfMemory ? BH_ERR_OOM : BH_ERR_DEVICE,
                     std::string(what) + ": " + hipGetErrorString(e));
}

// Waits for the counts of the reduction of generation `gen`: the kernel stores
// the eight counters in mapped host memory and then, after a system-scope
// fence, `gen` in word 8, so the host polls that word (no event marker on the
// stream).  A spin that has not seen it after 20 ms (the stream is far
// behind, or a launch failed) synchronises the stream instead, which reports
// a failed kernel; after that the word must be there.
static bh_status wait_counters(bh_ctx* ctx, uint32_t gen) {
    const auto seen = [&]() { return __atomic_load_n(ctx->h_counters + 8, __ATOMIC_ACQUIRE) == gen; };
    const auto t0 = std::chrono::steady_clock::now();
    for (uint32_t i = 1; !seen(); i++) {
        if ((i & 255u) == 0u && std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(20)) {
            const bh_status st = hip_check(ctx, hipStreamSynchronize(ctx->stream), "count readback");
            if (st != BH_OK) return st;
            if (!seen()) return set_error(ctx, BH_ERR_INTERNAL, "count readback: the reduction stored no counts");
            break;
        }
        __builtin_ia32_pause();
    }
    return BH_OK;
}

#define BH_TRY(expr)                      \
    do {                                  \
        bh_status _st = (expr);           \
        if (_st != BH_OK) return _st;     \
    } while (0)

// BH_DEBUG_POISON: a block handed out is first filled with 0xFF bytes (stream
// ordered, so before any kernel that uses it).  Blocks are at least 4-byte
// sized pool allocations, so rounding the byte count up to words stays inside.
static void poison(bh_ctx* ctx, void* p, size_t bytes) {
    if (ctx->debug & BH_DEBUG_POISON) launch_fill_u32(ctx, (uint32_t*)p, 0xFFFFFFFFu, (bytes + 3) / 4);
}

// RAII set of pool buffers released (stream ordered) at scope exit.
struct Scratch {
    bh_ctx* ctx;
    std::vector<void*> bufs;
    explicit Scratch(bh_ctx* c) : ctx(c) {}
    ~Scratch() {
        for (void* p : bufs) ctx->pool.release(p);
    }
    template <class T>
    bh_status get(T** out, size_t count) {
        void* p = nullptr;
        const size_t bytes = std::max<size_t>(count, 1) * sizeof(T);
        hipError_t e = ctx->pool.alloc(&p, bytes);
        if (e != hipSuccess) return hip_check(ctx, e, "workspace allocation");
        bufs.push_back(p);
        poison(ctx, p, bytes);
        *out = (T*)p;
        return BH_OK;
    }
};

// BH_DEBUG_VALIDATE: the first NaN or infinity of each array, reported as the
// reference's validation names it (validation.rs:6-84).  names[j] is the
// array's name, or nullptr for the transforms, whose columns are the means,
// rotations and log-scales.
static bh_status check_finite(bh_ctx* ctx, const char* what, const FiniteArrays& a, const char* const* names) {
    Scratch ws(ctx);
    unsigned long long* first;
    BH_TRY(ws.get(&first, kMaxFiniteArrays));
    launch_first_non_finite(ctx, a, first);
    BH_TRY(check_launch(ctx, "validation"));
    unsigned long long h[kMaxFiniteArrays];
    BH_TRY(hip_check(ctx, hipMemcpyAsync(h, first, sizeof(h), hipMemcpyDeviceToHost, ctx->stream), "validation"));
    BH_TRY(hip_check(ctx, hipStreamSynchronize(ctx->stream), "validation"));
    for (int j = 0; j < a.k; j++) {
        if (h[j] == ~0ull) continue;
        std::string name = names[j] ? names[j] : "";
        if (!names[j]) {
            const uint64_t col = h[j] % 10u;
            name = col < 3u ? "means" : col < 7u ? "rotations" : "log_scales";
        }
        return set_error(ctx, BH_ERR_NOT_FINITE,
                         std::string(what) + ": tensor '" + name + "' has a NaN or Inf (first @ flat index " +
                             std::to_string(h[j]) + ")");
    }
    return BH_OK;
}


// Workspace of bh_radix_argsort_noalloc: a fixed device array instead of the
// pool.  Each GPU the library runs on holds its own copy until the process
// ends.  In host code `scratch` names a host-side stand-in, never the device
// memory: its device address is looked up once per device
// (hipGetSymbolAddress, with that device current) and only that address is
// handed to kernels.  Every call on one device shares the array, so calls that
// overlap on one device race; each call clears what must start at zero.
constexpr size_t kNoAllocScratchBytes = (size_t)48 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mutex;
static void* g_scratch_addr[kMaxDevices];

// The device address of `scratch` on `device`, which must be current.
static hipError_t noalloc_scratch_address(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_addr[device]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return e;
        }
        g_scratch_addr[device] = ptr;
    }
    *out = g_scratch_addr[device];
    return hipSuccess;
}

// Hands out 256-byte aligned pieces of a fixed device region, front to back.
struct Bump {
    bh_ctx* ctx;
    char* base;
    size_t cap, used = 0;
    Bump(bh_ctx* c, void* b, size_t n) : ctx(c), base((char*)b), cap(n) {}
    template <class T>
    bh_status get(T** out, size_t count) {
        const size_t bytes = (std::max<size_t>(count, 1) * sizeof(T) + kAlign - 1) / kAlign * kAlign;
        if (bytes > cap - used)
            return set_error(ctx, BH_ERR_INVALID_ARG, "radix_argsort_noalloc: workspace exceeds the fixed scratch");
        *out = (T*)(base + used);
        used += bytes;
        poison(ctx, *out, bytes);
        return BH_OK;
    }
};

static uint32_t bit_length(uint32_t x) { return x ? 32u - (uint32_t)__builtin_clz(x) : 0u; }
// the largest splat count and depth-key width the depth sort's bucket path takes
constexpr uint32_t kBucketSortMaxSplats = 1u << 21;
constexpr uint32_t kBucketSortMaxKeyBits = 24;

// bh_radix_argsort's body over a workspace provider (the pool, or the fixed
// scratch of the allocation-free entry point).
template <class Ws>
static bh_status radix_argsort_with(bh_ctx* ctx, Ws& ws, const uint32_t* keys_in, const uint32_t* vals_in,
                                    uint32_t n, uint32_t sorting_bits, uint32_t* keys_out, uint32_t* vals_out) {
    // brush-sort runs ceil(bits/4) 4-bit passes, i.e. it orders by the low
    // 4*ceil(bits/4) key bits; keep exactly that key width.
    const uint32_t width = 4u * ((sorting_bits + 3u) / 4u);
    if (width == 0) {
        bh_status st = hip_check(
            ctx, hipMemcpyAsync(keys_out, keys_in, (size_t)n * 4, hipMemcpyDeviceToDevice, ctx->stream), "copy");
        if (st != BH_OK) return st;
        return hip_check(ctx, hipMemcpyAsync(vals_out, vals_in, (size_t)n * 4, hipMemcpyDeviceToDevice, ctx->stream),
                         "copy");
    }
    const uint32_t mask = width >= 32 ? 0xFFFFFFFFu : ((1u << width) - 1u);
    uint32_t *tk, *tv, *masked = nullptr;
    void* digit_scratch;
    BH_TRY(ws.get(&tk, n));
    BH_TRY(ws.get(&tv, n));
    BH_TRY(ws.get((char**)&digit_scratch, radix_sort_scratch_bytes(n, width)));
    if (mask != 0xFFFFFFFFu) {
        // Sort (key & mask, index) then gather: the emitted keys must be the
        // caller's original keys, including any bits above the key width.
        uint32_t *perm, *sk;
        BH_TRY(ws.get(&masked, n));
        BH_TRY(ws.get(&perm, n));
        BH_TRY(ws.get(&sk, n));
        launch_mask_u32(ctx, keys_in, mask, n, masked);
        BH_TRY(radix_sort_pairs(ctx, masked, nullptr, n, width, 0u, 0xFFFFFFFFu, sk, perm, tk, tv, digit_scratch));
        launch_gather_pairs(ctx, keys_in, vals_in, perm, n, keys_out, vals_out);
        return check_launch(ctx, "radix_argsort gather");
    }
    return radix_sort_pairs(ctx, keys_in, vals_in, n, width, 0u, 0xFFFFFFFFu, keys_out, vals_out, tk, tv,
                            digit_scratch);
}

// Below this many splats project backward zero-fills the dense gradients
// itself instead of the rasterize backward's fill workgroups.
#ifndef BH_FUSED_FILL_MIN
#define BH_FUSED_FILL_MIN 0
#endif
constexpr uint32_t kFusedFillMinSplats = BH_FUSED_FILL_MIN;

static bh_status check_device_error(bh_ctx* ctx, uint32_t flags) {
    if (flags & kErrOverflow) return set_error(ctx, BH_ERR_INTERNAL, "a device count overflowed");
    return BH_OK;
}

}  // namespace bh

using namespace bh;

extern "C" {

bh_status bh_ctx_create(int device, bh_ctx** out) {
    if (!out) return BH_ERR_INVALID_ARG;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) {
        (void)hipGetLastError();
        return BH_ERR_DEVICE;
    }
    if (hipSetDevice(device) != hipSuccess) return BH_ERR_DEVICE;
    bh_ctx* ctx = new (std::nothrow) bh_ctx();
    if (!ctx) return BH_ERR_OOM;
    ctx->device = device;
    // the allocation-free entry point's scratch on this device (looked up
    // once per device; a failure only disables that entry point)
    if (noalloc_scratch_address(device, &ctx->noalloc_scratch) != hipSuccess) ctx->noalloc_scratch = nullptr;
    // the counters' pinned host copy is written by the reduction kernel itself
    // (mapped, coherent host memory), so no copy runs between it and the reads
    if (hipMalloc(&ctx->d_counters, 64) != hipSuccess ||
        hipHostMalloc(&ctx->h_counters, 64, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess ||
        hipHostGetDevicePointer((void**)&ctx->h_counters_dev, ctx->h_counters, 0) != hipSuccess) {
        (void)hipGetLastError();
        if (ctx->d_counters) (void)hipFree(ctx->d_counters);
        if (ctx->h_counters) (void)hipHostFree(ctx->h_counters);
        delete ctx;
        return BH_ERR_OOM;
    }
    memset(ctx->h_counters, 0, 64);  // generation 0: no reduction has stored counts
    *out = ctx;
    return BH_OK;
}

void bh_ctx_destroy(bh_ctx* ctx) {
    if (!ctx) return;
    (void)hipStreamSynchronize(ctx->stream);
    for (auto& t : ctx->pending) {
        (void)hipEventDestroy(t.start);
        (void)hipEventDestroy(t.stop);
    }
    for (auto e : ctx->event_cache) (void)hipEventDestroy(e);
    ctx->pool.trim();
    for (auto& kv : ctx->pool.live) (void)hipFree(kv.first);
    (void)hipFree(ctx->d_counters);
    (void)hipHostFree(ctx->h_counters);
    delete ctx;
}

bh_status bh_ctx_set_stream(bh_ctx* ctx, void* hip_stream) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    hipStream_t s = (hipStream_t)hip_stream;
    if (s != ctx->stream) {
        BH_TRY(hip_check(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize"));
        ctx->stream = s;
    }
    return BH_OK;
}

const char* bh_last_error(const bh_ctx* ctx) { return ctx ? ctx->last_error.c_str() : "null context"; }

bh_status bh_ctx_set_timing(bh_ctx* ctx, int enable) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    ctx->timing = enable != 0;
    return BH_OK;
}

bh_status bh_ctx_set_timing_filter(bh_ctx* ctx, const char* name) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    ctx->timing_filter = name ? name : "";
    return BH_OK;
}

static bh_status collect_timings(bh_ctx* ctx) {
    BH_TRY(hip_check(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize"));
    for (auto& t : ctx->pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, t.start, t.stop) != hipSuccess) {
            (void)hipGetLastError();
            ms = 0.0f;
        }
        auto it = std::find_if(ctx->totals.begin(), ctx->totals.end(),
                               [&](const std::pair<std::string, TimingTotal>& kv) { return kv.first == t.name; });
        if (it == ctx->totals.end()) {
            ctx->totals.push_back({t.name, TimingTotal{}});
            it = ctx->totals.end() - 1;
        }
        it->second.launches += 1;
        it->second.total_ms += ms;
        ctx->event_cache.push_back(t.start);
        ctx->event_cache.push_back(t.stop);
    }
    ctx->pending.clear();
    return BH_OK;
}

bh_status bh_ctx_read_timings(bh_ctx* ctx, bh_kernel_timing* out, int max, int* count) {
    if (!ctx || !count) return BH_ERR_INVALID_ARG;
    BH_TRY(collect_timings(ctx));
    int n = 0;
    for (auto& kv : ctx->totals) {
        if (n >= max || !out) break;
        memset(out[n].name, 0, sizeof(out[n].name));
        strncpy(out[n].name, kv.first.c_str(), sizeof(out[n].name) - 1);
        out[n].launches = kv.second.launches;
        out[n].total_ms = kv.second.total_ms;
        n++;
    }
    *count = out ? n : (int)ctx->totals.size();
    return BH_OK;
}

bh_status bh_ctx_reset_timings(bh_ctx* ctx) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    BH_TRY(collect_timings(ctx));
    ctx->totals.clear();
    return BH_OK;
}

bh_status bh_ctx_set_debug(bh_ctx* ctx, uint32_t flags) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    if (flags & ~(BH_DEBUG_POISON | BH_DEBUG_VALIDATE | BH_DEBUG_EXACT_SIZES | BH_DEBUG_KEEP_LANES))
        return set_error(ctx, BH_ERR_INVALID_ARG, "set_debug: unknown flag");
    ctx->debug = flags;
    return BH_OK;
}

uint64_t bh_ctx_workspace_bytes(const bh_ctx* ctx) {
    if (!ctx) return 0;
    uint64_t b = ctx->pool.cached_bytes;
    for (auto& kv : ctx->pool.live) b += kv.second;
    return b;
}

bh_status bh_ctx_release_workspace(bh_ctx* ctx) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    BH_TRY(hip_check(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize"));
    ctx->pool.trim();
    return BH_OK;
}

bh_status bh_radix_argsort(bh_ctx* ctx, const uint32_t* keys_in, const uint32_t* vals_in, uint32_t n,
                           uint32_t sorting_bits, uint32_t* keys_out, uint32_t* vals_out) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    if (sorting_bits > 32) return set_error(ctx, BH_ERR_INVALID_ARG, "Can only sort up to 32 bits");
    if (n == 0) return BH_OK;
    if (!keys_in || !vals_in || !keys_out || !vals_out)
        return set_error(ctx, BH_ERR_INVALID_ARG, "radix_argsort: null pointer");
    if (keys_in == keys_out || vals_in == vals_out)
        return set_error(ctx, BH_ERR_INVALID_ARG, "radix_argsort: outputs must not alias inputs");
    Scratch ws(ctx);
    return radix_argsort_with(ctx, ws, keys_in, vals_in, n, sorting_bits, keys_out, vals_out);
}

bh_status bh_radix_argsort_noalloc(bh_ctx* ctx, const uint32_t* keys_in, const uint32_t* vals_in, uint32_t n,
                                   uint32_t sorting_bits, uint32_t* keys_out, uint32_t* vals_out) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    if (sorting_bits > 32) return set_error(ctx, BH_ERR_INVALID_ARG, "Can only sort up to 32 bits");
    if (n == 0) return BH_OK;
    if (!keys_in || !vals_in || !keys_out || !vals_out)
        return set_error(ctx, BH_ERR_INVALID_ARG, "radix_argsort_noalloc: null pointer");
    if (keys_in == keys_out || vals_in == vals_out)
        return set_error(ctx, BH_ERR_INVALID_ARG, "radix_argsort_noalloc: outputs must not alias inputs");
    if (n > BH_NOALLOC_SORT_MAX_KEYS)
        return set_error(ctx, BH_ERR_INVALID_ARG,
                         "radix_argsort_noalloc: n = " + std::to_string(n) + " exceeds the fixed scratch's maximum of " +
                             std::to_string(BH_NOALLOC_SORT_MAX_KEYS) + " keys");
    if (!ctx->noalloc_scratch)
        return set_error(ctx, BH_ERR_DEVICE, "radix_argsort_noalloc: the device scratch could not be located");
    Bump ws(ctx, ctx->noalloc_scratch, kNoAllocScratchBytes);
    return radix_argsort_with(ctx, ws, keys_in, vals_in, n, sorting_bits, keys_out, vals_out);
}

bh_status bh_prefix_sum(bh_ctx* ctx, const uint32_t* in, uint32_t* out, uint32_t n) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    if (n == 0) return BH_OK;
    if (!in || !out) return set_error(ctx, BH_ERR_INVALID_ARG, "prefix_sum: null pointer");
    Scratch ws(ctx);
    char* sums;
    BH_TRY(ws.get(&sums, scan_scratch_bytes(n)));
    return inclusive_scan(ctx, in, out, n, sums);
}

bh_status bh_get_tile_offsets(bh_ctx* ctx, const uint32_t* ids, uint32_t m, uint32_t num_tiles, uint32_t* offsets) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    if (!offsets || (m && !ids)) return set_error(ctx, BH_ERR_INVALID_ARG, "get_tile_offsets: null pointer");
    launch_tile_offsets(ctx, ids, m, num_tiles, offsets);
    return check_launch(ctx, "get_tile_offsets");
}

bh_status bh_render_forward(bh_ctx* ctx, const bh_project_uniforms* uin, const float background[3],
                            const float* transforms, const float* sh_coeffs, const float* raw_opacities,
                            uint32_t num_splats, uint32_t sh_degree, uint32_t flags, void* out_img, float* visible,
                            float* max_radius, uint32_t* tile_offsets, bh_fwd_state** state_out) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    if (!uin || !background || !state_out) return set_error(ctx, BH_ERR_INVALID_ARG, "render_forward: null argument");
    *state_out = nullptr;
    if (uin->img_w == 0 || uin->img_h == 0)
        return set_error(ctx, BH_ERR_INVALID_ARG, "Can't render images with 0 size.");
    {
        // the tile walks split a box's flattened tile index into row and
        // column through a float reciprocal, exact below 2^21 tiles an image
        const uint64_t tiles = (uint64_t)div_up(uin->img_w, BH_TILE_WIDTH) *
                               div_up(uin->img_h, (flags & BH_FLAG_TILE_16X8) ? 8u : BH_TILE_WIDTH);
        if (tiles >= (1ull << 21))
            return set_error(ctx, BH_ERR_INVALID_ARG, "render_forward: images are limited to 2^21 tiles");
    }
    if (sh_degree > 4) return set_error(ctx, BH_ERR_INVALID_ARG, "sh_degree must be <= 4");
    if (uin->camera_model > BH_CAMERA_TPF) return set_error(ctx, BH_ERR_INVALID_ARG, "unknown camera model");
    const bool bwd = (flags & BH_FLAG_BWD_INFO) != 0;
    const bool mip = (flags & BH_FLAG_MIP) != 0;
    if (!out_img || !tile_offsets || (num_splats && (!transforms || !sh_coeffs || !raw_opacities || !max_radius)) ||
        (bwd && num_splats && !visible))
        return set_error(ctx, BH_ERR_INVALID_ARG, "render_forward: null buffer");

    if ((ctx->debug & BH_DEBUG_VALIDATE) && num_splats) {
        // Splats::validate_values (gaussian_splats.rs:322-380): NaN / Inf in a
        // parameter fails the render before anything is drawn
        const uint32_t nc = (sh_degree + 1u) * (sh_degree + 1u);
        FiniteArrays a{};
        a.p[0] = transforms, a.n[0] = (uint64_t)num_splats * 10u;
        a.p[1] = sh_coeffs, a.n[1] = (uint64_t)num_splats * nc * 3u;
        a.p[2] = raw_opacities, a.n[2] = num_splats;
        a.k = 3;
        const char* names[] = {nullptr, "sh_coeffs", "raw_opacity"};
        BH_TRY(check_finite(ctx, "render", a, names));
    }

    bh_project_uniforms u = *uin;
    // calc_tile_bounds_for_dims (render.rs:36-47): 16x16 tiles, or 16x8 for the
    // candidate rasterizer
    const uint32_t tile_h = (flags & BH_FLAG_TILE_16X8) ? 8u : BH_TILE_WIDTH;
    u.tile_bw = div_up(u.img_w, BH_TILE_WIDTH);
    u.tile_bh = div_up(u.img_h, tile_h);
    u.sh_degree = sh_degree;
    u.total_splats = num_splats;
    u.num_visible = 0;
    const uint32_t num_tiles = u.tile_bw * u.tile_bh;

    bh_fwd_state* st = new (std::nothrow) bh_fwd_state();
    if (!st) return set_error(ctx, BH_ERR_OOM, "render_forward: host allocation");
    st->ctx = ctx;
    memset(&st->info, 0, sizeof(st->info));
    auto sget = [&](void** p, size_t bytes) -> bh_status {
        hipError_t e = ctx->pool.alloc(p, std::max<size_t>(bytes, 4));
        if (e != hipSuccess) return hip_check(ctx, e, "state allocation");
        st->buffers.push_back(*p);
        poison(ctx, *p, std::max<size_t>(bytes, 4));
        return BH_OK;
    };
    auto fail = [&](bh_status s) {
        for (void* p : st->buffers) ctx->pool.release(p);
        delete st;
        return s;
    };
#define BH_STRY(expr)                         \
    do {                                      \
        bh_status _st = (expr);               \
        if (_st != BH_OK) return fail(_st);   \
    } while (0)

    Scratch ws(ctx);
    // off_pre [T, 2], and with BWD_INFO the backward order's per-tile words
    // [T] (u64) and bucket counts behind it: one range that starts at zero
    // (bh_splat_record.h)
    uint32_t *counts = nullptr, *off_pre = nullptr;
    const uint64_t off_pre_words = (uint64_t)num_tiles * 2 + (bwd ? (uint64_t)num_tiles * 2 + kOrderBuckets : 0u);
    BH_STRY(sget((void**)&counts, (size_t)num_splats * 4));
    BH_STRY(sget((void**)&off_pre, (size_t)off_pre_words * 4));

    // The launches after project_forward depend on its counts (visible
    // splats, intersections, depth-key range).  A plan sizes them: the counts
    // themselves, read back first (the reference's order, render.rs:309-329),
    // or the previous forward's plan on this context, with the kernels reading
    // the actual counts from ctx->d_counters.  The host then reads the counts
    // only after everything is queued, while the GPU works, and queues the
    // exact launches again in the rare case that they do not fit the plan.
    struct Plan {
        bool device;          // kernels read the counts from ctx->d_counters
        uint32_t v;           // visible splats (a capacity when device)
        uint32_t m;           // intersections (a capacity when device)
        uint32_t key_bits;    // depth-key bits the depth sort covers
        uint32_t kmin, kcap;  // the depth keys' transform (host plan)
    };
    const bool planned = num_splats && ctx->plan_valid && !(ctx->debug & BH_DEBUG_EXACT_SIZES);

    char *depth_scr = nullptr, *scan_scr = nullptr;
    uint32_t* depth_keys = nullptr;
    float* vis_rows = nullptr;
    if (num_splats) {
        BH_STRY(ws.get(&depth_scr, radix_sort_scratch_bytes(num_splats, 32)));
        BH_STRY(ws.get(&scan_scr, scan_scratch_bytes(num_splats)));
    }
    // Everything the forward needs zeroed, in one launch: the counters' flags
    // word (the reduction kernel writes the others), the visible mask, the
    // depth sort's block sums (sized for 32 key bits, which covers the key
    // range found later), and both tile-offset arrays (empty tiles stay [0, 0]).
    auto zero_outputs = [&](bool counters) {
        const FillRange zero[] = {
            {ctx->d_counters + 1, 0u, counters && num_splats ? 1u : 0u},
            {(uint32_t*)visible, 0u, bwd ? (uint64_t)num_splats : 0u},
            {(uint32_t*)depth_scr, 0u, num_splats ? radix_sort_zeroed_words(num_splats, 32) : 0u},
            {off_pre, 0u, off_pre_words},
            {tile_offsets, 0u, bwd ? (uint64_t)num_tiles * 2 : 0u},
        };
        launch_fill_multi(ctx, zero, (int)(sizeof(zero) / sizeof(zero[0])));
    };
    // with splats, project_forward zeroes these beside its own work (its
    // reduction writes the counters, flags word included)
    ZeroRanges pf_zero{};
    if (num_splats) {
        pf_zero.p[0] = (uint32_t*)visible, pf_zero.count[0] = bwd ? (uint64_t)num_splats : 0u;
        pf_zero.p[1] = (uint32_t*)depth_scr, pf_zero.count[1] = radix_sort_zeroed_words(num_splats, 32);
        pf_zero.p[2] = off_pre, pf_zero.count[2] = off_pre_words;
        pf_zero.p[3] = tile_offsets, pf_zero.count[3] = bwd ? (uint64_t)num_tiles * 2 : 0u;
    } else {
        zero_outputs(true);
    }

    uint32_t num_visible = 0, kmin = 0, kmax = 0;
    uint64_t num_isect = 0;
    auto read_counts = [&]() -> bh_status {
        BH_TRY(wait_counters(ctx, ctx->count_generation));
        num_visible = ctx->h_counters[0];
        num_isect = (uint64_t)ctx->h_counters[2] | ((uint64_t)ctx->h_counters[3] << 32);
        kmin = ctx->h_counters[4];
        kmax = ctx->h_counters[5];
        BH_TRY(check_device_error(ctx, ctx->h_counters[1]));
        if (num_isect > 0xFFFFFFFFull)
            return set_error(ctx, BH_ERR_SHAPE, "more than 2^32 - 1 tile intersections");
        return BH_OK;
    };
    if (num_splats) {
        uint32_t* partials;
        BH_STRY(ws.get(&depth_keys, num_splats));
        BH_STRY(ws.get((char**)&partials, project_partials_bytes(num_splats)));
        BH_STRY(ws.get(&vis_rows, (size_t)num_splats * 12));
        StageRange stage("ProjectSplats");
        launch_project_forward(ctx, u, transforms, raw_opacities, sh_coeffs, sh_degree, num_splats, mip, tile_h, counts,
                               max_radius, depth_keys, vis_rows, partials, ctx->d_counters,
                               planned ? ctx->plan_isect_cap : 0u, pf_zero, ctx->h_counters_dev,
                               ++ctx->count_generation);
        BH_STRY(check_launch(ctx, "project_forward"));
    }

    uint32_t *gfc = nullptr, *cum = nullptr, *tile_ids = nullptr, *cgids = nullptr;
    float *projected = nullptr, *depths = nullptr;
    SplatRecord rec;
    auto enqueue = [&](const Plan& p) -> bh_status {
        const uint32_t* dc = p.device ? ctx->d_counters : nullptr;
        uint32_t* counts_sorted = nullptr;
        BH_TRY(sget((void**)&gfc, (size_t)std::max<uint32_t>(num_splats, 1u) * 4));
        BH_TRY(sget((void**)&cum, (size_t)p.v * 4));
        // up to 2^21 splats and a key range of up to 24 bits (depths within a
        // factor of about four), the depth sort is one top-digit pass and a
        // per-bucket sort that also writes cum_tiles_hit (four launches);
        // otherwise the LSD passes and the scan.  More splats would put more
        // than 8192 in a bucket at an even spread of depths; a wider range
        // (near floaters in front of a scene) leaves most splats in a few
        // top digits, buckets far above the 16384 pairs sorted in LDS.
        const bool buckets = num_splats <= kBucketSortMaxSplats && p.key_bits <= kBucketSortMaxKeyBits;
        if (p.v) {
            // depth sort: key' = min(bits - kmin, kmax - kmin + 1); culled splats
            // (all-ones key) map to the cap, and the first pass drops them, so
            // the later passes sort only the visible splats (render.rs:339-346
            // sorts the visible depths).  The LSD sort's last pass also gathers
            // each splat's tile count in depth order, so the scan below reads
            // them contiguously.  A plan with more key bits than the range
            // needs sorts the same: its extra passes see digit 0 only.
            uint32_t *sk, *tk, *tv;
            BH_TRY(ws.get(&sk, num_splats));
            BH_TRY(ws.get(&tk, num_splats));
            BH_TRY(ws.get(&tv, num_splats));
            SortDevice dev;
            if (dc) dev.key_sub = dc + 4, dev.key_cap = dc + 6, dev.n_rest = dc + 0;
            dev.drop_capped = true;
            dev.n_rest_host = p.v;
            StageRange stage("DepthSort");
            if (buckets) {
                BH_TRY(depth_sort_buckets(ctx, depth_keys, num_splats, p.kmin, p.kcap, sk, gfc, tk, tv, depth_scr,
                                          true, counts, cum, dev));
            } else {
                BH_TRY(ws.get(&counts_sorted, num_splats));
                BH_TRY(radix_sort_pairs(ctx, depth_keys, nullptr, num_splats, p.key_bits, p.kmin, p.kcap, sk, gfc, tk,
                                        tv, depth_scr, "depth_sort", true, counts, counts_sorted, dev));
            }
        }
        BH_TRY(sget((void**)&projected, (size_t)std::max<uint32_t>(p.v, 1u) * 40));
        BH_TRY(sget((void**)&depths, (size_t)p.v * 4));
        BH_TRY(sget((void**)&tile_ids, (size_t)std::max<uint32_t>(p.m, 1u) * 4));
        BH_TRY(sget((void**)&cgids, (size_t)std::max<uint32_t>(p.m, 1u) * 4));
        if (p.v) {
            if (!buckets) {
                StageRange stage("PrefixSumGaussHits");
                BH_TRY(inclusive_scan(ctx, counts_sorted, cum, p.v, scan_scr, dc));
            }
            // with intersections (and always under a device plan, which sizes
            // them for at least one), map_intersects orders the rows as it reads them
            if (p.m == 0) {
                StageRange stage("ProjectVisible");
                launch_project_visible(ctx, vis_rows, gfc, p.v, num_splats, projected, depths);
            }
            BH_TRY(check_launch(ctx, "project_visible"));
        } else {
            launch_fill_u32(ctx, (uint32_t*)projected, 0u, 10);
        }
        if (p.m) {
            // tile sort over bits(num_tiles) bits (render.rs:392-395); the map
            // kernel zeroes the sort's scratch.  Below 2^16 tiles (sentinel
            // included: 16 key bits) the map's tile ids and the sort's
            // intermediate keys are 16-bit, the sorted ones 32-bit.
            const uint32_t bits = bit_length(num_tiles);
            const bool k16 = bits <= 16;
            uint32_t *uc, *tv;
            void *ut, *tk;
            char* scr;
            if (k16) {
                BH_TRY(ws.get((uint16_t**)&ut, p.m));
                BH_TRY(ws.get((uint16_t**)&tk, p.m));
            } else {
                BH_TRY(ws.get((uint32_t**)&ut, p.m));
                BH_TRY(ws.get((uint32_t**)&tk, p.m));
            }
            BH_TRY(ws.get(&uc, p.m));
            BH_TRY(ws.get(&tv, p.m));
            BH_TRY(ws.get(&scr, radix_sort_scratch_bytes(p.m, bits)));
            {
                // project_visible's rows are ordered here too (ProjectVisible)
                StageRange stage("MapGaussiansToIntersect");
                launch_map_intersects(ctx, u.tile_bw, u.tile_bh, tile_h, vis_rows, gfc, num_splats, cum, p.v, projected,
                                  depths, ut, k16, uc, (uint32_t*)scr, (uint32_t)radix_sort_zeroed_words(p.m, bits),
                                  dc, p.m);
            }
            BH_TRY(check_launch(ctx, "map_intersects"));
            StageRange stage("Tile sort");
            SortDevice dev;
            if (dc) dev.n = dc + 7;
            if (k16)
                BH_TRY(radix_sort_pairs_k16(ctx, (const uint16_t*)ut, uc, p.m, bits, tile_ids, cgids, (uint16_t*)tk,
                                            tv, scr, "tile_sort", true, dev));
            else
                BH_TRY(radix_sort_pairs(ctx, (const uint32_t*)ut, uc, p.m, bits, 0u, 0xFFFFFFFFu, tile_ids, cgids,
                                        (uint32_t*)tk, tv, scr, "tile_sort", true, nullptr, nullptr, dev));
        } else {
            launch_fill_u32(ctx, tile_ids, 0u, 1);
            launch_fill_u32(ctx, cgids, 0u, 1);
        }
        {
            StageRange stage("GetTileOffsets");
            launch_tile_offsets(ctx, tile_ids, p.m, num_tiles, off_pre, true, dc ? dc + 7 : nullptr);
        }
        StageRange raster_stage(p.m ? "Rasterize" : "RasterizeEmpty");
        // the blend kernel starts the tiles with the most candidates first
        uint32_t* order = nullptr;
        if (p.m) {
            BH_TRY(ws.get(&order, num_tiles));
            launch_tile_order(ctx, off_pre, num_tiles, order);
        }
        // with BWD_INFO and intersections, the blend's last workgroups zero
        // the backward's gradient rows in the blend's tail
        st->bwd_rows = nullptr;
        st->bwd_rows_clean = false;
        if (bwd && p.m) BH_TRY(sget((void**)&st->bwd_rows, (size_t)num_splats * 11 * 4));
        rec = SplatRecord{};
        if (bwd) {
            // which pairs the blend used, for the fused backward.  Every BWD_INFO
            // blend writes block_end for every block (also with no intersections),
            // so the buffers exist whenever BWD_INFO is set.
            const uint32_t bpt = 2u * tile_h / 8u;
            BH_TRY(sget((void**)&rec.masks, std::max<size_t>(record_masks(p.m, bpt), 1) * sizeof(uint2)));
            BH_TRY(sget((void**)&rec.block_end, (size_t)num_tiles * bpt * 4));
            if (p.m) {
                // the backward's dispatch order, appended by the blend
                rec.order.word = reinterpret_cast<unsigned long long*>(off_pre + (size_t)num_tiles * 2);
                rec.order.count = off_pre + (size_t)num_tiles * 4;
                BH_TRY(sget((void**)&rec.order.list, (size_t)kOrderBuckets * num_tiles * 4));
            }
        }
        launch_rasterize(ctx, u.img_w, u.img_h, u.tile_bw, u.tile_bh, background, p.v, projected, cgids, gfc, off_pre,
                         order, flags, out_img, visible, tile_offsets, true, rec, (uint32_t*)st->bwd_rows,
                         st->bwd_rows ? (uint64_t)num_splats * 11 : 0u);
        st->bwd_rows_clean = st->bwd_rows != nullptr;
        return check_launch(ctx, "rasterize");
    };
    auto exact_plan = [&]() {
        Plan p{false, num_visible, (uint32_t)num_isect, 0u, kmin, kmax - kmin + 1u};
        if (num_visible) p.key_bits = std::max<uint32_t>(1u, bit_length(p.kcap));
        return p;
    };

    const size_t state_mark = st->buffers.size();
    if (planned) {
        const Plan p{true, num_splats, ctx->plan_isect_cap, ctx->plan_key_bits, 0u, 0u};
        BH_STRY(enqueue(p));
        BH_STRY(read_counts());
        const Plan exact = exact_plan();
        // a plan with no visible splat leaves the projected rows unwritten:
        // the exact launches write the zero row that case has
        if (num_visible == 0 || exact.m > p.m || exact.key_bits > p.key_bits) {
            // the exact launches reuse (stream ordered) the plan's buffers
            for (size_t i = state_mark; i < st->buffers.size(); i++) ctx->pool.release(st->buffers[i]);
            st->buffers.resize(state_mark);
            zero_outputs(false);
            BH_STRY(enqueue(exact));
        }
    } else {
        if (num_splats) BH_STRY(read_counts());
        BH_STRY(enqueue(exact_plan()));
    }
    if (num_splats) {
        // the next forward's plan: this key width, and room for 1/8 more
        // intersections (kept while within twice what is needed)
        if (num_visible) ctx->plan_key_bits = exact_plan().key_bits;
        const uint64_t want = num_isect + num_isect / 8 + 4096;
        if (!ctx->plan_valid || num_isect > ctx->plan_isect_cap || (uint64_t)ctx->plan_isect_cap > 2 * want)
            ctx->plan_isect_cap = (uint32_t)std::min<uint64_t>((want + 4095) / 4096 * 4096, 0xFFFFF000ull);
        ctx->plan_valid = true;
    }
    const uint32_t m = (uint32_t)num_isect;
#undef BH_STRY

    u.num_visible = num_visible;
    bh_fwd_info& in = st->info;
    in.num_splats = num_splats;
    in.num_visible = num_visible;
    in.num_intersections = m;
    in.num_tiles = num_tiles;
    in.tile_bw = u.tile_bw;
    in.tile_bh = u.tile_bh;
    in.img_w = u.img_w;
    in.img_h = u.img_h;
    in.sh_degree = sh_degree;
    in.flags = flags;
    in.uniforms = u;
    in.projected = projected;
    in.global_from_compact_gid = gfc;
    in.depths = depths;
    in.intersect_counts = counts;
    in.cum_tiles_hit = cum;
    in.tile_id_from_isect = tile_ids;
    in.compact_gid_from_isect = cgids;
    in.tile_offsets_pre = off_pre;
    st->record = rec;
    *state_out = st;
    return BH_OK;
}

bh_status bh_fwd_state_info(const bh_fwd_state* state, bh_fwd_info* out) {
    if (!state || !out) return BH_ERR_INVALID_ARG;
    *out = state->info;
    return BH_OK;
}

bh_status bh_fwd_state_backward_lanes(const bh_fwd_state* state, const float** lanes) {
    if (!state || !lanes) return BH_ERR_INVALID_ARG;
    *lanes = state->kept_lanes;
    return BH_OK;
}

void bh_fwd_state_release(bh_fwd_state* state) {
    if (!state) return;
    for (void* p : state->buffers) state->ctx->pool.release(p);
    delete state;
}

bh_status bh_rasterize_backward(bh_ctx* ctx, const float* out_img, const float* projected,
                                const uint32_t* compact_gid_from_isect, const uint32_t* tile_offsets,
                                uint32_t num_visible, const float background[3], uint32_t img_w, uint32_t img_h,
                                const float* v_output, uint32_t flags, float* v_combined) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    if (img_w == 0 || img_h == 0) return set_error(ctx, BH_ERR_INVALID_ARG, "Can't render images with 0 size.");
    if (!out_img || !projected || !compact_gid_from_isect || !tile_offsets || !background || !v_output ||
        !v_combined)
        return set_error(ctx, BH_ERR_INVALID_ARG, "rasterize_backward: null argument");
    const uint32_t tbw = div_up(img_w, BH_TILE_WIDTH);
    const uint32_t tbh = div_up(img_h, (flags & BH_FLAG_TILE_16X8) ? 8u : BH_TILE_WIDTH);
    StageRange stage("RasterizeBackwards");
    launch_fill_u32(ctx, (uint32_t*)v_combined, 0u, (uint64_t)std::max<uint32_t>(num_visible, 1) * 11);
    if (num_visible)
        launch_rasterize_backward(ctx, img_w, img_h, tbw, tbh, background, num_visible, out_img, projected,
                                  compact_gid_from_isect, tile_offsets, v_output, flags, nullptr, nullptr, v_combined);
    return check_launch(ctx, "rasterize_backward");
}

bh_status bh_project_backward(bh_ctx* ctx, const bh_project_uniforms* u, const float* transforms,
                              const float* sh_coeffs, const float* raw_opacities,
                              const uint32_t* global_from_compact_gid, const float* v_combined, uint32_t flags,
                              float* v_transforms, float* v_coeffs, float* v_raw_opac, float* v_refine) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    if (!u) return set_error(ctx, BH_ERR_INVALID_ARG, "project_backward: null uniforms");
    const uint32_t n = u->total_splats;
    if (n == 0) return BH_OK;
    if (u->sh_degree > 4) return set_error(ctx, BH_ERR_INVALID_ARG, "sh_degree must be <= 4");
    if (u->camera_model > BH_CAMERA_TPF) return set_error(ctx, BH_ERR_INVALID_ARG, "unknown camera model");
    if (u->num_visible > n) return set_error(ctx, BH_ERR_SHAPE, "num_visible > total_splats");
    if (!transforms || !sh_coeffs || !raw_opacities || !v_combined || !v_transforms || !v_coeffs || !v_raw_opac ||
        !v_refine || (u->num_visible && !global_from_compact_gid))
        return set_error(ctx, BH_ERR_INVALID_ARG, "project_backward: null argument");
    Scratch ws(ctx);
    uint32_t* cfg;
    BH_TRY(ws.get(&cfg, n));
    StageRange stage("ProjectBackwards");
    launch_invert_permutation(ctx, global_from_compact_gid, u->num_visible, n, cfg);
    launch_project_backward(ctx, *u, transforms, sh_coeffs, raw_opacities, cfg, n, u->sh_degree,
                            (flags & BH_FLAG_MIP) != 0, v_combined, v_transforms, v_coeffs, v_raw_opac, v_refine);
    return check_launch(ctx, "project_backward");
}

bh_status bh_render_backward(bh_ctx* ctx, const bh_fwd_state* state, const float* out_img,
                             const uint32_t* tile_offsets, const float background[3], const float* transforms,
                             const float* sh_coeffs, const float* raw_opacities, const float* v_output, uint32_t flags,
                             float* v_transforms, float* v_coeffs, float* v_raw_opac, float* v_refine) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    if (!state) return set_error(ctx, BH_ERR_INVALID_ARG, "render_backward: null forward state");
    const bh_fwd_info& in = state->info;
    if (!(in.flags & BH_FLAG_BWD_INFO))
        return set_error(ctx, BH_ERR_INVALID_ARG, "render_backward: the forward ran without BH_FLAG_BWD_INFO");
    // the cutoff and the image layout belong to the forward (burn_glue.rs:326-328
    // takes them from the forward state): a caller that asks for others is
    // rejected before anything is launched
    const uint32_t fwd_owned = BH_FLAG_SMOOTH_CUTOFF | BH_FLAG_RENDER_DEPTH;
    if ((flags & fwd_owned) != (in.flags & fwd_owned))
        return set_error(ctx, BH_ERR_INVALID_ARG,
                         "render_backward: BH_FLAG_SMOOTH_CUTOFF / BH_FLAG_RENDER_DEPTH differ from the forward's");
    const uint32_t n = in.num_splats;
    if (n == 0) return BH_OK;
    if (!out_img || !tile_offsets || !background || !transforms || !sh_coeffs || !raw_opacities || !v_output ||
        !v_transforms || !v_coeffs || !v_raw_opac || !v_refine)
        return set_error(ctx, BH_ERR_INVALID_ARG, "render_backward: null argument");
    // gradient lanes accumulated per global id, so project backward reads
    // them in order (no inverse permutation, no gathered rows).  The first
    // backward of a state takes the rows its forward zeroed and returns them
    // to the pool once project backward is queued; a later backward zeroes
    // rows of its own.  The call changes the state (it consumes those rows),
    // so backwards of one state are serialised like every call on a context.
    bh_fwd_state* st = const_cast<bh_fwd_state*>(state);
    const bool keep = (ctx->debug & BH_DEBUG_KEEP_LANES) != 0;
    Scratch ws(ctx);
    float* rows;
    const bool pre_zeroed = st->bwd_rows && st->bwd_rows_clean;
    if (pre_zeroed) {
        rows = st->bwd_rows;
        st->bwd_rows = nullptr;
        st->bwd_rows_clean = false;
    } else if (keep) {
        void* p = nullptr;
        hipError_t e = ctx->pool.alloc(&p, (size_t)n * 11 * sizeof(float));
        if (e != hipSuccess) return hip_check(ctx, e, "workspace allocation");
        st->buffers.push_back(p);
        poison(ctx, p, (size_t)n * 11 * sizeof(float));
        rows = (float*)p;
    } else {
        BH_TRY(ws.get(&rows, (size_t)n * 11));
    }
    if (st->kept_lanes) {
        st->drop(st->kept_lanes);
        st->kept_lanes = nullptr;
    }
    const uint32_t raster_flags = (in.flags & (fwd_owned | BH_FLAG_TILE_16X8)) | (flags & BH_FLAG_REFINE_WEIGHT);
    StageRange raster_stage("RasterizeBackwards");
    bool dense_zeroed = false;  // the four gradient arrays hold zeros
    if (in.num_visible && in.num_intersections && state->record.masks) {
        // the longest tiles (most splats the forward blended) start first: in
        // the order the forward's blend recorded, or one computed here (while
        // the gradient rows are zeroed)
        uint32_t* order = nullptr;
        if (state->record.order.list) {
            if (!pre_zeroed) launch_fill_u32(ctx, (uint32_t*)rows, 0u, (uint64_t)n * 11);
        } else {
            BH_TRY(ws.get(&order, in.num_tiles));
            if (pre_zeroed)
                launch_tile_order(ctx, tile_offsets, in.num_tiles, order);
            else
                launch_zero_and_tile_order(ctx, (uint32_t*)rows, (uint64_t)n * 11, tile_offsets, in.num_tiles, order);
        }
        // The dense gradients start as zeros, stored by workgroups of the
        // rasterize backward (bound by instruction issue, not memory) spread
        // among its blend's; project backward then writes only the rows of
        // splats with a gradient.
        const uint32_t nc = (in.sh_degree + 1u) * (in.sh_degree + 1u);
        const FillRange dense[] = {{(uint32_t*)v_transforms, 0u, (uint64_t)n * 10u},
                                   {(uint32_t*)v_coeffs, 0u, (uint64_t)n * 3u * nc},
                                   {(uint32_t*)v_raw_opac, 0u, (uint64_t)n},
                                   {(uint32_t*)v_refine, 0u, (uint64_t)n}};
        const int dense_k = n >= kFusedFillMinSplats ? 4 : 0;
        dense_zeroed = launch_rasterize_backward_recorded(
                           ctx, in.img_w, in.img_h, in.tile_bw, in.tile_bh, background, in.num_visible, out_img,
                           in.projected, in.compact_gid_from_isect, in.tile_offsets_pre, state->record, v_output,
                           raster_flags, in.global_from_compact_gid, order, rows, dense, dense_k) &&
                       dense_k != 0;
    } else {
        // no intersections: no pixel blended a splat, every gradient is zero
        if (!pre_zeroed) launch_fill_u32(ctx, (uint32_t*)rows, 0u, (uint64_t)n * 11);
    }
    BH_TRY(check_launch(ctx, "rasterize_backward"));
    {
        StageRange stage("ProjectBackwards");
        launch_project_backward(ctx, in.uniforms, transforms, sh_coeffs, raw_opacities, nullptr, n, in.sh_degree,
                                (in.flags & BH_FLAG_MIP) != 0, rows, v_transforms, v_coeffs, v_raw_opac, v_refine,
                                dense_zeroed);
    }
    BH_TRY(check_launch(ctx, "project_backward"));
    if (keep)
        st->kept_lanes = rows;
    else if (pre_zeroed)
        st->drop(rows);
    if (ctx->debug & BH_DEBUG_VALIDATE) {
        // Splats::bwd_validate (gaussian_splats.rs:384-415)
        const uint32_t nc = (in.sh_degree + 1u) * (in.sh_degree + 1u);
        FiniteArrays a{};
        a.p[0] = v_transforms, a.n[0] = (uint64_t)n * 10u;
        a.p[1] = v_coeffs, a.n[1] = (uint64_t)n * nc * 3u;
        a.p[2] = v_raw_opac, a.n[2] = n;
        a.k = 3;
        const char* names[] = {"gradient_transforms", "gradient_sh_coeffs", "gradient_raw_opacities"};
        BH_TRY(check_finite(ctx, "render_backward", a, names));
    }
    return BH_OK;
}

static bh_status check_loss_args(bh_ctx* ctx, const float* pred, uint32_t pred_stride, uint32_t channels,
                                 const uint32_t* gt, uint32_t w, uint32_t h, const bh_image_loss_config* cfg) {
    if (w == 0 || h == 0) return set_error(ctx, BH_ERR_INVALID_ARG, "image loss: zero image size");
    if (channels != 3 && channels != 4) return set_error(ctx, BH_ERR_SHAPE, "image loss: channels must be 3 or 4");
    if (pred_stride < channels) return set_error(ctx, BH_ERR_SHAPE, "image loss: pred_stride < channels");
    if (!pred || !gt || !cfg) return set_error(ctx, BH_ERR_INVALID_ARG, "image loss: null argument");
    return BH_OK;
}

bh_status bh_image_loss_forward(bh_ctx* ctx, const float* pred, uint32_t pred_stride, uint32_t channels,
                                const uint32_t* gt_packed, uint32_t img_w, uint32_t img_h,
                                const bh_image_loss_config* cfg, float* loss_map) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    BH_TRY(check_loss_args(ctx, pred, pred_stride, channels, gt_packed, img_w, img_h, cfg));
    if (!loss_map) return set_error(ctx, BH_ERR_INVALID_ARG, "image loss: null loss map");
    launch_image_loss_forward(ctx, pred, pred_stride, channels, gt_packed, img_w, img_h, *cfg, loss_map);
    return check_launch(ctx, "image_loss_forward");
}

bh_status bh_image_loss_backward(bh_ctx* ctx, const float* pred, uint32_t pred_stride, uint32_t channels,
                                 const uint32_t* gt_packed, uint32_t img_w, uint32_t img_h,
                                 const bh_image_loss_config* cfg, const float* dl_dmap, float* dl_dpred) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    BH_TRY(check_loss_args(ctx, pred, pred_stride, channels, gt_packed, img_w, img_h, cfg));
    if (!dl_dmap || !dl_dpred) return set_error(ctx, BH_ERR_INVALID_ARG, "image loss: null gradient buffer");
    launch_image_loss_backward(ctx, pred, pred_stride, channels, gt_packed, img_w, img_h, *cfg, dl_dmap, dl_dpred);
    return check_launch(ctx, "image_loss_backward");
}

bh_status bh_adam_scaled_step(bh_ctx* ctx, float* param, const float* grad, float* moment_1, float* moment_2,
                              const float* scaling, uint32_t rows, uint32_t row_len, uint32_t reduce_moment_2,
                              float lr, uint32_t time, const bh_adam_config* cfg) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    if (!cfg) return set_error(ctx, BH_ERR_INVALID_ARG, "adam: null config");
    if (time == 0) return set_error(ctx, BH_ERR_INVALID_ARG, "adam: time counts steps from 1");
    if ((uint64_t)rows * row_len == 0) return BH_OK;
    if (!param || !grad || !moment_1 || !moment_2) return set_error(ctx, BH_ERR_INVALID_ARG, "adam: null buffer");
    return launch_adam_step(ctx, param, grad, moment_1, moment_2, scaling, rows, row_len, reduce_moment_2 != 0, lr,
                            time, *cfg);
}

static bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0u; }

bh_status bh_ply_decode_rows(bh_ctx* ctx, const uint8_t* rows, uint64_t rows_bytes, uint32_t row_bytes,
                             uint64_t num_rows, uint32_t subsample, uint32_t flags, const bh_ply_column* columns,
                             uint32_t num_coeffs, float* transforms, float* sh_coeffs, float* raw_opac) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    if (subsample == 0) return set_error(ctx, BH_ERR_INVALID_ARG, "ply: subsample must be greater than zero");
    if (num_rows == 0) return BH_OK;
    if (!rows || !columns || !transforms || !sh_coeffs || !raw_opac)
        return set_error(ctx, BH_ERR_INVALID_ARG, "ply: null buffer");
    if (row_bytes == 0) return set_error(ctx, BH_ERR_INVALID_ARG, "ply: empty rows");
    if (!aligned4(rows)) return set_error(ctx, BH_ERR_INVALID_ARG, "ply: rows must be 4-byte aligned");
    if (rows_bytes < (num_rows * row_bytes + 3u) / 4u * 4u)
        return set_error(ctx, BH_ERR_INVALID_ARG, "ply: rows_bytes below num_rows * row_bytes (rounded up to 4)");
    const uint64_t n_out = (num_rows + subsample - 1) / subsample;
    return launch_ply_decode_rows(ctx, rows, rows_bytes, row_bytes, n_out, subsample, flags, columns, num_coeffs,
                                  transforms, sh_coeffs, raw_opac);
}

bh_status bh_ply_decode_compressed(bh_ctx* ctx, const float* chunks, uint64_t num_chunks, const uint8_t* vertex_rows,
                                   uint64_t vertex_bytes, const uint8_t* sh_rows, uint64_t sh_bytes,
                                   uint64_t num_rows, uint32_t subsample, uint32_t flags,
                                   const bh_ply_compressed_layout* layout, float* transforms, float* sh_coeffs,
                                   float* raw_opac) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    if (subsample == 0) return set_error(ctx, BH_ERR_INVALID_ARG, "ply: subsample must be greater than zero");
    if (!layout) return set_error(ctx, BH_ERR_INVALID_ARG, "ply: null layout");
    if (num_rows == 0) return BH_OK;
    const bh_ply_compressed_layout& L = *layout;
    if (!chunks || !vertex_rows || !transforms || !sh_coeffs || !raw_opac)
        return set_error(ctx, BH_ERR_INVALID_ARG, "ply: null buffer");
    if (num_chunks < (num_rows + 255u) / 256u)
        return set_error(ctx, BH_ERR_INVALID_ARG, "ply: fewer chunk rows than ceil(num_rows / 256)");
    const uint32_t offs[4] = {L.position_offset, L.scale_offset, L.rotation_offset, L.color_offset};
    for (uint32_t o : offs)
        if ((uint64_t)o + 4u > L.vertex_row_bytes)
            return set_error(ctx, BH_ERR_INVALID_ARG, "ply: packed word outside the vertex row");
    if (!aligned4(vertex_rows) || vertex_bytes < num_rows * L.vertex_row_bytes)
        return set_error(ctx, BH_ERR_INVALID_ARG, "ply: vertex rows unaligned or shorter than num_rows rows");
    if (L.sh_row_bytes == 0) {
        if (L.sh_rest_count != 0) return set_error(ctx, BH_ERR_INVALID_ARG, "ply: SH rest count without sh rows");
    } else {
        const uint32_t rc = L.sh_rest_count;
        if (!(rc == 0 || rc == 9 || rc == 24 || rc == 45 || rc == 72))
            return set_error(ctx, BH_ERR_INVALID_ARG, "ply: Unsupported SH rest property count");
        if (!sh_rows || sh_bytes < num_rows * L.sh_row_bytes)
            return set_error(ctx, BH_ERR_INVALID_ARG, "ply: sh rows missing or shorter than num_rows rows");
        for (uint32_t k = 0; k < rc; k++)
            if (L.sh_offsets[k] >= L.sh_row_bytes)
                return set_error(ctx, BH_ERR_INVALID_ARG, "ply: SH property outside the sh row");
    }
    const uint64_t n_out = (num_rows + subsample - 1) / subsample;
    return launch_ply_decode_compressed(ctx, chunks, vertex_rows, sh_rows, n_out, subsample, flags, L, transforms,
                                        sh_coeffs, raw_opac);
}

bh_status bh_ply_encode_rows(bh_ctx* ctx, const float* transforms, const float* sh_coeffs, const float* raw_opac,
                             uint64_t n, uint32_t num_coeffs, float* rows) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    if (n == 0) return BH_OK;
    if (!transforms || !sh_coeffs || !raw_opac || !rows) return set_error(ctx, BH_ERR_INVALID_ARG, "ply: null buffer");
    return launch_ply_encode_rows(ctx, transforms, sh_coeffs, raw_opac, n, num_coeffs, rows);
}

bh_status bh_copy_to_host(bh_ctx* ctx, void* dst, const void* src, uint64_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return BH_ERR_INVALID_ARG;
    if (!bytes) return BH_OK;
    BH_TRY(hip_check(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "copy to host"));
    return hip_check(ctx, hipStreamSynchronize(ctx->stream), "copy to host");
}

bh_status bh_copy_to_device(bh_ctx* ctx, void* dst, const void* src, uint64_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return BH_ERR_INVALID_ARG;
    if (!bytes) return BH_OK;
    BH_TRY(hip_check(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "copy to device"));
    return hip_check(ctx, hipStreamSynchronize(ctx->stream), "copy to device");
}

bh_status bh_copy_device(bh_ctx* ctx, void* dst, const void* src, uint64_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return BH_ERR_INVALID_ARG;
    if (!bytes) return BH_OK;
    return hip_check(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream), "copy on device");
}

bh_status bh_device_alloc(bh_ctx* ctx, void** out, uint64_t bytes) {
    if (!ctx || !out) return BH_ERR_INVALID_ARG;
    *out = nullptr;
    return hip_check(ctx, hipMalloc(out, std::max<uint64_t>(bytes, 4)), "hipMalloc");
}

bh_status bh_device_free(bh_ctx* ctx, void* ptr) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    if (!ptr) return BH_OK;
    return hip_check(ctx, hipFree(ptr), "hipFree");
}

bh_status bh_synchronize(bh_ctx* ctx) {
    if (!ctx) return BH_ERR_INVALID_ARG;
    return hip_check(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

}  // extern "C"
