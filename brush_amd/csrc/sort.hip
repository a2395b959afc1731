// sort.hip — fill, inclusive scan and stable radix sort for gfx950.
//
// Radix sort: LSD with 8-bit digits in the "onesweep" organisation
// (Adinets & Merrill, 2022): one histogram pass computes the digit counts of
// every pass up front, then each digit pass reads keys and values once and
// writes them once.  A partition of 4096 pairs is ranked stably inside the
// workgroup with wave64 ballots (an 8-ballot match of the digit gives each
// lane its peers; a per-wave running count orders slots), the block's digit
// counts are published to a look-back status array, and the pairs are written
// from LDS in digit order so each digit's run is a contiguous write.
//
// Forward progress of the look-back: a partition is its workgroup's id, and a
// workgroup only waits on lower ids.  Workgroups go to the XCDs round robin
// and each XCD dispatches its share in increasing id order, so whenever some
// partition waits, every lower partition already has a resident workgroup or
// has finished (an atomic ticket per workgroup gives the same guarantee
// without relying on dispatch order, but serialises workgroup starts on one
// counter: measured 14 us of a 93 us tile-sort pass).  The spin is bounded;
// on exhaustion the kernel raises an error flag that the host turns into
// BH_ERR_INTERNAL, and the kernel still completes.
//
// Replaces brush-sort (crates/brush-sort/src/lib.rs:16-129, which runs five
// kernels per 4-bit pass with a single-workgroup scan) and brush-prefix-sum
// (crates/brush-prefix-sum/src/lib.rs:11-87, a multi-level Hillis-Steele scan).
#include <hip/hip_runtime.h>

#include "bh_internal.h"
#include "bh_lookback.h"

namespace bh {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kItems = 16;
constexpr int kPart = kThreads * kItems;  // 4096
constexpr int kRadix = 256;
// p[0, count) = value: 16-byte stores from the first 16-byte boundary, single
// words for the unaligned head and the tail.
__global__ void fill_u32_kernel(uint32_t* p, uint32_t value, uint64_t count) {
    const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    const uint64_t head = min<uint64_t>(count, ((16u - (reinterpret_cast<uintptr_t>(p) & 15u)) & 15u) / 4u);
    if (tid < head) p[tid] = value;
    const uint64_t quads = (count - head) / 4u;
    uint4* q = reinterpret_cast<uint4*>(p + head);
    const uint4 v4 = make_uint4(value, value, value, value);
    for (uint64_t i = tid; i < quads; i += stride) q[i] = v4;
    for (uint64_t i = head + quads * 4u + tid; i < count; i += stride) p[i] = value;
}

void launch_fill_u32(bh_ctx* ctx, uint32_t* p, uint32_t value, uint64_t count) {
    if (count == 0) return;
    KernelTimer t(ctx, "fill");
    uint32_t blocks = (uint32_t)std::min<uint64_t>((count / 4 + 255) / 256 + 1, 2048);
    fill_u32_kernel<<<blocks, 256, 0, ctx->stream>>>(p, value, count);
}

struct FillRanges {
    FillRange r[kMaxFillRanges];
    int k;
};

// Every range filled by the whole grid in turn (the range index is uniform),
// each as fill_u32_kernel fills one.
__global__ void fill_multi_kernel(FillRanges ranges) {
    const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (int j = 0; j < ranges.k; j++) {
        uint32_t* p = ranges.r[j].p;
        const uint32_t value = ranges.r[j].value;
        const uint64_t count = ranges.r[j].count;
        const uint64_t head = min<uint64_t>(count, ((16u - (reinterpret_cast<uintptr_t>(p) & 15u)) & 15u) / 4u);
        if (tid < head) p[tid] = value;
        const uint64_t quads = (count - head) / 4u;
        uint4* q = reinterpret_cast<uint4*>(p + head);
        const uint4 v4 = make_uint4(value, value, value, value);
        for (uint64_t i = tid; i < quads; i += stride) q[i] = v4;
        for (uint64_t i = head + quads * 4u + tid; i < count; i += stride) p[i] = value;
    }
}

void launch_fill_multi(bh_ctx* ctx, const FillRange* ranges, int k) {
    FillRanges fr{};
    uint64_t total = 0;
    for (int j = 0; j < k; j++) {
        if (ranges[j].count == 0 || !ranges[j].p) continue;
        if (fr.k == kMaxFillRanges) {  // more than one launch holds
            launch_fill_multi(ctx, ranges + j, k - j);
            break;
        }
        fr.r[fr.k++] = ranges[j];
        total += ranges[j].count;
    }
    if (fr.k == 0) return;
    KernelTimer t(ctx, "fill");
    const uint32_t blocks = (uint32_t)std::min<uint64_t>((total / 4 + 255) / 256 + 1, 2048);
    fill_multi_kernel<<<blocks, 256, 0, ctx->stream>>>(fr);
}


// Digit layout of a sort by the low `key_bits` bits: ceil(key_bits / 8)
// passes of equal width (13 bits -> 7 + 6), so every pass has at most 256
// buckets and the runs each partition writes per bucket are as long as the
// bit count allows.
struct DigitPlan {
    uint32_t key_bits, passes, width;
    uint32_t shift(uint32_t p) const { return p * width; }
    uint32_t bits(uint32_t p) const { return p * width >= key_bits ? 0u : min(width, key_bits - p * width); }
};
static DigitPlan digit_plan(uint32_t key_bits) {
    DigitPlan d;
    d.key_bits = key_bits;
    d.passes = key_bits == 0 ? 1u : (key_bits + 7u) / 8u;
    d.width = key_bits == 0 ? 1u : (key_bits + d.passes - 1u) / d.passes;
    return d;
}

// ---- histogram of all digit passes -------------------------------------------

// Each wave counts into its own LDS copy (less contention on the few buckets
// of a narrow digit); a modest grid keeps the global atomics on the 256 *
// passes bucket words few.
__global__ __launch_bounds__(kThreads) void radix_hist_kernel(const uint32_t* __restrict__ keys, uint32_t n,
                                                               uint32_t passes, uint32_t width, uint32_t key_sub,
                                                               uint32_t key_cap, uint32_t* __restrict__ hist) {
    __shared__ uint32_t sh[kWaves][4 * kRadix];
    const uint32_t wave = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < kWaves * 4 * kRadix; i += kThreads) (&sh[0][0])[i] = 0;
    __syncthreads();
    const uint32_t mask = (1u << width) - 1u;
    uint32_t* mine = sh[wave];
    // 16-byte loads when the keys are 16-byte aligned (every internal buffer
    // is); a caller's misaligned view is counted one key at a time
    const bool vec = (reinterpret_cast<uintptr_t>(keys) & 15u) == 0u;
    const uint32_t n4 = vec ? n / 4u : 0u;
    const uint4* k4 = reinterpret_cast<const uint4*>(keys);
    for (uint32_t idx = blockIdx.x * kThreads + threadIdx.x; idx < n4; idx += gridDim.x * kThreads) {
        const uint4 q = k4[idx];
        const uint32_t kk[4] = {min(q.x - key_sub, key_cap), min(q.y - key_sub, key_cap), min(q.z - key_sub, key_cap),
                                min(q.w - key_sub, key_cap)};
#pragma unroll
        for (int e = 0; e < 4; e++)
            for (uint32_t p = 0; p < passes; p++) atomicAdd(&mine[p * kRadix + ((kk[e] >> (p * width)) & mask)], 1u);
    }
    // the keys after the last full group of four
    for (uint32_t idx = n4 * 4u + blockIdx.x * kThreads + threadIdx.x; idx < n; idx += gridDim.x * kThreads) {
        const uint32_t kk = min(keys[idx] - key_sub, key_cap);
        for (uint32_t p = 0; p < passes; p++) atomicAdd(&mine[p * kRadix + ((kk >> (p * width)) & mask)], 1u);
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < passes * kRadix; i += kThreads) {
        uint32_t c = 0;
#pragma unroll
        for (int w = 0; w < kWaves; w++) c += sh[w][i];
        if (c) atomicAdd(&hist[i], c);
    }
}

// ---- one digit pass ------------------------------------------------------------

template <bool FIRST, int ITEMS>
__global__ __launch_bounds__(kThreads) void onesweep_kernel(const uint32_t* __restrict__ keys_in,
                                                             const uint32_t* __restrict__ vals_in,
                                                             uint32_t* __restrict__ keys_out,
                                                             uint32_t* __restrict__ vals_out, uint32_t n,
                                                             uint32_t shift, uint32_t digit_bits, uint32_t key_sub,
                                                             uint32_t key_cap, const uint32_t* __restrict__ hist,
                                                             uint64_t* status, uint32_t* err) {
    constexpr int PART = kThreads * ITEMS;
    __shared__ uint32_t s_wave_hist[kWaves][kRadix];
    __shared__ uint32_t s_local_start[kRadix];
    __shared__ uint32_t s_global_off[kRadix];
    __shared__ uint32_t s_buf[PART];  // keys, then values, in digit order
    __shared__ uint32_t s_tot[kWaves];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < kWaves * kRadix; i += kThreads) (&s_wave_hist[0][0])[i] = 0;
    __syncthreads();
    const uint32_t part = blockIdx.x;
    const uint64_t base = (uint64_t)part * PART;
    const uint64_t wave_base = base + (uint64_t)wave * (64 * ITEMS);
    const uint32_t dmask = (1u << digit_bits) - 1u;

    uint32_t k[ITEMS], v[ITEMS], pos[ITEMS];
#pragma unroll
    for (int j = 0; j < ITEMS; j++) {
        uint64_t idx = wave_base + (uint64_t)j * 64 + lane;
        bool valid = idx < n;
        uint32_t kk = valid ? keys_in[idx] : 0u;
        if (FIRST) kk = min(kk - key_sub, key_cap);
        k[j] = kk;
        v[j] = valid ? (vals_in ? vals_in[idx] : (uint32_t)idx) : 0u;
    }
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
    for (int j = 0; j < ITEMS; j++) {
        uint64_t idx = wave_base + (uint64_t)j * 64 + lane;
        bool valid = idx < n;
        uint32_t d = (k[j] >> shift) & dmask;
        uint64_t peers = __ballot(valid);
        for (uint32_t b = 0; b < digit_bits; b++) {
            bool bit = (d >> b) & 1u;
            uint64_t bal = __ballot(bit);
            peers &= bit ? bal : ~bal;
        }
        uint32_t prefix = 0;
        if (valid) prefix = s_wave_hist[wave][d];
        pos[j] = prefix + (uint32_t)__popcll(peers & lt_mask);
        // the highest lane of each peer group advances the wave's running count
        if (valid && (peers >> lane) == 1ull) s_wave_hist[wave][d] = prefix + (uint32_t)__popcll(peers);
    }
    __syncthreads();

    // per-digit counts of the partition and each wave's offset inside them
    const uint32_t d = tid;
    uint32_t c[kWaves];
#pragma unroll
    for (int w = 0; w < kWaves; w++) c[w] = s_wave_hist[w][d];
    uint32_t total = 0;
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
        s_wave_hist[w][d] = total;
        total += c[w];
    }
    uint64_t* my_status = status + (uint64_t)part * kRadix + d;
    uint32_t excl = 0;
    if (part == 0) {
        status_store(my_status, kFlagPrefix | total);
    } else {
        status_store(my_status, kFlagAgg | total);
        excl = look_back(status, part, kRadix, d, err);
        status_store(my_status, kFlagPrefix | (uint64_t)(excl + total));
    }
    uint32_t tot_dummy;
    uint32_t bin_base = block_exclusive_scan<kThreads>(hist[d], s_tot, &tot_dummy);
    uint32_t local_start = block_exclusive_scan<kThreads>(total, s_tot, &tot_dummy);
    s_local_start[d] = local_start;
    s_global_off[d] = bin_base + excl;
    __syncthreads();

    // keys into LDS in digit order, then out; the destination of each LDS slot
    // is kept for the values
#pragma unroll
    for (int j = 0; j < ITEMS; j++) {
        uint64_t idx = wave_base + (uint64_t)j * 64 + lane;
        uint32_t dd = (k[j] >> shift) & dmask;
        pos[j] = s_local_start[dd] + s_wave_hist[wave][dd] + pos[j];
        if (idx < n) s_buf[pos[j]] = k[j];
    }
    __syncthreads();
    const uint32_t count = (uint32_t)min<uint64_t>((uint64_t)PART, (uint64_t)n - base);
    uint32_t dst[ITEMS];
#pragma unroll
    for (int j = 0; j < ITEMS; j++) {
        const uint32_t i = (uint32_t)(j * kThreads + tid);
        dst[j] = 0xFFFFFFFFu;
        if (i < count) {
            const uint32_t key = s_buf[i];
            const uint32_t dd = (key >> shift) & dmask;
            const uint32_t g = s_global_off[dd] + (i - s_local_start[dd]);
            if (g < n) {  // always true unless a look-back gave up (reported through err)
                keys_out[g] = key;
                dst[j] = g;
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < ITEMS; j++) {
        uint64_t idx = wave_base + (uint64_t)j * 64 + lane;
        if (idx < n) s_buf[pos[j]] = v[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < ITEMS; j++) {
        const uint32_t i = (uint32_t)(j * kThreads + tid);
        if (dst[j] != 0xFFFFFFFFu) vals_out[dst[j]] = s_buf[i];
    }
}

// Partitions of 4096 pairs (smaller partitions measured slower: more
// look-back traffic for the same data).
static uint32_t sort_part(uint32_t) { return (uint32_t)kPart; }

// scratch layout: hist[4*256] | status[passes][parts][256] (u64)
size_t radix_sort_scratch_bytes(uint32_t n, uint32_t key_bits) {
    const uint64_t parts = div_up(n, sort_part(n));
    return (size_t)(4 * kRadix) * 4 + (size_t)digit_plan(key_bits).passes * parts * kRadix * 8;
}

size_t radix_sort_zeroed_words(uint32_t n, uint32_t key_bits) {
    const uint64_t parts = div_up(n, sort_part(n));
    return (size_t)(4 * kRadix) + (size_t)digit_plan(key_bits).passes * parts * kRadix * 2;
}

bh_status radix_sort_pairs(bh_ctx* ctx, const uint32_t* keys_in, const uint32_t* vals_in, uint32_t n,
                           uint32_t key_bits, uint32_t key_sub, uint32_t key_cap, uint32_t* keys_out,
                           uint32_t* vals_out, uint32_t* tmp_keys, uint32_t* tmp_vals, void* scratch,
                           const char* tag, bool scratch_zeroed) {
    const std::string hist_name = std::string(tag) + "_hist", pass_name = std::string(tag) + "_onesweep";
    if (n == 0) return BH_OK;
    if (key_bits > 32) return set_error(ctx, BH_ERR_INVALID_ARG, "radix sort: more than 32 key bits");
    const DigitPlan plan = digit_plan(key_bits);
    const uint32_t part_size = sort_part(n);
    const uint32_t parts = div_up(n, part_size);
    uint32_t* hist = (uint32_t*)scratch;
    uint64_t* status = (uint64_t*)(hist + 4 * kRadix);
    if (!scratch_zeroed) launch_fill_u32(ctx, hist, 0u, radix_sort_zeroed_words(n, key_bits));
    {
        KernelTimer t(ctx, hist_name.c_str());
        uint32_t blocks = std::min<uint32_t>(div_up(div_up(n, 4), kThreads * 8), 512);
        radix_hist_kernel<<<blocks, kThreads, 0, ctx->stream>>>(keys_in, n, plan.passes, plan.width, key_sub, key_cap,
                                                                hist);
    }
    const uint32_t* src_k = keys_in;
    const uint32_t* src_v = vals_in;
    for (uint32_t p = 0; p < plan.passes; p++) {
        // the last pass lands in the output buffers
        bool to_out = ((plan.passes - 1 - p) % 2) == 0;
        uint32_t* dk = to_out ? keys_out : tmp_keys;
        uint32_t* dv = to_out ? vals_out : tmp_vals;
        uint64_t* st = status + (uint64_t)p * parts * kRadix;
        const uint32_t sh = plan.shift(p), bits = plan.bits(p);
        const uint32_t sub = p == 0 ? key_sub : 0u, cap = p == 0 ? key_cap : 0xFFFFFFFFu;
        KernelTimer t(ctx, pass_name.c_str());
#define BH_PASS(F, I)                                                                                               \
    onesweep_kernel<F, I><<<parts, kThreads, 0, ctx->stream>>>(src_k, src_v, dk, dv, n, sh, bits, sub, cap,        \
                                                               hist + p * kRadix, st, ctx->d_counters + 1)
        if (part_size == (uint32_t)kPart) {
            if (p == 0) BH_PASS(true, kItems); else BH_PASS(false, kItems);
        } else {
            if (p == 0) BH_PASS(true, 4); else BH_PASS(false, 4);
        }
#undef BH_PASS
        src_k = dk;
        src_v = dv;
    }
    return check_launch(ctx, "radix sort");
}

__global__ void mask_u32_kernel(const uint32_t* __restrict__ in, uint32_t mask, uint32_t n,
                                uint32_t* __restrict__ out) {
    uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i < n) out[i] = in[i] & mask;
}

void launch_mask_u32(bh_ctx* ctx, const uint32_t* in, uint32_t mask, uint32_t n, uint32_t* out) {
    if (n == 0) return;
    KernelTimer t(ctx, "mask");
    mask_u32_kernel<<<div_up(n, 256), 256, 0, ctx->stream>>>(in, mask, n, out);
}

__global__ void gather_pairs_kernel(const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in,
                                    const uint32_t* __restrict__ perm, uint32_t n, uint32_t* __restrict__ keys_out,
                                    uint32_t* __restrict__ vals_out) {
    uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i < n) {
        uint32_t j = perm[i];
        keys_out[i] = keys_in[j];
        vals_out[i] = vals_in[j];
    }
}

void launch_gather_pairs(bh_ctx* ctx, const uint32_t* keys_in, const uint32_t* vals_in, const uint32_t* perm,
                         uint32_t n, uint32_t* keys_out, uint32_t* vals_out) {
    if (n == 0) return;
    KernelTimer t(ctx, "gather_pairs");
    gather_pairs_kernel<<<div_up(n, 256), 256, 0, ctx->stream>>>(keys_in, vals_in, perm, n, keys_out, vals_out);
}

// ---- single-pass inclusive scan ----------------------------------------------------

__global__ __launch_bounds__(kThreads) void scan_kernel(const uint32_t* __restrict__ in,
                                                         const uint32_t* __restrict__ gather,
                                                         uint32_t* __restrict__ out, uint32_t n, uint64_t* status,
                                                         uint32_t* err) {
    __shared__ uint32_t s_tot[kWaves];
    __shared__ uint32_t s_prefix;
    const int tid = threadIdx.x;
    const uint32_t part = blockIdx.x;
    const uint64_t first = (uint64_t)part * kPart + (uint64_t)tid * kItems;
    uint32_t x[kItems];
    uint32_t run = 0;
#pragma unroll
    for (int j = 0; j < kItems; j++) {
        uint64_t idx = first + j;
        uint32_t val = 0;
        if (idx < n) val = gather ? in[gather[idx]] : in[idx];
        run += val;
        x[j] = run;
    }
    uint32_t block_total;
    uint32_t thread_excl = block_exclusive_scan<kThreads>(run, s_tot, &block_total);
    if (tid == 0) {
        uint32_t excl = 0;
        if (part == 0) {
            status_store(status, kFlagPrefix | block_total);
        } else {
            status_store(status + part, kFlagAgg | block_total);
            excl = look_back(status, part, 1, 0, err);
            status_store(status + part, kFlagPrefix | (uint64_t)(excl + block_total));
        }
        s_prefix = excl;
    }
    __syncthreads();
    const uint32_t add = s_prefix + thread_excl;
#pragma unroll
    for (int j = 0; j < kItems; j++) {
        uint64_t idx = first + j;
        if (idx < n) out[idx] = x[j] + add;
    }
}

size_t scan_scratch_bytes(uint32_t n) { return 64 + (size_t)div_up(n, kPart) * 8; }

size_t scan_zeroed_words(uint32_t n) { return (size_t)div_up(n, kPart) * 2; }

bh_status inclusive_scan(bh_ctx* ctx, const uint32_t* in, const uint32_t* gather, uint32_t* out, uint32_t n,
                         void* scratch, bool status_zeroed) {
    if (n == 0) return BH_OK;
    uint32_t parts = div_up(n, kPart);
    uint64_t* status = (uint64_t*)((char*)scratch + 64);
    if (!status_zeroed) launch_fill_u32(ctx, (uint32_t*)status, 0u, scan_zeroed_words(n));
    KernelTimer t(ctx, "scan");
    scan_kernel<<<parts, kThreads, 0, ctx->stream>>>(in, gather, out, n, status, ctx->d_counters + 1);
    return check_launch(ctx, "scan");
}

}  // namespace bh
