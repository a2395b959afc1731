// sort.hip — fill, inclusive scan and stable radix sort for gfx950.
//
// Radix sort: LSD with digits of at most 8 bits, each pass in three kernels
// (reduce-then-scan).  An upsweep counts the digits of every partition of 4096
// keys; a small scan turns the counts into each partition's output offset per
// digit (digit totals below it plus the same digit in earlier partitions);
// the digit pass then ranks a partition's pairs stably inside the workgroup
// with wave64 ballots (an 8-ballot match of the digit gives each lane its
// peers; a per-wave running count orders slots) and writes them from LDS in
// digit order, so each digit's run is a contiguous write.  No workgroup waits
// on another: a decoupled look-back over the ~2500 partitions of a tile sort
// was measured to cost 31 of a pass's 76 us (a chain that advances a few
// partitions per coherent round trip), more than the extra read of the keys.
//
// The inclusive scan below keeps a decoupled look-back.  A partition is
// its workgroup's id and waits only on lower ids.  Workgroups go
// to the XCDs round robin and each XCD dispatches its share in increasing id
// order, so whenever some partition waits, every lower partition already has
// a resident workgroup or has finished.  The spin is bounded; on exhaustion
// the kernel raises an error flag that the host turns into BH_ERR_INTERNAL,
// and the kernel still completes.
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

// Offset geometry of a sort: `parts` partitions of 256 * `items` pairs,
// `radix` counters per partition (2^width), and partitions grouped into
// `blocks` of `rows` (a power of two >= sqrt(parts)) for the offset scan, so
// that both the block sums every scan workgroup reads and the rows it walks
// stay short.  Partitions are as large as still gives about four workgroups
// per CU: 4096 pairs from 4M keys, 1024 for a 1M-key depth sort (4096 would
// leave it 245 workgroups for 256 CUs).
struct ScanPlan {
    uint32_t items, parts, rows, blocks, radix;
};
static ScanPlan scan_plan(uint32_t n, const DigitPlan& d) {
    ScanPlan s;
    s.items = n >= (4096u << 10) ? 16u : n >= (2048u << 10) ? 8u : 4u;
    s.parts = div_up(n, (uint64_t)kThreads * s.items);
    s.rows = 16;
    while ((uint64_t)s.rows * s.rows < s.parts) s.rows *= 2;
    s.blocks = div_up(s.parts, s.rows);
    s.radix = 1u << d.width;
    return s;
}

// ---- reduce-then-scan: digit counts of each partition ----------------------------

// One workgroup per partition: the digit counts of its keys (per-wave LDS
// copies, 16-byte loads for a whole aligned partition) go to its row of
// `counts` and are added to its block's sums.
template <bool FIRST, int ITEMS>
__global__ __launch_bounds__(kThreads) void radix_upsweep_kernel(const uint32_t* __restrict__ keys, uint32_t n,
                                                                  uint32_t shift, uint32_t digit_bits,
                                                                  uint32_t key_sub, uint32_t key_cap, uint32_t radix,
                                                                  uint32_t rows, uint32_t* __restrict__ counts,
                                                                  uint32_t* __restrict__ blk) {
    __shared__ uint32_t s_hist[kWaves][kRadix];
    const int tid = threadIdx.x, wave = tid >> 6;
    for (int i = tid; i < kWaves * kRadix; i += kThreads) (&s_hist[0][0])[i] = 0;
    __syncthreads();
    constexpr int PART = kThreads * ITEMS;
    const uint32_t part = blockIdx.x;
    const uint64_t base = (uint64_t)part * PART;
    const uint32_t dmask = (1u << digit_bits) - 1u;
    uint32_t* mine = s_hist[wave];
    if (base + PART <= n && (reinterpret_cast<uintptr_t>(keys) & 15u) == 0u) {
        const uint4* k4 = reinterpret_cast<const uint4*>(keys + base);
        uint4 q[ITEMS / 4];
#pragma unroll
        for (int j = 0; j < ITEMS / 4; j++) q[j] = k4[j * kThreads + tid];
#pragma unroll
        for (int j = 0; j < ITEMS / 4; j++) {
            const uint32_t kk[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t k = FIRST ? min(kk[e] - key_sub, key_cap) : kk[e];
                atomicAdd(&mine[(k >> shift) & dmask], 1u);
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < ITEMS; j++) {
            const uint64_t idx = base + (uint64_t)j * kThreads + tid;
            if (idx < n) {
                const uint32_t k = FIRST ? min(keys[idx] - key_sub, key_cap) : keys[idx];
                atomicAdd(&mine[(k >> shift) & dmask], 1u);
            }
        }
    }
    __syncthreads();
    if ((uint32_t)tid < radix) {
        uint32_t c = 0;
#pragma unroll
        for (int w = 0; w < kWaves; w++) c += s_hist[w][tid];
        counts[(size_t)part * radix + tid] = c;
        if (c) atomicAdd(&blk[(size_t)(part / rows) * radix + tid], c);
    }
}

// counts[q][d] becomes the output position of partition q's first pair of
// digit d: the totals of the digits below d plus the counts of digit d in the
// partitions before q.  One workgroup of 1024 threads per block of `rows`
// partitions; each digit column is shared by 1024 / radix thread groups, which
// split the block sums and the block's rows between them, so a thread issues
// its few loads together (a handful of memory round trips in all).
constexpr int kScanThreads = 1024;
__global__ __launch_bounds__(kScanThreads) void radix_scan_kernel(uint32_t* __restrict__ counts,
                                                                   const uint32_t* __restrict__ blk, uint32_t parts,
                                                                   uint32_t rows, uint32_t blocks, uint32_t radix) {
    __shared__ uint32_t s_tot[kScanThreads / 64];
    __shared__ uint32_t s_all[kScanThreads];     // a thread's share of its digit's total
    __shared__ uint32_t s_before[kScanThreads];  // ... of the blocks before this one
    __shared__ uint32_t s_rows[kScanThreads];    // ... of this block's rows
    __shared__ uint32_t s_base[kRadix];
    constexpr int kChunk = 16;
    const uint32_t tid = threadIdx.x, b = blockIdx.x;
    const uint32_t d = tid & (radix - 1u), grp = tid / radix, groups = kScanThreads / radix;
    // block sums: group g reads blocks g, g + groups, ...
    uint32_t all = 0, before = 0;
    for (uint32_t q0 = grp; q0 < blocks; q0 += groups * kChunk) {
        uint32_t x[kChunk];
#pragma unroll
        for (int i = 0; i < kChunk; i++) {
            const uint32_t q = q0 + i * groups;
            x[i] = q < blocks ? blk[(size_t)q * radix + d] : 0u;
        }
#pragma unroll
        for (int i = 0; i < kChunk; i++) {
            all += x[i];
            before += q0 + i * groups < b ? x[i] : 0u;
        }
    }
    // this block's rows: group g takes a contiguous run of them
    const uint32_t r0 = b * rows, r1 = min(parts, r0 + rows);
    const uint32_t sub = (rows + groups - 1u) / groups;
    const uint32_t lo = min(r1, r0 + grp * sub), hi = min(r1, lo + sub);
    uint32_t mine = 0;
    for (uint32_t q0 = lo; q0 < hi; q0 += kChunk) {
        uint32_t x[kChunk];
#pragma unroll
        for (int i = 0; i < kChunk; i++) x[i] = q0 + i < hi ? counts[(size_t)(q0 + i) * radix + d] : 0u;
#pragma unroll
        for (int i = 0; i < kChunk; i++) mine += x[i];
    }
    s_all[tid] = all;
    s_before[tid] = before;
    s_rows[tid] = mine;
    __syncthreads();
    uint32_t total = 0, pre = 0;
    if (grp == 0) {
        for (uint32_t g = 0; g < groups; g++) {
            total += s_all[g * radix + d];
            pre += s_before[g * radix + d];
        }
    }
    uint32_t dummy;
    const uint32_t bin_base = block_exclusive_scan<kScanThreads>(grp == 0 ? total : 0u, s_tot, &dummy);
    if (grp == 0) s_base[d] = bin_base + pre;
    __syncthreads();
    uint32_t run = s_base[d];
    for (uint32_t g = 0; g < grp; g++) run += s_rows[g * radix + d];
    for (uint32_t q0 = lo; q0 < hi; q0 += kChunk) {
        uint32_t x[kChunk];
#pragma unroll
        for (int i = 0; i < kChunk; i++) x[i] = q0 + i < hi ? counts[(size_t)(q0 + i) * radix + d] : 0u;
#pragma unroll
        for (int i = 0; i < kChunk; i++) {
            if (q0 + i < hi) counts[(size_t)(q0 + i) * radix + d] = run;
            run += x[i];
        }
    }
}

// ---- one digit pass ------------------------------------------------------------

// One workgroup per partition of 256 * ITEMS pairs: stable ranking inside the
// partition, then every pair written to offs[part][digit] + its rank among the
// partition's pairs of that digit, through LDS in digit order.
template <bool FIRST, int ITEMS>
__global__ __launch_bounds__(kThreads) void onesweep_kernel(const uint32_t* __restrict__ keys_in,
                                                             const uint32_t* __restrict__ vals_in,
                                                             uint32_t* __restrict__ keys_out,
                                                             uint32_t* __restrict__ vals_out, uint32_t n,
                                                             uint32_t shift, uint32_t digit_bits, uint32_t key_sub,
                                                             uint32_t key_cap, uint32_t radix,
                                                             const uint32_t* __restrict__ offs) {
    __shared__ uint32_t s_wave_hist[kWaves][kRadix];
    __shared__ uint32_t s_local_start[kRadix];
    __shared__ uint32_t s_global_off[kRadix];
    constexpr int PART = kThreads * ITEMS;
    __shared__ uint32_t s_buf[PART];  // keys, then values, in digit order
    __shared__ uint32_t s_tot[kWaves];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t part = blockIdx.x;
    // this partition's output offset of digit `tid`, loaded while the pairs are ranked
    const uint32_t my_off = (uint32_t)tid < radix ? offs[(size_t)part * radix + tid] : 0u;
    for (int i = tid; i < kWaves * kRadix; i += kThreads) (&s_wave_hist[0][0])[i] = 0;
    __syncthreads();
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
    uint32_t tot_dummy;
    const uint32_t local_start = block_exclusive_scan<kThreads>(total, s_tot, &tot_dummy);
    s_local_start[d] = local_start;
    s_global_off[d] = my_off;
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
            if (g < n) {  // always true: the offsets partition [0, n)
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

// scratch layout: block sums blk[passes][blocks][radix] (zeroed before the
// sort) | offsets counts[parts][radix] (rewritten by every pass)
size_t radix_sort_scratch_bytes(uint32_t n, uint32_t key_bits) {
    const DigitPlan plan = digit_plan(key_bits);
    const ScanPlan sp = scan_plan(n, plan);
    return ((size_t)plan.passes * sp.blocks + sp.parts) * sp.radix * 4;
}

size_t radix_sort_zeroed_words(uint32_t n, uint32_t key_bits) {
    const DigitPlan plan = digit_plan(key_bits);
    const ScanPlan sp = scan_plan(n, plan);
    return (size_t)plan.passes * sp.blocks * sp.radix;
}

bh_status radix_sort_pairs(bh_ctx* ctx, const uint32_t* keys_in, const uint32_t* vals_in, uint32_t n,
                           uint32_t key_bits, uint32_t key_sub, uint32_t key_cap, uint32_t* keys_out,
                           uint32_t* vals_out, uint32_t* tmp_keys, uint32_t* tmp_vals, void* scratch,
                           const char* tag, bool scratch_zeroed) {
    const std::string up_name = std::string(tag) + "_up", scan_name = std::string(tag) + "_scan",
                      pass_name = std::string(tag) + "_onesweep";
    if (n == 0) return BH_OK;
    if (key_bits > 32) return set_error(ctx, BH_ERR_INVALID_ARG, "radix sort: more than 32 key bits");
    const DigitPlan plan = digit_plan(key_bits);
    const ScanPlan sp = scan_plan(n, plan);
    uint32_t* blk = (uint32_t*)scratch;
    uint32_t* offs = blk + (size_t)plan.passes * sp.blocks * sp.radix;
    if (!scratch_zeroed) launch_fill_u32(ctx, blk, 0u, radix_sort_zeroed_words(n, key_bits));
    const uint32_t* src_k = keys_in;
    const uint32_t* src_v = vals_in;
    for (uint32_t p = 0; p < plan.passes; p++) {
        // the last pass lands in the output buffers
        bool to_out = ((plan.passes - 1 - p) % 2) == 0;
        uint32_t* dk = to_out ? keys_out : tmp_keys;
        uint32_t* dv = to_out ? vals_out : tmp_vals;
        uint32_t* pblk = blk + (size_t)p * sp.blocks * sp.radix;
        const uint32_t sh = plan.shift(p), bits = plan.bits(p);
        const uint32_t sub = p == 0 ? key_sub : 0u, cap = p == 0 ? key_cap : 0xFFFFFFFFu;
        const dim3 grid(sp.parts), block(kThreads);
#define BH_SORT_PASS(I)                                                                                          \
    do {                                                                                                        \
        {                                                                                                       \
            KernelTimer t(ctx, up_name.c_str());                                                                \
            if (p == 0)                                                                                         \
                radix_upsweep_kernel<true, I><<<grid, block, 0, ctx->stream>>>(src_k, n, sh, bits, sub, cap,   \
                                                                               sp.radix, sp.rows, offs, pblk); \
            else                                                                                                \
                radix_upsweep_kernel<false, I><<<grid, block, 0, ctx->stream>>>(src_k, n, sh, bits, sub, cap,  \
                                                                                sp.radix, sp.rows, offs, pblk); \
        }                                                                                                       \
        {                                                                                                       \
            KernelTimer t(ctx, scan_name.c_str());                                                              \
            radix_scan_kernel<<<sp.blocks, kScanThreads, 0, ctx->stream>>>(offs, pblk, sp.parts, sp.rows,       \
                                                                           sp.blocks, sp.radix);               \
        }                                                                                                       \
        {                                                                                                       \
            KernelTimer t(ctx, pass_name.c_str());                                                              \
            if (p == 0)                                                                                         \
                onesweep_kernel<true, I><<<grid, block, 0, ctx->stream>>>(src_k, src_v, dk, dv, n, sh, bits,   \
                                                                          sub, cap, sp.radix, offs);           \
            else                                                                                                \
                onesweep_kernel<false, I><<<grid, block, 0, ctx->stream>>>(src_k, src_v, dk, dv, n, sh, bits,  \
                                                                           sub, cap, sp.radix, offs);          \
        }                                                                                                       \
    } while (0)
        if (sp.items == 16)
            BH_SORT_PASS(16);
        else if (sp.items == 8)
            BH_SORT_PASS(8);
        else
            BH_SORT_PASS(4);
#undef BH_SORT_PASS
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
