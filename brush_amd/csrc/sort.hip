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
// The inclusive scan is reduce-then-scan as well (partition sums, then the
// in-partition scan plus the sums before it).
//
// Replaces brush-sort (crates/brush-sort/src/lib.rs:16-129, which runs five
// kernels per 4-bit pass with a single-workgroup scan) and brush-prefix-sum
// (crates/brush-prefix-sum/src/lib.rs:11-87, a multi-level Hillis-Steele scan).
#include <hip/hip_runtime.h>

#include "bh_internal.h"
#include "bh_wave.h"

namespace bh {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kRadix = 256;

// Exclusive scan of one value per thread over a block of THREADS threads
// (a multiple of 64); *total receives the block's sum.
template <int THREADS>
__device__ inline uint32_t block_exclusive_scan(uint32_t v, uint32_t* s_wave_tot, uint32_t* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        uint32_t y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) s_wave_tot[wave] = x;
    __syncthreads();
    uint32_t off = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < THREADS / 64; w++) {
        uint32_t t = s_wave_tot[w];
        if (w < wave) off += t;
        tot += t;
    }
    __syncthreads();
    *total = tot;
    return off + x - v;
}

// Stable ranks of a wave's pairs among its pairs of the same digit
// (k >> sh) & (2^bits - 1): item j of lane l is the wave's (64 j + l)-th pair,
// valid where bit j of `valid` is set, for j < items (wave-uniform).  On
// return pos[j] = hist[d] before the call plus the wave's earlier pairs of
// digit d, and hist[d] (the wave's running count in LDS) has advanced by the
// wave's pairs of each digit.  A lane's peers (the lanes that share its
// digit) come from a match over the digit's bit planes; the highest lane of
// each peer group advances the running count.  BITS > 0 matches exactly BITS
// planes, unrolled (digits must be below 2^BITS); BITS == 0 the runtime `bits`.
template <int ITEMS, int BITS = 0>
__device__ __forceinline__ void wave_rank(const uint32_t (&k)[ITEMS], uint32_t valid, uint32_t items, uint32_t sh,
                                          uint32_t bits, uint32_t* hist, uint32_t (&pos)[ITEMS]) {
    const int lane = threadIdx.x & 63;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const uint32_t dmask = (1u << bits) - 1u;
#pragma unroll
    for (int j = 0; j < ITEMS; j++) {
        if ((uint32_t)j < items) {
            const bool ok = (valid >> j) & 1u;
            const uint32_t d = (k[j] >> sh) & dmask;
            uint64_t peers = __ballot(ok);
            if constexpr (BITS > 0) {
#pragma unroll
                for (int b = 0; b < BITS; b++) {
                    const bool bit = (d >> b) & 1u;
                    const uint64_t bal = __ballot(bit);
                    peers &= bit ? bal : ~bal;
                }
            } else {
                for (uint32_t b = 0; b < bits; b++) {
                    const bool bit = (d >> b) & 1u;
                    const uint64_t bal = __ballot(bit);
                    peers &= bit ? bal : ~bal;
                }
            }
            uint32_t prefix = 0;
            if (ok) prefix = hist[d];
            pos[j] = prefix + (uint32_t)__popcll(peers & lt_mask);
            if (ok && (peers >> lane) == 1ull) hist[d] = prefix + (uint32_t)__popcll(peers);
        }
    }
}

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
    launch(ctx, fill_u32_kernel, dim3(blocks), dim3(256), 0u, p, value, count);
}

// Every range filled by the whole grid in turn (fill_ranges_strided).
__global__ void fill_multi_kernel(FillRanges ranges) {
    fill_ranges_strided<false>(ranges, (uint64_t)blockIdx.x * blockDim.x + threadIdx.x,
                               (uint64_t)gridDim.x * blockDim.x);
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
    launch(ctx, fill_multi_kernel, dim3(blocks), dim3(256), 0u, fr);
}

// ---- debug validation: the first non-finite value of each array ----------------------

// first[i] = the smallest index of a NaN or infinite value in array i (or
// stays ~0 when it holds none): one grid-stride pass, atomics only on a hit.
__global__ void first_non_finite_kernel(FiniteArrays a, unsigned long long* __restrict__ first) {
    const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (int j = 0; j < a.k; j++) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(a.p[j]);
        for (uint64_t i = tid; i < a.n[j]; i += stride)
            if ((p[i] & 0x7F800000u) == 0x7F800000u) atomicMin(&first[j], (unsigned long long)i);
    }
}

void launch_first_non_finite(bh_ctx* ctx, const FiniteArrays& a, unsigned long long* first) {
    launch_fill_u32(ctx, reinterpret_cast<uint32_t*>(first), 0xFFFFFFFFu, 2u * kMaxFiniteArrays);
    uint64_t total = 0;
    for (int j = 0; j < a.k; j++) total += a.n[j];
    if (total == 0) return;
    KernelTimer t(ctx, "first_non_finite");
    const uint32_t blocks = (uint32_t)std::min<uint64_t>((total + 255) / 256, 4096);
    launch(ctx, first_non_finite_kernel, dim3(blocks), dim3(256), 0u, a, first);
}

// Digit layout of a sort by the low `key_bits` bits: ceil(key_bits / 8)
// passes of near-equal width, so every pass has at most 256
// buckets and the runs each partition writes per bucket are as long as the
// bit count allows.
// The narrower digits come first: the first pass reads the unsorted input
// and writes the shortest runs, so it gets the fewest buckets (13 bits -> 6 + 7).
struct DigitPlan {
    uint32_t key_bits, passes, width;
    // passes [0, narrow) have width - 1 bits, the others width
    uint32_t narrow() const { return passes * width - key_bits; }
    uint32_t bits(uint32_t p) const { return key_bits == 0 ? 0u : (p < narrow() ? width - 1u : width); }
    uint32_t shift(uint32_t p) const { return p * width - min(p, narrow()); }
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
// `blocks` of `rows` (a power of two >= sqrt(parts), or >= sqrt(parts / 2)
// above 2^14 partitions) for the offset scan, so
// that both the block sums every scan workgroup reads and the rows it walks
// stay short.  Partitions hold 2048 pairs from 2M keys (the 10M-pair tile
// sort of a 1080p frame: 4096-pair partitions need 112 VGPRs, four waves per
// SIMD, and measured 10 us per frame slower) and 1024 below (a 1M-key depth
// sort in 4096-pair partitions would have 245 workgroups for 256 CUs).
struct ScanPlan {
    uint32_t items, parts, rows, blocks, radix;
};
static ScanPlan scan_plan(uint32_t n, const DigitPlan& d) {
    ScanPlan s;
    s.items = n >= (2048u << 10) ? 8u : 4u;
    s.parts = div_up(n, (uint64_t)kThreads * s.items);
    // above 2^14 partitions (a 4K frame's tile sort) rows ~ sqrt(parts / 2):
    // twice the scan workgroups, so more of the chip walks the counts
    s.rows = 16;
    while ((uint64_t)s.rows * s.rows < s.parts &&
           (s.parts <= (1u << 14) || (uint64_t)s.rows * s.rows * 2u < s.parts))
        s.rows *= 2;
    s.blocks = div_up(s.parts, s.rows);
    s.radix = 1u << d.width;
    return s;
}

// A first pass over 32-bit keys whose shift is kShiftTop sorts by the top 8
// bits of the transformed key range instead: bit_length(key_cap) - 8 (0 below
// 9 bits), taken from the key cap the kernel reads, so the digit follows a
// device-held range.
constexpr uint32_t kShiftTop = 0xFFFFFFFFu;
__device__ __forceinline__ uint32_t top_digit_shift(uint32_t cap) {
    const uint32_t bl = cap ? 32u - (uint32_t)__clz((int)cap) : 0u;
    return bl > 8u ? bl - 8u : 0u;
}

// ---- reduce-then-scan: digit counts of each partition ----------------------------

// One workgroup per partition: the digit counts of its keys (per-wave LDS
// copies, 16-byte loads for a whole aligned partition; 8-byte ones for four
// 16-bit keys) go to its row of `counts` and are added to its block's sums.
// K is the stored key type: uint32_t, or uint16_t for keys below 2^16.
template <bool FIRST, int ITEMS, typename K>
__global__ __launch_bounds__(kThreads) void radix_upsweep_kernel(const K* __restrict__ keys, uint32_t n,
                                                                  uint32_t shift, uint32_t digit_bits,
                                                                  uint32_t key_sub, uint32_t key_cap, uint32_t radix,
                                                                  uint32_t rows, uint32_t* __restrict__ counts,
                                                                  uint32_t* __restrict__ blk, SortDevice dev) {
    __shared__ uint32_t s_hist[kWaves][kRadix];
    // with dev.weight, each digit's sum of the keys' weights (weight[index])
    constexpr bool WEIGHTS = FIRST && sizeof(K) == 4;
    __shared__ uint32_t s_whist[WEIGHTS ? kWaves : 1][kRadix];
    const int tid = threadIdx.x, wave = tid >> 6;
    if (dev.n) n = min(n, *dev.n);
    if (FIRST && dev.key_sub) {
        key_sub = *dev.key_sub;
        key_cap = *dev.key_cap;
    }
    if constexpr (FIRST && sizeof(K) == 4)
        if (shift == kShiftTop) shift = top_digit_shift(key_cap);
    const uint32_t* __restrict__ weight = WEIGHTS ? dev.weight : nullptr;
    for (int i = tid; i < kWaves * kRadix; i += kThreads) (&s_hist[0][0])[i] = 0;
    if (WEIGHTS && weight)
        for (int i = tid; i < kWaves * kRadix; i += kThreads) (&s_whist[0][0])[i] = 0;
    __syncthreads();
    constexpr int PART = kThreads * ITEMS;
    const uint32_t part = blockIdx.x;
    const uint64_t base = (uint64_t)part * PART;
    const uint32_t dmask = (1u << digit_bits) - 1u;
    uint32_t* mine = s_hist[wave];
    // the first pass of a dropping sort does not count capped keys
    const bool drop = FIRST && dev.drop_capped;
    if (base + PART <= n && (reinterpret_cast<uintptr_t>(keys) & 15u) == 0u &&
        (reinterpret_cast<uintptr_t>(weight) & 15u) == 0u) {
        // this thread's ITEMS keys as 32-bit words: 16-byte loads (8-byte
        // ones for four 16-bit keys), interleaved across the threads
        constexpr int WORDS = ITEMS * (int)sizeof(K) / 4;
        constexpr int VW = WORDS >= 4 ? 4 : 2;
        uint32_t w[WORDS];
        uint32_t wt[WEIGHTS ? ITEMS : 1];
        if constexpr (VW == 4) {
            const uint4* k4 = reinterpret_cast<const uint4*>(keys + base);
#pragma unroll
            for (int j = 0; j < WORDS / 4; j++) {
                const uint4 q = k4[j * kThreads + tid];
                w[4 * j] = q.x, w[4 * j + 1] = q.y, w[4 * j + 2] = q.z, w[4 * j + 3] = q.w;
            }
            if constexpr (WEIGHTS) {
                // weights of the same indices (keys are 32-bit here: item e is word e)
                if (weight) {
                    const uint4* w4 = reinterpret_cast<const uint4*>(weight + base);
#pragma unroll
                    for (int j = 0; j < ITEMS / 4; j++) {
                        const uint4 q = w4[j * kThreads + tid];
                        wt[4 * j] = q.x, wt[4 * j + 1] = q.y, wt[4 * j + 2] = q.z, wt[4 * j + 3] = q.w;
                    }
                }
            }
        } else {
            const uint2* k2 = reinterpret_cast<const uint2*>(keys + base);
#pragma unroll
            for (int j = 0; j < WORDS / 2; j++) {
                const uint2 q = k2[j * kThreads + tid];
                w[2 * j] = q.x, w[2 * j + 1] = q.y;
            }
        }
#pragma unroll
        for (int e = 0; e < ITEMS; e++) {
            const uint32_t kw = sizeof(K) == 4 ? w[e] : (w[e / 2] >> (16 * (e & 1))) & 0xFFFFu;
            const uint32_t k = FIRST ? min(kw - key_sub, key_cap) : kw;
            if (!(drop && k == key_cap)) {
                atomicAdd(&mine[(k >> shift) & dmask], 1u);
                if constexpr (WEIGHTS)
                    if (weight && wt[e]) atomicAdd(&s_whist[wave][(k >> shift) & dmask], wt[e]);
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < ITEMS; j++) {
            const uint64_t idx = base + (uint64_t)j * kThreads + tid;
            if (idx < n) {
                const uint32_t kw = keys[idx];
                const uint32_t k = FIRST ? min(kw - key_sub, key_cap) : kw;
                if (!(drop && k == key_cap)) {
                    atomicAdd(&mine[(k >> shift) & dmask], 1u);
                    if constexpr (WEIGHTS)
                        if (weight && weight[idx]) atomicAdd(&s_whist[wave][(k >> shift) & dmask], weight[idx]);
                }
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
        if constexpr (WEIGHTS) {
            if (weight) {
                uint32_t ws = 0;
#pragma unroll
                for (int w = 0; w < kWaves; w++) ws += s_whist[w][tid];
                if (ws) atomicAdd(&dev.wsum[(size_t)(part / rows) * radix + tid], ws);
            }
        }
    }
}

// counts[q][d] becomes the output position of partition q's first pair of
// digit d: the totals of the digits below d plus the counts of digit d in the
// partitions before q.  One workgroup of 1024 threads per block of `rows`
// partitions; each digit column is shared by 1024 / radix thread groups, which
// split the block sums and the block's rows between them.  A thread issues the
// loads of its first 16 block sums and 16 rows together and keeps the rows in
// registers for the stores, so a common sort (up to 16 of each per thread)
// costs one memory round trip; larger ones loop over further chunks.
constexpr int kScanThreads = 1024;
__global__ __launch_bounds__(kScanThreads) void radix_scan_kernel(uint32_t* __restrict__ counts,
                                                                   const uint32_t* __restrict__ blk, uint32_t parts,
                                                                   uint32_t rows, uint32_t blocks, uint32_t radix) {
    __shared__ uint32_t s_tot[kScanThreads / 64];
    __shared__ uint32_t s_all[kScanThreads];     // a thread's share of its digit's total
    __shared__ uint32_t s_before[kScanThreads];  // ... of the blocks before this one
    __shared__ uint32_t s_rows[kScanThreads];    // ... of this block's rows
    __shared__ uint32_t s_base[kRadix];
    constexpr uint32_t kChunk = 16;
    const uint32_t tid = threadIdx.x, b = blockIdx.x;
    const uint32_t d = tid & (radix - 1u), grp = tid / radix, groups = kScanThreads / radix;
    // block sums: group g reads blocks g, g + groups, ...; this block's rows:
    // group g takes a contiguous run of them
    const uint32_t r0 = b * rows, r1 = min(parts, r0 + rows);
    const uint32_t sub = (rows + groups - 1u) / groups;
    const uint32_t lo = min(r1, r0 + grp * sub), hi = min(r1, lo + sub);
    uint32_t xb[kChunk], xr[kChunk];
#pragma unroll
    for (uint32_t i = 0; i < kChunk; i++) {
        const uint32_t q = grp + i * groups;
        xb[i] = q < blocks ? blk[(size_t)q * radix + d] : 0u;
    }
#pragma unroll
    for (uint32_t i = 0; i < kChunk; i++) xr[i] = lo + i < hi ? counts[(size_t)(lo + i) * radix + d] : 0u;
    uint32_t all = 0, before = 0, mine = 0;
#pragma unroll
    for (uint32_t i = 0; i < kChunk; i++) {
        all += xb[i];
        before += grp + i * groups < b ? xb[i] : 0u;
        mine += xr[i];
    }
    for (uint32_t q = grp + kChunk * groups; q < blocks; q += groups) {
        const uint32_t x = blk[(size_t)q * radix + d];
        all += x;
        before += q < b ? x : 0u;
    }
    for (uint32_t q = lo + kChunk; q < hi; q++) mine += counts[(size_t)q * radix + d];
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
#pragma unroll
    for (uint32_t i = 0; i < kChunk; i++) {
        if (lo + i < hi) counts[(size_t)(lo + i) * radix + d] = run;
        run += xr[i];
    }
    for (uint32_t q = lo + kChunk; q < hi; q++) {
        const uint32_t x = counts[(size_t)q * radix + d];
        counts[(size_t)q * radix + d] = run;
        run += x;
    }
}

// ---- one digit pass ------------------------------------------------------------

// Partition of workgroup b of a grid of g: the dispatcher deals workgroups to
// the eight XCDs in turn, so XCD x runs b = x, x + 8, ...; giving those
// workgroups consecutive partitions keeps the two halves of a 128-byte line
// that neighbouring partitions write for one digit in the same L2, where they
// merge (with partitions dealt round robin, a 1080p tile sort's first pass
// wrote 114 MB for 80 MB of pairs).  Only locality depends on this order.
__device__ __forceinline__ uint32_t xcd_partition(uint32_t b, uint32_t g) {
    const uint32_t x = b & 7u, q = g >> 3, r = g & 7u;
    return x * q + min(x, r) + (b >> 3);
}

// One workgroup per partition of 256 * ITEMS pairs: stable ranking inside the
// partition, then every pair written to offs[part][digit] + its rank among the
// partition's pairs of that digit, through LDS in digit order.  With GATHER,
// each output value v also writes gather_out[g] = gather_src[v]: the gather
// loads are issued with the pair loads (their latency hides behind the
// ranking) and go out through LDS like the values.
template <bool FIRST, int ITEMS, bool GATHER, typename KI, typename KO>
__global__ __launch_bounds__(kThreads) void onesweep_kernel(const KI* __restrict__ keys_in,
                                                             const uint32_t* __restrict__ vals_in,
                                                             KO* __restrict__ keys_out,
                                                             uint32_t* __restrict__ vals_out, uint32_t n,
                                                             uint32_t shift, uint32_t digit_bits, uint32_t key_sub,
                                                             uint32_t key_cap, uint32_t radix,
                                                             const uint32_t* __restrict__ offs,
                                                             const uint32_t* __restrict__ gather_src,
                                                             uint32_t* __restrict__ gather_out, SortDevice dev) {
    __shared__ uint32_t s_wave_hist[kWaves][kRadix];
    __shared__ uint32_t s_local_start[kRadix];
    __shared__ uint32_t s_global_off[kRadix];
    constexpr int PART = kThreads * ITEMS;
    __shared__ uint32_t s_buf[PART];  // keys, then values, in digit order
    __shared__ uint32_t s_tot[kWaves];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t part = xcd_partition(blockIdx.x, gridDim.x);
    if (dev.n) n = min(n, *dev.n);
    if (FIRST && dev.key_sub) {
        key_sub = *dev.key_sub;
        key_cap = *dev.key_cap;
    }
    if constexpr (FIRST && sizeof(KI) == 4)
        if (shift == kShiftTop) shift = top_digit_shift(key_cap);
    // a partition past a device-held count has no pairs (the grid is sized
    // for the capacity); the upsweep wrote its counts as zeros
    if ((uint64_t)part * (kThreads * ITEMS) >= n) return;
    // this partition's output offset of digit `tid`, loaded while the pairs are ranked
    const uint32_t my_off = (uint32_t)tid < radix ? offs[(size_t)part * radix + tid] : 0u;
    for (int i = tid; i < kWaves * kRadix; i += kThreads) (&s_wave_hist[0][0])[i] = 0;
    __syncthreads();
    const uint64_t base = (uint64_t)part * PART;
    const uint64_t wave_base = base + (uint64_t)wave * (64 * ITEMS);
    const uint32_t dmask = (1u << digit_bits) - 1u;

    uint32_t k[ITEMS], v[ITEMS], pos[ITEMS];
    uint32_t gv[GATHER ? ITEMS : 1];
    // the first pass of a dropping sort neither ranks nor writes capped keys
    const bool drop = FIRST && dev.drop_capped;
    uint32_t kept = 0;  // bit j: item j is a pair of this pass
    // every key, value and gather load first, none conditional on a loaded
    // key (a load behind the drop test would wait for its key: one memory
    // round trip per item), then the transform and the drop test
#pragma unroll
    for (int j = 0; j < ITEMS; j++) {
        const uint64_t idx = wave_base + (uint64_t)j * 64 + lane;
        const bool in_range = idx < n;
        k[j] = in_range ? keys_in[idx] : 0u;
        v[j] = in_range ? (vals_in ? vals_in[idx] : (uint32_t)idx) : 0u;
        if (GATHER) gv[j] = gather_src[v[j]];  // v = 0 out of range: in bounds
        if (in_range) kept |= 1u << j;
    }
#pragma unroll
    for (int j = 0; j < ITEMS; j++) {
        if (FIRST) k[j] = min(k[j] - key_sub, key_cap);
        if (drop && k[j] == key_cap) {
            kept &= ~(1u << j);
            v[j] = 0u;
        }
        if (GATHER) gv[j] = (kept >> j) & 1u ? gv[j] : 0u;
    }
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
    for (int j = 0; j < ITEMS; j++) {
        const bool valid = (kept >> j) & 1u;
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
    uint32_t count;  // the partition's pairs (dropped keys excluded)
    const uint32_t local_start = block_exclusive_scan<kThreads>(total, s_tot, &count);
    s_local_start[d] = local_start;
    s_global_off[d] = my_off;
    __syncthreads();

    // keys into LDS in digit order, then out; the destination of each LDS slot
    // is kept for the values
#pragma unroll
    for (int j = 0; j < ITEMS; j++) {
        uint32_t dd = (k[j] >> shift) & dmask;
        pos[j] = s_local_start[dd] + s_wave_hist[wave][dd] + pos[j];
        if ((kept >> j) & 1u) s_buf[pos[j]] = k[j];
    }
    __syncthreads();
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
                keys_out[g] = (KO)key;
                dst[j] = g;
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < ITEMS; j++)
        if ((kept >> j) & 1u) s_buf[pos[j]] = v[j];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < ITEMS; j++) {
        const uint32_t i = (uint32_t)(j * kThreads + tid);
        if (dst[j] != 0xFFFFFFFFu) vals_out[dst[j]] = s_buf[i];
    }
    if (GATHER) {
        __syncthreads();
#pragma unroll
        for (int j = 0; j < ITEMS; j++)
            if ((kept >> j) & 1u) s_buf[pos[j]] = gv[j];
        __syncthreads();
#pragma unroll
        for (int j = 0; j < ITEMS; j++) {
            const uint32_t i = (uint32_t)(j * kThreads + tid);
            if (dst[j] != 0xFFFFFFFFu) gather_out[dst[j]] = s_buf[i];
        }
    }
}

// ---- depth sort: one top-digit pass, then each bucket sorted by one workgroup -------
//
// A stable pass by the top 8 bits of the key range (the digit passes above, with
// kShiftTop) leaves 256 buckets, each the run of one top digit in input order.
// One workgroup per bucket then sorts it stably by the key bits below that
// digit, in 8-bit LSD passes: a bucket of up to kBsCap pairs is ranked and
// reordered in LDS without touching memory between passes; a larger one makes
// the same passes over its chunks through global memory (ping-ponging with
// the temporaries).  The result is the stable sort by the whole key, in four
// launches instead of three per 8-bit digit.
constexpr int kBsThreads = 1024;
constexpr int kBsWaves = kBsThreads / 64;
constexpr int kBsItems = 16;
constexpr uint32_t kBsCap = kBsThreads * kBsItems;
constexpr uint32_t kBsBuckets = 256;

// Stable rank of the chunk of `cnt` pairs the workgroup holds (item j of a
// lane is chunk element e = wave * 64 * iw + j * 64 + lane, j < iw, valid
// below cnt) by the digit (k >> sh) & (2^bits - 1).  On return pos[j] is the
// element's position in the digit-ordered chunk, and s_start[d] / s_cnt[d]
// the chunk's first position and count of digit d.
__device__ __forceinline__ void bucket_rank(const uint32_t (&k)[kBsItems], uint32_t (&pos)[kBsItems], uint32_t iw,
                                            uint32_t cnt, uint32_t sh, uint32_t bits,
                                            uint32_t (*s_hist)[kRadix], uint32_t* s_start, uint32_t* s_cnt,
                                            uint32_t* s_tot) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < kBsWaves * kRadix; i += kBsThreads) (&s_hist[0][0])[i] = 0;
    __syncthreads();
    const uint32_t dmask = (1u << bits) - 1u;
    const uint32_t wbase = (uint32_t)wave * 64u * iw;
    uint32_t valid = 0;
#pragma unroll
    for (int j = 0; j < kBsItems; j++)
        if (wbase + (uint32_t)j * 64u + (uint32_t)lane < cnt) valid |= 1u << j;
    wave_rank<kBsItems, 8>(k, valid, iw, sh, bits, s_hist[wave], pos);
    __syncthreads();
    // digit d = tid: each wave's offset inside the digit, the digit's total
    uint32_t total = 0;
    if (tid < kRadix) {
#pragma unroll
        for (int w = 0; w < kBsWaves; w++) {
            const uint32_t c = s_hist[w][tid];
            s_hist[w][tid] = total;
            total += c;
        }
    }
    uint32_t all;
    const uint32_t start = block_exclusive_scan<kBsThreads>(total, s_tot, &all);
    if (tid < kRadix) {
        s_start[tid] = start;
        s_cnt[tid] = total;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kBsItems; j++) {
        if ((uint32_t)j < iw) {
            if (wbase + (uint32_t)j * 64u + (uint32_t)lane < cnt) {
                const uint32_t d = (k[j] >> sh) & dmask;
                pos[j] += s_start[d] + s_hist[wave][d];
            }
        }
    }
}

// Longest run of equal keys that the counting path orders (one thread per
// run, insertion sort in LDS), and the widest key it counts: a bucket with a
// longer run or wider keys takes the LSD passes instead.
constexpr uint32_t kBsMaxRun = 32;
constexpr uint32_t kBsCountBits = 15;

// One chunk of cum_tiles_hit: vv holds the chunk's sorted values (cnt <=
// kBsCap of them, wave-major items, ipt per lane); out[e] = offset + the
// workgroup's sum of `part` + the inclusive prefix sum of weight[vv] through
// chunk element e (a wave scan per item row, the waves' totals and shares of
// `part` through LDS).  Returns the chunk's weight plus the sum of `part`.
template <int N>
__device__ uint32_t cum_chunk_w(uint32_t (&w)[N], uint32_t ipt, uint32_t cnt, uint32_t* __restrict__ out,
                                uint32_t offset, uint32_t part, uint32_t* s_w);

template <int N>
__device__ uint32_t cum_chunk(const uint32_t (&vv)[N], uint32_t ipt, uint32_t cnt,
                              const uint32_t* __restrict__ weight, uint32_t* __restrict__ out, uint32_t offset,
                              uint32_t part, uint32_t* s_w) {
    // (every item's weight load issued before the first is used: vv holds a
    // valid index, 0, past the chunk's end)
    uint32_t w[N];
#pragma unroll
    for (int j = 0; j < N; j++)
        if ((uint32_t)j < ipt) w[j] = weight[vv[j]];
    return cum_chunk_w<N>(w, ipt, cnt, out, offset, part, s_w);
}

// cum_chunk from the weights of the chunk's sorted elements, w[j] (item j of
// the lane, as vv above; entries past the chunk are ignored).
template <int N>
__device__ uint32_t cum_chunk_w(uint32_t (&w)[N], uint32_t ipt, uint32_t cnt, uint32_t* __restrict__ out,
                                uint32_t offset, uint32_t part, uint32_t* s_w) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t wb = (uint32_t)wave * 64u * ipt;
#pragma unroll
    for (int j = 0; j < N; j++) {
        const uint32_t e = wb + (uint32_t)j * 64u + (uint32_t)lane;
        if ((uint32_t)j >= ipt || e >= cnt) w[j] = 0u;
    }
    uint32_t run = 0u;  // the wave's running total (uniform)
#pragma unroll
    for (int j = 0; j < N; j++) {
        if ((uint32_t)j < ipt) {  // uniform
            const uint32_t x = wave_incl_add_u32(w[j]);
            w[j] = x + run;
            run += (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
        }
    }
    const uint32_t pw = (uint32_t)__builtin_amdgcn_readlane((int)wave_incl_add_u32(part), 63);
    if (lane == 0) {
        s_w[wave] = run;
        s_w[kBsWaves + wave] = pw;
    }
    __syncthreads();
    uint32_t before = 0u, all = 0u, base = 0u;
#pragma unroll
    for (int q = 0; q < kBsWaves; q++) {
        const uint32_t t = s_w[q];
        before += q < wave ? t : 0u;
        all += t;
        base += s_w[kBsWaves + q];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < N; j++) {
        const uint32_t e = wb + (uint32_t)j * 64u + (uint32_t)lane;
        if ((uint32_t)j < ipt && e < cnt) out[e] = offset + base + before + w[j];
    }
    return all + base;
}

// Counting sort of a bucket of `size` <= IW * kBsThreads pairs by the low
// `low` <= 15 bits of its keys, and everything the bucket needs after it.
// Items are wave-major, IW per lane (element e = wave * 64 * IW + j * 64 +
// lane), and every item loop is unrolled over IW with no per-item branch, so
// each phase's loads and LDS operations are in flight together:
//   * the keys (loads clamped into the bucket);
//   * a histogram of the keys in packed 16-bit LDS counters (lanes past the
//     bucket add 0 to a counter of their own) and its exclusive scan;
//   * one returning LDS add per pair for its slot;
//   * the runs of equal keys (a run of slots) put back in input order, each
//     by the thread that holds its first slot, after every thread has read
//     the keys around its slots at once;
//   * the values and their weights (wts: the weights in the bucket's input
//     order, which the top-digit pass wrote beside the values) gathered into
//     sorted order from the bucket's own range, the values written in place,
//     and cum_tiles_hit formed over the weights (cum_chunk_w).
// Returns false, having written nothing, when a key occurs more than
// kBsMaxRun times.  s_raw holds the counters (up to 16384 words), then each
// slot's input position and key (16384 uint16_t each).
template <int IW>
__device__ bool bucket_counted(const uint32_t* __restrict__ keys, uint32_t* __restrict__ vals, uint32_t start,
                               uint32_t size, uint32_t low, const uint32_t* __restrict__ wts,
                               uint32_t* __restrict__ cum, uint32_t part, uint32_t* s_raw, uint32_t* s_tot,
                               uint32_t* s_flag, uint32_t* s_w) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t wbase = (uint32_t)wave * 64u * IW;
    uint32_t* words = s_raw;                                         // counters, two per word
    uint16_t* s_idx = reinterpret_cast<uint16_t*>(s_raw + 16384);  // slot -> input position
    uint16_t* s_bin = s_idx + kBsCap;                                // slot -> key
    const uint32_t lowmask = (1u << low) - 1u;
    const uint32_t nwords = 1u << (low - 1u);
    // counter word i lives at word swz(i): the scan's threads each read 16
    // consecutive words, which would put a wave's 64 lanes on 4 LDS banks;
    // the swizzle (inside each aligned group of 16) spreads them over all
    auto swz = [](uint32_t i) { return (i & ~15u) | ((i & 15u) ^ ((i >> 6) & 15u)); };
    uint32_t k[IW];
#pragma unroll
    for (int j = 0; j < IW; j++) k[j] = keys[start + min(wbase + (uint32_t)j * 64u + (uint32_t)lane, size - 1u)];
    for (uint32_t i = (uint32_t)tid; i < nwords; i += kBsThreads) words[i] = 0u;
    if (tid == 0) *s_flag = 0u;
    // an item's counter word and increment (past the bucket: 0, added to a
    // word of the lane's own, so that no item needs a branch)
    auto word_of = [&](int j) {
        return wbase + (uint32_t)j * 64u + (uint32_t)lane < size ? swz(k[j] >> 1)
                                                                 : swz((uint32_t)tid & (nwords - 1u));
    };
    auto inc_of = [&](int j) {
        return wbase + (uint32_t)j * 64u + (uint32_t)lane < size ? 1u << ((k[j] & 1u) * 16u) : 0u;
    };
#pragma unroll
    for (int j = 0; j < IW; j++) k[j] &= lowmask;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < IW; j++) atomicAdd(&words[word_of(j)], inc_of(j));
    __syncthreads();
    // exclusive scan of the counters (thread t: words [t * wpt, (t + 1) * wpt))
    // and the largest count
    const uint32_t wpt = (nwords + kBsThreads - 1u) / kBsThreads;  // <= 16
    uint32_t loc[16], sum = 0u, mx = 0u;
#pragma unroll
    for (uint32_t w = 0; w < 16u; w++) loc[w] = words[swz(min((uint32_t)tid * wpt + w, nwords - 1u))];
#pragma unroll
    for (uint32_t w = 0; w < 16u; w++) {
        if (w >= wpt || (uint32_t)tid * wpt + w >= nwords) loc[w] = 0u;
        const uint32_t lo = loc[w] & 0xFFFFu, hi = loc[w] >> 16;
        sum += lo + hi;
        mx = max(mx, max(lo, hi));
    }
    if (mx > kBsMaxRun) *s_flag = 1u;
    uint32_t all;
    uint32_t run = block_exclusive_scan<kBsThreads>(sum, s_tot, &all);
#pragma unroll
    for (uint32_t w = 0; w < 16u; w++) {
        const uint32_t i = (uint32_t)tid * wpt + w;
        if (w < wpt && i < nwords) {
            const uint32_t lo = loc[w] & 0xFFFFu, hi = loc[w] >> 16;
            words[swz(i)] = run | ((run + lo) << 16);
            run += lo + hi;
        }
    }
    __syncthreads();
    if (*s_flag) return false;  // uniform: a run too long for one thread
    // every pair takes its key's next slot (any order among equal keys)
    uint32_t slot[IW];
#pragma unroll
    for (int j = 0; j < IW; j++) {
        const uint32_t half = (k[j] & 1u) * 16u;
        slot[j] = (atomicAdd(&words[word_of(j)], inc_of(j)) >> half) & 0xFFFFu;
    }
#pragma unroll
    for (int j = 0; j < IW; j++) {
        const uint32_t e = wbase + (uint32_t)j * 64u + (uint32_t)lane;
        if (e < size) {
            s_idx[slot[j]] = (uint16_t)e;
            s_bin[slot[j]] = (uint16_t)k[j];
        }
    }
    __syncthreads();
    // runs of equal keys into input order: thread t looks at slots t + q *
    // kBsThreads, reading the keys of up to eight slots and of their
    // neighbours at once
    constexpr int RQ = IW < 8 ? IW : 8;
#pragma unroll
    for (int q0 = 0; q0 < IW; q0 += RQ) {
        uint32_t bq[RQ], bl[RQ], br[RQ];
#pragma unroll
        for (int q = 0; q < RQ; q++) {
            const uint32_t i = min((uint32_t)tid + (uint32_t)(q0 + q) * kBsThreads, size - 1u);
            bq[q] = s_bin[i];
            bl[q] = s_bin[i ? i - 1u : 0u];
            br[q] = s_bin[min(i + 1u, size - 1u)];
        }
#pragma unroll
        for (int q = 0; q < RQ; q++) {
            const uint32_t i = (uint32_t)tid + (uint32_t)(q0 + q) * kBsThreads;
            if (i + 1u < size && br[q] == bq[q] && (i == 0u || bl[q] != bq[q])) {
                uint32_t r = 2u;
                while (i + r < size && s_bin[i + r] == bq[q]) r++;
                for (uint32_t a = i + 1u; a < i + r; a++) {
                    const uint32_t x = s_idx[a];
                    uint32_t c = a;
                    while (c > i && s_idx[c - 1u] > x) {
                        s_idx[c] = s_idx[c - 1u];
                        c--;
                    }
                    s_idx[c] = (uint16_t)x;
                }
            }
        }
    }
    __syncthreads();
    // values and weights in sorted order (past the bucket: the last slot's),
    // read before any value is overwritten, then out
    uint32_t v[IW], w[IW];
#pragma unroll
    for (int j = 0; j < IW; j++) v[j] = s_idx[min(wbase + (uint32_t)j * 64u + (uint32_t)lane, size - 1u)];
#pragma unroll
    for (int j = 0; j < IW; j++) {
        w[j] = wts[start + v[j]];
        v[j] = vals[start + v[j]];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < IW; j++) {
        const uint32_t i = wbase + (uint32_t)j * 64u + (uint32_t)lane;
        if (i < size) vals[start + i] = v[j];
    }
    // cum_tiles_hit from the sorted weights
    cum_chunk_w<IW>(w, IW, size, cum + start, 0u, part, s_w);
    return true;
}

// Bucket b = [offs[b], offs[b + 1]) (the last one ends at the pair count; n
// and cap are the pair count and the key cap, from n_dev / cap_dev when
// given) and its key bits below the top digit.
struct BucketSpan {
    uint32_t start, size, low;
};
__device__ __forceinline__ BucketSpan bucket_span(uint32_t b, const uint32_t* __restrict__ offs, uint32_t n,
                                                  const uint32_t* __restrict__ n_dev, uint32_t cap,
                                                  const uint32_t* __restrict__ cap_dev) {
    if (n_dev) n = min(n, *n_dev);
    if (cap_dev) cap = *cap_dev;
    const uint32_t end = min(n, b + 1u < kBsBuckets ? offs[b + 1] : n);
    const uint32_t start = min(offs[b], end);
    return BucketSpan{start, end - start, top_digit_shift(cap)};
}

// This thread's share of the weights of the buckets before bucket b: the
// first pass's per-block digit sums wsum[wsum_words / 256][256] over the
// blocks and the digits below b (summed over the workgroup by cum_chunk;
// eight loads in flight per round, at clamped indices).
__device__ __forceinline__ uint32_t bucket_part(uint32_t b, const uint32_t* __restrict__ wsum, uint32_t wsum_words) {
    const uint32_t tid = threadIdx.x;
    uint32_t part = 0u;
    if ((tid & (kBsBuckets - 1u)) < b && wsum_words) {
        for (uint32_t i0 = tid; i0 < wsum_words; i0 += 8u * kBsThreads) {
            uint32_t x[8];
#pragma unroll
            for (int q = 0; q < 8; q++) x[q] = wsum[min(i0 + (uint32_t)q * kBsThreads, wsum_words - 1u)];
#pragma unroll
            for (int q = 0; q < 8; q++) part += i0 + (uint32_t)q * kBsThreads < wsum_words ? x[q] : 0u;
        }
    }
    return part;
}

// Workgroup b counts bucket b into order (bucket_counted, with wts the
// weights in the order of the top-digit pass's output) when its keys have
// 1 to 15 bits below the top digit and it holds at most kBcItems pairs a
// lane, and sets done[b] (also for an empty bucket); otherwise, or when a
// key occurs too often, it writes nothing but done[b] = 0 and
// bucket_sort_kernel sorts the bucket.
constexpr uint32_t kBcItems = 8;  // (12 or 16 items a lane spill registers)
__global__ __launch_bounds__(kBsThreads) void bucket_count_kernel(const uint32_t* __restrict__ keys,
                                                                   uint32_t* __restrict__ vals,
                                                                   const uint32_t* __restrict__ offs, uint32_t n,
                                                                   const uint32_t* __restrict__ n_dev, uint32_t cap,
                                                                   const uint32_t* __restrict__ cap_dev,
                                                                   const uint32_t* __restrict__ wts,
                                                                   const uint32_t* __restrict__ wsum,
                                                                   uint32_t wsum_words, uint32_t* __restrict__ cum,
                                                                   uint32_t* __restrict__ done) {
    // the counters (up to 16384 words), then each slot's input position and
    // key (16384 uint16_t each)
    __shared__ uint32_t s_raw[2 * kBsCap];
    __shared__ uint32_t s_tot[kBsWaves];
    __shared__ uint32_t s_w[2 * kBsWaves];
    __shared__ uint32_t s_flag;
    const uint32_t b = blockIdx.x;
    const BucketSpan sp = bucket_span(b, offs, n, n_dev, cap, cap_dev);
    bool ok = sp.size == 0u;
    if (sp.size && sp.low > 0u && sp.low <= kBsCountBits && sp.size <= kBcItems * kBsThreads) {
        const uint32_t part = bucket_part(b, wsum, wsum_words);
        const uint32_t iw = (sp.size + kBsThreads - 1u) / kBsThreads;
        if (iw <= 4u)
            ok = bucket_counted<4>(keys, vals, sp.start, sp.size, sp.low, wts, cum, part, s_raw, s_tot, &s_flag, s_w);
        else
            ok = bucket_counted<kBcItems>(keys, vals, sp.start, sp.size, sp.low, wts, cum, part, s_raw, s_tot,
                                          &s_flag, s_w);
    }
    if (threadIdx.x == 0) done[b] = ok ? 1u : 0u;
}

// Workgroup b sorts bucket b, unless bucket_count_kernel has (done[b]), stably
// by the key bits below the top digit in 8-bit LSD passes, writes vals in
// place and cum[i] = the inclusive prefix sum of weight[vals[.]] over the
// whole sorted order: the bucket's own prefix plus the weights of the buckets
// before it (bucket_part).
__global__ __launch_bounds__(kBsThreads) void bucket_sort_kernel(uint32_t* __restrict__ keys,
                                                                  uint32_t* __restrict__ vals,
                                                                  const uint32_t* __restrict__ offs, uint32_t n,
                                                                  const uint32_t* __restrict__ n_dev, uint32_t cap,
                                                                  const uint32_t* __restrict__ cap_dev,
                                                                  const uint32_t* __restrict__ weight,
                                                                  const uint32_t* __restrict__ wsum,
                                                                  uint32_t wsum_words, uint32_t* __restrict__ cum,
                                                                  uint32_t* __restrict__ tmp_k,
                                                                  uint32_t* __restrict__ tmp_v,
                                                                  const uint32_t* __restrict__ done) {
    // keys, values and per-wave histograms
    __shared__ uint32_t s_raw[2 * kBsCap + kBsWaves * kRadix];
    uint32_t* s_k = s_raw;
    uint32_t* s_v = s_raw + kBsCap;
    uint32_t(*s_hist)[kRadix] = reinterpret_cast<uint32_t(*)[kRadix]>(s_raw + 2 * kBsCap);
    __shared__ uint32_t s_start[kRadix], s_cnt[kRadix], s_run[kRadix];
    __shared__ uint32_t s_tot[kBsWaves];
    __shared__ uint32_t s_w[2 * kBsWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t b = blockIdx.x;
    if (done[b]) return;
    const BucketSpan sp = bucket_span(b, offs, n, n_dev, cap, cap_dev);
    if (sp.size == 0u) return;
    const uint32_t start = sp.start, size = sp.size, low = sp.low, passes = (low + 7u) / 8u;
    uint32_t k[kBsItems], v[kBsItems], pos[kBsItems];
    const uint32_t part = bucket_part(b, wsum, wsum_words);

    if (size <= kBsCap) {
        // the whole bucket in registers, reordered through LDS by each LSD pass
        const uint32_t iw = (size + kBsThreads - 1u) / kBsThreads;
        {
            const uint32_t wbase = (uint32_t)wave * 64u * iw;
#pragma unroll
            for (int j = 0; j < kBsItems; j++) {
                if ((uint32_t)j < iw) {
                    const uint32_t e = wbase + (uint32_t)j * 64u + (uint32_t)lane;
                    k[j] = e < size ? keys[start + e] : 0u;
                    v[j] = e < size ? vals[start + e] : 0u;
                }
            }
            for (uint32_t p = 0; p < passes; p++) {
                const uint32_t sh = 8u * p, bits = min(8u, low - sh);
                bucket_rank(k, pos, iw, size, sh, bits, s_hist, s_start, s_cnt, s_tot);
#pragma unroll
                for (int j = 0; j < kBsItems; j++) {
                    if ((uint32_t)j < iw) {
                        if (wbase + (uint32_t)j * 64u + (uint32_t)lane < size) {
                            s_k[pos[j]] = k[j];
                            s_v[pos[j]] = v[j];
                        }
                    }
                }
                __syncthreads();
#pragma unroll
                for (int j = 0; j < kBsItems; j++) {
                    if ((uint32_t)j < iw) {
                        const uint32_t e = wbase + (uint32_t)j * 64u + (uint32_t)lane;
                        if (e < size) {
                            k[j] = s_k[e];
                            v[j] = s_v[e];
                        }
                    }
                }
                __syncthreads();
            }
#pragma unroll
            for (int j = 0; j < kBsItems; j++) {
                if ((uint32_t)j < iw) {
                    const uint32_t e = wbase + (uint32_t)j * 64u + (uint32_t)lane;
                    if (e < size) vals[start + e] = v[j];
                }
            }
            // cum_tiles_hit from the sorted values still in registers
            cum_chunk(v, iw, size, weight, cum + start, 0u, part, s_w);
        }
    } else {
        // A bucket above the LDS capacity: each pass counts the bucket's digits,
        // then ranks its chunks in order and writes every pair to the digit's
        // running offset, from (keys, vals) to (tmp_k, tmp_v) and back.
        uint32_t *src_k = keys, *src_v = vals, *dst_k = tmp_k, *dst_v = tmp_v;
        for (uint32_t p = 0; p < passes; p++) {
            const uint32_t sh = 8u * p, bits = min(8u, low - sh), dmask = (1u << bits) - 1u;
            if (tid < kRadix) s_run[tid] = 0u;
            __syncthreads();
            for (uint32_t e = (uint32_t)tid; e < size; e += kBsThreads) atomicAdd(&s_run[(src_k[start + e] >> sh) & dmask], 1u);
            __syncthreads();
            const uint32_t c = tid < kRadix ? s_run[tid] : 0u;
            uint32_t all;
            const uint32_t before = block_exclusive_scan<kBsThreads>(c, s_tot, &all);
            if (tid < kRadix) s_run[tid] = before;
            __syncthreads();
            for (uint32_t c0 = 0; c0 < size; c0 += kBsCap) {
                const uint32_t cnt = min(kBsCap, size - c0);
                const uint32_t iw = (cnt + kBsThreads - 1u) / kBsThreads;
                const uint32_t wbase = (uint32_t)wave * 64u * iw;
    #pragma unroll
                for (int j = 0; j < kBsItems; j++) {
                    if ((uint32_t)j < iw) {
                        const uint32_t e = wbase + (uint32_t)j * 64u + (uint32_t)lane;
                        k[j] = e < cnt ? src_k[start + c0 + e] : 0u;
                        v[j] = e < cnt ? src_v[start + c0 + e] : 0u;
                    }
                }
                bucket_rank(k, pos, iw, cnt, sh, bits, s_hist, s_start, s_cnt, s_tot);
    #pragma unroll
                for (int j = 0; j < kBsItems; j++) {
                    if ((uint32_t)j < iw) {
                        if (wbase + (uint32_t)j * 64u + (uint32_t)lane < cnt) {
                            const uint32_t d = (k[j] >> sh) & dmask;
                            const uint32_t dst = start + s_run[d] + (pos[j] - s_start[d]);
                            dst_k[dst] = k[j];
                            dst_v[dst] = v[j];
                        }
                    }
                }
                __syncthreads();
                if (tid < kRadix) s_run[tid] += s_cnt[tid];
                __syncthreads();
            }
            uint32_t* t = src_k;
            src_k = dst_k;
            dst_k = t;
            t = src_v;
            src_v = dst_v;
            dst_v = t;
        }
        // the sorted values into vals, and cum_tiles_hit over them, by chunks
        uint32_t carry = 0u;
        for (uint32_t c0 = 0; c0 < size; c0 += kBsCap) {
            const uint32_t cnt = min(kBsCap, size - c0);
            const uint32_t iw = (cnt + kBsThreads - 1u) / kBsThreads;
            const uint32_t wbase = (uint32_t)wave * 64u * iw;
#pragma unroll
            for (int j = 0; j < kBsItems; j++) {
                if ((uint32_t)j < iw) {
                    const uint32_t e = wbase + (uint32_t)j * 64u + (uint32_t)lane;
                    v[j] = e < cnt ? src_v[start + c0 + e] : 0u;
                    if (e < cnt && src_v != vals) vals[start + c0 + e] = v[j];
                }
            }
            carry += cum_chunk(v, iw, cnt, weight, cum + start + c0, carry, c0 == 0u ? part : 0u, s_w);
        }
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

template <bool FIRST, int ITEMS, typename KI, typename KO>
static void launch_digit_pass(bh_ctx* ctx, uint32_t parts, const KI* src_k, const uint32_t* src_v, KO* dk,
                              uint32_t* dv, uint32_t n, uint32_t sh, uint32_t bits, uint32_t sub, uint32_t cap,
                              uint32_t radix, const uint32_t* offs, const uint32_t* gs, uint32_t* go,
                              const SortDevice& dev) {
    if constexpr (sizeof(KI) == 4 && sizeof(KO) == 4) {
        if (go) {
            launch(ctx, onesweep_kernel<FIRST, ITEMS, true, KI, KO>, dim3(parts), dim3(kThreads), 0u, src_k, src_v, dk,
                   dv, n, sh, bits, sub, cap, radix, offs, gs, go, dev);
            return;
        }
    }
    launch(ctx, onesweep_kernel<FIRST, ITEMS, false, KI, KO>, dim3(parts), dim3(kThreads), 0u, src_k, src_v, dk, dv, n,
           sh, bits, sub, cap, radix, offs, nullptr, nullptr, dev);
}

// One digit pass: upsweep, offset scan, scatter.  Keys are read as uint16_t
// or uint32_t (in_w bytes) and written as out_w bytes; 16-bit keys carry at
// most 16 key bits.
template <bool FIRST, int I>
static bh_status sort_pass(bh_ctx* ctx, const ScanPlan& sp, const std::string& up_name,
                           const std::string& scan_name, const std::string& pass_name, const void* src_k,
                           int in_w, const uint32_t* src_v, void* dk, int out_w, uint32_t* dv, uint32_t n,
                           uint32_t sh, uint32_t bits, uint32_t sub, uint32_t cap, uint32_t* offs, uint32_t* pblk,
                           const uint32_t* gs, uint32_t* go, const SortDevice& pdev) {
    const dim3 grid(sp.parts), block(kThreads);
    {
        KernelTimer t(ctx, up_name.c_str());
        if (in_w == 2)
            launch(ctx, radix_upsweep_kernel<FIRST, I, uint16_t>, grid, block, 0u, (const uint16_t*)src_k, n, sh, bits,
                   sub, cap, sp.radix, sp.rows, offs, pblk, pdev);
        else
            launch(ctx, radix_upsweep_kernel<FIRST, I, uint32_t>, grid, block, 0u, (const uint32_t*)src_k, n, sh, bits,
                   sub, cap, sp.radix, sp.rows, offs, pblk, pdev);
    }
    {
        KernelTimer t(ctx, scan_name.c_str());
        launch(ctx, radix_scan_kernel, dim3(sp.blocks), dim3(kScanThreads), 0u, offs, pblk, sp.parts, sp.rows,
               sp.blocks, sp.radix);
    }
    KernelTimer t(ctx, pass_name.c_str());
    if (in_w == 4 && out_w == 4)
        launch_digit_pass<FIRST, I, uint32_t, uint32_t>(ctx, sp.parts, (const uint32_t*)src_k, src_v, (uint32_t*)dk,
                                                        dv, n, sh, bits, sub, cap, sp.radix, offs, gs, go, pdev);
    else if (in_w == 2 && out_w == 2 && !go)
        launch_digit_pass<FIRST, I, uint16_t, uint16_t>(ctx, sp.parts, (const uint16_t*)src_k, src_v, (uint16_t*)dk,
                                                        dv, n, sh, bits, sub, cap, sp.radix, offs, gs, go, pdev);
    else if (in_w == 2 && out_w == 4 && !go)
        launch_digit_pass<FIRST, I, uint16_t, uint32_t>(ctx, sp.parts, (const uint16_t*)src_k, src_v, (uint32_t*)dk,
                                                        dv, n, sh, bits, sub, cap, sp.radix, offs, gs, go, pdev);
    else
        return set_error(ctx, BH_ERR_INVALID_ARG, "radix sort: unsupported key widths");
    return BH_OK;
}

// The sort over keys stored as in_w / tmp_w / out_w bytes (keys_in, the
// temporaries and keys_out).
static bh_status radix_sort_impl(bh_ctx* ctx, const void* keys_in, int in_w, const uint32_t* vals_in, uint32_t n,
                                 uint32_t key_bits, uint32_t key_sub, uint32_t key_cap, void* keys_out, int out_w,
                                 uint32_t* vals_out, void* tmp_keys, int tmp_w, uint32_t* tmp_vals, void* scratch,
                                 const char* tag, bool scratch_zeroed, const uint32_t* gather_src,
                                 uint32_t* gather_out, const SortDevice& dev) {
    const std::string up_name = std::string(tag) + "_up", scan_name = std::string(tag) + "_scan",
                      pass_name = std::string(tag) + "_onesweep";
    if (n == 0) return BH_OK;
    if (key_bits > 32) return set_error(ctx, BH_ERR_INVALID_ARG, "radix sort: more than 32 key bits");
    if (std::min(std::min(in_w, out_w), tmp_w) < 4 && (key_bits > 16 || key_sub != 0u))
        return set_error(ctx, BH_ERR_INVALID_ARG, "radix sort: 16-bit keys carry at most 16 key bits");
    const DigitPlan plan = digit_plan(key_bits);
    const ScanPlan sp = scan_plan(n, plan);
    uint32_t* blk = (uint32_t*)scratch;
    uint32_t* offs = blk + (size_t)plan.passes * sp.blocks * sp.radix;
    if (!scratch_zeroed) launch_fill_u32(ctx, blk, 0u, radix_sort_zeroed_words(n, key_bits));
    const void* src_k = keys_in;
    int src_w = in_w;
    const uint32_t* src_v = vals_in;
    // a dropping sort: the first pass sees n pairs, the later ones n_rest
    SortDevice dev_rest = dev;
    dev_rest.drop_capped = false;
    if (dev.drop_capped && dev.n_rest) dev_rest.n = dev.n_rest;
    const uint32_t n_first = n, n_later = dev.drop_capped ? std::min(n, dev.n_rest_host) : n;
    for (uint32_t p = 0; p < plan.passes; p++) {
        const SortDevice& pdev = p == 0 ? dev : dev_rest;
        n = p == 0 ? n_first : n_later;
        // the last pass lands in the output buffers
        bool to_out = ((plan.passes - 1 - p) % 2) == 0;
        void* dk = to_out ? keys_out : tmp_keys;
        const int dst_w = to_out ? out_w : tmp_w;
        uint32_t* dv = to_out ? vals_out : tmp_vals;
        uint32_t* pblk = blk + (size_t)p * sp.blocks * sp.radix;
        const uint32_t sh = plan.shift(p), bits = plan.bits(p);
        const uint32_t sub = p == 0 ? key_sub : 0u, cap = p == 0 ? key_cap : 0xFFFFFFFFu;
        const bool last = p + 1 == plan.passes;
        const uint32_t* gs = last ? gather_src : nullptr;
        uint32_t* go = last ? gather_out : nullptr;
#define BH_SORT_PASS(F, I)                                                                                   \
    do {                                                                                                         \
        const bh_status st_ = sort_pass<F, I>(ctx, sp, up_name, scan_name, pass_name, src_k, src_w, src_v, dk,   \
                                              dst_w, dv, n, sh, bits, sub, cap, offs, pblk, gs, go, pdev);      \
        if (st_ != BH_OK) return st_;                                                                            \
    } while (0)
        if (sp.items == 8) {
            if (p == 0) BH_SORT_PASS(true, 8); else BH_SORT_PASS(false, 8);
        } else {
            if (p == 0) BH_SORT_PASS(true, 4); else BH_SORT_PASS(false, 4);
        }
#undef BH_SORT_PASS
        src_k = dk;
        src_w = dst_w;
        src_v = dv;
    }
    return check_launch(ctx, "radix sort");
}

bh_status radix_sort_pairs(bh_ctx* ctx, const uint32_t* keys_in, const uint32_t* vals_in, uint32_t n,
                           uint32_t key_bits, uint32_t key_sub, uint32_t key_cap, uint32_t* keys_out,
                           uint32_t* vals_out, uint32_t* tmp_keys, uint32_t* tmp_vals, void* scratch,
                           const char* tag, bool scratch_zeroed, const uint32_t* gather_src,
                           uint32_t* gather_out, const SortDevice& dev) {
    return radix_sort_impl(ctx, keys_in, 4, vals_in, n, key_bits, key_sub, key_cap, keys_out, 4, vals_out, tmp_keys,
                           4, tmp_vals, scratch, tag, scratch_zeroed, gather_src, gather_out, dev);
}

bh_status radix_sort_pairs_k16(bh_ctx* ctx, const uint16_t* keys_in, const uint32_t* vals_in, uint32_t n,
                               uint32_t key_bits, uint32_t* keys_out, uint32_t* vals_out, uint16_t* tmp_keys,
                               uint32_t* tmp_vals, void* scratch, const char* tag, bool scratch_zeroed,
                               const SortDevice& dev) {
    return radix_sort_impl(ctx, keys_in, 2, vals_in, n, key_bits, 0u, 0xFFFFFFFFu, keys_out, 4, vals_out, tmp_keys,
                           2, tmp_vals, scratch, tag, scratch_zeroed, nullptr, nullptr, dev);
}

bh_status depth_sort_buckets(bh_ctx* ctx, const uint32_t* keys_in, uint32_t n, uint32_t key_sub, uint32_t key_cap,
                             uint32_t* keys_tmp, uint32_t* vals_out, uint32_t* tmp_keys, uint32_t* tmp_vals,
                             void* scratch, bool scratch_zeroed, const uint32_t* weight, uint32_t* cum,
                             const SortDevice& dev) {
    if (n == 0) return BH_OK;
    const DigitPlan plan = digit_plan(8);
    const ScanPlan sp = scan_plan(n, plan);
    // block sums | per-block digit weight sums (both zeroed) | offsets
    const size_t blk_words = (size_t)sp.blocks * sp.radix;
    uint32_t* blk = (uint32_t*)scratch;
    uint32_t* wsum = blk + blk_words;
    uint32_t* offs = wsum + blk_words;
    // the buckets bucket_count_kernel sorted, after the offsets
    uint32_t* done = offs + (size_t)sp.parts * sp.radix;
    if ((2 * blk_words + (size_t)sp.parts * sp.radix + kBsBuckets) * 4 > radix_sort_scratch_bytes(n, 32))
        return set_error(ctx, BH_ERR_INTERNAL, "depth sort: scratch too small for the bucket flags");
    if (!scratch_zeroed) launch_fill_u32(ctx, blk, 0u, 2 * blk_words);
    SortDevice d = dev;
    d.weight = weight;
    d.wsum = wsum;
    // the top-digit pass: keys to keys_tmp, values (input indices) to
    // vals_out, their weights beside them to tmp_vals (read by the count
    // kernel; the LSD kernel's larger buckets reuse their own ranges of it)
    bh_status st;
    if (sp.items == 8)
        st = sort_pass<true, 8>(ctx, sp, "depth_sort_up", "depth_sort_scan", "depth_sort_onesweep", keys_in, 4,
                                nullptr, keys_tmp, 4, vals_out, n, kShiftTop, 8u, key_sub, key_cap, offs, blk, weight,
                                tmp_vals, d);
    else
        st = sort_pass<true, 4>(ctx, sp, "depth_sort_up", "depth_sort_scan", "depth_sort_onesweep", keys_in, 4,
                                nullptr, keys_tmp, 4, vals_out, n, kShiftTop, 8u, key_sub, key_cap, offs, blk, weight,
                                tmp_vals, d);
    if (st != BH_OK) return st;
    {
        const uint32_t n_rest = dev.drop_capped ? std::min(n, dev.n_rest_host) : n;
        const uint32_t* n_dev = dev.drop_capped ? dev.n_rest : dev.n;
        {
            KernelTimer t(ctx, "depth_sort_count");
            launch(ctx, bucket_count_kernel, dim3(kBsBuckets), dim3(kBsThreads), 0u, keys_tmp, vals_out, offs, n_rest,
                   n_dev, key_cap, dev.key_cap, (const uint32_t*)tmp_vals, wsum, (uint32_t)blk_words, cum, done);
        }
        KernelTimer t(ctx, "depth_sort_buckets");
        launch(ctx, bucket_sort_kernel, dim3(kBsBuckets), dim3(kBsThreads), 0u, keys_tmp, vals_out, offs, n_rest,
               n_dev, key_cap, dev.key_cap, weight, wsum, (uint32_t)blk_words, cum, tmp_keys, tmp_vals, done);
    }
    return check_launch(ctx, "depth sort");
}

size_t depth_sort_buckets_zeroed_words(uint32_t n) {
    const ScanPlan sp = scan_plan(n, digit_plan(8));
    return 2 * (size_t)sp.blocks * sp.radix;
}

__global__ void mask_u32_kernel(const uint32_t* __restrict__ in, uint32_t mask, uint32_t n,
                                uint32_t* __restrict__ out) {
    uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i < n) out[i] = in[i] & mask;
}

void launch_mask_u32(bh_ctx* ctx, const uint32_t* in, uint32_t mask, uint32_t n, uint32_t* out) {
    if (n == 0) return;
    KernelTimer t(ctx, "mask");
    launch(ctx, mask_u32_kernel, dim3(div_up(n, 256)), dim3(256), 0u, in, mask, n, out);
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
    launch(ctx, gather_pairs_kernel, dim3(div_up(n, 256)), dim3(256), 0u, keys_in, vals_in, perm, n, keys_out,
           vals_out);
}

// ---- inclusive scan (reduce-then-scan) -------------------------------------------

// A partition is 256 threads x 4 * `chunks` consecutive values, with `chunks`
// chosen so that there are at most 4096 partitions: one reduce kernel writes
// each partition's sum, then the scan kernel adds the sums of the partitions
// before it (at most 16 loads per thread, issued with the value loads) to the
// in-partition scan.  The values are read twice, the second time mostly from
// cache.  `out` may alias `in`: every value is read by the thread that writes
// it, before it writes it.  (The forward's scan of tile counts in depth order
// reads counts that the depth sort's last pass gathered, so no scan kernel
// gathers: a gather in each of the two kernels measured 25 us at 1M splats.)
struct ScanGeom {
    uint32_t chunks, part, parts;
};
static ScanGeom scan_geom(uint32_t n) {
    ScanGeom g;
    g.chunks = std::max<uint32_t>(1u, div_up(n, (uint64_t)4096 * kThreads * 4));
    g.part = kThreads * 4u * g.chunks;
    g.parts = div_up(n, g.part);
    return g;
}

__device__ __forceinline__ uint32_t scan_value(const uint32_t* in, uint64_t idx, uint32_t n) {
    return idx < n ? in[idx] : 0u;
}

__global__ __launch_bounds__(kThreads) void scan_reduce_kernel(const uint32_t* in, uint32_t n, uint32_t chunks,
                                                                uint32_t* __restrict__ sums,
                                                                const uint32_t* __restrict__ dev_n) {
    __shared__ uint32_t s_tot[kWaves];
    if (dev_n) n = min(n, *dev_n);
    const uint64_t first = ((uint64_t)blockIdx.x * kThreads + threadIdx.x) * 4u * chunks;
    uint32_t run = 0;
    for (uint32_t c = 0; c < chunks; c++) {
        uint32_t x[4];
#pragma unroll
        for (int j = 0; j < 4; j++) x[j] = scan_value(in, first + c * 4u + j, n);
        run += x[0] + x[1] + x[2] + x[3];
    }
    uint32_t total;
    (void)block_exclusive_scan<kThreads>(run, s_tot, &total);
    if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

__global__ __launch_bounds__(kThreads) void scan_down_kernel(const uint32_t* in, uint32_t* out, uint32_t n,
                                                              uint32_t chunks, const uint32_t* __restrict__ sums,
                                                              const uint32_t* __restrict__ dev_n) {
    __shared__ uint32_t s_tot[kWaves];
    if (dev_n) n = min(n, *dev_n);
    const uint32_t part = blockIdx.x, tid = threadIdx.x;
    const uint64_t first = ((uint64_t)part * kThreads + tid) * 4u * chunks;
    // the sums of the partitions before this one (part < 4096: 16 per thread)
    uint32_t prev[16];
#pragma unroll
    for (uint32_t i = 0; i < 16; i++) {
        const uint32_t q = tid + i * kThreads;
        prev[i] = q < part ? sums[q] : 0u;
    }
    uint32_t run = 0;
    for (uint32_t c = 0; c < chunks; c++) {
        uint32_t x[4];
#pragma unroll
        for (int j = 0; j < 4; j++) x[j] = scan_value(in, first + c * 4u + j, n);
        run += x[0] + x[1] + x[2] + x[3];
    }
    uint32_t before = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) before += prev[i];
    uint32_t part_excl;
    (void)block_exclusive_scan<kThreads>(before, s_tot, &part_excl);
    uint32_t dummy;
    uint32_t acc = part_excl + block_exclusive_scan<kThreads>(run, s_tot, &dummy);
    for (uint32_t c = 0; c < chunks; c++) {
        uint32_t x[4];
#pragma unroll
        for (int j = 0; j < 4; j++) x[j] = scan_value(in, first + c * 4u + j, n);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            acc += x[j];
            if (first + c * 4u + j < n) out[first + c * 4u + j] = acc;
        }
    }
}

// at most 4096 partition sums for any n (so a caller may size it for an upper
// bound of n)
size_t scan_scratch_bytes(uint32_t) { return (size_t)4096 * 4; }

bh_status inclusive_scan(bh_ctx* ctx, const uint32_t* in, uint32_t* out, uint32_t n, void* scratch,
                         const uint32_t* dev_n) {
    if (n == 0) return BH_OK;
    const ScanGeom g = scan_geom(n);
    uint32_t* sums = (uint32_t*)scratch;
    {
        KernelTimer t(ctx, "scan_reduce");
        launch(ctx, scan_reduce_kernel, dim3(g.parts), dim3(kThreads), 0u, in, n, g.chunks, sums, dev_n);
    }
    {
        KernelTimer t(ctx, "scan");
        launch(ctx, scan_down_kernel, dim3(g.parts), dim3(kThreads), 0u, in, out, n, g.chunks, sums, dev_n);
    }
    return check_launch(ctx, "scan");
}

}  // namespace bh
