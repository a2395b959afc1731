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
// `blocks` of `rows` (a power of two >= sqrt(parts)) for the offset scan, so
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
    s.rows = 16;
    while ((uint64_t)s.rows * s.rows < s.parts) s.rows *= 2;
    s.blocks = div_up(s.parts, s.rows);
    s.radix = 1u << d.width;
    return s;
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
    const int tid = threadIdx.x, wave = tid >> 6;
    if (dev.n) n = min(n, *dev.n);
    if (FIRST && dev.key_sub) {
        key_sub = *dev.key_sub;
        key_cap = *dev.key_cap;
    }
    for (int i = tid; i < kWaves * kRadix; i += kThreads) (&s_hist[0][0])[i] = 0;
    __syncthreads();
    constexpr int PART = kThreads * ITEMS;
    const uint32_t part = blockIdx.x;
    const uint64_t base = (uint64_t)part * PART;
    const uint32_t dmask = (1u << digit_bits) - 1u;
    uint32_t* mine = s_hist[wave];
    // the first pass of a dropping sort does not count capped keys
    const bool drop = FIRST && dev.drop_capped;
    if (base + PART <= n && (reinterpret_cast<uintptr_t>(keys) & 15u) == 0u) {
        // this thread's ITEMS keys as 32-bit words: 16-byte loads (8-byte
        // ones for four 16-bit keys), interleaved across the threads
        constexpr int WORDS = ITEMS * (int)sizeof(K) / 4;
        constexpr int VW = WORDS >= 4 ? 4 : 2;
        uint32_t w[WORDS];
        if constexpr (VW == 4) {
            const uint4* k4 = reinterpret_cast<const uint4*>(keys + base);
#pragma unroll
            for (int j = 0; j < WORDS / 4; j++) {
                const uint4 q = k4[j * kThreads + tid];
                w[4 * j] = q.x, w[4 * j + 1] = q.y, w[4 * j + 2] = q.z, w[4 * j + 3] = q.w;
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
            if (!(drop && k == key_cap)) atomicAdd(&mine[(k >> shift) & dmask], 1u);
        }
    } else {
#pragma unroll
        for (int j = 0; j < ITEMS; j++) {
            const uint64_t idx = base + (uint64_t)j * kThreads + tid;
            if (idx < n) {
                const uint32_t kw = keys[idx];
                const uint32_t k = FIRST ? min(kw - key_sub, key_cap) : kw;
                if (!(drop && k == key_cap)) atomicAdd(&mine[(k >> shift) & dmask], 1u);
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
    // the first pass of a dropping sort neither ranks nor writes capped keys
    const bool drop = FIRST && dev.drop_capped;
    uint32_t kept = 0;  // bit j: item j is a pair of this pass
#pragma unroll
    for (int j = 0; j < ITEMS; j++) {
        uint64_t idx = wave_base + (uint64_t)j * 64 + lane;
        bool valid = idx < n;
        uint32_t kk = valid ? keys_in[idx] : 0u;
        if (FIRST) kk = min(kk - key_sub, key_cap);
        if (drop && kk == key_cap) valid = false;
        if (valid) kept |= 1u << j;
        k[j] = kk;
        v[j] = valid ? (vals_in ? vals_in[idx] : (uint32_t)idx) : 0u;
    }
    uint32_t gv[GATHER ? ITEMS : 1];
    if (GATHER) {
#pragma unroll
        for (int j = 0; j < ITEMS; j++) gv[j] = (kept >> j) & 1u ? gather_src[v[j]] : 0u;
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
