// bh_splat_record.h — the forward blend's record of which (splat, pixel) pairs
// contributed, read by the fused backward.
//
// The forward (rasterize_kernel with BWD_INFO) decides, pixel by pixel and
// front to back, which splats a pixel blends: alpha >= 1/255 (or the smooth
// band), sigma >= 0, and the transmittance test.  The reference's backward
// replays those decisions with the same arithmetic
// (crates/brush-render-bwd/src/kernels/rasterize_backwards.rs:308-441).  Here
// the forward writes them down instead, one bit per pair, and the fused
// backward reads them: it evaluates only pairs that contributed and needs no
// bit-exact replay of the forward's alpha and transmittance.
//
// Layout, per 8x8 block of a tile whose candidate list is [lo, hi) (len =
// hi - lo, BPT blocks per tile):
//   masks[BPT lo + blk len + (k - lo)]  bit p: candidate k contributed to
//                                       pixel p of the block (p = lane =
//                                       x + 8 y within the block)
//   block_end[tile BPT + blk]           one past the last candidate any
//                                       pixel of the block consumed (lo when
//                                       none did)
// Candidate runs are in tile order, so the tiles' regions [BPT lo, BPT hi)
// partition [0, BPT M) (M candidates).  The forward writes the masks of every
// batch of 64 candidates it walks; the backward reads candidates below
// block_end only, all of which lie in walked batches.
#pragma once

#include "bh_wave.h"

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bh {

// The backward's dispatch order, built by the forward blend: tiles grouped
// into kOrderBuckets buckets by the candidates their pixels blended (longest
// first; the order inside a bucket is arbitrary), and the backward's
// workgroup for slot i takes the i-th tile of the concatenated bucket lists.
// count[b] hands out slots of list[b][...].  Each of a tile's BPT blocks adds
// (1 << 32) | its bucket << (8 blk) to word[tile] (one 64-bit atomic), so the
// last block finds every block's bucket in the returned word and appends the
// tile under the smallest (its longest block's), with no fence between the
// blocks; tiles that blended nothing are left out.  word and count start at
// zero.  (Tile offsets building the forward's order the same way, from the
// two ends of each run, took 54 instead of 11 us: its appends arrive close
// together on a few hot bucket counters.)
constexpr uint32_t kOrderBuckets = 64;

struct TileOrder {
    unsigned long long* word = nullptr;  // [num_tiles]
    uint32_t* count = nullptr;           // [kOrderBuckets]
    uint32_t* list = nullptr;            // [kOrderBuckets][num_tiles]; null: no order
};

struct SplatRecord {
    uint2* masks = nullptr;
    uint32_t* block_end = nullptr;
    TileOrder order;  // the backward's dispatch order
};

inline size_t record_masks(uint64_t m, uint32_t bpt) { return (size_t)bpt * (size_t)m; }

// A tile (or block) of len candidates: 63 - q with q = len below 4 and a
// quarter-octave index above (q = 4 at len = 4, 8 at 8, 12 at 16, ...), so
// that longer ones fall in smaller buckets; len 0 gives 63, and lengths
// from ~114k up share bucket 0.
__device__ __forceinline__ uint32_t order_bucket(uint32_t len) {
    uint32_t q = len;
    if (len >= 4u) {
        const uint32_t msb = 31u - (uint32_t)__builtin_clz(len);
        q = msb * 4u + ((len >> (msb - 2u)) & 3u) - 4u;
    }
    return (kOrderBuckets - 1u) - min(q, kOrderBuckets - 1u);
}

// The tile of dispatch slot `slot`, or num_tiles when the slot lies past the
// last recorded tile.  Called by a whole wave (64 lanes) with a uniform slot:
// lane b holds bucket b's count, a wave scan gives each bucket's end, and the
// slot's bucket is the first whose end lies past it.
static_assert(kOrderBuckets == 64, "one order bucket per lane of a wave");
__device__ __forceinline__ uint32_t ordered_tile(uint32_t slot, const uint32_t* __restrict__ count,
                                                 const uint32_t* __restrict__ list, uint32_t num_tiles) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t c = count[lane];
    const uint32_t end = wave_incl_add_u32(c);
    const uint64_t past = __builtin_amdgcn_ballot_w64(slot < end);
    if (past == 0ull) return num_tiles;
    const uint32_t bucket = (uint32_t)__builtin_ctzll(past);
    const uint32_t start = (uint32_t)__builtin_amdgcn_readlane((int)(end - c), (int)bucket);
    return list[(size_t)bucket * num_tiles + (slot - start)];
}

// Appends tile t to bucket b of an order.
__device__ __forceinline__ void order_append(const TileOrder& o, uint32_t b, uint32_t t, uint32_t num_tiles) {
    const uint32_t k = atomicAdd(&o.count[b], 1u);
    o.list[(size_t)b * num_tiles + k] = t;
}

// index of candidate lo's mask in the block's region
template <uint32_t BPT>
__device__ __forceinline__ size_t record_base(uint32_t blk, uint32_t lo, uint32_t hi) {
    return (size_t)BPT * lo + (size_t)blk * (hi - lo);
}

}  // namespace bh
