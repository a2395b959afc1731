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

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bh {

struct SplatRecord {
    uint2* masks = nullptr;
    uint32_t* block_end = nullptr;
};

inline size_t record_masks(uint64_t m, uint32_t bpt) { return (size_t)bpt * (size_t)m; }

// index of candidate lo's mask in the block's region
template <uint32_t BPT>
__device__ __forceinline__ size_t record_base(uint32_t blk, uint32_t lo, uint32_t hi) {
    return (size_t)BPT * lo + (size_t)blk * (hi - lo);
}

}  // namespace bh
