// bh_lookback.h — decoupled look-back building blocks shared by the sort,
// the scan and the kernels that fuse a scan into their own pass.
//
// A partition publishes its aggregate (flag kFlagAgg) as soon as it knows it
// and its inclusive prefix (kFlagPrefix) once its look-back is done; a status
// word holds the flag in its top two bits and the value in its low 32 bits,
// and a zero word means "not published".  A partition is its workgroup's id
// and only waits on lower ids, which the in-order dispatch of each XCD has
// already made resident.  Spins are bounded: on exhaustion the kernel raises
// kErrSpin and still completes.
#pragma once

#include <hip/hip_runtime.h>

#include "bh_internal.h"

namespace bh {

constexpr uint64_t kFlagAgg = 1ull << 62;
constexpr uint64_t kFlagPrefix = 2ull << 62;
constexpr uint32_t kSpinLimit = 1u << 24;

__device__ __forceinline__ uint64_t status_load(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void status_store(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Sum of the values published by partitions [0, part) for one status column.
// Walks backwards accumulating aggregates until an inclusive prefix is found,
// reading four predecessors per round trip (the loads are independent).
__device__ inline uint32_t look_back(const uint64_t* status, uint32_t part, uint32_t stride, uint32_t col,
                              uint32_t* err) {
    uint32_t excl = 0;
    int64_t p = (int64_t)part - 1;
    uint32_t spins = 0;
    while (p >= 0) {
        uint64_t s[4];
#pragma unroll
        for (int i = 0; i < 4; i++) s[i] = p - i >= 0 ? status_load(status + (uint64_t)(p - i) * stride + col) : 0ull;
        bool stalled = false, found = false;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if (stalled || found || p - i < 0) continue;
            const uint64_t flag = s[i] & (3ull << 62);
            if (flag == 0) {
                stalled = true;  // wait for this one, keeping what was summed
                p -= i;
                continue;
            }
            excl += (uint32_t)s[i];
            if (flag == kFlagPrefix) found = true;
        }
        if (found) break;
        if (!stalled) {
            p -= 4;
            continue;
        }
        if (++spins >= kSpinLimit) {
            atomicOr(err, kErrSpin);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    return excl;
}

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

}  // namespace bh
