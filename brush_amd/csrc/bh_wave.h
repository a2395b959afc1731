// bh_wave.h — wave64 scans over DPP lane moves.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace bh {

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROW_MASK, 0xF, true);
}

// Inclusive wave64 scans: shifts within 16-lane rows, then row broadcasts of
// lanes 15 and 31 into the following rows.
__device__ __forceinline__ uint32_t wave_incl_add_u32(uint32_t x) {
    x += dpp_u32<0x111, 0xF>(x);  // row_shr:1
    x += dpp_u32<0x112, 0xF>(x);  // row_shr:2
    x += dpp_u32<0x114, 0xF>(x);  // row_shr:4
    x += dpp_u32<0x118, 0xF>(x);  // row_shr:8
    x += dpp_u32<0x142, 0xA>(x);  // row_bcast:15 into rows 1 and 3
    x += dpp_u32<0x143, 0xC>(x);  // row_bcast:31 into rows 2 and 3
    return x;
}
__device__ __forceinline__ uint32_t wave_incl_max_u32(uint32_t x) {
    x = max(x, dpp_u32<0x111, 0xF>(x));
    x = max(x, dpp_u32<0x112, 0xF>(x));
    x = max(x, dpp_u32<0x114, 0xF>(x));
    x = max(x, dpp_u32<0x118, 0xF>(x));
    x = max(x, dpp_u32<0x142, 0xA>(x));
    x = max(x, dpp_u32<0x143, 0xC>(x));
    return x;
}

}  // namespace bh
