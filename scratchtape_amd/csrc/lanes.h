// Cross-lane exchanges within a wave64 that stay in the VALU.
//
// __shfl_xor compiles to ds_bpermute_b32, which goes through the LDS unit:
// roughly a hundred cycles per exchange, and a butterfly or bitonic network
// chains many of them.  xor_lane(v, j, lane) returns lane (lane ^ j)'s v for
// j a power of two below 64 with
//   j = 1, 2   a DPP quad permutation ([1,0,3,2], [2,3,0,1]);
//   j = 4      DPP row_shl:4 (lane i reads i + 4) or row_shr:4 (i - 4) within
//              the 16-lane row, picked by lane bit 2 (the lanes a shift leaves
//              without a source are never picked);
//   j = 8      DPP row_ror:8 (rotation by 8 within the row);
//   j = 15     DPP row_mirror (lane i of a row reads lane 15 - i); 63 is
//              15, then 16, then 32;
//   j = 16, 32 v_permlane16_swap / v_permlane32_swap of v with itself: the
//              swap returns (v with the odd rows / upper half replaced,
//              v with the even rows / lower half replaced), and a lane takes
//              the one holding its partner's value.
// Each of these is checked on the device against lane ^ j by st_lane_selftest.  Inside an
// unrolled loop j is a constant and the switch folds away; any other j falls
// back to __shfl_xor.  The partner lane must be active (a DPP read from a
// disabled lane does not return its register): callers use these in
// wave-uniform code, or (j < 16, which stays within a row of 16 lanes) in code
// uniform over each row.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace st {

__device__ __forceinline__ uint32_t xor_lane(uint32_t v, int j, int lane) {
    switch (j) {
        case 1:
            return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
        case 2:
            return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);
        case 4: {
            const uint32_t up = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x104, 0xF, 0xF, false);
            const uint32_t dn = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x114, 0xF, 0xF, false);
            return (lane & 4) ? dn : up;
        }
        case 8:
            return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, false);
        case 15:
            return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, false);
        case 63: {
            const uint32_t m = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, false);
            const auto r = __builtin_amdgcn_permlane16_swap(m, m, false, false);
            const uint32_t t = (lane & 16) ? r[0] : r[1];
            const auto q = __builtin_amdgcn_permlane32_swap(t, t, false, false);
            return (lane & 32) ? q[0] : q[1];
        }
        case 16: {
            const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
            return (lane & 16) ? r[0] : r[1];
        }
        case 32: {
            const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
            return (lane & 32) ? r[0] : r[1];
        }
        default:
            return (uint32_t)__shfl_xor((int)v, j, 64);
    }
}

__device__ __forceinline__ int32_t xor_lane(int32_t v, int j, int lane) {
    return (int32_t)xor_lane((uint32_t)v, j, lane);
}

__device__ __forceinline__ float xor_lane(float v, int j, int lane) {
    return __builtin_bit_cast(float, xor_lane(__builtin_bit_cast(uint32_t, v), j, lane));
}

__device__ __forceinline__ uint64_t xor_lane(uint64_t v, int j, int lane) {
    const uint32_t lo = xor_lane((uint32_t)v, j, lane), hi = xor_lane((uint32_t)(v >> 32), j, lane);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ double xor_lane(double v, int j, int lane) {
    return __builtin_bit_cast(double, xor_lane(__builtin_bit_cast(uint64_t, v), j, lane));
}

// Inclusive prefix sum over the wave's 64 lanes: DPP row_shr 1, 2, 4, 8
// within each row of 16 (a shift past the row's start reads 0), then
// row_bcast:15 adds each even row's last lane to the row after it (rows 1, 3)
// and row_bcast:31 adds lane 31 to rows 2 and 3.  Checked by st_lane_selftest.
__device__ __forceinline__ int32_t wave_incl_scan(int32_t x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);
    return x;
}

// A wave-uniform lane's value (index known to be the same in every lane).
__device__ __forceinline__ uint32_t lane_value(uint32_t v, int src) { return (uint32_t)__builtin_amdgcn_readlane((int)v, src); }
__device__ __forceinline__ int32_t lane_value(int32_t v, int src) { return __builtin_amdgcn_readlane(v, src); }

// This lane's index in its wave64.
__device__ __forceinline__ int lane_id() { return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

}  // namespace st
