// Wavefront-level reductions for wave64 (gfx950).  Reductions inside a
// 16-lane row use DPP modifiers (one VALU op per step); wider steps use
// ds_bpermute through __shfl_xor.
#pragma once
#include <hip/hip_runtime.h>

namespace ullm {

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
// DPP controls: quad_perm [1,0,3,2] / [2,3,0,1], row_half_mirror, row_mirror.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

// Sum over aligned groups of N lanes (N a power of two <= 64); every lane of a
// group receives the group total.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
    if constexpr (N >= 2) x += dpp<kDppXor1>(x);
    if constexpr (N >= 4) x += dpp<kDppXor2>(x);
    if constexpr (N >= 8) x += dpp<kDppHalfMirror>(x);
    if constexpr (N >= 16) x += dpp<kDppMirror>(x);
    if constexpr (N >= 32) x += __shfl_xor(x, 16, 64);
    if constexpr (N >= 64) x += __shfl_xor(x, 32, 64);
    return x;
}

// Full-wave sum in VALU only: DPP inside 16-lane rows, then the gfx950 lane
// swaps across rows (x + the lane 16 / 32 away); every lane gets the total.
__device__ __forceinline__ float wave_sum(float x) {
    x += dpp<kDppXor1>(x);
    x += dpp<kDppXor2>(x);
    x += dpp<kDppHalfMirror>(x);
    x += dpp<kDppMirror>(x);
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

// The value of lane l ^ 32.
__device__ __forceinline__ float xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((__lane_id() & 32) ? r[0] : r[1]);
}

}  // namespace ullm
