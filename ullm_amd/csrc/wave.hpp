// Wavefront-level reductions for wave64 (gfx950).  Reductions inside a
// 16-lane row use DPP modifiers (one VALU op per step); wider steps use
// the gfx950 row swaps (v_permlane16_swap / v_permlane32_swap): no LDS round
// trips.
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
    if constexpr (N >= 32) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    if constexpr (N >= 64) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
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

// max / sum of x over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four 16-lane rows),
// in VALU only (the gfx950 row swaps), every lane getting the result.
__device__ __forceinline__ float rows_max(float x) {
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

// Full-wave max in VALU only (as wave_sum).
__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp<kDppXor1>(x));
    x = fmaxf(x, dpp<kDppXor2>(x));
    x = fmaxf(x, dpp<kDppHalfMirror>(x));
    x = fmaxf(x, dpp<kDppMirror>(x));
    return rows_max(x);
}

// Sum over the lanes congruent to l modulo N (N a power of two, 1 <= N <= 16):
// row rotations by N, 2N, .. 8 inside each 16-lane row, then the row swaps.
template <int N>
__device__ __forceinline__ float class_sum(float x) {
    static_assert(N >= 1 && N <= 16 && (N & (N - 1)) == 0, "class size");
    if constexpr (N <= 1) x += dpp<0x121>(x);
    if constexpr (N <= 2) x += dpp<0x122>(x);
    if constexpr (N <= 4) x += dpp<0x124>(x);
    if constexpr (N <= 8) x += dpp<0x128>(x);  // row_ror:8 = lane ^ 8 in the row
    return rows_sum(x);
}

// The value of lane l ^ 32.
__device__ __forceinline__ float xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((__lane_id() & 32) ? r[0] : r[1]);
}

// The value of lane l ^ OFF, OFF in {8, 16, 32}, without an LDS round trip
// (8: a row rotation by 8 within each 16-lane row, which is l ^ 8 there).
template <int OFF>
__device__ __forceinline__ float lane_xor(float x) {
    static_assert(OFF == 8 || OFF == 16 || OFF == 32, "lane_xor offset");
    if constexpr (OFF == 8) {
        return dpp<0x128>(x);
    } else if constexpr (OFF == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        return __uint_as_float((__lane_id() & 16) ? r[0] : r[1]);
    } else {
        return xor32(x);
    }
}

}  // namespace ullm
