// Shared helpers for the gfx950 attention kernels: element types, 16-byte
// vector loads, conversions and the error/status plumbing of the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>

#include "../../include/ullm_hip.h"

namespace ullm {

// Storage tags.  Caches hold raw 16-bit patterns; conversion is explicit so
// that bf16 and f16 never go through a compiler-chosen path.
struct F32 { using raw = float; static constexpr int bytes = 4; };
struct F16 { using raw = uint16_t; static constexpr int bytes = 2; };
struct BF16 { using raw = uint16_t; static constexpr int bytes = 2; };

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float f16_lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
}
__device__ __forceinline__ float f16_hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

// Round-to-nearest-even f32 -> bf16 bits (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Two f32 -> packed 16-bit pair (low = a), round-to-nearest-even in hardware
// (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 on gfx950).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, f16x2_t));
}

// Widen one 16-byte chunk (4 f32 or 8 half-precision values) to f32.
template <class T> struct Chunk;
template <> struct Chunk<F32> {
    static constexpr int n = 4;
    __device__ __forceinline__ static void widen(const u32x4 &r, float *o) {
        o[0] = __uint_as_float(r[0]); o[1] = __uint_as_float(r[1]);
        o[2] = __uint_as_float(r[2]); o[3] = __uint_as_float(r[3]);
    }
};
template <> struct Chunk<F16> {
    static constexpr int n = 8;
    __device__ __forceinline__ static void widen(const u32x4 &r, float *o) {
#pragma unroll
        for (int i = 0; i < 4; i++) { o[2 * i] = f16_lo(r[i]); o[2 * i + 1] = f16_hi(r[i]); }
    }
};
template <> struct Chunk<BF16> {
    static constexpr int n = 8;
    __device__ __forceinline__ static void widen(const u32x4 &r, float *o) {
#pragma unroll
        for (int i = 0; i < 4; i++) { o[2 * i] = bf16_lo(r[i]); o[2 * i + 1] = bf16_hi(r[i]); }
    }
};

__device__ __forceinline__ u32x4 ld16(const void *p) { return *(const u32x4 *)p; }
// Streaming load: the KV cache is read exactly once per decode call, so keep
// it from displacing reusable lines.
__device__ __forceinline__ u32x4 ld16_stream(const void *p) {
    return __builtin_nontemporal_load((const u32x4 *)p);
}

// Tuning override from the environment (0 when unset), read once when the
// library loads rather than on every call.
inline int env_override(const char *name) {
    const char *e = getenv(name);
    return e ? atoi(e) : 0;
}

// Host-side status plumbing -------------------------------------------------
int set_error(int code, const char *fmt, ...);
inline int check_hip(hipError_t e, const char *what) {
    if (e != hipSuccess) return set_error(ULLM_HIP_E_HIP, "%s: %s", what, hipGetErrorString(e));
    return ULLM_HIP_OK;
}
inline int dtype_bytes(int dt) { return dt == ULLM_DT_F32 ? 4 : 2; }
inline bool dtype_ok(int dt) { return dt == ULLM_DT_F32 || dt == ULLM_DT_F16 || dt == ULLM_DT_BF16; }

// Merge of split-KV partials (decode_mfma.hip): acc [units][splits][gt][D]
// and (m, l) [units][splits][gt][2] f32, units = batch * n_units.
void decode_merge_launch(int D, const float *ws_ml, const float *ws_acc, int splits, int gt,
                         int n_units, int batch, int n_head, float *out, hipStream_t st);
// MFMA decode path for f16/bf16 caches, and f32 caches on short splits
// (decode_mfma.hip).
size_t decode_mfma_plan_bytes(int batch, int n_head, int n_kv_head, int D, int max_len, int window);
size_t decode_mfma_workspace(int batch, int n_head, int n_kv_head, int D, int max_len, int window);
int decode_mfma(int dtype, const float *q, const void *kc, const void *vc, int64_t kvs,
                int64_t ss, const int32_t *lens, int max_len, int win, int batch, int nh, int nkv,
                int D, float qs, float *out, void *ws, size_t ws_bytes, hipStream_t st);
// Whether an f32-cache decode runs on the MFMA block kernel (decode_mfma
// with ULLM_DT_F32), and that plan's workspace bytes.
bool decode_f32_block_plan(int batch, int n_head, int n_kv_head, int D, int max_len, int window,
                           size_t *bytes);

// f32-cache split-KV decode over a paged cache (decode.hip).
size_t decode_f32_workspace(int batch, int n_head, int n_kv_head, int D, int max_len, int window);
int decode_f32_paged(const float *q, const void *kp, const void *vp, int64_t kvs,
                     const int32_t *tab, int tab_stride, int shift, int n_pages,
                     const int32_t *lens, int max_len, int win, int batch, int nh, int nkv, int D,
                     float qs, float *out, void *ws, size_t ws_bytes, hipStream_t st);

constexpr float kLog2e = 1.4426950408889634f;

}  // namespace ullm
