// Fused Q/K/V preparation + KV-cache append, and the host RoPE table.
//
// One wave owns one head vector of one token row:
//   slots [0, n_head)                 -> a query head
//   slots [n_head, n_head+n_kv_head)  -> a key head
//   slots [.., n_head+2*n_kv_head)    -> a value head
// and applies, in the reference's order (crates/ullm-model/src/lib.rs:
// 1027-1058, decode :877-914): bias add, per-head RMSNorm (math.rs:82-86),
// RoPE (math.rs:116-161) via the precomputed (cos, sin) table, then the
// store -- q to q_out, K/V straight into the cache slot of position
// start_pos + row.  This replaces the bias, rmsnorm_heads and rope_* Metal
// dispatches (forward.rs:416-447, :799-853; shader.metal:828-941) with one
// launch.
#include <cmath>
#include "common.hpp"
#include "wave.hpp"

namespace ullm {

template <int OUT_DT>
__device__ __forceinline__ void store_elem(void *base, int64_t idx, float v) {
    if constexpr (OUT_DT == ULLM_DT_F32) ((float *)base)[idx] = v;
    else if constexpr (OUT_DT == ULLM_DT_F16) ((uint16_t *)base)[idx] = f32_to_f16_bits(v);
    else ((uint16_t *)base)[idx] = f32_to_bf16_bits(v);
}

constexpr int kAppendWaves = 4;

template <int D, int QDT, int KVDT>
__global__ __launch_bounds__(kAppendWaves * 64) void qkv_append_kernel(
    const float *__restrict__ q_in, const float *__restrict__ k_in, const float *__restrict__ v_in,
    const float *__restrict__ q_bias, const float *__restrict__ k_bias,
    const float *__restrict__ v_bias, const float *__restrict__ q_norm,
    const float *__restrict__ k_norm, float eps, const float *__restrict__ cs, int neox,
    int rotary_dim, int rows, int start_pos, int n_head, int n_kv_head, void *q_out,
    void *k_cache, void *v_cache, int64_t kv_stride) {
    constexpr int NE = D / 64;
    __shared__ float buf[kAppendWaves][D];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int slots = n_head + 2 * n_kv_head;
    const int64_t gslot = (int64_t)blockIdx.x * kAppendWaves + wave;
    const bool active = gslot < (int64_t)rows * slots;
    const int row = active ? (int)(gslot / slots) : 0;
    const int slot = active ? (int)(gslot % slots) : 0;
    const int kind = slot < n_head ? 0 : (slot < n_head + n_kv_head ? 1 : 2);
    const int head = kind == 0 ? slot : (kind == 1 ? slot - n_head : slot - n_head - n_kv_head);
    const int64_t q_dim = (int64_t)n_head * D, kv_dim = (int64_t)n_kv_head * D;
    const float *src = kind == 0 ? q_in + row * q_dim : (kind == 1 ? k_in : v_in) + row * kv_dim;
    src += (int64_t)head * D;
    const float *bias = kind == 0 ? q_bias : (kind == 1 ? k_bias : v_bias);
    const float *nw = kind == 0 ? q_norm : (kind == 1 ? k_norm : nullptr);

    float x[NE];
#pragma unroll
    for (int i = 0; i < NE; i++) {
        const int e = lane + 64 * i;
        x[i] = active ? src[e] : 0.f;
        if (bias) x[i] += bias[(int64_t)head * D + e];
    }
    if (nw) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < NE; i++) ss += x[i] * x[i];
        ss = group_sum<64>(ss);
        const float inv = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
        for (int i = 0; i < NE; i++) x[i] = x[i] * inv * nw[lane + 64 * i];
    }
    const int pos = start_pos + row;
    // RoPE needs the partner element of each pair: exchange through LDS.
#pragma unroll
    for (int i = 0; i < NE; i++) buf[wave][lane + 64 * i] = x[i];
    __syncthreads();
    if (kind != 2) {
        const int half = rotary_dim / 2;
        const float *cp = cs + (int64_t)pos * half * 2;
#pragma unroll
        for (int i = 0; i < NE; i++) {
            const int e = lane + 64 * i;
            if (neox) {
                if (e < rotary_dim) {
                    const int j = e < half ? e : e - half;
                    const float c = cp[2 * j], s = cp[2 * j + 1];
                    const float a = buf[wave][j], b = buf[wave][j + half];
                    x[i] = e < half ? a * c - b * s : a * s + b * c;
                }
            } else if (e < rotary_dim) {
                const int j = e >> 1;
                const float c = cp[2 * j], s = cp[2 * j + 1];
                const float a = buf[wave][e & ~1], b = buf[wave][e | 1];
                x[i] = (e & 1) ? a * s + b * c : a * c - b * s;
            }
        }
    }
    if (!active) return;
#pragma unroll
    for (int i = 0; i < NE; i++) {
        const int e = lane + 64 * i;
        if (kind == 0) store_elem<QDT>(q_out, row * q_dim + (int64_t)head * D + e, x[i]);
        else store_elem<KVDT>(kind == 1 ? k_cache : v_cache,
                              (int64_t)pos * kv_stride + (int64_t)head * D + e, x[i]);
    }
}

template <int D, int QDT>
static void launch_kv(int kvdt, dim3 g, dim3 b, hipStream_t st, const float *qi, const float *ki,
                      const float *vi, const float *qb, const float *kb, const float *vb,
                      const float *qn, const float *kn, float eps, const float *cs, int neox,
                      int rd, int rows, int sp, int nh, int nkv, void *qo, void *kc, void *vc,
                      int64_t kvs) {
    if (kvdt == ULLM_DT_F32)
        hipLaunchKernelGGL((qkv_append_kernel<D, QDT, ULLM_DT_F32>), g, b, 0, st, qi, ki, vi, qb, kb, vb, qn, kn, eps, cs, neox, rd, rows, sp, nh, nkv, qo, kc, vc, kvs);
    else if (kvdt == ULLM_DT_F16)
        hipLaunchKernelGGL((qkv_append_kernel<D, QDT, ULLM_DT_F16>), g, b, 0, st, qi, ki, vi, qb, kb, vb, qn, kn, eps, cs, neox, rd, rows, sp, nh, nkv, qo, kc, vc, kvs);
    else
        hipLaunchKernelGGL((qkv_append_kernel<D, QDT, ULLM_DT_BF16>), g, b, 0, st, qi, ki, vi, qb, kb, vb, qn, kn, eps, cs, neox, rd, rows, sp, nh, nkv, qo, kc, vc, kvs);
}

template <int D>
static void launch_q(int qdt, int kvdt, dim3 g, dim3 b, hipStream_t st, const float *qi,
                     const float *ki, const float *vi, const float *qb, const float *kb,
                     const float *vb, const float *qn, const float *kn, float eps,
                     const float *cs, int neox, int rd, int rows, int sp, int nh, int nkv,
                     void *qo, void *kc, void *vc, int64_t kvs) {
    if (qdt == ULLM_DT_F32) launch_kv<D, ULLM_DT_F32>(kvdt, g, b, st, qi, ki, vi, qb, kb, vb, qn, kn, eps, cs, neox, rd, rows, sp, nh, nkv, qo, kc, vc, kvs);
    else if (qdt == ULLM_DT_F16) launch_kv<D, ULLM_DT_F16>(kvdt, g, b, st, qi, ki, vi, qb, kb, vb, qn, kn, eps, cs, neox, rd, rows, sp, nh, nkv, qo, kc, vc, kvs);
    else launch_kv<D, ULLM_DT_BF16>(kvdt, g, b, st, qi, ki, vi, qb, kb, vb, qn, kn, eps, cs, neox, rd, rows, sp, nh, nkv, qo, kc, vc, kvs);
}

}  // namespace ullm

using namespace ullm;

// Host RoPE table with the reference's f32 formula (math.rs:118-121, :150-154).
// Kept out of any FMA contraction: every step is a single rounding, as in Rust.
#pragma clang fp contract(off)
extern "C" int ullm_hip_rope_table(float *cs, int n_pos, int rotary_dim, float theta) {
    if (!cs || n_pos < 1 || rotary_dim < 2 || (rotary_dim & 1))
        return set_error(ULLM_HIP_E_INVALID, "rope_table: bad n_pos=%d rotary_dim=%d", n_pos,
                         rotary_dim);
    const int half = rotary_dim / 2;
    for (int j = 0; j < half; j++) {
        volatile float expo = 2.0f * (float)j / (float)rotary_dim;
        const float freq = 1.0f / powf(theta, expo);
        for (int p = 0; p < n_pos; p++) {
            volatile float ang = (float)p * freq;
            const float s = sinf(ang);
            const float c = cosf(ang);
            cs[((size_t)p * half + j) * 2] = c;
            cs[((size_t)p * half + j) * 2 + 1] = s;
        }
    }
    return ULLM_HIP_OK;
}

extern "C" int ullm_hip_qkv_append(const float *q_in, const float *k_in, const float *v_in,
                                   const float *q_bias, const float *k_bias, const float *v_bias,
                                   const float *q_norm, const float *k_norm, float eps,
                                   const float *rope_cs, int rope_n_pos, int rope_neox,
                                   int rotary_dim, int rows, int start_pos, int n_head,
                                   int n_kv_head, int head_dim, void *q_out, int q_dtype,
                                   void *k_cache, void *v_cache, int kv_dtype, int64_t kv_stride,
                                   void *stream) {
    if (!dtype_ok(q_dtype) || !dtype_ok(kv_dtype))
        return set_error(ULLM_HIP_E_UNSUPPORTED, "qkv_append: dtype q=%d kv=%d", q_dtype, kv_dtype);
    if (head_dim != 64 && head_dim != 128 && head_dim != 256)
        return set_error(ULLM_HIP_E_UNSUPPORTED, "qkv_append: head_dim %d not in {64,128,256}",
                         head_dim);
    if (rows < 0 || start_pos < 0 || n_head < 1 || n_kv_head < 1 || n_head % n_kv_head)
        return set_error(ULLM_HIP_E_INVALID, "qkv_append: bad rows/heads");
    if (rotary_dim < 2 || rotary_dim > head_dim || (rotary_dim & 1))
        return set_error(ULLM_HIP_E_INVALID, "qkv_append: rotary_dim %d", rotary_dim);
    if (kv_stride < (int64_t)n_kv_head * head_dim)
        return set_error(ULLM_HIP_E_INVALID, "qkv_append: kv_stride too small");
    if (rows == 0) return ULLM_HIP_OK;
    if (!q_in || !k_in || !v_in || !rope_cs || !q_out || !k_cache || !v_cache)
        return set_error(ULLM_HIP_E_INVALID, "qkv_append: null tensor pointer");
    if (rope_n_pos < start_pos + rows)
        return set_error(ULLM_HIP_E_INVALID, "qkv_append: rope table has %d positions, need %d",
                         rope_n_pos, start_pos + rows);
    if (q_out == (void *)q_in && q_dtype != ULLM_DT_F32)
        return set_error(ULLM_HIP_E_INVALID, "qkv_append: in-place q needs q_dtype f32");
    const int64_t waves = (int64_t)rows * (n_head + 2 * n_kv_head);
    dim3 grid((unsigned)((waves + kAppendWaves - 1) / kAppendWaves)), block(kAppendWaves * 64);
    hipStream_t st = (hipStream_t)stream;
    switch (head_dim) {
        case 64: launch_q<64>(q_dtype, kv_dtype, grid, block, st, q_in, k_in, v_in, q_bias, k_bias, v_bias, q_norm, k_norm, eps, rope_cs, rope_neox, rotary_dim, rows, start_pos, n_head, n_kv_head, q_out, k_cache, v_cache, kv_stride); break;
        case 128: launch_q<128>(q_dtype, kv_dtype, grid, block, st, q_in, k_in, v_in, q_bias, k_bias, v_bias, q_norm, k_norm, eps, rope_cs, rope_neox, rotary_dim, rows, start_pos, n_head, n_kv_head, q_out, k_cache, v_cache, kv_stride); break;
        default: launch_q<256>(q_dtype, kv_dtype, grid, block, st, q_in, k_in, v_in, q_bias, k_bias, v_bias, q_norm, k_norm, eps, rope_cs, rope_neox, rotary_dim, rows, start_pos, n_head, n_kv_head, q_out, k_cache, v_cache, kv_stride); break;
    }
    return check_hip(hipGetLastError(), "qkv_append launch");
}
