// Device helpers shared by the MFMA attention kernels: 16-bit packing, MFMA
// wrappers, buffer resources, LDS DMA and LDS reads that bypass the
// compiler's LDS-DMA alias tracking.
#pragma once
#include "common.hpp"

namespace ullm {

constexpr int kRsrcWord3 = 0x00020000;  // raw buffer resource word 3 (gfx9 data format)

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Pointer known to be wave-uniform, kept in SGPRs.
__device__ __forceinline__ void *uniform_ptr(const void *p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (void *)(((uint64_t)hi << 32) | lo);
}

// Compile-time loop: f(Int<0>{}) ... f(Int<N-1>{}).
template <int V>
struct Int { static constexpr int value = V; };
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(Int<I>{});
        static_for<I + 1, N>(f);
    }
}

// Compiler-only ordering point for wave-private LDS traffic.
__device__ __forceinline__ void lds_order() { asm volatile("" ::: "memory"); }

template <class T>
__device__ __forceinline__ f32x4 mfma16(const u32x4 &a, const u32x4 &b, const f32x4 &c) {
    if constexpr (__is_same(T, BF16))
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                      __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// Pair of f32 -> packed 16-bit pair of T (hardware RNE), and back.
template <class T>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (__is_same(T, BF16)) return pack_bf16x2(a, b);
    else return pack_f16x2(a, b);
}
template <class T>
__device__ __forceinline__ void unpack2(uint32_t w, float &a, float &b) {
    if constexpr (__is_same(T, BF16)) { a = bf16_lo(w); b = bf16_hi(w); }
    else { a = f16_lo(w); b = f16_hi(w); }
}
// x = hi + lo with hi, lo in T: ~2x the mantissa bits of T.
// Returns {hi, lo} packed pairs.
template <class T>
__device__ __forceinline__ u32x2 split2(float x0, float x1) {
    const uint32_t hi = pack2<T>(x0, x1);
    float h0, h1;
    unpack2<T>(hi, h0, h1);
    return u32x2{hi, pack2<T>(x0 - h0, x1 - h1)};
}

// s_waitcnt immediate that waits until at most n vector-memory operations
// are outstanding (gfx9 encoding: vmcnt[3:0] | vmcnt[5:4] << 14; expcnt and
// lgkmcnt left at their maxima).
constexpr int vm_wait(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }


typedef __attribute__((address_space(3))) void lds_void;

// LDS reads of DMA-filled tiles, issued as inline asm: the compiler would
// otherwise treat every LDS read as possibly aliasing in-flight LDS DMA and
// wait for all of it (vmcnt(0)), serialising the two-stage pipeline.  The
// caller waits with lds_wait() (tied to the destination registers) before use.
// One 16-byte-per-lane buffer load straight into LDS (lane i -> dst + 16 i),
// nontemporal.  Offsets past the resource's range read zero; the range check
// covers the per-lane offset, so callers put every variable part there and
// keep the scalar offset at 0.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, char *dst, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)dst, 16, voff, soff, 0, 2);
}
// Same load with the default cache policy, for operands that other
// workgroups re-read from L2 (GEMM tiles).
__device__ __forceinline__ void dma16_cached(__amdgpu_buffer_rsrc_t r, char *dst, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)dst, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)p;
}
__device__ __forceinline__ u32x4 lds_read_b128(uint32_t a) {
    u32x4 r;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(a));
    return r;
}
__device__ __forceinline__ void lds_write_b128(uint32_t a, const u32x4 &v) {
    asm volatile("ds_write_b128 %0, %1" ::"v"(a), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_write_b64(uint32_t a, const u32x2 &v) {
    asm volatile("ds_write_b64 %0, %1" ::"v"(a), "v"(v) : "memory");
}
__device__ __forceinline__ u32x2 lds_read_tr16_b64(uint32_t a) {
    u32x2 r;
    asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(a));
    return r;
}
// 16-byte-per-lane raw buffer load that the compiler does not track: it
// would otherwise make every later use wait for all vector-memory traffic
// issued after it (vmcnt retires in order, LDS DMA included).  The caller
// waits with an explicit vmcnt wait and ties the registers before use.  The
// resource is a raw descriptor {base lo, base hi, bytes, word3} in SGPRs.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 raw_rsrc(const void *base, int bytes) {
    const uint64_t v = (uint64_t)base;
    return i32x4{(int)__builtin_amdgcn_readfirstlane((uint32_t)v),
                 (int)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32) & 0xffff),
                 __builtin_amdgcn_readfirstlane(bytes), kRsrcWord3};
}
__device__ __forceinline__ u32x4 buffer_load_b128_untracked(const i32x4 &rsrc, int voff) {
    u32x4 v;
    asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=v"(v) : "v"(voff), "s"(rsrc) : "memory");
    return v;
}

// Same reads with a compile-time byte offset in the instruction's immediate
// field (0..65535), so per-lane addresses can be computed once.
template <int OFF>
__device__ __forceinline__ u32x4 lds_read_b128_at(uint32_t a) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset");
    u32x4 r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(OFF));
    return r;
}
template <int OFF>
__device__ __forceinline__ u32x2 lds_read_tr16_b64_at(uint32_t a) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset");
    u32x2 r;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(OFF));
    return r;
}
// Waits until at most N LDS reads of this wave are outstanding (they retire
// in order, so the earlier ones are complete).
template <int N>
__device__ __forceinline__ void lds_wait_n() {
    static_assert(N >= 0 && N < 16, "lgkmcnt");
    asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N) : "memory");
}
// max(x[l], x[l ^ 32]) across the wave halves, without an LDS round trip.
__device__ __forceinline__ float max_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
template <int N>
__device__ __forceinline__ void lds_wait(u32x4 (&r)[N]) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < N; i++) asm volatile("" : "+v"(r[i]));
}

}  // namespace ullm

namespace ullm {

template <class T>
__device__ __forceinline__ f32x16 mfma32(const u32x4 &a, const u32x4 &b, const f32x16 &c) {
    if constexpr (__is_same(T, BF16))
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                      __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// Waits for this wave's outstanding LDS reads and ties the results to the
// wait so the compiler cannot use them earlier.
__device__ __forceinline__ void lds_wait_any() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void tie(u32x4 &r) { asm volatile("" : "+v"(r)); }
__device__ __forceinline__ void tie_f(float &r) { asm volatile("" : "+v"(r)); }
// One 4-byte LDS read per lane, not tracked by the compiler (see the 16-byte
// reads above); the caller waits with lds_wait_any() and ties the result.
__device__ __forceinline__ uint32_t lds_read_b32(uint32_t a) {
    uint32_t r;
    asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(a));
    return r;
}
__device__ __forceinline__ void tie(u32x2 &r) { asm volatile("" : "+v"(r)); }

// Workgroup barrier without a memory fence (LDS DMA visibility is ensured by
// each wave's own vmcnt wait before it).
__device__ __forceinline__ void wg_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Paged K/V (tab == nullptr: the contiguous cache).  Key t of the sequence
// is row t % P of page tab[t / P] (P = 2^shift, a multiple of every prefill
// kernel's key tile), so a tile's DMA goes through a buffer resource based at its page
// whose range ends at the sequence length: rows past it, and pages outside
// the table or [0, n_pages), read as zeros.
struct KvPages {
    const int32_t *tab;
    int tab_len, shift, n_pages;
};

// Buffer resources and scalar offset of the key tile starting at key0 (a
// tile never crosses a page).  EB: bytes per cache element.
template <int D, int EB = 2>
__device__ __forceinline__ void page_tile(const KvPages &pg, const char *kc, const char *vc,
                                          int kvh, int rbg, int kv_len, int key0,
                                          __amdgpu_buffer_rsrc_t &kr, __amdgpu_buffer_rsrc_t &vr,
                                          int &so) {
    const int pi = key0 >> pg.shift;
    const int phys = key0 < kv_len && pi < pg.tab_len ? pg.tab[pi] : -1;
    const bool ok = phys >= 0 && phys < pg.n_pages;
    const int64_t pb = ((int64_t)(ok ? phys : 0) << pg.shift) * rbg + (int64_t)kvh * D * EB;
    const int rows = min(1 << pg.shift, kv_len - (pi << pg.shift));
    const int range = ok ? (rows - 1) * rbg + D * EB : 0;
    kr = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(kc + pb), 0, range, kRsrcWord3);
    vr = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(vc + pb), 0, range, kRsrcWord3);
    so = __builtin_amdgcn_readfirstlane((key0 & ((1 << pg.shift) - 1)) * rbg);
}

// Head_dim-256 prefill on 16-row waves, two per SIMD (prefill16.hip);
// pgs.tab == nullptr for a contiguous cache.
int launch_prefill16(int dtype, const void *q, const void *kc, const void *vc, int64_t kvs, int S,
                     int start_pos, int window, int n_head, int kv_mul, float qs, float *out,
                     hipStream_t st, KvPages pgs);
int launch_prefill16_128(int dtype, const void *q, const void *kc, const void *vc, int64_t kvs,
                         int S, int start_pos, int window, int n_head, int kv_mul, float qs,
                         float *out, hipStream_t st, KvPages pgs);

}  // namespace ullm
