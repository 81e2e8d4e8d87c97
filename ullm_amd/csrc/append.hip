// Fused Q/K/V preparation + KV-cache append, and the host RoPE table.
//
// qkv_append_kernel: a workgroup of kAppendWaves waves owns one token row.
// Each head vector gets, in the reference's order
// (crates/ullm-model/src/lib.rs:1027-1058, decode :877-914): bias add,
// per-head RMSNorm (math.rs:82-86), RoPE (math.rs:116-161) via the
// precomputed (cos, sin) table, then the store -- q to q_out, K/V straight
// into the cache slot of position start_pos + row.  The kernel streams
// ~4 x D x 4 bytes per head; its VALU work per element is what limits it
// once the loads are in flight, so a lane holds the two halves of a RoPE
// pair (SplitEpi) and one RMS reduction serves 256/D heads.
// This replaces the bias, rmsnorm_heads and rope_* Metal dispatches
// (forward.rs:416-447, :799-853; shader.metal:828-941) with one launch.
#include <cmath>
#include "common.hpp"
#include "mfma_util.hpp"
#include "wave.hpp"
// The split projection's cross-workgroup exchange (qkv_proj_kernel) relies
// on gfx950's cache policy for system-scope stores and on its L2 topology;
// this library is built for gfx950 only.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "append.hip: the split projection exchange is written for gfx950"
#endif


namespace ullm {

template <int N>
struct VecF;
template <> struct VecF<1> { typedef float t; };
template <> struct VecF<2> { typedef float2 t; };
template <> struct VecF<4> { typedef float4 t; };

template <int E>
__device__ __forceinline__ void load_e(const float *p, float (&x)[E]) {
    if constexpr (E == 1) x[0] = p[0];
    else if constexpr (E == 2) { const float2 v = *(const float2 *)p; x[0] = v.x; x[1] = v.y; }
    else { const float4 v = *(const float4 *)p; x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w; }
}

// Store E consecutive elements converted to OUT_DT.
template <int OUT_DT, int E>
__device__ __forceinline__ void store_e(void *base, int64_t idx, const float (&x)[E]) {
    if constexpr (OUT_DT == ULLM_DT_F32) {
        float *p = (float *)base + idx;
        if constexpr (E == 1) p[0] = x[0];
        else if constexpr (E == 2) *(float2 *)p = float2{x[0], x[1]};
        else *(float4 *)p = float4{x[0], x[1], x[2], x[3]};
    } else {
        // hardware round-to-nearest-even packs
        auto pk = [](float a, float b) {
            return OUT_DT == ULLM_DT_F16 ? pack_f16x2(a, b) : pack_bf16x2(a, b);
        };
        uint16_t *p = (uint16_t *)base + idx;
        if constexpr (E == 1) p[0] = (uint16_t)pk(x[0], 0.f);
        else if constexpr (E == 2) *(uint32_t *)p = pk(x[0], x[1]);
        else *(uint2 *)p = uint2{pk(x[0], x[1]), pk(x[2], x[3])};
    }
}

constexpr int kAppendWaves = 4;
constexpr int kBatch = 3;  // groups per wave with loads in flight together
constexpr int kAppendSplitBelow = 256;  // rows under which a row's groups spread over workgroups

// Per-lane state of the head epilogue of one token row: the (cos, sin) of
// this lane's elements at the row's position and the Q/K norm weights.  A
// lane holds E = D/64 consecutive elements of a head vector.
template <int D>
struct HeadEpi {
    static constexpr int E = D / 64;
    int lane, e0, rotary_dim, half, neox;
    float eps;
    float rc[E], rs[E], wq[E], wk[E];
    const float *q_norm, *k_norm;

    __device__ __forceinline__ HeadEpi(const float *cs, int pos, int rotary_dim_, int neox_,
                                       const float *qn, const float *kn, float eps_)
        : lane((int)(threadIdx.x & 63)), e0((int)(threadIdx.x & 63) * E), rotary_dim(rotary_dim_),
          half(rotary_dim_ / 2), neox(neox_), eps(eps_), q_norm(qn), k_norm(kn) {
        const float *cp = cs + (int64_t)pos * half * 2;
#pragma unroll
        for (int i = 0; i < E; i++) {
            const int e = e0 + i;
            const int j = e < rotary_dim ? (neox ? (e < half ? e : e - half) : e >> 1) : 0;
            rc[i] = cp[2 * j];
            rs[i] = cp[2 * j + 1];
            wq[i] = 1.f;
            wk[i] = 1.f;
        }
        if (q_norm) load_e<E>(q_norm + e0, wq);
        if (k_norm) load_e<E>(k_norm + e0, wk);
    }

    // Bias (already added by the caller), per-head RMSNorm (math.rs:82-86)
    // and RoPE (math.rs:116-161) of one head vector of kind 0 (q), 1 (k) or
    // 2 (v), in the reference's order.  lds_row: D floats private to the
    // wave, used only for partial-rotary pairs.
    __device__ __forceinline__ void norm_rope(float (&x)[E], int kind, float *lds_row) const {
        const float *nw = kind == 0 ? q_norm : (kind == 1 ? k_norm : nullptr);
        if (nw) {
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < E; i++) ss += x[i] * x[i];
            ss = wave_sum(ss);
            // v_rsq_f32 (~1 ulp) for (sum/n + eps).sqrt().recip()
            const float inv = __builtin_amdgcn_rsqf(ss / (float)D + eps);
#pragma unroll
            for (int i = 0; i < E; i++) x[i] = x[i] * inv * (kind == 0 ? wq[i] : wk[i]);
        }
        if (kind == 2) return;
        float y[E];
        if (rotary_dim == D) {
            // Full-width RoPE: a NeoX partner (e +- D/2) sits in lane l ^ 32 at
            // the same element index; an interleaved partner (e ^ 1) in the same
            // lane, or in lane l ^ 1 when a lane holds one element.
#pragma unroll
            for (int i = 0; i < E; i++) {
                float pa;
                if (neox) pa = xor32(x[i]);
                else if constexpr (E == 1) pa = dpp<kDppXor1>(x[i]);
                else pa = x[i ^ 1];
                const bool lo = neox ? lane < 32 : ((e0 + i) & 1) == 0;
                // lo: a*c - b*s with a = own, b = partner; hi: a*s + b*c with a = partner
                y[i] = lo ? x[i] * rc[i] - pa * rs[i] : pa * rs[i] + x[i] * rc[i];
            }
        } else {
            // Partial rotary: the partner of each pair comes from the wave's
            // LDS row (LDS operations of one wave complete in order).
#pragma unroll
            for (int i = 0; i < E; i++) lds_row[e0 + i] = x[i];
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int i = 0; i < E; i++) {
                const int e = e0 + i;
                y[i] = x[i];
                if (e < rotary_dim) {
                    if (neox) {
                        const int j = e < half ? e : e - half;
                        const float a = lds_row[j], c = lds_row[j + half];
                        y[i] = e < half ? a * rc[i] - c * rs[i] : a * rs[i] + c * rc[i];
                    } else {
                        const float a = lds_row[e & ~1], c = lds_row[e | 1];
                        y[i] = (e & 1) ? a * rs[i] + c * rc[i] : a * rc[i] - c * rs[i];
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();  // the row may be rewritten next
        }
#pragma unroll
        for (int i = 0; i < E; i++) x[i] = y[i];
    }
};

// Store one finished head vector: q to q_out (row-major [rows][n_head*D]),
// k / v into cache row crow (the position, or its paged slot).
template <int D, int QDT, int KVDT>
__device__ __forceinline__ void store_head(const float (&x)[D / 64], int kind, int head, int row,
                                           int64_t crow, int e0, int64_t q_dim, void *q_out,
                                           void *k_cache, void *v_cache, int64_t kv_stride) {
    constexpr int E = D / 64;
    if (kind == 0)
        store_e<QDT, E>(q_out, row * q_dim + (int64_t)head * D + e0, x);
    else
        store_e<KVDT, E>(kind == 1 ? k_cache : v_cache,
                         crow * kv_stride + (int64_t)head * D + e0, x);
}

// Paged destination of the K/V rows (pos == nullptr: the contiguous cache,
// row r at position start_pos + r).  Row r of a paged call is one token of
// sequence r at position pos[r], stored in slot pos % P of page
// tab[r * stride + pos / P] (P = 2^shift); a row whose position falls
// outside [0, rope_n_pos) or whose page index is outside the table or the
// pool is skipped (nothing written).
struct PageMap {
    const int32_t *pos, *tab;
    int stride, shift, n_pages, rope_n_pos;
};

// Head epilogue of qkv_append_kernel in its split-half lane layout: a head
// vector of D elements is held by L = D/4 lanes, lane m of the head holding
// elements {2m, 2m+1} (x[0], x[1]) and {D/2+2m, D/2+2m+1} (x[2], x[3]), so a
// wave holds HPW = 256/D heads.  Both full-width RoPE pairings are then
// inside the lane: NeoX pairs e with e + D/2 (x[0]/x[2], x[1]/x[3]),
// interleaved pairs 2j with 2j+1 (x[0]/x[1], x[2]/x[3]); only partial rotary
// goes through LDS.  The RMS sum is a group_sum over the head's L lanes, one
// reduction for HPW heads.
template <int D>
struct SplitEpi {
    static constexpr int L = D / 4, HPW = 64 / L;
    int m, rotary_dim, half, neox;
    float eps;
    float rc[4], rs[4], wq[4], wk[4];
    const float *q_norm, *k_norm;

    // Element index of x[i] of lane m.
    __device__ __forceinline__ static int elem(int m, int i) { return (i >> 1) * (D / 2) + 2 * m + (i & 1); }

    __device__ __forceinline__ SplitEpi(const float *cs, int pos, int rotary_dim_, int neox_,
                                        const float *qn, const float *kn, float eps_)
        : m((int)(threadIdx.x & 63) % L), rotary_dim(rotary_dim_), half(rotary_dim_ / 2),
          neox(neox_), eps(eps_), q_norm(qn), k_norm(kn) {
        const float *cp = cs + (int64_t)pos * half * 2;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int e = elem(m, i);
            const int j = e < rotary_dim ? (neox ? (e < half ? e : e - half) : e >> 1) : 0;
            rc[i] = cp[2 * j];
            rs[i] = cp[2 * j + 1];
            wq[i] = q_norm ? q_norm[e] : 1.f;
            wk[i] = k_norm ? k_norm[e] : 1.f;
        }
    }

    // Per-head RMSNorm (math.rs:82-86) and RoPE (math.rs:116-161) of one head
    // vector of KIND 0 (q) or 1 (k), in the reference's order, the bias
    // already added.  lds_head: D floats private to this head of the wave,
    // used only for partial-rotary pairs.
    template <int KIND>
    __device__ __forceinline__ void norm_rope(float (&x)[4], float *lds_head) const {
        if (KIND == 0 ? q_norm != nullptr : k_norm != nullptr) {
            float ss = x[0] * x[0];
#pragma unroll
            for (int i = 1; i < 4; i++) ss += x[i] * x[i];
            ss = group_sum<L>(ss);
            // v_rsq_f32 (~1 ulp) for (sum/n + eps).sqrt().recip()
            const float inv = __builtin_amdgcn_rsqf(ss / (float)D + eps);
#pragma unroll
            for (int i = 0; i < 4; i++) x[i] = x[i] * inv * (KIND == 0 ? wq[i] : wk[i]);
        }
        float y[4];
        if (rotary_dim == D) {
            // (a, b) a pair, a the lower element: a' = a*c - b*s, b' = a*s + b*c
            // with (c, s) of the pair (equal in both lanes of the pair's table).
            auto pair = [&](int a, int b) {
                y[a] = x[a] * rc[a] - x[b] * rs[a];
                y[b] = x[a] * rs[b] + x[b] * rc[b];
            };
            if (neox) {  // wave-uniform
                pair(0, 2);
                pair(1, 3);
            } else {
                pair(0, 1);
                pair(2, 3);
            }
        } else {
            // Partial rotary: the partner of each pair comes from LDS (LDS
            // operations of one wave complete in order).
#pragma unroll
            for (int i = 0; i < 4; i++) lds_head[elem(m, i)] = x[i];
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int e = elem(m, i);
                y[i] = x[i];
                if (e < rotary_dim) {
                    if (neox) {
                        const int j = e < half ? e : e - half;
                        const float a = lds_head[j], c = lds_head[j + half];
                        y[i] = e < half ? a * rc[i] - c * rs[i] : a * rs[i] + c * rc[i];
                    } else {
                        const float a = lds_head[e & ~1], c = lds_head[e | 1];
                        y[i] = (e & 1) ? a * rs[i] + c * rc[i] : a * rc[i] - c * rs[i];
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();  // the row may be rewritten next
        }
#pragma unroll
        for (int i = 0; i < 4; i++) x[i] = y[i];
    }
};

// Token row blockIdx.x; the row's head vectors are taken in groups of HPW
// heads of one kind (q heads, then K heads, then V heads; a kind's last group
// may be partly empty), groups [blockIdx.y * gpw, +gpw) by this workgroup,
// group g by wave g % kAppendWaves, kBatch groups at a time with every load
// of a batch issued before any is used.
template <int D, int QDT, int KVDT>
__global__ __launch_bounds__(kAppendWaves * 64) void qkv_append_kernel(
    const float *__restrict__ q_in, const float *__restrict__ k_in, const float *__restrict__ v_in,
    const float *__restrict__ q_bias, const float *__restrict__ k_bias,
    const float *__restrict__ v_bias, const float *__restrict__ q_norm,
    const float *__restrict__ k_norm, float eps, const float *__restrict__ cs, int neox,
    int rotary_dim, int rows, int start_pos, int n_head, int n_kv_head, void *q_out,
    void *k_cache, void *v_cache, int64_t kv_stride, PageMap pm, int gpw) {
    using Epi = SplitEpi<D>;
    constexpr int L = Epi::L, HPW = Epi::HPW;
    __shared__ float buf[kAppendWaves][HPW * D];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: group math in SGPRs
    const int hl = (int)(threadIdx.x & 63) / L;                          // head of the lane within a group
    const int row = blockIdx.x;
    const int gq = (n_head + HPW - 1) / HPW, gk = (n_kv_head + HPW - 1) / HPW;
    const int groups = gq + 2 * gk;
    const int64_t q_dim = (int64_t)n_head * D, kv_dim = (int64_t)n_kv_head * D;
    int pos = start_pos + row;
    int64_t crow = pos;
    if (pm.pos) {  // wave-uniform
        pos = __builtin_amdgcn_readfirstlane(pm.pos[row]);
        const int pg = pos >> pm.shift;
        const bool in = pos >= 0 && pos < pm.rope_n_pos && pg < pm.stride;
        const int phys = in ? __builtin_amdgcn_readfirstlane(pm.tab[(int64_t)row * pm.stride + pg]) : -1;
        if (phys < 0 || phys >= pm.n_pages) return;
        crow = ((int64_t)phys << pm.shift) + (pos & ((1 << pm.shift) - 1));
    }
    const Epi epi(cs, pos, rotary_dim, neox, q_norm, k_norm, eps);
    const int c0 = 2 * epi.m, c1 = D / 2 + 2 * epi.m;  // element offsets of x[0..1], x[2..3]
    const unsigned loff = (unsigned)(hl * D + c0);      // of x[0..1] from the group's first head
    const bool has_bias = q_bias || k_bias || v_bias;

    // This workgroup's groups: [gbeg, gend) of the row (gpw per workgroup
    // along blockIdx.y; all of them when gridDim.y == 1).
    const int gbeg = (int)blockIdx.y * gpw, gend = min(groups, gbeg + gpw);
    for (int g0 = gbeg + wave; g0 < gend; g0 += kAppendWaves * kBatch) {
        float x[kBatch][4], bv[kBatch][4];
        int kind[kBatch], head[kBatch];
        bool ok[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; b++) {
            const int g = g0 + b * kAppendWaves;
            kind[b] = g >= gend ? 3 : (g < gq ? 0 : (g < gq + gk ? 1 : 2));  // wave-uniform
            const int first = kind[b] == 0 ? 0 : (kind[b] == 1 ? gq : gq + gk);
            const int h0 = (g - first) * HPW;  // wave-uniform first head of the group
            head[b] = h0 + hl;
            ok[b] = kind[b] != 3 && head[b] < (kind[b] == 0 ? n_head : n_kv_head);
            // uniform base + a 32-bit lane offset; a lane past the kind's last
            // head re-reads head h0 (in bounds) and stores nothing
            const float *src = (kind[b] == 0 ? q_in + row * q_dim : (kind[b] == 1 ? k_in : v_in) + row * kv_dim) + (int64_t)h0 * D;
            const float *bias = kind[b] == 0 ? q_bias : (kind[b] == 1 ? k_bias : v_bias);
            const unsigned lo = ok[b] ? loff : (unsigned)c0;
            float2 a{0.f, 0.f}, c{0.f, 0.f}, ba{0.f, 0.f}, bc{0.f, 0.f};
            if (kind[b] != 3) {
                a = *(const float2 *)(src + lo);
                c = *(const float2 *)(src + lo + D / 2);
                if (bias) {
                    ba = *(const float2 *)(bias + (int64_t)h0 * D + lo);
                    bc = *(const float2 *)(bias + (int64_t)h0 * D + lo + D / 2);
                }
            }
            x[b][0] = a.x, x[b][1] = a.y, x[b][2] = c.x, x[b][3] = c.y;
            bv[b][0] = ba.x, bv[b][1] = ba.y, bv[b][2] = bc.x, bv[b][3] = bc.y;
        }
#pragma unroll
        for (int b = 0; b < kBatch; b++) {
            if (kind[b] == 3) continue;  // wave-uniform
            if (has_bias)
#pragma unroll
                for (int i = 0; i < 4; i++) x[b][i] += bv[b][i];
            if (kind[b] == 0) epi.template norm_rope<0>(x[b], &buf[wave][hl * D]);
            else if (kind[b] == 1) epi.template norm_rope<1>(x[b], &buf[wave][hl * D]);
            if (!ok[b]) continue;
            const float lo[2] = {x[b][0], x[b][1]}, hi[2] = {x[b][2], x[b][3]};
            const int h0 = head[b] - hl;  // wave-uniform
            if (kind[b] == 0) {
                void *dst = (char *)q_out + (row * q_dim + (int64_t)h0 * D) * (QDT == ULLM_DT_F32 ? 4 : 2);
                store_e<QDT, 2>(dst, loff, lo);
                store_e<QDT, 2>(dst, loff + D / 2, hi);
            } else {
                void *dst = (char *)(kind[b] == 1 ? k_cache : v_cache) +
                            (crow * kv_stride + (int64_t)h0 * D) * (KVDT == ULLM_DT_F32 ? 4 : 2);
                store_e<KVDT, 2>(dst, loff, lo);
                store_e<KVDT, 2>(dst, loff + D / 2, hi);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Decode-side Q/K/V projection with the append fused into its epilogue
// (crates/ullm-model/src/lib.rs:857-914; the Metal forward's wq/wk/wv
// matvecs into q and the cache slot, bias, q/k norm and RoPE,
// forward.rs:415-447): y = W x per head vector, W row-major [out][in_dim] in
// f32, f16 or bf16 (math.rs:9-21 matvec_q: dequantised row times x, f32
// sums), then the head epilogue HeadEpi (bias, norm, RoPE, store).
//
// A workgroup owns one head vector (slot) of one token row, or 1/NSP of its
// rows in split mode: its proj_waves(NSP) waves each compute RPW rows of W,
// every lane accumulating 16-byte chunks of a row in f32 with x's matching
// chunk (loaded once per chunk for all of the wave's rows), then a wave sum
// per row.  The results meet in LDS and wave 0 finishes the head.  The
// kernel streams W once (HBM-bound); a CU pulls the D x in_dim slice of one
// head (a quarter of it in split mode).  Split mode runs 8 waves of D/32 rows
// (x re-read by half as many waves: 10.8 against 11.1 us at the Qwen3-4B
// decode shape); whole heads 16 waves of D/16 rows (the rows' loads in
// flight stay within the register file at head_dim 256).
constexpr int proj_waves(int nsp) { return nsp > 1 ? 8 : 16; }

template <int WDT>
struct WVec;
template <> struct WVec<ULLM_DT_F32> { static constexpr int n = 4; };
template <> struct WVec<ULLM_DT_F16> { static constexpr int n = 8; };
template <> struct WVec<ULLM_DT_BF16> { static constexpr int n = 8; };

// Widen one 16-byte chunk of W to f32.
template <int WDT>
__device__ __forceinline__ void widen_w(const u32x4 &r, float *o) {
    if constexpr (WDT == ULLM_DT_F32) {
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] = __uint_as_float(r[i]);
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if constexpr (WDT == ULLM_DT_BF16) { o[2 * i] = bf16_lo(r[i]); o[2 * i + 1] = bf16_hi(r[i]); }
            else { o[2 * i] = f16_lo(r[i]); o[2 * i + 1] = f16_hi(r[i]); }
        }
    }
}

template <int D, int WDT, int QDT, int KVDT, int NSP>
__global__ __launch_bounds__(proj_waves(NSP) * 64) void qkv_proj_kernel(
    const float *__restrict__ x, int in_dim, const char *__restrict__ wq,
    const char *__restrict__ wk, const char *__restrict__ wv, const float *__restrict__ q_bias,
    const float *__restrict__ k_bias, const float *__restrict__ v_bias,
    const float *__restrict__ q_norm, const float *__restrict__ k_norm, float eps,
    const float *__restrict__ cs, int neox, int rotary_dim, int start_pos, int n_head,
    int n_kv_head, void *q_out, void *k_cache, void *v_cache, int64_t kv_stride,
    float *__restrict__ ws_y, uint32_t *__restrict__ ws_cnt) {
    constexpr int E = D / 64, RPW = D / proj_waves(NSP) / NSP, VEC = WVec<WDT>::n;
    constexpr int WB = WDT == ULLM_DT_F32 ? 4 : 2;  // bytes per weight
    static_assert(RPW >= 1, "rows per wave");
    __shared__ float ys[D];
    __shared__ float lrow[D];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slot = blockIdx.x / NSP, part = blockIdx.x % NSP, row = blockIdx.y;
    const int slots = n_head + 2 * n_kv_head;
    const int kind = slot < n_head ? 0 : (slot < n_head + n_kv_head ? 1 : 2);
    const int head = kind == 0 ? slot : (kind == 1 ? slot - n_head : slot - n_head - n_kv_head);
    const int r0 = part * (D / NSP) + wave * RPW;  // first W row of this wave in the head
    const char *w = (kind == 0 ? wq : (kind == 1 ? wk : wv)) +
                    ((int64_t)head * D + r0) * in_dim * WB;
    const float *xr = x + (int64_t)row * in_dim;

    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) acc[r] = 0.f;
    // Software pipeline over 16-byte chunks of the rows: chunk i+1's loads
    // are in flight while chunk i is multiplied (chunks past in_dim read 0).
    auto load = [&](int c, u32x4 (&wr)[RPW], float (&xv)[VEC]) {
        const bool ok = c < in_dim;
#pragma unroll
        for (int r = 0; r < RPW; r++)
            wr[r] = ok ? *(const u32x4 *)(w + ((int64_t)r * in_dim + c) * WB) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int h = 0; h < VEC / 4; h++) {
            const float4 t = ok ? *(const float4 *)(xr + c + 4 * h) : float4{0.f, 0.f, 0.f, 0.f};
            xv[4 * h] = t.x; xv[4 * h + 1] = t.y; xv[4 * h + 2] = t.z; xv[4 * h + 3] = t.w;
        }
    };
    auto mac = [&](const u32x4 (&wr)[RPW], const float (&xv)[VEC]) {
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            float wf[VEC];
            widen_w<WDT>(wr[r], wf);
#pragma unroll
            for (int i = 0; i < VEC; i++) acc[r] = __builtin_fmaf(wf[i], xv[i], acc[r]);
        }
    };
    constexpr int STEP = 64 * VEC;
    u32x4 wa[RPW], wb[RPW];
    float xa[VEC], xb[VEC];
    int c = lane * VEC;
    load(c, wa, xa);
    for (; c < in_dim; c += 2 * STEP) {
        load(c + STEP, wb, xb);
        mac(wa, xa);
        if (c + STEP >= in_dim) break;
        load(c + 2 * STEP, wa, xa);
        mac(wb, xb);
    }
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const float t = wave_sum(acc[r]);
        if (lane == 0) ys[r0 + r] = t;
    }
    __syncthreads();
    if (wave != 0) return;
    if constexpr (NSP > 1) {
        // NSP workgroups share a head vector: wave 0 of each stores its part
        // to the workspace and counts itself in; the last to arrive reads
        // the whole vector back, finishes the head and resets the counter
        // for the next call.  Nobody waits, so no co-residency is assumed.
        //
        // Ordering (LLVM AMDGPU memory model, gfx950: one L2 per XCD, the
        // L2s not coherent with each other for ordinary accesses):
        //  * the parts are system-scope atomic stores, which gfx950 issues
        //    with sc0 sc1: written through every cache level to memory;
        //  * `s_waitcnt vmcnt(0)` completes them before the counter update is
        //    issued, so they are performed at memory before the count is.
        //    This is the agent-scope release sequence (`buffer_wbl2 sc1;
        //    s_waitcnt vmcnt(0)`) minus the L2 write-back, which has nothing
        //    of this exchange to write back: the parts never sit dirty in an
        //    L2.  The write-back would cost 1.5 us per call at the Qwen3-4B
        //    decode shape (12.4 against 10.9 us, acquire-release counter);
        //  * the counter is an agent-scope atomic, performed at memory;
        //  * only the last arriver, having read n - 1, issues the agent-scope
        //    ACQUIRE fence (`buffer_inv sc1`: its CU's L1 and its XCD's L2
        //    drop their lines) before it reloads the parts, so no stale copy
        //    can serve them.
        // The workspace is zeroed once by the caller; every call leaves its
        // counters at zero.
        constexpr int PART = D / NSP;
        float *yh = ws_y + ((int64_t)row * slots + slot) * D;
        for (int i = lane; i < PART; i += 64)
            __hip_atomic_store(yh + part * PART + i, ys[part * PART + i], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_SYSTEM);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        uint32_t prev = 0;
        if (lane == 0) {
            uint32_t *cnt = ws_cnt + (int64_t)row * slots + slot;
            prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (prev == NSP - 1) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        prev = __builtin_amdgcn_readfirstlane(prev);
        if (prev != NSP - 1) return;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        for (int i = lane; i < D; i += 64)
            ys[i] = __hip_atomic_load(yh + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_wave_barrier();
    }
    const int pos = start_pos + row;
    const HeadEpi<D> epi(cs, pos, rotary_dim, neox, q_norm, k_norm, eps);
    float v[E];
    load_e<E>(ys + epi.e0, v);
    const float *bias = kind == 0 ? q_bias : (kind == 1 ? k_bias : v_bias);
    if (bias) {
        float bv[E];
        load_e<E>(bias + (int64_t)head * D + epi.e0, bv);
#pragma unroll
        for (int i = 0; i < E; i++) v[i] += bv[i];
    }
    epi.norm_rope(v, kind, lrow);
    store_head<D, QDT, KVDT>(v, kind, head, row, (int64_t)pos, epi.e0, (int64_t)n_head * D, q_out,
                             k_cache, v_cache, kv_stride);
}

template <int D, int QDT>
static void launch_kv(int kvdt, dim3 g, dim3 b, hipStream_t st, const float *qi, const float *ki,
                      const float *vi, const float *qb, const float *kb, const float *vb,
                      const float *qn, const float *kn, float eps, const float *cs, int neox,
                      int rd, int rows, int sp, int nh, int nkv, void *qo, void *kc, void *vc,
                      int64_t kvs, PageMap pm, int gpw) {
    if (kvdt == ULLM_DT_F32)
        hipLaunchKernelGGL((qkv_append_kernel<D, QDT, ULLM_DT_F32>), g, b, 0, st, qi, ki, vi, qb, kb, vb, qn, kn, eps, cs, neox, rd, rows, sp, nh, nkv, qo, kc, vc, kvs, pm, gpw);
    else if (kvdt == ULLM_DT_F16)
        hipLaunchKernelGGL((qkv_append_kernel<D, QDT, ULLM_DT_F16>), g, b, 0, st, qi, ki, vi, qb, kb, vb, qn, kn, eps, cs, neox, rd, rows, sp, nh, nkv, qo, kc, vc, kvs, pm, gpw);
    else
        hipLaunchKernelGGL((qkv_append_kernel<D, QDT, ULLM_DT_BF16>), g, b, 0, st, qi, ki, vi, qb, kb, vb, qn, kn, eps, cs, neox, rd, rows, sp, nh, nkv, qo, kc, vc, kvs, pm, gpw);
}

template <int D>
static void launch_q(int qdt, int kvdt, dim3 g, dim3 b, hipStream_t st, const float *qi,
                     const float *ki, const float *vi, const float *qb, const float *kb,
                     const float *vb, const float *qn, const float *kn, float eps,
                     const float *cs, int neox, int rd, int rows, int sp, int nh, int nkv,
                     void *qo, void *kc, void *vc, int64_t kvs, PageMap pm, int gpw) {
    if (qdt == ULLM_DT_F32) launch_kv<D, ULLM_DT_F32>(kvdt, g, b, st, qi, ki, vi, qb, kb, vb, qn, kn, eps, cs, neox, rd, rows, sp, nh, nkv, qo, kc, vc, kvs, pm, gpw);
    else if (qdt == ULLM_DT_F16) launch_kv<D, ULLM_DT_F16>(kvdt, g, b, st, qi, ki, vi, qb, kb, vb, qn, kn, eps, cs, neox, rd, rows, sp, nh, nkv, qo, kc, vc, kvs, pm, gpw);
    else launch_kv<D, ULLM_DT_BF16>(kvdt, g, b, st, qi, ki, vi, qb, kb, vb, qn, kn, eps, cs, neox, rd, rows, sp, nh, nkv, qo, kc, vc, kvs, pm, gpw);
}

// Grid of qkv_append_kernel: one token row per blockIdx.x; a row's head
// groups spread over blockIdx.y in parts of gpw groups.  Few rows (decode, a
// short chunk) leave CUs idle and each workgroup's waves would run several
// rounds of loads, so each part is one round (kAppendWaves * kBatch groups);
// many rows keep a row per workgroup.
static dim3 append_grid(int rows, int n_head, int n_kv_head, int head_dim, int &gpw) {
    static const int env = env_override("ULLM_HIP_APPEND_GPW");  // tuning override
    const int hpw = 256 / head_dim;
    const int groups = (n_head + hpw - 1) / hpw + 2 * ((n_kv_head + hpw - 1) / hpw);
    gpw = rows < kAppendSplitBelow ? kAppendWaves * kBatch : groups;
    if (env > 0) gpw = env;
    return dim3((unsigned)rows, (unsigned)((groups + gpw - 1) / gpw));
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
    int gpw;
    const dim3 grid = append_grid(rows, n_head, n_kv_head, head_dim, gpw), block(kAppendWaves * 64);
    hipStream_t st = (hipStream_t)stream;
    switch (head_dim) {
        case 64: launch_q<64>(q_dtype, kv_dtype, grid, block, st, q_in, k_in, v_in, q_bias, k_bias, v_bias, q_norm, k_norm, eps, rope_cs, rope_neox, rotary_dim, rows, start_pos, n_head, n_kv_head, q_out, k_cache, v_cache, kv_stride, PageMap{}, gpw); break;
        case 128: launch_q<128>(q_dtype, kv_dtype, grid, block, st, q_in, k_in, v_in, q_bias, k_bias, v_bias, q_norm, k_norm, eps, rope_cs, rope_neox, rotary_dim, rows, start_pos, n_head, n_kv_head, q_out, k_cache, v_cache, kv_stride, PageMap{}, gpw); break;
        default: launch_q<256>(q_dtype, kv_dtype, grid, block, st, q_in, k_in, v_in, q_bias, k_bias, v_bias, q_norm, k_norm, eps, rope_cs, rope_neox, rotary_dim, rows, start_pos, n_head, n_kv_head, q_out, k_cache, v_cache, kv_stride, PageMap{}, gpw); break;
    }
    return check_hip(hipGetLastError(), "qkv_append launch");
}

extern "C" int ullm_hip_qkv_append_paged(const float *q_in, const float *k_in, const float *v_in,
                                         const float *q_bias, const float *k_bias,
                                         const float *v_bias, const float *q_norm,
                                         const float *k_norm, float eps, const float *rope_cs,
                                         int rope_n_pos, int rope_neox, int rotary_dim, int rows,
                                         const int32_t *positions, int n_head, int n_kv_head,
                                         int head_dim, void *q_out, int q_dtype, void *k_pages,
                                         void *v_pages, int kv_dtype, int64_t kv_stride,
                                         int page_size, int n_pages, const int32_t *block_table,
                                         int table_stride, void *stream) {
    if (!dtype_ok(q_dtype) || !dtype_ok(kv_dtype))
        return set_error(ULLM_HIP_E_UNSUPPORTED, "qkv_append_paged: dtype q=%d kv=%d", q_dtype, kv_dtype);
    if (head_dim != 64 && head_dim != 128 && head_dim != 256)
        return set_error(ULLM_HIP_E_UNSUPPORTED, "qkv_append_paged: head_dim %d not in {64,128,256}",
                         head_dim);
    if (rows < 0 || rows > 0x7fffffff / 4 || n_head < 1 || n_kv_head < 1 || n_head % n_kv_head)
        return set_error(ULLM_HIP_E_INVALID, "qkv_append_paged: bad rows/heads");
    if (rotary_dim < 2 || rotary_dim > head_dim || (rotary_dim & 1))
        return set_error(ULLM_HIP_E_INVALID, "qkv_append_paged: rotary_dim %d", rotary_dim);
    if (kv_stride < (int64_t)n_kv_head * head_dim)
        return set_error(ULLM_HIP_E_INVALID, "qkv_append_paged: kv_stride too small");
    if (page_size < 1 || (page_size & (page_size - 1)))
        return set_error(ULLM_HIP_E_INVALID, "qkv_append_paged: page_size %d must be a power of two",
                         page_size);
    if (n_pages < 1 || table_stride < 1 || rope_n_pos < 1)
        return set_error(ULLM_HIP_E_INVALID, "qkv_append_paged: n_pages/table_stride/rope_n_pos < 1");
    if (rows == 0) return ULLM_HIP_OK;
    if (!q_in || !k_in || !v_in || !rope_cs || !q_out || !k_pages || !v_pages || !positions ||
        !block_table)
        return set_error(ULLM_HIP_E_INVALID, "qkv_append_paged: null tensor pointer");
    if (q_out == (void *)q_in && q_dtype != ULLM_DT_F32)
        return set_error(ULLM_HIP_E_INVALID, "qkv_append_paged: in-place q needs q_dtype f32");
    const PageMap pm{positions, block_table, table_stride, __builtin_ctz(page_size), n_pages,
                     rope_n_pos};
    int gpw;
    const dim3 grid = append_grid(rows, n_head, n_kv_head, head_dim, gpw), block(kAppendWaves * 64);
    hipStream_t st = (hipStream_t)stream;
    switch (head_dim) {
        case 64: launch_q<64>(q_dtype, kv_dtype, grid, block, st, q_in, k_in, v_in, q_bias, k_bias, v_bias, q_norm, k_norm, eps, rope_cs, rope_neox, rotary_dim, rows, 0, n_head, n_kv_head, q_out, k_pages, v_pages, kv_stride, pm, gpw); break;
        case 128: launch_q<128>(q_dtype, kv_dtype, grid, block, st, q_in, k_in, v_in, q_bias, k_bias, v_bias, q_norm, k_norm, eps, rope_cs, rope_neox, rotary_dim, rows, 0, n_head, n_kv_head, q_out, k_pages, v_pages, kv_stride, pm, gpw); break;
        default: launch_q<256>(q_dtype, kv_dtype, grid, block, st, q_in, k_in, v_in, q_bias, k_bias, v_bias, q_norm, k_norm, eps, rope_cs, rope_neox, rotary_dim, rows, 0, n_head, n_kv_head, q_out, k_pages, v_pages, kv_stride, pm, gpw); break;
    }
    return check_hip(hipGetLastError(), "qkv_append_paged launch");
}

namespace ullm {

// A head vector is split over kProjSplit workgroups when the grid would
// otherwise leave most CUs idle (decode: a few dozen head vectors).
constexpr int kProjSplit = 4;
constexpr int kProjSplitBelow = 256;  // rows * slots under which to split

static bool proj_split(int rows, int slots) { return (int64_t)rows * slots < kProjSplitBelow; }

struct ProjArgs {
    const float *x;
    int in_dim;
    const char *wq, *wk, *wv;
    const float *qb, *kb, *vb, *qn, *kn;
    float eps;
    const float *cs;
    int neox, rd, sp, nh, nkv;
    void *qo, *kc, *vc;
    int64_t kvs;
    float *ws_y;
    uint32_t *ws_cnt;
};

template <int D, int WDT, int QDT, int KVDT>
static void launch_proj(bool split, int rows, hipStream_t st, const ProjArgs &a) {
    const int slots = a.nh + 2 * a.nkv;
    auto go = [&](auto nspc) {
        constexpr int NSP = decltype(nspc)::value;
        hipLaunchKernelGGL((qkv_proj_kernel<D, WDT, QDT, KVDT, NSP>),
                           dim3((unsigned)(slots * NSP), (unsigned)rows), dim3(proj_waves(NSP) * 64), 0, st,
                           a.x, a.in_dim, a.wq, a.wk, a.wv, a.qb, a.kb, a.vb, a.qn, a.kn, a.eps, a.cs,
                           a.neox, a.rd, a.sp, a.nh, a.nkv, a.qo, a.kc, a.vc, a.kvs, a.ws_y, a.ws_cnt);
    };
    if (split) go(Int<kProjSplit>{});
    else go(Int<1>{});
}

template <int D, int WDT, int QDT>
static void launch_proj_kv(int kvdt, bool split, int rows, hipStream_t st, const ProjArgs &a) {
    if (kvdt == ULLM_DT_F32) launch_proj<D, WDT, QDT, ULLM_DT_F32>(split, rows, st, a);
    else if (kvdt == ULLM_DT_F16) launch_proj<D, WDT, QDT, ULLM_DT_F16>(split, rows, st, a);
    else launch_proj<D, WDT, QDT, ULLM_DT_BF16>(split, rows, st, a);
}

template <int D, int WDT>
static void launch_proj_q(int qdt, int kvdt, bool split, int rows, hipStream_t st, const ProjArgs &a) {
    if (qdt == ULLM_DT_F32) launch_proj_kv<D, WDT, ULLM_DT_F32>(kvdt, split, rows, st, a);
    else if (qdt == ULLM_DT_F16) launch_proj_kv<D, WDT, ULLM_DT_F16>(kvdt, split, rows, st, a);
    else launch_proj_kv<D, WDT, ULLM_DT_BF16>(kvdt, split, rows, st, a);
}

template <int D>
static void launch_proj_w(int wdt, int qdt, int kvdt, bool split, int rows, hipStream_t st,
                          const ProjArgs &a) {
    if (wdt == ULLM_DT_F32) launch_proj_q<D, ULLM_DT_F32>(qdt, kvdt, split, rows, st, a);
    else if (wdt == ULLM_DT_F16) launch_proj_q<D, ULLM_DT_F16>(qdt, kvdt, split, rows, st, a);
    else launch_proj_q<D, ULLM_DT_BF16>(qdt, kvdt, split, rows, st, a);
}

static size_t proj_ws_bytes(int rows, int slots, int D) {
    if (!proj_split(rows, slots)) return 0;
    const size_t n = (size_t)rows * slots;
    return n * D * 4 + (n * 4 + 255) / 256 * 256;
}

}  // namespace ullm

extern "C" int ullm_hip_qkv_proj_append(const float *x, int in_dim, const void *w_q,
                                        const void *w_k, const void *w_v, int w_dtype,
                                        const float *q_bias, const float *k_bias,
                                        const float *v_bias, const float *q_norm,
                                        const float *k_norm, float eps, const float *rope_cs,
                                        int rope_n_pos, int rope_neox, int rotary_dim, int rows,
                                        int start_pos, int n_head, int n_kv_head, int head_dim,
                                        void *q_out, int q_dtype, void *k_cache, void *v_cache,
                                        int kv_dtype, int64_t kv_stride, void *workspace,
                                        size_t workspace_bytes, void *stream) {
    if (!dtype_ok(w_dtype) || !dtype_ok(q_dtype) || !dtype_ok(kv_dtype))
        return set_error(ULLM_HIP_E_UNSUPPORTED, "qkv_proj_append: dtype w=%d q=%d kv=%d",
                         w_dtype, q_dtype, kv_dtype);
    if (head_dim != 64 && head_dim != 128 && head_dim != 256)
        return set_error(ULLM_HIP_E_UNSUPPORTED, "qkv_proj_append: head_dim %d not in {64,128,256}",
                         head_dim);
    if (rows < 0 || start_pos < 0 || n_head < 1 || n_kv_head < 1 || n_head % n_kv_head)
        return set_error(ULLM_HIP_E_INVALID, "qkv_proj_append: bad rows/heads");
    if (in_dim < 8 || in_dim % 8)
        return set_error(ULLM_HIP_E_INVALID, "qkv_proj_append: in_dim %d must be a positive multiple of 8",
                         in_dim);
    if (rotary_dim < 2 || rotary_dim > head_dim || (rotary_dim & 1))
        return set_error(ULLM_HIP_E_INVALID, "qkv_proj_append: rotary_dim %d", rotary_dim);
    if (kv_stride < (int64_t)n_kv_head * head_dim)
        return set_error(ULLM_HIP_E_INVALID, "qkv_proj_append: kv_stride too small");
    if (rows == 0) return ULLM_HIP_OK;
    if (!x || !w_q || !w_k || !w_v || !rope_cs || !q_out || !k_cache || !v_cache)
        return set_error(ULLM_HIP_E_INVALID, "qkv_proj_append: null tensor pointer");
    if (((uintptr_t)x | (uintptr_t)w_q | (uintptr_t)w_k | (uintptr_t)w_v) & 15)
        return set_error(ULLM_HIP_E_INVALID, "qkv_proj_append: x and weights must be 16-byte aligned");
    if (rope_n_pos < start_pos + rows)
        return set_error(ULLM_HIP_E_INVALID, "qkv_proj_append: rope table has %d positions, need %d",
                         rope_n_pos, start_pos + rows);
    if (rows > 65535)
        return set_error(ULLM_HIP_E_INVALID, "qkv_proj_append: rows %d > 65535", rows);
    const int slots = n_head + 2 * n_kv_head;
    const bool split = proj_split(rows, slots);
    const size_t need = proj_ws_bytes(rows, slots, head_dim);
    if (need > 0 && (!workspace || workspace_bytes < need))
        return set_error(ULLM_HIP_E_WORKSPACE, "qkv_proj_append: workspace of %zu bytes needed, %zu given",
                         need, workspace_bytes);
    ProjArgs a{x, in_dim, (const char *)w_q, (const char *)w_k, (const char *)w_v, q_bias, k_bias,
               v_bias, q_norm, k_norm, eps, rope_cs, rope_neox, rotary_dim, start_pos, n_head,
               n_kv_head, q_out, k_cache, v_cache, kv_stride,
               split ? (float *)workspace : nullptr,
               split ? (uint32_t *)((char *)workspace + (size_t)rows * slots * head_dim * 4) : nullptr};
    hipStream_t st = (hipStream_t)stream;
    switch (head_dim) {
        case 64: launch_proj_w<64>(w_dtype, q_dtype, kv_dtype, split, rows, st, a); break;
        case 128: launch_proj_w<128>(w_dtype, q_dtype, kv_dtype, split, rows, st, a); break;
        default: launch_proj_w<256>(w_dtype, q_dtype, kv_dtype, split, rows, st, a); break;
    }
    return check_hip(hipGetLastError(), "qkv_proj_append launch");
}

extern "C" size_t ullm_hip_qkv_proj_workspace_bytes(int rows, int n_head, int n_kv_head,
                                                    int head_dim) {
    if (rows < 1 || n_head < 1 || n_kv_head < 1 || head_dim < 1) return 0;
    return proj_ws_bytes(rows, n_head + 2 * n_kv_head, head_dim);
}
