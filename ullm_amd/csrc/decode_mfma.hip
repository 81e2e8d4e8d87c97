// Split-KV single-query GQA decode attention on MFMA (gfx950), f16/bf16 KV.
//
// Computes what the CPU reference computes at
// crates/ullm-model/src/lib.rs:916-938 (window start: :1183-1186):
//   out[b,h] = softmax_t(scale * q[b,h] . K[t]) . V[t],  t in start..len-1.
//
// Why MFMA for a bandwidth-bound op: a VALU formulation spends ~50 wave64
// instructions per key (dot products, cross-lane sums, widening, exp), which
// caps one CU far below its share of HBM bandwidth.  Here both contractions
// run on v_mfma_f32_16x16x32_{f16,bf16} and the VALU only does the softmax:
//  * A "unit" is up to 16 query heads sharing one kv head (GQA group).
//  * S^T[16 keys x 16 heads] = K . Q^T: the K tile is the A operand and comes
//    straight from 16-byte global loads (lane = key, 8 consecutive d); Q^T is
//    the B operand, held in registers for the whole call.  q (f32) is split
//    into hi + lo halves of the cache dtype, two MFMAs per step, so the
//    product keeps ~f32 accuracy.
//  * O^T[16 d x 16 heads] += V^T . P^T: V^T is the A operand.  Each lane
//    loads 8 keys x 8 d of V, transposes them in registers and stores them in
//    a wave-private LDS tile [d][key]; one 16-byte LDS read per d tile then
//    gives the operand.  P^T (the B operand) is exactly the S^T accumulator of
//    two key tiles, exponentiated: the key order inside a k-step is free, so
//    the LDS tile is written in accumulator order and P never moves between
//    lanes.  f16 caches use P in f16 (2^-11); bf16 caches split P into
//    hi + lo bf16 (two MFMAs) to stay inside a 1e-3 rel-L2 budget.
//  * In both accumulators a lane's column is one head, so the running max,
//    sum and rescale of a head live in the lanes that own its output.
//  * Waves of a workgroup stream disjoint key blocks and merge through LDS;
//    splits merge in-launch: the last workgroup of a unit (agent-scope
//    counter) combines the partials and writes `out`.
#include <cstdlib>
#include "common.hpp"
#include "wave.hpp"

namespace ullm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

constexpr int kMW = 4;          // waves per workgroup
constexpr int kTok = 32;        // keys per wave iteration (two 16-key tiles)
constexpr int kMaxUnitHeads = 16;
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer, gfx9 data format
constexpr int kMfmaTargetWG = 512;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

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

// f32 -> 16-bit storage of T (RNE) and back.
template <class T>
__device__ __forceinline__ uint32_t to16(float f) {
    if constexpr (__is_same(T, BF16)) return f32_to_bf16_bits(f);
    else return f32_to_f16_bits(f);
}
template <class T>
__device__ __forceinline__ float from16(uint32_t h) {
    if constexpr (__is_same(T, BF16)) return __uint_as_float(h << 16);
    else return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

template <class T, int D>
__global__ __launch_bounds__(kMW * 64, D <= 128 ? 2 : 1) void decode_mfma_kernel(
    const float *__restrict__ q, const char *__restrict__ kc, const char *__restrict__ vc,
    int64_t kv_stride, int64_t seq_stride, const int32_t *__restrict__ seq_lens, int window,
    int n_head, int kv_mul, int gt, int n_units, int chunk, int splits, float qscale,
    float *__restrict__ out, float *__restrict__ ws_ml, float *__restrict__ ws_acc) {
    constexpr int NS = D / 32;      // QK k-steps (32 d each)
    constexpr int NDT = D / 16;     // 16-wide d tiles of O^T
    constexpr int CPR = D / 8;      // 16-byte chunks per key row
    constexpr int VP = D + 16;      // LDS V row pitch (halves): conflict-free rows
    constexpr bool SPLITP = __is_same(T, BF16);

    const int split = blockIdx.x, unit = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n16 = lane & 15, kg = lane >> 4;
    const int head0 = unit * gt, kvh = head0 / kv_mul;
    const bool head_ok = n16 < gt;

    const int len = seq_lens[b];
    const int start = (window > 0 && len > window) ? len - window : 0;
    const int c0 = start + split * chunk;
    const int c1 = min(c0 + chunk, len);

    __shared__ __attribute__((aligned(16))) uint16_t vt_all[kMW][kTok * VP];
    uint16_t *vt = vt_all[wave];

    // Q^T operand, hi/lo split: step s, lane (head n16, chunk c = s*4 + kg).
    // All q loads are issued before any is used (one round trip).
    u32x4 qh[NS], ql[NS];
    {
        const float *qp = q + ((int64_t)b * n_head + head0 + (head_ok ? n16 : 0)) * D;
        f32x4 qa[NS][2];
#pragma unroll
        for (int s = 0; s < NS; s++) {
            qa[s][0] = *(const f32x4 *)(qp + (s * 4 + kg) * 8);
            qa[s][1] = *(const f32x4 *)(qp + (s * 4 + kg) * 8 + 4);
        }
#pragma unroll
        for (int s = 0; s < NS; s++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float x0 = head_ok ? qa[s][j >> 1][(2 * j) & 3] * qscale : 0.f;
                const float x1 = head_ok ? qa[s][j >> 1][(2 * j + 1) & 3] * qscale : 0.f;
                const uint32_t h0 = to16<T>(x0), h1 = to16<T>(x1);
                const uint32_t l0 = to16<T>(x0 - from16<T>(h0)), l1 = to16<T>(x1 - from16<T>(h1));
                qh[s][j] = h0 | (h1 << 16);
                ql[s][j] = l0 | (l1 << 16);
            }
    }

    f32x4 oacc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; i++) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_part = 0.f;

    const int rb = (int)(kv_stride * 2);  // bytes per key row
    // Buffer resources over this sequence's kv head, ending at key c1: loads
    // of keys >= c1 fall outside the range and return zero.
    const char *kb0 = kc + (int64_t)b * seq_stride * 2 + (int64_t)kvh * D * 2;
    const char *vb0 = vc + (int64_t)b * seq_stride * 2 + (int64_t)kvh * D * 2;
    const int range = c1 > 0 ? (c1 - 1) * rb + D * 2 : 0;
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void *)kb0, 0, range, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void *)vb0, 0, range, kRsrcWord3);

    // V is staged row-major: lane l loads 16-byte chunk (l % CPR) of key
    // (l / CPR) + KPI*i of the block and writes it unchanged to the wave's LDS
    // tile; the transposing LDS read (ds_read_b64_tr_b16) later turns it into
    // the V^T operand.
    constexpr int KPI = 64 / CPR;          // keys covered by one load instruction
    constexpr int VL = kTok / KPI;         // V loads per lane per block
    const int vcol = lane % CPR, vrow0 = lane / CPR;

    struct Tile {
        u32x4 k[2][NS];
        u32x4 v[VL];
    };
    // Loop-invariant lane offsets; the block start goes in a scalar offset.
    int koffb[2];
#pragma unroll
    for (int t = 0; t < 2; t++) koffb[t] = (t * 16 + n16) * rb + kg * 16;
    const int voffb = vrow0 * rb + vcol * 16;
    // Issue the loads of the block starting at key tb (nontemporal).
    auto issue = [&](Tile &T_, int tb) {
        const int so = tb * rb;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int s = 0; s < NS; s++)
                T_.k[t][s] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, koffb[t] + s * 64, so, 2));
#pragma unroll
        for (int i = 0; i < VL; i++)
            T_.v[i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, voffb + i * KPI * rb, so, 2));
    };
    // Consume a loaded block.
    auto consume = [&](Tile &T_, int tb) {
        // S^T = K . Q^T (two 16-key tiles), q split hi + lo
        f32x4 sacc[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            sacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < NS; s++) {
                sacc[t] = mfma16<T>(T_.k[t][s], qh[s], sacc[t]);
                sacc[t] = mfma16<T>(T_.k[t][s], ql[s], sacc[t]);
            }
        }
        // V rows into the wave's LDS tile (row-major, padded pitch)
#pragma unroll
        for (int i = 0; i < VL; i++)
            *(u32x4 *)(vt + (vrow0 + i * KPI) * VP + vcol * 8) = T_.v[i];
        // online softmax: lane = head n16, keys kg*4+i (tile 0) and 16+kg*4+i
        float sv[8];
        const bool full = tb + kTok <= c1;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                sv[t * 4 + i] = (full || tb + t * 16 + kg * 4 + i < c1) ? sacc[t][i] : -INFINITY;
        float mt = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                         fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
        mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
        const float m_new = fmaxf(m_run, mt);
        const float mu = m_new == -INFINITY ? 0.f : m_new;
        if (__any(m_new != m_run)) {  // rescale only when some head's max moved
            const float corr = __builtin_amdgcn_exp2f(m_run - mu);
            l_part *= corr;
#pragma unroll
            for (int i = 0; i < NDT; i++) oacc[i] *= corr;
        }
        m_run = m_new;
        float p[8];
#pragma unroll
        for (int i = 0; i < 8; i++) { p[i] = __builtin_amdgcn_exp2f(sv[i] - mu); l_part += p[i]; }
        u32x4 ph, pl;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t h0 = to16<T>(p[2 * j]), h1 = to16<T>(p[2 * j + 1]);
            ph[j] = h0 | (h1 << 16);
            if constexpr (SPLITP) {
                const uint32_t l0 = to16<T>(p[2 * j] - from16<T>(h0));
                const uint32_t l1 = to16<T>(p[2 * j + 1] - from16<T>(h1));
                pl[j] = l0 | (l1 << 16);
            }
        }
        // O^T += V^T . P^T.  The LDS tile is private to this wave and a wave's
        // LDS instructions execute in issue order, so only the compiler must
        // be kept from reordering; a memory fence here would also wait for
        // the next block's global loads and serialise the pipeline.
        lds_order();
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            // lane n16 of key group kg receives V[keys c*16 + kg*4 + j][d = dt*16 + n16]
            const uint16_t *r0 = vt + (kg * 4 + (n16 >> 2)) * VP + dt * 16 + 4 * (n16 & 3);
            const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)r0);
            const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(r0 + 16 * VP));
            const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
            const u32x4 a = {l2[0], l2[1], h2[0], h2[1]};
            oacc[dt] = mfma16<T>(a, ph, oacc[dt]);
            if constexpr (SPLITP) oacc[dt] = mfma16<T>(a, pl, oacc[dt]);
        }
        lds_order();  // the tile is rewritten by the next block
    };

    // Two-stage pipeline: the next block's loads are in flight while the
    // current block computes (head_dim 256 has no registers for a second
    // stage and streams one block at a time).
    constexpr int STEP = kMW * kTok;
    int tb = c0 + wave * kTok;
    if constexpr (D <= 128) {
        Tile A_, B_;
        if (tb < c1) {
            issue(A_, tb);
            for (;;) {
                const int tn = tb + STEP;
                issue(B_, tn);
                consume(A_, tb);
                if (tn >= c1) break;
                const int tn2 = tn + STEP;
                issue(A_, tn2);
                consume(B_, tn);
                if (tn2 >= c1) break;
                tb = tn2;
            }
        }
    } else {
        for (; tb < c1; tb += STEP) {
            Tile A_;
            issue(A_, tb);
            consume(A_, tb);
        }
    }

    // ---- wave result: head n16, d = dt*16 + kg*4 + i ----
    l_part += __shfl_xor(l_part, 16, 64);
    l_part += __shfl_xor(l_part, 32, 64);

    __syncthreads();  // all waves done with their V^T tiles: reuse the LDS
    float *sm = (float *)&vt_all[0][0];
    float *sm_m = sm;                                 // [kMW][16]
    float *sm_l = sm + kMW * 16;                      // [kMW][16]
    float *sm_o = sm + 2 * kMW * 16;                  // [kMW][16][D]
    if (kg == 0) { sm_m[wave * 16 + n16] = m_run; sm_l[wave * 16 + n16] = l_part; }
#pragma unroll
    for (int dt = 0; dt < NDT; dt++)
#pragma unroll
        for (int i = 0; i < 4; i++) sm_o[(wave * 16 + n16) * D + dt * 16 + kg * 4 + i] = oacc[dt][i];
    __syncthreads();

    const int64_t u = (int64_t)b * n_units + unit;
    const int GD = gt * D;
    for (int idx = tid; idx < GD; idx += kMW * 64) {
        const int g = idx / D, d = idx % D;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < kMW; w++) mx = fmaxf(mx, sm_m[w * 16 + g]);
        const float mu = mx == -INFINITY ? 0.f : mx;
        float num = 0.f, den = 0.f;
#pragma unroll
        for (int w = 0; w < kMW; w++) {
            const float c = exp2f(sm_m[w * 16 + g] - mu);
            num += sm_o[(w * 16 + g) * D + d] * c;
            den += sm_l[w * 16 + g] * c;
        }
        if (splits == 1) {
            out[((int64_t)b * n_head + head0 + g) * D + d] = den > 0.f ? num / den : 0.f;
        } else {
            ws_acc[(u * splits + split) * GD + idx] = num;
            if (d == 0) {
                ws_ml[((u * splits + split) * gt + g) * 2] = mx;
                ws_ml[((u * splits + split) * gt + g) * 2 + 1] = den;
            }
        }
    }
}

}  // namespace ullm

namespace ullm {

constexpr int kMaxSplits = 128;
constexpr int kMergeLoads = 32;  // per-thread partial loads kept in flight

// Combines the split partials of one (sequence, head): all loads are issued
// at once -- m/l of every split into LDS, and thread (column of 4 d, split
// residue r) holds its splits' partial rows in registers -- then the
// log-sum-exp weights are applied and the residues summed through LDS.
template <int D>
__global__ __launch_bounds__(256) void decode_merge_kernel(const float *__restrict__ ws_ml,
                                                           const float *__restrict__ ws_acc,
                                                           int splits, int gt, int n_units,
                                                           int n_head, float *__restrict__ out) {
    constexpr int NC = D / 4, R = 256 / NC;
    const int g = blockIdx.x, unit = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, col = tid % NC, r = tid / NC;
    const int64_t u = (int64_t)b * n_units + unit;
    const int GD = gt * D;
    __shared__ float sm_m[kMaxSplits], sm_l[kMaxSplits];
    __shared__ f32x4 red[R][NC];
    for (int sp = tid; sp < splits; sp += 256) {
        sm_m[sp] = ws_ml[((u * splits + sp) * gt + g) * 2];
        sm_l[sp] = ws_ml[((u * splits + sp) * gt + g) * 2 + 1];
    }
    f32x4 v[kMergeLoads];
#pragma unroll
    for (int i = 0; i < kMergeLoads; i++) {
        const int sp = r + i * R;
        v[i] = sp < splits ? *(const f32x4 *)(ws_acc + (u * splits + sp) * GD + g * D + col * 4)
                           : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int sp = 0; sp < splits; sp++) mx = fmaxf(mx, sm_m[sp]);
    const float mu = mx == -INFINITY ? 0.f : mx;
    f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kMergeLoads; i++) {
        const int sp = r + i * R;
        if (sp < splits) a += v[i] * exp2f(sm_m[sp] - mu);
    }
    red[r][col] = a;
    __syncthreads();
    if (tid < NC) {
        f32x4 t = red[0][tid];
#pragma unroll
        for (int rr = 1; rr < R; rr++) t += red[rr][tid];
        float den = 0.f;
        for (int sp = 0; sp < splits; sp++) den += sm_l[sp] * exp2f(sm_m[sp] - mu);
        const float inv = den > 0.f ? 1.0f / den : 0.f;
        *(f32x4 *)(out + ((int64_t)b * n_head + unit * gt + g) * D + tid * 4) = t * inv;
    }
}

}  // namespace ullm

namespace ullm {

struct MfmaPlan {
    int gt, n_units, chunk, splits;
    size_t off_ml, off_acc, bytes;
};

static MfmaPlan plan_mfma(int batch, int n_head, int n_kv_head, int D, int max_len, int window) {
    MfmaPlan p{};
    const int kv_mul = n_head / n_kv_head;
    p.gt = kv_mul;
    if (p.gt > kMaxUnitHeads)
        for (p.gt = kMaxUnitHeads; kv_mul % p.gt; p.gt--) {}
    p.n_units = n_head / p.gt;
    const int visible = (window > 0 && max_len > window) ? window : max_len;
    const int units = batch * p.n_units;
    const int tile = kMW * kTok;
    int splits = (visible + tile - 1) / tile;
    const int want = (kMfmaTargetWG + units - 1) / units;
    if (splits > want) splits = want;
    const int cap = kMaxSplits;
    if (splits > cap) splits = cap;
    if (const char *e = getenv("ULLM_HIP_DECODE_SPLITS")) {  // tuning override
        const int f = atoi(e);
        if (f >= 1) splits = f < cap ? f : cap;
    }
    if (splits < 1) splits = 1;
    int chunk = (visible + splits - 1) / splits;
    chunk = (chunk + kTok - 1) / kTok * kTok;
    p.chunk = chunk;
    p.splits = (visible + chunk - 1) / chunk;
    const size_t ml = ((size_t)units * p.splits * p.gt * 2 * 4 + 255) / 256 * 256;
    const size_t ac = (size_t)units * p.splits * p.gt * D * 4;
    p.off_ml = 0;
    p.off_acc = ml;
    p.bytes = p.splits > 1 ? ml + ac : 0;
    return p;
}

size_t decode_mfma_workspace(int batch, int n_head, int n_kv_head, int D, int max_len,
                             int window) {
    return plan_mfma(batch, n_head, n_kv_head, D, max_len, window).bytes;
}

template <class T, int D>
static void launch_mfma(const MfmaPlan &p, const float *q, const void *kc, const void *vc,
                        int64_t kvs, int64_t ss, const int32_t *lens, int win, int batch, int nh,
                        int kv_mul, float qs, float *out, char *ws, hipStream_t st) {
    hipLaunchKernelGGL((decode_mfma_kernel<T, D>), dim3(p.splits, p.n_units, batch),
                       dim3(kMW * 64), 0, st, q, (const char *)kc, (const char *)vc, kvs, ss,
                       lens, win, nh, kv_mul, p.gt, p.n_units, p.chunk, p.splits, qs, out,
                       (float *)(ws + p.off_ml), (float *)(ws + p.off_acc));
    if (p.splits > 1)
        hipLaunchKernelGGL((decode_merge_kernel<D>), dim3(p.gt, p.n_units, batch), dim3(256), 0,
                           st, (const float *)(ws + p.off_ml), (const float *)(ws + p.off_acc),
                           p.splits, p.gt, p.n_units, nh, out);
}

int decode_mfma(int dtype, const float *q, const void *kc, const void *vc, int64_t kvs,
                int64_t ss, const int32_t *lens, int max_len, int win, int batch, int nh,
                int nkv, int D, float qs, float *out, void *ws, size_t ws_bytes,
                hipStream_t st) {
    const MfmaPlan p = plan_mfma(batch, nh, nkv, D, max_len, win);
    if (p.bytes > 0 && (!ws || ws_bytes < p.bytes))
        return set_error(ULLM_HIP_E_WORKSPACE, "decode: workspace of %zu bytes needed, %zu given",
                         p.bytes, ws_bytes);
    const int kv_mul = nh / nkv;
    char *w = (char *)ws;
#define ULLM_MFMA_CASE(TT, DD) \
    launch_mfma<TT, DD>(p, q, kc, vc, kvs, ss, lens, win, batch, nh, kv_mul, qs, out, w, st)
    if (dtype == ULLM_DT_F16) {
        if (D == 64) ULLM_MFMA_CASE(F16, 64);
        else if (D == 128) ULLM_MFMA_CASE(F16, 128);
        else ULLM_MFMA_CASE(F16, 256);
    } else {
        if (D == 64) ULLM_MFMA_CASE(BF16, 64);
        else if (D == 128) ULLM_MFMA_CASE(BF16, 128);
        else ULLM_MFMA_CASE(BF16, 256);
    }
#undef ULLM_MFMA_CASE
    return check_hip(hipGetLastError(), "decode (mfma) launch");
}

}  // namespace ullm
