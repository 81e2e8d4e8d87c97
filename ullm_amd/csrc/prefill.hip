// Causal multi-token prefill attention on CDNA4 MFMA (gfx950).
//
// Computes, for query row s at pos = start_pos + s and head h (kv head
// h / kv_mul), out[s,h] = softmax_t(scale * q[s,h] . K[t]) . V[t] over
// t in start..pos (start = 0, or the sliding-window start) -- the CPU
// reference loop crates/ullm-model/src/lib.rs:1061-1087, with the window rule
// of lib.rs:1183-1186 applied per row as the Metal kernel does
// (shader.metal:1051).
//
// Design:
//  * A workgroup is 4 waves and owns BM = 128 query rows of one head; each
//    wave owns 32 rows.  Per iteration the workgroup stages BN keys of K
//    (as stored) and V (transposed to [d][key] and widened to f16) in LDS.
//  * S^T = K . Q^T runs on v_mfma_f32_32x32x16_{bf16,f16}: K tiles from LDS
//    are the A operand, the wave's Q rows stay in registers as the B operand.
//    In the S^T accumulator every lane holds ONE query row (lane % 32) and 16
//    keys, so the row max needs a single cross-lane exchange (lane ^ 32) and
//    the row sum stays lane-local until the end.
//  * The same accumulator, exponentiated and rounded to f16, IS the B operand
//    of O^T += V^T . P^T (v_mfma_f32_32x32x16_f16): the keys' order inside a
//    k-step is free, so V^T is read from LDS in the accumulator's key order
//    and no register shuffle of P is needed.  P.V in f16 keeps the rounding of
//    P at 2^-11 (bf16 would cost 2^-8 relative, beyond a 1e-3 rel-L2 budget).
//  * Online softmax in the exp2 domain (scale*log2(e) folded into one
//    multiply), f32 statistics and accumulators.
//  * Tiles are ordered kv-head major and, within a kv head, longest causal
//    row block first; blocks are dealt to the 8 XCDs so that all query heads
//    of one kv head share one XCD's L2 (workgroup i runs on XCD i % 8).
#include "common.hpp"
#include "mfma_util.hpp"
#include "wave.hpp"

namespace ullm {

template <int D>
struct PrefillCfg {
    static constexpr int BM = 128;                    // query rows per workgroup
    static constexpr int BN = D <= 128 ? 64 : 32;     // keys per iteration
    static constexpr int KP = D + 8;                  // K row pitch in LDS (elements)
    static constexpr int VP = BN + 8;                 // V^T row pitch in LDS (elements)
    static constexpr int CPR = D / 8;                 // 16-byte chunks per key row
    static constexpr int NCH = BN * CPR / 256;        // chunks (rows) per thread per tile
    static constexpr int NKT = BN / 32;               // 32-key MFMA tiles per iteration
    static constexpr int NDT = D / 32;                // 32-wide d tiles of the output
    static constexpr int NKS = D / 16;                // 16-deep k steps of Q.K
    static_assert(NCH >= 1 && 256 % CPR == 0, "staging map");
};

template <class T>
__device__ __forceinline__ f32x16 mfma_qk(const u32x4 &a, const u32x4 &b, const f32x16 &c) {
    if constexpr (sizeof(T) && T::bytes == 2 && __is_same(T, BF16))
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t to_f16_pair(float lo, float hi) {
    return (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
}

template <class T, int D>
__global__ __launch_bounds__(256, D >= 256 ? 1 : 2) void prefill_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ kc,
    const uint16_t *__restrict__ vc, int64_t kv_stride, int S, int start_pos, int window,
    int n_head, int kv_mul, float qscale, float *__restrict__ out) {
    using C = PrefillCfg<D>;
    constexpr int BM = C::BM, BN = C::BN, KP = C::KP, VP = C::VP, CPR = C::CPR, NCH = C::NCH;
    constexpr int NKT = C::NKT, NDT = C::NDT, NKS = C::NKS;
    __shared__ __attribute__((aligned(16))) uint16_t Ks[BN * KP];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[D * VP];

    // ---- tile assignment (XCD-aware, longest first) ----
    const int nqb = (S + BM - 1) / BM;
    const int total = n_head * nqb;
    const int per_xcd = (total + 7) / 8;
    const int t = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (t >= total) return;
    const int per_kvh = nqb * kv_mul;
    const int kvh = t / per_kvh, r = t % per_kvh;
    const int qb = nqb - 1 - r / kv_mul;
    const int h = kvh * kv_mul + r % kv_mul;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = lane & 31, h2 = lane >> 5;
    const int q0 = qb * BM, qw = q0 + wave * 32;
    const int64_t q_dim = (int64_t)n_head * D;
    const int kv_len = start_pos + S;

    // ---- Q rows of this wave as the B operand (d = s*16 + h2*8 + j) ----
    const int qrow = qw + c;
    const bool row_ok = qrow < S;
    u32x4 qreg[NKS];
    {
        const uint16_t *qp = q + (int64_t)(row_ok ? qrow : 0) * q_dim + (int64_t)h * D + h2 * 8;
#pragma unroll
        for (int s = 0; s < NKS; s++) qreg[s] = row_ok ? ld16(qp + s * 16) : u32x4{0, 0, 0, 0};
    }
    const int pos_row = start_pos + qrow;

    // ---- key range of the workgroup and of this wave ----
    const int wg_last = start_pos + min(q0 + BM, S) - 1;  // largest position in the block
    const int kv_hi = wg_last + 1;
    int kv_lo = 0;
    if (window > 0) kv_lo = max(0, start_pos + q0 + 1 - window);
    kv_lo = (kv_lo / BN) * BN;
    const int w_first = start_pos + qw;                   // smallest position of the wave
    const int w_last = start_pos + min(qw + 32, S) - 1;   // largest (may be < w_first)

    f32x16 oacc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; i++) oacc[i] = f32x16{};
    float m_run = -INFINITY, l_part = 0.f;

    // ---- staging map: thread -> (column chunk cc, rows rg*NCH .. +NCH) ----
    const int cc = tid % CPR, rg = tid / CPR;
    const uint16_t *kg = kc + (int64_t)kvh * D + cc * 8;
    const uint16_t *vg = vc + (int64_t)kvh * D + cc * 8;
    u32x4 kpre[NCH], vpre[NCH];
    auto prefetch = [&](int kb) {
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            const int key = kb + rg * NCH + i;
            const bool ok = key < kv_len;
            kpre[i] = ok ? ld16(kg + (int64_t)key * kv_stride) : u32x4{0, 0, 0, 0};
            vpre[i] = ok ? ld16(vg + (int64_t)key * kv_stride) : u32x4{0, 0, 0, 0};
        }
    };
    prefetch(kv_lo);

    for (int kb = kv_lo; kb < kv_hi; kb += BN) {
        __syncthreads();  // previous tile fully consumed
#pragma unroll
        for (int i = 0; i < NCH; i++)
            *(u32x4 *)&Ks[(rg * NCH + i) * KP + cc * 8] = kpre[i];
        // V^T: element (d = cc*8 + j, key = rg*NCH + i), widened to f16.
#pragma unroll
        for (int j = 0; j < 8; j++) {
            float vf[NCH];
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                const uint32_t w = vpre[i][j >> 1];
                if constexpr (__is_same(T, BF16)) vf[i] = (j & 1) ? bf16_hi(w) : bf16_lo(w);
                else vf[i] = (j & 1) ? f16_hi(w) : f16_lo(w);
            }
            uint16_t *dst = &Vt[(cc * 8 + j) * VP + rg * NCH];
            if constexpr (NCH == 4) {
                *(u32x2 *)dst = u32x2{to_f16_pair(vf[0], vf[1]), to_f16_pair(vf[2], vf[3])};
            } else if constexpr (NCH == 2) {
                *(uint32_t *)dst = to_f16_pair(vf[0], vf[1]);
            } else {
#pragma unroll
                for (int i = 0; i < NCH; i++) dst[i] = f32_to_f16_bits(vf[i]);
            }
        }
        __syncthreads();
        if (kb + BN < kv_hi) prefetch(kb + BN);

        // Skip the MFMA work when the whole tile is masked for this wave.
        const bool causal_dead = kb > w_last;
        const bool window_dead = window > 0 && kb + BN - 1 < w_first + 1 - window;
        if (causal_dead || window_dead || qw >= S) continue;

        // ---- S^T = K . Q^T ----
        f32x16 sacc[NKT];
#pragma unroll
        for (int kt = 0; kt < NKT; kt++) {
            sacc[kt] = f32x16{};
            const uint16_t *kr = &Ks[(kt * 32 + c) * KP + h2 * 8];
#pragma unroll
            for (int s = 0; s < NKS; s++)
                sacc[kt] = mfma_qk<T>(*(const u32x4 *)(kr + s * 16), qreg[s], sacc[kt]);
        }

        // ---- online softmax over this tile (lane = one query row) ----
        const bool need_mask = (kb + BN - 1 > w_first) || (window > 0 && kb < w_last + 1 - window);
        float mloc = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < NKT; kt++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                float sv = sacc[kt][i] * qscale;
                if (need_mask) {
                    const int key = kb + kt * 32 + (i >> 2) * 8 + h2 * 4 + (i & 3);
                    const bool dead = key > pos_row || (window > 0 && key <= pos_row - window);
                    sv = dead ? -INFINITY : sv;
                }
                sacc[kt][i] = sv;
                mloc = fmaxf(mloc, sv);
            }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
        const float m_new = fmaxf(m_run, mloc);
        const float mu = m_new == -INFINITY ? 0.f : m_new;
        const float corr = exp2f(m_run - mu);
        m_run = m_new;
        float psum = 0.f;
        u32x4 pk[NKT][2];
#pragma unroll
        for (int kt = 0; kt < NKT; kt++)
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const float p0 = exp2f(sacc[kt][ks * 8 + 2 * jj] - mu);
                    const float p1 = exp2f(sacc[kt][ks * 8 + 2 * jj + 1] - mu);
                    psum += p0 + p1;
                    pk[kt][ks][jj] = to_f16_pair(p0, p1);
                }
        l_part = l_part * corr + psum;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) oacc[dt] *= corr;

        // ---- O^T += V^T . P^T (keys in accumulator order) ----
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            const uint16_t *vr = &Vt[(dt * 32 + c) * VP + h2 * 4];
#pragma unroll
            for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                for (int ks = 0; ks < 2; ks++) {
                    const int kofs = kt * 32 + ks * 16;
                    const u32x2 lo = *(const u32x2 *)(vr + kofs);
                    const u32x2 hi = *(const u32x2 *)(vr + kofs + 8);
                    const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
                    oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, pk[kt][ks]),
                        oacc[dt], 0, 0, 0);
                }
        }
    }

    // ---- normalise and store: lane holds row qrow, d = dt*32 + g*8 + h2*4 + 0..3 ----
    const float l_tot = l_part + __shfl_xor(l_part, 32, 64);
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    if (!row_ok) return;
    float *op = out + (int64_t)qrow * q_dim + (int64_t)h * D + h2 * 4;
#pragma unroll
    for (int dt = 0; dt < NDT; dt++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            f32x4 v = {oacc[dt][g * 4] * inv, oacc[dt][g * 4 + 1] * inv, oacc[dt][g * 4 + 2] * inv,
                       oacc[dt][g * 4 + 3] * inv};
            *(f32x4 *)(op + dt * 32 + g * 8) = v;
        }
}

// ---------------------------------------------------------------------------
// Prefill v2: K/V tiles shared by 8 waves through a 3-stage LDS ring filled by
// buffer_load ... lds (whole contiguous head rows per instruction, 16-byte
// slots XOR-swizzled by row); K operands via ds_read_b128, V^T operands via
// the transposing ds_read_b64_tr_b16 from the row-major V tile.
//
// Work: a "unit" is HW query heads of one kv head (HW = 4, 2 or 1 heads,
// dividing the GQA group) and a "group" is RW = 4/HW consecutive 32-row
// blocks, so 4 waves cover one group.  A workgroup = 8 waves = two groups:
// without a window they are g and NG-1-g, so every workgroup carries the same
// causal work (no tail of short workgroups); with a window they are adjacent.
// Each wave owns 32 query rows of one head.
template <int D>
struct PF2 {
    static constexpr int NW = 8;
    static constexpr int BN = D <= 128 ? 64 : 32;   // keys per tile
    static constexpr int RB = D * 2;                // LDS bytes per key row
    static constexpr int SLOTS = D / 8;             // 16-byte slots per row
    static constexpr int RPI = 1024 / RB;           // rows per DMA instruction
    static constexpr int NI = BN / RPI;             // DMA instructions per K (or V) tile
    static constexpr int NIW = NI / NW;             // ... per wave
    static constexpr int TILE = BN * RB;
    static constexpr int STAGE = 2 * TILE;
    static constexpr int NSTG = 3;
    static constexpr int NKT = BN / 32;             // 32-key MFMA tiles per tile
    static constexpr int NKS = D / 16;              // QK k-steps
    static constexpr int NDT = D / 32;              // output d tiles
    static_assert(NIW >= 1 && NI % NW == 0, "DMA split");
};

template <class T, int D>
__global__ __launch_bounds__(512) void prefill2_kernel(
    const uint16_t *__restrict__ q, const char *__restrict__ kc, const char *__restrict__ vc,
    int64_t kv_stride, int S, int start_pos, int window, int n_head, int kv_mul, int hw,
    int rw, int n_units, int ng, int np, int paired, float qscale, float *__restrict__ out) {
    using C = PF2<D>;
    constexpr int BN = C::BN, RB = C::RB, SLOTS = C::SLOTS, RPI = C::RPI, NIW = C::NIW;
    constexpr int TILE = C::TILE, STAGE = C::STAGE, NKT = C::NKT, NKS = C::NKS, NDT = C::NDT;
    constexpr bool CVTV = __is_same(T, BF16);  // bf16 V is widened to f16 in LDS
    __shared__ __attribute__((aligned(1024))) char lds[C::NSTG * STAGE];

    // ---- work assignment (XCD-aware: one unit's workgroups share an L2) ----
    const int total = n_units * np;
    const int per_xcd = (total + 7) / 8;
    const int t = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (t >= total) return;
    const int unit = t / np, pair = t % np;
    const int n_sub = kv_mul / hw;
    const int kvh = unit / n_sub;
    const int head0 = kvh * kv_mul + (unit % n_sub) * hw;
    const int gA = paired ? pair : 2 * pair;
    const int gB = paired ? ng - 1 - pair : 2 * pair + 1;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int half = wave >> 2, slot = wave & 3;
    const int kv_len = start_pos + S;

    // Key range of one wave (uniform): rows of block (group, slot).
    auto wave_rows = [&](int w, int &row0, int &lo, int &hi) {
        const int g = (w >> 2) ? gB : gA;
        const bool dup = (w >> 2) && gB == gA;
        row0 = (g * rw + (w & 3) / hw) * 32;
        if (g >= ng || dup || row0 >= S) { lo = 1 << 30; hi = -1; return; }
        hi = start_pos + min(row0 + 32, S);
        lo = window > 0 ? max(0, start_pos + row0 + 1 - window) : 0;
    };
    int lo = 1 << 30, hi = -1;
#pragma unroll
    for (int w = 0; w < 8; w++) {
        int r0, l0, h0;
        wave_rows(w, r0, l0, h0);
        lo = min(lo, l0);
        hi = max(hi, h0);
    }
    int row0, wlo, whi;
    wave_rows(wave, row0, wlo, whi);
    const int head = head0 + slot % hw;
    const bool active = whi > 0;

    // ---- buffer resources (out-of-range reads return zero) ----
    const int rbg = (int)(kv_stride * 2);
    const int range = (kv_len - 1) * rbg + D * 2;
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(kc + (int64_t)kvh * D * 2), 0, range, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(vc + (int64_t)kvh * D * 2), 0, range, kRsrcWord3);

    // DMA lane map: this wave writes instructions wave*NIW + i of each tile.
    int dofs[NIW];
#pragma unroll
    for (int i = 0; i < NIW; i++) {
        const int r = (wave * NIW + i) * RPI + lane / SLOTS;
        dofs[i] = r * rbg + (((lane % SLOTS) ^ (r & (SLOTS - 1))) * 16);
    }
    const int kt0 = hi > 0 ? (max(lo, 0) / BN) : 0;
    const int nt = hi > 0 ? (hi + BN - 1) / BN - kt0 : 0;
    auto issue = [&](int tt) {
        const int so = __builtin_amdgcn_readfirstlane((kt0 + tt) * BN * rbg);
        char *st = lds + (tt % C::NSTG) * STAGE;
#pragma unroll
        for (int i = 0; i < NIW; i++) {
            dma16(krs, st + (wave * NIW + i) * 1024, dofs[i] + so, 0);
            dma16(vrs, st + TILE + (wave * NIW + i) * 1024, dofs[i] + so, 0);
        }
    };

    // ---- Q rows of this wave: B operand, d = s*16 + (lane/32)*8 + j ----
    const int c32 = lane & 31, h2 = lane >> 5;
    const int64_t q_dim = (int64_t)n_head * D;
    u32x4 qreg[NKS];
    {
        const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc(
            uniform_ptr(q), 0, (int)((int64_t)S * q_dim * 2), kRsrcWord3);
        const int qo = (int)(((int64_t)(row0 + c32) * q_dim + (int64_t)head * D + h2 * 8) * 2);
#pragma unroll
        for (int s = 0; s < NKS; s++)
            qreg[s] = active ? __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                   qrs, qo + s * 32, 0, 0))
                             : u32x4{0, 0, 0, 0};
    }
    const int pos_row = start_pos + row0 + c32;

    f32x16 oacc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; i++) oacc[i] = f32x16{};
    float m_run = -INFINITY, l_part = 0.f;

    // bf16 -> f16 of one V tile in LDS: each thread widens 16-byte chunks
    // (exact for |v| < 65504: bf16's 8-bit mantissa fits f16's 11 bits).
    auto widen_v = [&](int tt) {
        if constexpr (CVTV) {
            const uint32_t vb = lds_addr(lds + (tt % C::NSTG) * STAGE + TILE);
            constexpr int CH = TILE / 16 / (C::NW * 64);  // chunks per thread
            u32x4 w[CH];
#pragma unroll
            for (int c = 0; c < CH; c++) w[c] = lds_read_b128(vb + (c * C::NW * 64 + tid) * 16);
            lds_wait_any();
#pragma unroll
            for (int c = 0; c < CH; c++) {
                tie(w[c]);
                u32x4 o;
#pragma unroll
                for (int j = 0; j < 4; j++) o[j] = pack_f16x2(bf16_lo(w[c][j]), bf16_hi(w[c][j]));
                lds_write_b128(vb + (c * C::NW * 64 + tid) * 16, o);
            }
        }
    };
    // Ring: tiles tt+1 and tt+2 are in flight while tile tt computes; the V of
    // tile tt+1 is widened during iteration tt, before the barrier that
    // publishes it.
    if (nt > 0) {
        issue(0);
        issue(1);
        __builtin_amdgcn_s_waitcnt(vm_wait(2 * NIW));  // own DMA of tile 0 landed
        wg_barrier();
        widen_v(0);  // published by the first barrier of the loop
    }
    for (int tt = 0; tt < nt; tt++) {
        // own DMA of tile tt+1 landed and own LDS writes (widened V) retired
        __builtin_amdgcn_s_waitcnt(vm_wait(0) & ~(15 << 8));
        wg_barrier();  // tile tt+1 landed everywhere; V(tt) widened; tile tt-1 consumed
        issue(tt + 2);
        widen_v(tt + 1);
        const int kb = (kt0 + tt) * BN;
        if (!active || kb >= whi || kb + BN <= wlo) continue;
        const char *kt_ = lds + (tt % C::NSTG) * STAGE, *vt_ = kt_ + TILE;
        const uint32_t kbase = lds_addr(kt_), vbase = lds_addr(vt_);

        // ---- S^T = K . Q^T ----
        f32x16 sacc[NKT];
#pragma unroll
        for (int kt = 0; kt < NKT; kt++) {
            const int r = kt * 32 + c32;
            u32x4 ka[NKS];
#pragma unroll
            for (int s = 0; s < NKS; s++)
                ka[s] = lds_read_b128(kbase + r * RB + (((s * 2 + h2) ^ (r & (SLOTS - 1))) * 16));
            lds_wait_any();
#pragma unroll
            for (int s = 0; s < NKS; s++) tie(ka[s]);
            sacc[kt] = f32x16{};
#pragma unroll
            for (int s = 0; s < NKS; s++) sacc[kt] = mfma32<T>(ka[s], qreg[s], sacc[kt]);
        }

        // ---- online softmax (lane = query row c32; keys (i/4)*8 + h2*4 + i%4) ----
        // Scores stay unscaled; qscale > 0 so the max commutes with scaling,
        // and scaling is folded into the exp2 argument (one FMA per score).
        const bool need_mask = (kb + BN - 1 > start_pos + row0) ||
                               (window > 0 && kb <= start_pos + row0 + 31 - window);
        if (need_mask) {
#pragma unroll
            for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int key = kb + kt * 32 + (i >> 2) * 8 + h2 * 4 + (i & 3);
                    const bool dead = key > pos_row || (window > 0 && key <= pos_row - window);
                    sacc[kt][i] = dead ? -INFINITY : sacc[kt][i];
                }
        }
        float mloc = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < NKT; kt++)
#pragma unroll
            for (int i = 0; i < 16; i++) mloc = fmaxf(mloc, sacc[kt][i]);
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64)) * qscale;
        const float m_new = fmaxf(m_run, mloc);
        const float mu = m_new == -INFINITY ? 0.f : m_new;
        if (__any(m_new != m_run)) {
            const float corr = __builtin_amdgcn_exp2f(m_run - mu);
            l_part *= corr;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) oacc[dt] *= corr;
        }
        m_run = m_new;
        u32x4 ph[NKT][2];
#pragma unroll
        for (int kt = 0; kt < NKT; kt++)
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kt][ks * 8 + 2 * jj], qscale, -mu));
                    const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kt][ks * 8 + 2 * jj + 1], qscale, -mu));
                    l_part += p0 + p1;
                    ph[kt][ks][jj] = pack_f16x2(p0, p1);
                }

        // ---- O^T += V^T . P^T: two transposing reads per 16-key k-step ----
        const int g16 = lane >> 4, i16 = lane & 15, hh = g16 >> 1;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            const int e0 = dt * 32 + (g16 & 1) * 16 + 4 * (i16 & 3);
            const int chq = e0 >> 3, boff = (e0 & 7) * 2;
            u32x4 va[NKT][2];
#pragma unroll
            for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                for (int ks = 0; ks < 2; ks++) {
                    const int R0 = kt * 32 + ks * 16 + hh * 4 + (i16 >> 2);
                    const int R1 = R0 + 8;
                    const u32x2 a0 = lds_read_tr16_b64(vbase + R0 * RB + ((chq ^ (R0 & (SLOTS - 1))) * 16) + boff);
                    const u32x2 a1 = lds_read_tr16_b64(vbase + R1 * RB + ((chq ^ (R1 & (SLOTS - 1))) * 16) + boff);
                    va[kt][ks] = u32x4{a0[0], a0[1], a1[0], a1[1]};
                }
            lds_wait_any();
#pragma unroll
            for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                for (int ks = 0; ks < 2; ks++) {
                    tie(va[kt][ks]);
                    oacc[dt] = mfma32<F16>(va[kt][ks], ph[kt][ks], oacc[dt]);
                }
        }
    }
    __builtin_amdgcn_s_waitcnt(vm_wait(0));  // no DMA may outlive the workgroup

    if (!active) return;
    const float l_tot = l_part + __shfl_xor(l_part, 32, 64);
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    const int qrow = row0 + c32;
    if (qrow >= S) return;
    float *op = out + (int64_t)qrow * q_dim + (int64_t)head * D + h2 * 4;
#pragma unroll
    for (int dt = 0; dt < NDT; dt++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            f32x4 v = {oacc[dt][g * 4] * inv, oacc[dt][g * 4 + 1] * inv, oacc[dt][g * 4 + 2] * inv,
                       oacc[dt][g * 4 + 3] * inv};
            *(f32x4 *)(op + dt * 32 + g * 8) = v;
        }
}

// ---------------------------------------------------------------------------
// Prefill v4 (head_dim <= 128, GQA groups of 4k heads, no binding window):
// split-K inside the workgroup so that both waves of every SIMD compute at
// every step.
//
// A workgroup owns 4 heads of one kv head and the causal pair of 32-row
// blocks A = g, B = NG-1-g.  The key tiles stream in the rotated order
// 0..TB-1, 0..TA-1 (A on tiles [0, TA), B on [TA, TB) then [0, TA): the online
// softmax is order-free), two stream positions per step: set 0 (waves 0-3)
// takes the even positions and set 1 (waves 4-7) the odd ones, each wave
// keeping its own (m, l, O) for the same 32 query rows of one head.  When a
// block is done, set 1 hands its partial over -- O/l into the output rows,
// (m, l) through LDS -- and set 0 merges at the next step.  Every workgroup
// streams TA+TB tiles, a constant for the causal pair, and no SIMD runs a
// lone wave.
//
// LDS: K tiles of the 4 ring stages at [0, 4 TILE), V tiles at
// [4 TILE, 8 TILE).  A wave of set s only reads stages s and s+2, so every
// per-lane LDS address is fixed at start and the stage, key-row and k-step
// parts go into the instructions' immediate offsets.  Each wave widens (bf16
// -> f16) exactly the V bytes its own DMA wrote, so one barrier per step
// orders DMA, widening and reads.
//
// The running max is raised only when a row's tile max exceeds it by more
// than 2^8 (in the exp2 domain): P = exp2(s - m) then stays <= 256, exact in
// f16's range, and the O/l rescale runs a handful of times per block instead
// of on every new maximum.
template <class T, int D>
__global__ __launch_bounds__(512) void prefill4_kernel(
    const uint16_t *__restrict__ q, const char *__restrict__ kc, const char *__restrict__ vc,
    int64_t kv_stride, int S, int start_pos, int n_head, int kv_mul, int ng, int np,
    float qscale, float *__restrict__ out) {
    using C = PF2<D>;
    constexpr int BN = C::BN, RB = C::RB, SLOTS = C::SLOTS, RPI = C::RPI, NIW = C::NIW;
    constexpr int TILE = C::TILE, NKT = C::NKT, NKS = C::NKS, NDT = C::NDT;
    constexpr int NSTG = 4, VREG = NSTG * TILE;
    constexpr bool CVTV = __is_same(T, BF16);
    constexpr float kLazy = 8.0f;  // log2 headroom before the max is raised
    static_assert(D <= 128 && BN == 64, "v4 tiling");
    static_assert(2 * TILE + (NKT * 32) * RB <= 65535, "immediate offsets");
    // 16-byte slot swizzle of key row r.  A 256-byte row (D = 128) spans all
    // 64 banks, so the four rows one 16-lane transpose read touches must land
    // on different slot pairs: XOR with 2r, not r.  128-byte rows (D = 64)
    // alternate bank halves and use r itself.
    auto swz = [](int r) { return D == 128 ? (r << 1) & (SLOTS - 1) : r & (SLOTS - 1); };
    __shared__ __attribute__((aligned(1024))) char lds[2 * VREG];
    __shared__ float hand_ml[2][4][32][2];

    const int n_units = (n_head / kv_mul) * (kv_mul / 4);
    const int total = n_units * np;
    const int per_xcd = (total + 7) / 8;
    const int tsk = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (tsk >= total) return;
    const int unit = tsk / np, pair = tsk % np;
    const int kvh = unit / (kv_mul / 4);
    const int head0 = kvh * kv_mul + (unit % (kv_mul / 4)) * 4;
    const int gA = pair, gB = ng - 1 - pair != pair ? ng - 1 - pair : -1;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int set = wave >> 2, slot = wave & 3;
    const int c32 = lane & 31, h2 = lane >> 5;
    const int kv_len = start_pos + S;
    const int64_t q_dim = (int64_t)n_head * D;
    const int head = head0 + slot;

    const int rowA = gA * 32, rowB = gB >= 0 ? gB * 32 : S;
    auto tiles_hi = [&](int row) {
        return row < S ? (start_pos + min(row + 32, S) + BN - 1) / BN : 0;
    };
    const int TA = tiles_hi(rowA), TB = tiles_hi(rowB);
    const int TB1 = max(TB, TA);
    const int P = TB1 + (TB > 0 ? TA : 0);
    auto stream_tile = [&](int p) { return p < TB1 ? p : p - TB1; };
    auto task_blk = [&](int p) {  // 0 = A, 1 = B, -1 = idle
        if (p >= P) return -1;
        const int t = stream_tile(p);
        if (p < TB1) return t < TA ? 0 : (t < TB ? 1 : -1);
        return t < TA ? 1 : -1;
    };

    // ---- K/V DMA (each wave loads NIW 1 KiB chunks of every K and V tile) ----
    const int rbg = (int)(kv_stride * 2);
    const int range = (kv_len - 1) * rbg + D * 2;
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(kc + (int64_t)kvh * D * 2), 0, range, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(vc + (int64_t)kvh * D * 2), 0, range, kRsrcWord3);
    int dofs[NIW];
#pragma unroll
    for (int i = 0; i < NIW; i++) {
        const int r = (wave * NIW + i) * RPI + lane / SLOTS;
        dofs[i] = r * rbg + (((lane % SLOTS) ^ swz(r)) * 16);
    }
    auto issue = [&](int p) {
        const int t = p < P ? stream_tile(p) : (kv_len + BN) / BN;  // past P: zeros
        const int so = t * BN * rbg;
        char *st = lds + (p % NSTG) * TILE;
#pragma unroll
        for (int i = 0; i < NIW; i++) {
            dma16(krs, st + (wave * NIW + i) * 1024, dofs[i] + so, 0);
            dma16(vrs, st + VREG + (wave * NIW + i) * 1024, dofs[i] + so, 0);
        }
    };
    auto widen_own = [&](int p) {
        if constexpr (CVTV) {
            const uint32_t vb = lds_addr(lds + VREG + (p % NSTG) * TILE) + wave * NIW * 1024 + lane * 16;
            u32x4 w[NIW];
#pragma unroll
            for (int i = 0; i < NIW; i++) w[i] = lds_read_b128(vb + i * 1024);
            lds_wait_any();
#pragma unroll
            for (int i = 0; i < NIW; i++) {
                tie(w[i]);
                u32x4 o;
#pragma unroll
                for (int j = 0; j < 4; j++) o[j] = pack_f16x2(bf16_lo(w[i][j]), bf16_hi(w[i][j]));
                lds_write_b128(vb + i * 1024, o);
            }
        }
    };

    // ---- fixed per-lane LDS read addresses (stage `set`, key row 0) ----
    const uint32_t lds0 = lds_addr(lds);
    uint32_t ka_addr[NKS];
#pragma unroll
    for (int s = 0; s < NKS; s++)
        ka_addr[s] = lds0 + set * TILE + c32 * RB + (((s * 2 + h2) ^ swz(c32)) * 16);
    const int g16 = lane >> 4, i16 = lane & 15;
    uint32_t va_addr[NDT][2];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int e0 = dt * 32 + (g16 & 1) * 16 + 4 * (i16 & 3);
            const int chq = e0 >> 3, boff = (e0 & 7) * 2;
            const int R = (g16 >> 1) * 4 + (i16 >> 2) + h * 8;
            va_addr[dt][h] = lds0 + VREG + set * TILE + R * RB + ((chq ^ swz(R)) * 16) + boff;
        }

    // ---- Q of the block being computed (reloaded once, at the A -> B switch) ----
    const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(q), 0, (int)((int64_t)S * q_dim * 2), kRsrcWord3);
    u32x4 qv[NKS];
    auto load_q = [&](int row) {
        const int o = (int)((min(row + c32, S) * q_dim + (int64_t)head * D + h2 * 8) * 2);
#pragma unroll
        for (int s = 0; s < NKS; s++)
            qv[s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qrs, o + s * 32, 0, 0));
    };

    f32x16 oacc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; i++) oacc[i] = f32x16{};
    float m_run = -INFINITY, l_part = 0.f;

    auto compute = [&](auto par, int p, int blk) {
        constexpr int SOFF = decltype(par)::value * 2 * TILE;  // stage s or s+2
        const int row = blk ? rowB : rowA;
        const int kb = stream_tile(p) * BN;
        f32x16 sacc[NKT];
        static_for<0, NKT>([&](auto ktc) {
            constexpr int kt = decltype(ktc)::value;
            u32x4 ka[NKS];
            static_for<0, NKS>([&](auto sc) {
                constexpr int s = decltype(sc)::value;
                ka[s] = lds_read_b128_at<SOFF + kt * 32 * RB>(ka_addr[s]);
            });
            lds_wait_any();
            sacc[kt] = f32x16{};
#pragma unroll
            for (int s = 0; s < NKS; s++) {
                tie(ka[s]);
                sacc[kt] = mfma32<T>(ka[s], qv[s], sacc[kt]);
            }
        });
        const int pos_row = start_pos + row + c32;
        if (kb + BN - 1 > start_pos + row) {  // tile reaches past the block's first row
#pragma unroll
            for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int key = kb + kt * 32 + (i >> 2) * 8 + h2 * 4 + (i & 3);
                    sacc[kt][i] = key > pos_row ? -INFINITY : sacc[kt][i];
                }
        }
        float mloc = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < NKT; kt++)
#pragma unroll
            for (int i = 0; i < 16; i++) mloc = fmaxf(mloc, sacc[kt][i]);
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64)) * qscale;
        if (__any(mloc > m_run + kLazy)) {
            const float m_new = fmaxf(m_run, mloc);
            const float corr = __builtin_amdgcn_exp2f(m_run - (m_new == -INFINITY ? 0.f : m_new));
            l_part *= corr;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) oacc[dt] *= corr;
            m_run = m_new;
        }
        const float mu = m_run == -INFINITY ? 0.f : m_run;
        u32x4 ph[NKT][2];
#pragma unroll
        for (int kt = 0; kt < NKT; kt++)
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kt][ks * 8 + 2 * jj], qscale, -mu));
                    const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kt][ks * 8 + 2 * jj + 1], qscale, -mu));
                    l_part += p0 + p1;
                    ph[kt][ks][jj] = pack_f16x2(p0, p1);
                }
        static_for<0, NDT>([&](auto dtc) {
            constexpr int dt = decltype(dtc)::value;
            u32x4 va[NKT][2];
            static_for<0, NKT>([&](auto ktc) {
                constexpr int kt = decltype(ktc)::value;
                static_for<0, 2>([&](auto ksc) {
                    constexpr int ks = decltype(ksc)::value;
                    constexpr int off = SOFF + (kt * 32 + ks * 16) * RB;
                    const u32x2 a0 = lds_read_tr16_b64_at<off>(va_addr[dt][0]);
                    const u32x2 a1 = lds_read_tr16_b64_at<off>(va_addr[dt][1]);
                    va[kt][ks] = u32x4{a0[0], a0[1], a1[0], a1[1]};
                });
            });
            lds_wait_any();
#pragma unroll
            for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                for (int ks = 0; ks < 2; ks++) {
                    tie(va[kt][ks]);
                    oacc[dt] = mfma32<F16>(va[kt][ks], ph[kt][ks], oacc[dt]);
                }
        });
    };

    auto reset = [&]() {
#pragma unroll
        for (int i = 0; i < NDT; i++) oacc[i] = f32x16{};
        m_run = -INFINITY;
        l_part = 0.f;
    };
    // Set 1 hands its partial of block `b` to set 0: O/l into the output rows
    // (f32), (m, l) into LDS.
    auto hand_over = [&](int b) {
        const int row = b ? rowB : rowA;
        const float l_tot = l_part + __shfl_xor(l_part, 32, 64);
        const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
        const int qrow = row + c32;
        if (h2 == 0) { hand_ml[b][slot][c32][0] = m_run; hand_ml[b][slot][c32][1] = l_tot; }
        if (qrow < S) {
            float *op = out + (int64_t)qrow * q_dim + (int64_t)head * D + h2 * 4;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                for (int g = 0; g < 4; g++)
                    *(f32x4 *)(op + dt * 32 + g * 8) =
                        f32x4{oacc[dt][g * 4] * inv, oacc[dt][g * 4 + 1] * inv,
                              oacc[dt][g * 4 + 2] * inv, oacc[dt][g * 4 + 3] * inv};
        }
        reset();
    };
    // Set 0 merges the handed-over partial of block `b` with its own and
    // writes the result.
    auto merge_out = [&](int b) {
        const int row = b ? rowB : rowA;
        const float l0 = l_part + __shfl_xor(l_part, 32, 64);
        const float m1 = hand_ml[b][slot][c32][0], l1 = hand_ml[b][slot][c32][1];
        const float M = fmaxf(m_run, m1);
        const float mu = M == -INFINITY ? 0.f : M;
        const float a0 = __builtin_amdgcn_exp2f(m_run - mu), a1 = __builtin_amdgcn_exp2f(m1 - mu);
        const float den = l0 * a0 + l1 * a1;
        const float inv = den > 0.f ? 1.0f / den : 0.f;
        const float w1 = l1 * a1 * inv, w0 = a0 * inv;
        const int qrow = row + c32;
        if (qrow < S) {
            float *op = out + (int64_t)qrow * q_dim + (int64_t)head * D + h2 * 4;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const f32x4 o1 = __builtin_nontemporal_load((const f32x4 *)(op + dt * 32 + g * 8));
                    *(f32x4 *)(op + dt * 32 + g * 8) =
                        f32x4{oacc[dt][g * 4] * w0 + o1[0] * w1, oacc[dt][g * 4 + 1] * w0 + o1[1] * w1,
                              oacc[dt][g * 4 + 2] * w0 + o1[2] * w1, oacc[dt][g * 4 + 3] * w0 + o1[3] * w1};
                }
        }
        reset();
    };

    const int nj = (P + 1) / 2;
    const int jA = (TA - 1) / 2;  // step in which block A's last tile is computed
    int qblk = task_blk(set) == 1 ? 1 : 0;
    load_q(qblk ? rowB : rowA);
    issue(0);
    issue(1);
    __builtin_amdgcn_s_waitcnt(vm_wait(0));
    widen_own(0);
    widen_own(1);
    auto step = [&](auto par, int j) {
        __builtin_amdgcn_s_waitcnt(vm_wait(63) & ~(15 << 8));  // own LDS writes done
        wg_barrier();  // positions 2j, 2j+1 ready everywhere; 2j-2, 2j-1 consumed
        issue(2 * j + 2);
        issue(2 * j + 3);
        if (set == 0 && j == jA + 1) merge_out(0);
        const int p = 2 * j + set;
        const int blk = task_blk(p);
        if (set == 1 && j == jA && blk != 0) hand_over(0);
        if (blk >= 0) compute(par, p, blk);
        if (set == 1 && j == jA && blk == 0) hand_over(0);
        const int nb = task_blk(p + 2);
        if (nb >= 0 && nb != qblk) {
            qblk = nb;
            load_q(nb ? rowB : rowA);
        }
        __builtin_amdgcn_s_waitcnt(vm_wait(0));  // DMA of 2j+2, 2j+3, Q and stores retired
        widen_own(2 * j + 2);
        widen_own(2 * j + 3);
    };
    for (int j = 0; j < nj; j += 2) {
        step(Int<0>{}, j);
        if (j + 1 < nj) step(Int<1>{}, j + 1);
    }
    if (set == 1 && gB >= 0) hand_over(1);
    __builtin_amdgcn_s_waitcnt(vm_wait(0) & ~(15 << 8));
    wg_barrier();
    if (set == 0) {
        if (jA + 1 == nj) merge_out(0);
        if (gB >= 0) merge_out(1);
    }
}

// head_dim 256 keeps the register-staged kernel (the LDS-ring variant needs
// more than the 256 registers two waves per SIMD allow).
template <class T, int D, bool V2 = (D <= 128)>
struct PrefillLaunch {
    static void run(const void *q, const void *kc, const void *vc, int64_t kvs, int S, int sp,
                    int win, int nh, int kv_mul, float qs, float *out, hipStream_t st) {
        const int nqb = (S + PrefillCfg<D>::BM - 1) / PrefillCfg<D>::BM;
        const int total = nh * nqb;
        const int per_xcd = (total + 7) / 8;
        hipLaunchKernelGGL((prefill_kernel<T, D>), dim3(per_xcd * 8), dim3(256), 0, st,
                           (const uint16_t *)q, (const uint16_t *)kc, (const uint16_t *)vc, kvs,
                           S, sp, win, nh, kv_mul, qs, out);
    }
};
template <class T, int D>
struct PrefillLaunch<T, D, true> {
    static void run(const void *q, const void *kc, const void *vc, int64_t kvs, int S, int sp,
                    int win, int nh, int kv_mul, float qs, float *out, hipStream_t st);
};

template <class T, int D>
void PrefillLaunch<T, D, true>::run(const void *q, const void *kc, const void *vc, int64_t kvs,
                                    int S, int sp, int win, int nh, int kv_mul, float qs,
                                    float *out, hipStream_t st) {
    // Units of HW heads (HW | kv_mul, at most 4) x groups of RW = 4/HW 32-row blocks.
    const int hw = kv_mul % 4 == 0 ? 4 : (kv_mul % 2 == 0 ? 2 : 1);
    const int rw = 4 / hw;
    const int n_units = (nh / kv_mul) * (kv_mul / hw);
    const int ng = (S + 32 * rw - 1) / (32 * rw);
    const int np = (ng + 1) / 2;
    // Without an effective window the causal work of group g grows with g, so
    // a workgroup takes g and ng-1-g; with a window it takes 2g and 2g+1.
    const int paired = !(win > 0 && win < sp + S);
    const int total = n_units * np;
    const int per_xcd = (total + 7) / 8;
    if (D <= 128 && kv_mul % 4 == 0 && paired) {
        hipLaunchKernelGGL((prefill4_kernel<T, D>), dim3(per_xcd * 8), dim3(512), 0, st,
                           (const uint16_t *)q, (const char *)kc, (const char *)vc, kvs, S, sp,
                           nh, kv_mul, ng, np, qs, out);
        return;
    }
    hipLaunchKernelGGL((prefill2_kernel<T, D>), dim3(per_xcd * 8), dim3(512), 0, st,
                       (const uint16_t *)q, (const char *)kc, (const char *)vc, kvs, S, sp, win,
                       nh, kv_mul, hw, rw, n_units, ng, np, paired, qs, out);
}

template <class T, int D>
static int launch_prefill(const void *q, const void *kc, const void *vc, int64_t kvs, int S,
                          int sp, int win, int nh, int kv_mul, float qs, float *out,
                          hipStream_t st) {
    PrefillLaunch<T, D>::run(q, kc, vc, kvs, S, sp, win, nh, kv_mul, qs, out, st);
    return check_hip(hipGetLastError(), "prefill launch");
}

template <class T>
static int dispatch_prefill(int D, const void *q, const void *kc, const void *vc, int64_t kvs,
                            int S, int sp, int win, int nh, int kv_mul, float qs, float *out,
                            hipStream_t st) {
    switch (D) {
        case 64: return launch_prefill<T, 64>(q, kc, vc, kvs, S, sp, win, nh, kv_mul, qs, out, st);
        case 128: return launch_prefill<T, 128>(q, kc, vc, kvs, S, sp, win, nh, kv_mul, qs, out, st);
        case 256: return launch_prefill<T, 256>(q, kc, vc, kvs, S, sp, win, nh, kv_mul, qs, out, st);
        default: return set_error(ULLM_HIP_E_UNSUPPORTED, "prefill: head_dim %d not in {64,128,256}", D);
    }
}

}  // namespace ullm

using namespace ullm;

extern "C" int ullm_hip_attn_prefill(const void *q, const void *k_cache, const void *v_cache,
                                     int dtype, int64_t kv_stride, int S, int start_pos,
                                     int window, int n_head, int n_kv_head, int head_dim,
                                     float scale, float *out, void *stream) {
    if (dtype != ULLM_DT_F16 && dtype != ULLM_DT_BF16)
        return set_error(ULLM_HIP_E_UNSUPPORTED, "prefill: dtype %d (MFMA path takes f16/bf16)", dtype);
    if (n_head < 1 || n_kv_head < 1 || n_head % n_kv_head || S < 0 || start_pos < 0)
        return set_error(ULLM_HIP_E_INVALID, "prefill: bad shape S=%d start_pos=%d heads=%d/%d", S,
                         start_pos, n_head, n_kv_head);
    if (head_dim != 64 && head_dim != 128 && head_dim != 256)
        return set_error(ULLM_HIP_E_UNSUPPORTED, "prefill: head_dim %d not in {64,128,256}", head_dim);
    if (kv_stride < (int64_t)n_kv_head * head_dim || (kv_stride * 2) % 16)
        return set_error(ULLM_HIP_E_INVALID, "prefill: kv_stride must be >= n_kv_head*head_dim and 16-byte aligned");
    if (S == 0) return ULLM_HIP_OK;
    if (!q || !k_cache || !v_cache || !out)
        return set_error(ULLM_HIP_E_INVALID, "prefill: null tensor pointer");
    if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out) & 15)
        return set_error(ULLM_HIP_E_INVALID, "prefill: tensors must be 16-byte aligned");
    const float qs = scale * kLog2e;
    const int kv_mul = n_head / n_kv_head;
    hipStream_t st = (hipStream_t)stream;
    if (dtype == ULLM_DT_BF16)
        return dispatch_prefill<BF16>(head_dim, q, k_cache, v_cache, kv_stride, S, start_pos, window, n_head, kv_mul, qs, out, st);
    return dispatch_prefill<F16>(head_dim, q, k_cache, v_cache, kv_stride, S, start_pos, window, n_head, kv_mul, qs, out, st);
}
