// Causal multi-token prefill attention on CDNA4 MFMA (gfx950).
//
// Computes, for query row s at pos = start_pos + s and head h (kv head
// h / kv_mul), out[s,h] = softmax_t(scale * q[s,h] . K[t]) . V[t] over
// t in start..pos (start = 0, or the sliding-window start) -- the CPU
// reference loop crates/ullm-model/src/lib.rs:1061-1087, with the window rule
// of lib.rs:1183-1186 applied per row as the Metal kernel does
// (shader.metal:1051).
//
// Three kernels, all with f32 softmax statistics and accumulators, the
// online softmax in the exp2 domain (scale*log2(e) folded into one multiply),
// QK^T on v_mfma_f32_32x32x16_{bf16,f16} and P.V on the f16 variant (P and a
// bf16 V rounded to f16: 2^-11 relative, where bf16 P would cost 2^-8):
//  * prefill16_kernel (prefill16.hip) for head_dim 256, and for head_dim 128
//    when a prompt is too short for prefill4_kernel's pairs to fill the chip;
//  * prefill4_kernel (head_dim <= 128, no binding window): 8-wave
//    workgroups over a pair of causal row blocks, split-K between two
//    4-wave sets, K/V tiles shared through an LDS ring filled by DMA;
//  * prefill2_kernel (head_dim <= 128, binding sliding window): the same
//    staging without the split;
//  * prefill_sk_kernel (head_dim 256): one 32-row block of one head per
//    workgroup, split-K over its 4 waves, merged through LDS.  Kept as a
//    comparison point (ULLM_HIP_PREFILL256=1): head_dim 256 runs
//    prefill16_kernel (prefill16.hip), faster at every measured shape.
// In every kernel the S^T = K.Q^T accumulator holds ONE query row per lane
// (lane % 32) and 16 keys, so the row max needs a single cross-lane exchange
// (lane ^ 32); exponentiated and rounded to f16 it IS the B operand of
// O^T += V^T.P^T (the keys' order inside a k-step is free, so V^T is read
// from LDS in the accumulator's key order).  Work is dealt to the 8 XCDs so
// that the query heads of one kv head share an XCD's L2 (workgroup i runs on
// XCD i % 8).
#include "common.hpp"
#include "mfma_util.hpp"
#include "wave.hpp"

namespace ullm {

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
// 16-byte slot swizzle of key row r in an LDS K/V tile (slot p of row r
// holds chunk p ^ kv_swz(r)); LDS serves 64 banks x 4 bytes per cycle.  Two
// read patterns must be conflict-free:
//  * K operand, ds_read_b128, taken 16 lanes (256 bytes) per cycle: 16
//    consecutive rows reading the same chunk, so kv_swz must be a bijection
//    on 16 rows (on the 8 rows of one parity for D = 64, two rows per bank
//    line);
//  * V^T operand, ds_read_b64_tr_b16, taken 32 lanes (256 bytes) per cycle:
//    an aligned group of 4 rows x the same 4 chunks (one 64-byte quarter of
//    a 256-byte line), so the 4 rows must land in 4 different quarters.
// D = 128 and 256 (every row starts a bank line): bits 2-3 <- r bits 0-1
// (the quarter), bits 0-1 <- r bits 2-3 (the bijection).  D = 64 (rows r and
// r+1 share a line): bit 2 <- r bit 1, bits 0-1 <- r bits 2-3.  Measured in
// isolation: the transposing reads run at 147 TB/s chip-wide with this
// swizzle against 77 TB/s (two conflict cycles per read) with a swizzle
// that spread the rows over chunk pairs.
template <int D>
__device__ __forceinline__ int kv_swz(int r) {
    if constexpr (D >= 128) return ((r & 3) << 2) | ((r >> 2) & 3);
    else return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
}

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
    int rw, int n_units, int ng, int np, int paired, float qscale, float *__restrict__ out,
    KvPages pgs) {
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
    const int slot = wave & 3;
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
        dofs[i] = r * rbg + (((lane % SLOTS) ^ kv_swz<D>(r)) * 16);
    }
    const int kt0 = hi > 0 ? (max(lo, 0) / BN) : 0;
    const int nt = hi > 0 ? (hi + BN - 1) / BN - kt0 : 0;
    auto issue = [&](int tt) {
        __amdgpu_buffer_rsrc_t kr = krs, vr = vrs;
        int so;
        if (pgs.tab) page_tile<D>(pgs, kc, vc, kvh, rbg, kv_len, (kt0 + tt) * BN, kr, vr, so);
        else so = __builtin_amdgcn_readfirstlane((kt0 + tt) * BN * rbg);
        char *st = lds + (tt % C::NSTG) * STAGE;
#pragma unroll
        for (int i = 0; i < NIW; i++) {
            dma16(kr, st + (wave * NIW + i) * 1024, dofs[i] + so, 0);
            dma16(vr, st + TILE + (wave * NIW + i) * 1024, dofs[i] + so, 0);
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
                ka[s] = lds_read_b128(kbase + r * RB + (((s * 2 + h2) ^ kv_swz<D>(r)) * 16));
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
        float m4[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};  // independent chains
#pragma unroll
        for (int kt = 0; kt < NKT; kt++)
#pragma unroll
            for (int i = 0; i < 16; i++) m4[i & 3] = fmaxf(m4[i & 3], sacc[kt][i]);
        float mloc = fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]));
        mloc = fmaxf(mloc, xor32(mloc)) * qscale;
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
        float ls[4] = {0.f, 0.f, 0.f, 0.f};  // independent partial sums
#pragma unroll
        for (int kt = 0; kt < NKT; kt++)
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kt][ks * 8 + 2 * jj], qscale, -mu));
                    const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kt][ks * 8 + 2 * jj + 1], qscale, -mu));
                    ls[jj] += p0 + p1;
                    ph[kt][ks][jj] = pack_f16x2(p0, p1);
                }
        l_part += (ls[0] + ls[1]) + (ls[2] + ls[3]);

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
                    const u32x2 a0 = lds_read_tr16_b64(vbase + R0 * RB + ((chq ^ kv_swz<D>(R0)) * 16) + boff);
                    const u32x2 a1 = lds_read_tr16_b64(vbase + R1 * RB + ((chq ^ kv_swz<D>(R1)) * 16) + boff);
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
    const float l_tot = l_part + xor32(l_part);
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
// Prefill v4 (head_dim <= 128, no binding window; any GQA ratio):
// split-K inside the workgroup so that both waves of every SIMD compute at
// every step.
//
// A workgroup owns hw heads of one kv head (hw = 4, 2 or 1, the largest that
// divides the GQA ratio) and the causal pair of 32 * (4 / hw)-row blocks
// A = g, B = NG-1-g (TA and TB key tiles); the 4 waves of a set cover the
// hw heads x 4 / hw row groups of 32, all sharing each K/V tile.  Its TA+TB tile-units are
// cut into two streams (set 0 slightly longer): set 0 (waves 0-3) runs A's tiles [0, TA) and
// then B's tiles [TA, n0); set 1 (waves 4-7) runs B's tiles [n0, TB) and
// [0, TA).  Every wave keeps (m, l, O) for the 32 query rows of one head.
// A's output is written by set 0 as soon as its last tile is done; B's two
// partials (the online softmax is order-free) are merged once after the loop
// through the idle K/V ring, which also turns the MFMA-layout output into
// contiguous 2 KiB row stores.  The middle block of an odd block count (no
// partner) is split the same way.
//
// The sets are independent in the main loop: each loads its own stream into
// its own ring stages and synchronises its 4 waves with an LDS arrival
// counter, so one set's barrier, DMA and widening overlap the other's MFMAs.
// Per wave the loop is software-pipelined: step j computes exp(S_j) and the
// MFMAs of S_{j+1} = QK(j+1), then PV(j) and max(S_{j+1}); K is loaded two
// items ahead and V one.
//
// LDS: K tiles of the 4 ring stages at [0, 4 TILE), V tiles at
// [4 TILE, 8 TILE); set s's item i lives in stage 2 (i & 1) + s.  Every
// per-lane LDS address is therefore fixed at start and the stage, key-row and
// k-step parts go into the instructions' immediate offsets.  Each wave widens
// (bf16 -> f16) exactly the V bytes its own DMA wrote, so the one set barrier
// per step orders DMA, widening and reads.
//
// The running max is raised only when a row's tile max exceeds it by more
// than 2^8 (in the exp2 domain): P = exp2(s - m) then stays <= 256, exact in
// f16's range, and the O/l rescale runs a handful of times per block instead
// of on every new maximum.
template <class T, int D>
__global__ __launch_bounds__(512) void prefill4_kernel(
    const uint16_t *__restrict__ q, const char *__restrict__ kc, const char *__restrict__ vc,
    int64_t kv_stride, int S, int start_pos, int n_head, int kv_mul, int lhw, int ng, int np,
    float qscale, float *__restrict__ out, KvPages pgs) {
    using C = PF2<D>;
    constexpr int BN = C::BN, RB = C::RB, SLOTS = C::SLOTS, RPI = C::RPI, NIW = C::NIW;
    constexpr int TILE = C::TILE, NKT = C::NKT, NKS = C::NKS, NDT = C::NDT;
    constexpr int NSTG = 4, VREG = NSTG * TILE;
    constexpr bool CVTV = __is_same(T, BF16);
    constexpr float kLazy = 8.0f;  // log2 headroom before the max is raised
    constexpr int OROW = 4 * D * 4;  // bytes of staged output per 32-row group (4 heads of f32)
    static_assert(D <= 128 && BN == 64, "v4 tiling");
    static_assert(2 * TILE + (NKT * 32) * RB <= 65535, "immediate offsets");
    static_assert(4 * 64 * NDT * 64 + 32 * OROW <= 2 * VREG, "epilogue staging");
    auto swz = [](int r) { return kv_swz<D>(r); };
    __shared__ __attribute__((aligned(1024))) char lds[2 * VREG];
    __shared__ float hand_ml[4][32][2];
    __shared__ uint32_t set_bar[2];

    // A set's 4 waves cover hw heads x rw row groups of 32 (hw * rw = 4): a
    // "block" is 32 rw query rows of hw heads sharing one kv head.
    const int hw = 1 << lhw, rw = 4 >> lhw, BLK = 32 * rw;
    const int upk = kv_mul >> lhw;  // units per kv head
    const int n_units = (n_head / kv_mul) * upk;
    const int total = n_units * np;
    const int per_xcd = (total + 7) / 8;
    const int tsk = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (tsk >= total) return;
    const int unit = tsk / np, pair = tsk % np;
    const int kvh = unit / upk;
    const int head0 = kvh * kv_mul + (unit % upk) * hw;
    const int gA = pair, gB = ng - 1 - pair != pair ? ng - 1 - pair : -1;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int set = wave >> 2, slot = wave & 3;
    const int c32 = lane & 31, h2 = lane >> 5;
    const int kv_len = start_pos + S;
    const int64_t q_dim = (int64_t)n_head * D;
    const int head = head0 + (slot & (hw - 1));
    const int sub = (slot >> lhw) * 32;  // this wave's row offset inside the block

    // ---- the two tile streams ----
    const int rowA = gA * BLK, rowB = gB >= 0 ? gB * BLK : rowA;  // rowB: merged block
    const int TA = (start_pos + min(rowA + BLK, S) + BN - 1) / BN;
    const int TB = gB >= 0 ? (start_pos + min(rowB + BLK, S) + BN - 1) / BN : 0;
    const int n_tot = TA + TB;
    // Set 0 takes 34/64 of the tiles: set 1's waves are younger and lose
    // issue arbitration to set 0's, so its steps run ~15 % slower (measured
    // 1-3 % faster overall than an even split).  n0 >= TA holds (TA <= TB)
    // and n0 <= TB keeps set 1's first tile inside block B.
    const int n0 = min((n_tot * 34 + 63) / 64, gB >= 0 ? TB : n_tot);
    const int n1 = n_tot - n0;
    // item i of stream s -> key tile, and whether it belongs to block A
    // (only set 0 has A items when the block has a partner).
    auto item_tile = [&](int s_, int i) {
        if (gB < 0) return s_ ? n0 + i : i;
        if (s_ == 0) return i;
        const int t = n0 + i;
        return t < TB ? t : t - TB;
    };

    const int n_me = set ? n1 : n0;

    // ---- K/V DMA: each set loads its own stream, NIWS 1 KiB chunks per wave ----
    constexpr int NIWS = 2 * NIW;
    const int rbg = (int)(kv_stride * 2);
    const int range = (kv_len - 1) * rbg + D * 2;
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(kc + (int64_t)kvh * D * 2), 0, range, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(vc + (int64_t)kvh * D * 2), 0, range, kRsrcWord3);
    int dofs[NIWS];
#pragma unroll
    for (int i = 0; i < NIWS; i++) {
        const int r = (slot * NIWS + i) * RPI + lane / SLOTS;
        dofs[i] = r * rbg + (((lane % SLOTS) ^ swz(r)) * 16);
    }
    // Paged: buffer resources of the items in flight, by item parity.
    struct PageSlot { __amdgpu_buffer_rsrc_t k, v; int so; };
    PageSlot pslot[2] = {{krs, vrs, 0}, {krs, vrs, 0}};
    // This wave's chunks of item i of its set's stream: K (kv = 0) or V (kv = 1).
    auto load_tile = [&](int kv, int i) {
        const int t = i < n_me ? item_tile(set, i) : (kv_len + BN) / BN;  // past: zeros
        __amdgpu_buffer_rsrc_t kr = krs, vr = vrs;
        int so;
        if (pgs.tab) {
            // The page of item i is looked up once, when its K goes out; its
            // V (one step later) reuses it from the item's parity slot.
            PageSlot &ps = (i & 1) ? pslot[1] : pslot[0];
            if (kv == 0) page_tile<D>(pgs, kc, vc, kvh, rbg, kv_len, t * BN, ps.k, ps.v, ps.so);
            kr = ps.k;
            vr = ps.v;
            so = ps.so;
        } else {
            so = t * BN * rbg;
        }
        char *st = lds + kv * VREG + (2 * (i & 1) + set) * TILE + slot * NIWS * 1024;
#pragma unroll
        for (int c = 0; c < NIWS; c++) dma16(kv ? vr : kr, st + c * 1024, dofs[c] + so, 0);
    };
    // bf16 -> f16 in place, for the V chunks this wave loaded of item j + 1.
    auto widen_own = [&](int j) {
        if constexpr (CVTV) {
            const uint32_t vb = lds_addr(lds + VREG + (2 * ((j + 1) & 1) + set) * TILE) +
                                slot * NIWS * 1024 + lane * 16;
            u32x4 w[NIWS];
#pragma unroll
            for (int i = 0; i < NIWS; i++) w[i] = lds_read_b128(vb + i * 1024);
            lds_wait_any();
#pragma unroll
            for (int i = 0; i < NIWS; i++) {
                tie(w[i]);
                u32x4 o;
#pragma unroll
                for (int e = 0; e < 4; e++) o[e] = pack_f16x2(bf16_lo(w[i][e]), bf16_hi(w[i][e]));
                lds_write_b128(vb + i * 1024, o);
            }
        }
    };
    // Barrier of the 4 waves of this set (the sets run independently in the
    // main loop): a monotonic LDS arrival counter.  Callers have retired
    // their DMA (vmcnt) and LDS writes (lgkmcnt) before arriving.
    uint32_t bar_target = 0;
    auto set_barrier = [&]() {
        bar_target += 4;
        asm volatile("" ::: "memory");
        if (lane == 0)
            __hip_atomic_fetch_add(&set_bar[set], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        while (__hip_atomic_load(&set_bar[set], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < bar_target)
            __builtin_amdgcn_s_sleep(1);
        asm volatile("" ::: "memory");
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

    // ---- Q of the block being computed (set 0 reloads once, at A -> B) ----
    // Untracked loads: the reload at the A -> B switch would otherwise make
    // every QK MFMA wait for the step's K/V DMA.  Each load_q is followed by
    // a vmcnt(0) wait and tie_q before the next QK.
    const i32x4 qrs = raw_rsrc(q, (int)((int64_t)S * q_dim * 2));
    u32x4 qv[NKS];
    auto load_q = [&](int row) {
        const int o = (int)((min(row + sub + c32, S) * q_dim + (int64_t)head * D + h2 * 8) * 2);
#pragma unroll
        for (int s = 0; s < NKS; s++) qv[s] = buffer_load_b128_untracked(qrs, o + s * 32);
    };
    auto tie_q = [&]() {
#pragma unroll
        for (int s = 0; s < NKS; s++) tie(qv[s]);
    };

    f32x16 oacc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; i++) oacc[i] = f32x16{};
    float m_run = -INFINITY, l_part = 0.f;

    // S of two consecutive items: item i lives in s2[i & 1].
    f32x16 s2[2][NKT];
    u32x4 ph[NKT][2];  // P (f16) of the item awaiting PV
    // S = K Q^T of the item in K stage 2 KPAR + set, into s2[DST].  The K
    // reads run two groups of G ahead of the MFMAs that use them.
    auto qk = [&](auto kparc, auto dstc) {
        constexpr int SOFF = decltype(kparc)::value * 2 * TILE, DST = decltype(dstc)::value;
        constexpr int G = 4, NG = NKT * NKS / G;
        u32x4 kbuf[2][G];
        auto rd = [&](auto gc) {
            constexpr int g = decltype(gc)::value, kt = g * G / NKS, s0 = g * G % NKS;
            static_for<0, G>([&](auto ic) {
                constexpr int i = decltype(ic)::value;
                kbuf[g & 1][i] = lds_read_b128_at<SOFF + kt * 32 * RB>(ka_addr[s0 + i]);
            });
        };
        rd(Int<0>{});
        rd(Int<1>{});
        static_for<0, NG>([&](auto gc) {
            constexpr int g = decltype(gc)::value, kt = g * G / NKS, s0 = g * G % NKS;
            lds_wait_n<(g + 1 < NG ? G : 0)>();
            if constexpr (s0 == 0) s2[DST][kt] = f32x16{};
#pragma unroll
            for (int i = 0; i < G; i++) {
                tie(kbuf[g & 1][i]);
                s2[DST][kt] = mfma32<T>(kbuf[g & 1][i], qv[s0 + i], s2[DST][kt]);
            }
            if constexpr (g + 2 < NG) rd(Int<g + 2>{});
        });
    };
    // Causal mask of s2[SRC] for key tile `tile` and query block `row`
    // (only the tiles that reach past the block's first row need it).
    auto mask = [&](auto srcc, int row, int tile) {
        constexpr int SRC = decltype(srcc)::value;
        const int kb = tile * BN;
        if (kb + BN - 1 > start_pos + row + sub) {
            const int pos_row = start_pos + row + sub + c32;
#pragma unroll
            for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int key = kb + kt * 32 + (i >> 2) * 8 + h2 * 4 + (i & 3);
                    s2[SRC][kt][i] = key > pos_row ? -INFINITY : s2[SRC][kt][i];
                }
        }
    };
    // Row max of s2[SRC], in the exp2 domain.
    auto rowmax = [&](auto srcc) {
        constexpr int SRC = decltype(srcc)::value;
        float m4[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};  // independent chains
#pragma unroll
        for (int kt = 0; kt < NKT; kt++)
#pragma unroll
            for (int i = 0; i < 16; i++) m4[i & 3] = fmaxf(m4[i & 3], s2[SRC][kt][i]);
        return max_xor32(fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]))) * qscale;
    };
    // Lazy online-softmax max update before an item's exponentials.
    auto raise_max = [&](float mloc) {
        if (__any(mloc > m_run + kLazy)) {
            const float m_new = fmaxf(m_run, mloc);
            const float corr = __builtin_amdgcn_exp2f(m_run - (m_new == -INFINITY ? 0.f : m_new));
            l_part *= corr;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) oacc[dt] *= corr;
            m_run = m_new;
        }
    };
    // P = exp2(S scale - m) of s2[SRC] as f16, and l += sum(P) in f32.
    auto exps = [&](auto srcc) {
        constexpr int SRC = decltype(srcc)::value;
        const float mu = m_run == -INFINITY ? 0.f : m_run;
        // Four independent partial sums: one running sum would chain every
        // add of the step behind the previous one.
        float ls[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kt = 0; kt < NKT; kt++)
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s2[SRC][kt][ks * 8 + 2 * jj], qscale, -mu));
                    const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s2[SRC][kt][ks * 8 + 2 * jj + 1], qscale, -mu));
                    ph[kt][ks][jj] = pack_f16x2(p0, p1);
                    ls[jj] += p0 + p1;
                }
        l_part += (ls[0] + ls[1]) + (ls[2] + ls[3]);
    };
    // O += V^T P with the item's V in V stage 2 VPAR + set.  The V^T reads of
    // d tile dt + 1 are in flight during dt's MFMAs.
    auto pv = [&](auto vparc) {
        constexpr int SOFF = decltype(vparc)::value * 2 * TILE;
        constexpr int RPD = NKT * 2 * 2;  // transpose reads per d tile
        u32x2 vbuf[2][NKT][2][2];
        auto rd = [&](auto dtc) {
            constexpr int dt = decltype(dtc)::value;
            static_for<0, NKT>([&](auto ktc) {
                constexpr int kt = decltype(ktc)::value;
                static_for<0, 2>([&](auto ksc) {
                    constexpr int ks = decltype(ksc)::value;
                    constexpr int off = SOFF + (kt * 32 + ks * 16) * RB;
                    vbuf[dt & 1][kt][ks][0] = lds_read_tr16_b64_at<off>(va_addr[dt][0]);
                    vbuf[dt & 1][kt][ks][1] = lds_read_tr16_b64_at<off>(va_addr[dt][1]);
                });
            });
        };
        rd(Int<0>{});
        if constexpr (NDT > 1) rd(Int<1>{});
        static_for<0, NDT>([&](auto dtc) {
            constexpr int dt = decltype(dtc)::value;
            lds_wait_n<(dt + 1 < NDT ? RPD : 0)>();
#pragma unroll
            for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                for (int ks = 0; ks < 2; ks++) {
                    tie(vbuf[dt & 1][kt][ks][0]);
                    tie(vbuf[dt & 1][kt][ks][1]);
                    const u32x2 a0 = vbuf[dt & 1][kt][ks][0], a1 = vbuf[dt & 1][kt][ks][1];
                    oacc[dt] = mfma32<F16>(u32x4{a0[0], a0[1], a1[0], a1[1]}, ph[kt][ks], oacc[dt]);
                }
            if constexpr (dt + 2 < NDT) rd(Int<dt + 2>{});
        });
    };

    // ---- main loop ----
    // Software pipeline per wave: step j runs exp(S_j) interleaved with the
    // MFMAs of S_{j+1} = QK(j+1), then PV(j) interleaved with max(S_{j+1}).
    // K is therefore loaded two items ahead and V one: step j loads K of
    // item j+2 (into item j's K stage) and V of item j+1.
    auto row_of = [&](int i) { return set == 0 && gB >= 0 && i < TA ? rowA : rowB; };
    if (tid < 2) set_bar[tid] = 0;
    load_q(set == 0 ? rowA : rowB);
    load_tile(0, 0);
    load_tile(0, 1);
    load_tile(1, 0);
    __builtin_amdgcn_s_waitcnt(vm_wait(0));
    tie_q();
    widen_own(-1);
    __builtin_amdgcn_s_waitcnt(vm_wait(63) & ~(15 << 8));
    wg_barrier();
    if (n_me > 0) {
        qk(Int<0>{}, Int<0>{});
        mask(Int<0>{}, row_of(0), item_tile(set, 0));
        raise_max(rowmax(Int<0>{}));
        if (set == 0 && gB >= 0 && TA == 1) {
            load_q(rowB);
            __builtin_amdgcn_s_waitcnt(vm_wait(0));
            tie_q();
        }
    }
    auto step = [&](auto par, int j) {
        constexpr int P = decltype(par)::value;
        constexpr Int<P ^ 1> npar{};
        __builtin_amdgcn_s_waitcnt(vm_wait(63) & ~(15 << 8));  // own LDS writes done
        set_barrier();  // item j's V and item j+1's K ready; item j's K and j-1's V consumed
        load_tile(0, j + 2);
        {
            // The exp + QK phase runs at raised wave priority, so the SIMD's
            // other wave (the other set, often in its PV phase) fills the
            // gaps this phase leaves.  The compiler sinks the exponentials
            // next to the PV MFMAs that use them, so the window holds the QK
            // MFMAs; measured on cfg3 against no priority change or a window
            // around PV instead: 49.0 / 49.3 / 49.0 us, within noise.
            __builtin_amdgcn_s_setprio(3);
            exps(par);
            qk(npar, npar);  // item j+1 (an idle tile of zeros past the end)
            if (set == 0 && gB >= 0 && j + 1 == TA - 1) load_q(rowB);
            __builtin_amdgcn_s_setprio(0);
        }
        load_tile(1, j + 1);
        {
            mask(npar, row_of(j + 1), item_tile(set, j + 1));
            pv(par);
            const float m_next = rowmax(npar);
            if (set == 0 && gB >= 0 && j == TA - 1) {  // block A complete: write it, switch to B
                const float l_tot = l_part + xor32(l_part);
                const float inv = 1.0f / l_tot;
                const int qrow = rowA + sub + c32;
                if (qrow < S) {
                    float *op = out + (int64_t)qrow * q_dim + (int64_t)head * D + h2 * 4;
#pragma unroll
                    for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                        for (int g = 0; g < 4; g++)
                            __builtin_nontemporal_store(
                                f32x4{oacc[dt][g * 4] * inv, oacc[dt][g * 4 + 1] * inv,
                                      oacc[dt][g * 4 + 2] * inv, oacc[dt][g * 4 + 3] * inv},
                                (f32x4 *)(op + dt * 32 + g * 8));
                }
#pragma unroll
                for (int i = 0; i < NDT; i++) oacc[i] = f32x16{};
                m_run = -INFINITY;
                l_part = 0.f;
            }
            if (j + 1 < n_me) raise_max(m_next);
        }
        // Item j+2's K, j+1's V and Q retired.  In the step that wrote block
        // A's rows, its NDT*4 stores (issued last) may still drain: they are
        // counted, in order, after the DMA.
        if (set == 0 && gB >= 0 && j == TA - 1) __builtin_amdgcn_s_waitcnt(vm_wait(NDT * 4));
        else __builtin_amdgcn_s_waitcnt(vm_wait(0));
        tie_q();
        widen_own(j);
    };
    for (int j = 0; j < n_me; j += 2) {
        step(Int<0>{}, j);
        if (j + 1 < n_me) step(Int<1>{}, j + 1);
    }

    // ---- merge the merged block's two partials through LDS ----
    __builtin_amdgcn_s_waitcnt(vm_wait(0) & ~(15 << 8));
    wg_barrier();  // ring idle
    const uint32_t part = lds0 + (slot * 64 + lane) * 16;  // [slot][dt][g][lane] f32x4
    if (set == 1) {
        const float l_tot = l_part + xor32(l_part);
        if (h2 == 0) { hand_ml[slot][c32][0] = m_run; hand_ml[slot][c32][1] = l_tot; }
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                lds_write_b128(part + (dt * 4 + g) * 4 * 64 * 16,
                               __builtin_bit_cast(u32x4, f32x4{oacc[dt][g * 4], oacc[dt][g * 4 + 1],
                                                               oacc[dt][g * 4 + 2], oacc[dt][g * 4 + 3]}));
    }
    __builtin_amdgcn_s_waitcnt(vm_wait(63) & ~(15 << 8));
    wg_barrier();
    const uint32_t stg = lds0 + 4 * 64 * NDT * 64;  // staged rows [32][OROW]
    if (set == 0) {
        const float l0 = l_part + xor32(l_part);
        const float m1 = hand_ml[slot][c32][0], l1 = hand_ml[slot][c32][1];
        const float M = fmaxf(m_run, m1);
        const float mu = M == -INFINITY ? 0.f : M;
        const float a0 = __builtin_amdgcn_exp2f(m_run - mu), a1 = __builtin_amdgcn_exp2f(m1 - mu);
        const float den = l0 * a0 + l1 * a1;
        const float inv = den > 0.f ? 1.0f / den : 0.f;
        const float w0 = a0 * inv, w1 = a1 * inv;
        u32x4 o1[NDT][4];
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
#pragma unroll
            for (int g = 0; g < 4; g++) o1[dt][g] = lds_read_b128(part + (dt * 4 + g) * 4 * 64 * 16);
        lds_wait_any();
        const int srow = sub + c32;  // staged row: hw heads x D f32
        const uint32_t dst = stg + srow * (hw * D * 4);
        const int c0 = (slot & (hw - 1)) * (D / 4) + h2;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                tie(o1[dt][g]);
                const f32x4 b = __builtin_bit_cast(f32x4, o1[dt][g]);
                lds_write_b128(dst + ((c0 + dt * 8 + g * 2) ^ (srow & 15)) * 16,
                               __builtin_bit_cast(u32x4, f32x4{oacc[dt][g * 4] * w0 + b[0] * w1,
                                                               oacc[dt][g * 4 + 1] * w0 + b[1] * w1,
                                                               oacc[dt][g * 4 + 2] * w0 + b[2] * w1,
                                                               oacc[dt][g * 4 + 3] * w0 + b[3] * w1}));
            }
    }
    __builtin_amdgcn_s_waitcnt(vm_wait(63) & ~(15 << 8));
    wg_barrier();
    // BLK rows x (hw heads x D f32), contiguous in the output row: each wave
    // stores BLK / 8 rows.
    const int cpr = hw * D / 4;  // 16-byte chunks per staged row
    for (int r4 = 0; r4 < rw * 4; r4++) {
        const int r = wave * rw * 4 + r4;
        const int qrow = rowB + r;
        for (int c = lane; c < cpr; c += 64) {
            const u32x4 v = lds_read_b128(stg + r * (hw * D * 4) + (c ^ (r & 15)) * 16);
            lds_wait_any();
            if (qrow < S)
                __builtin_nontemporal_store(__builtin_bit_cast(f32x4, v),
                                            (f32x4 *)(out + (int64_t)qrow * q_dim + (int64_t)head0 * D) + c);
        }
    }
}

// ---------------------------------------------------------------------------
// Prefill with split-K inside the workgroup (head_dim 256).
//
// A workgroup owns one 32-row block of one query head; its 4 waves split the
// block's key tiles (32 keys each) into 4 contiguous ranges, each wave keeps
// (m, l, O) of all 32 rows over its range, and the 4 partials are merged
// through LDS at the end (the online softmax is order-free).  That makes
// n_head * ceil(S / 32) workgroups: at S = 1024 with 8 heads, 256, one per CU,
// where 128-row workgroups would leave three quarters of the CUs idle.  One
// wave per SIMD: the D = 256 output (128 registers), Q (64) and a K tile (64)
// exceed what two waves per SIMD may hold.
// Per wave and tile, K goes global -> registers in the MFMA A-operand layout
// (lane = key row, 16-byte chunks); tile t+1's K is requested as soon as
// tile t's QK MFMAs have read theirs.  V goes global -> the wave's own LDS
// stage by buffer_load ... lds (row-major, 16-byte chunks XOR-swizzled by row
// kv_swz, bf16 widened to f16 in place) and is read transposed
// as the V^T operand; two stages, V of tile t+1 in flight while t computes.
template <class T, int D>
__global__ __launch_bounds__(256, 1) void prefill_sk_kernel(
    const uint16_t *__restrict__ q, const char *__restrict__ kc, const char *__restrict__ vc,
    int64_t kv_stride, int S, int start_pos, int window, int n_head, int kv_mul, int nb,
    float qscale, float *__restrict__ out, KvPages pgs) {
    constexpr int BN = 32, RB = D * 2, SLOTS = D / 8, RPI = 1024 / RB, NI = BN / RPI;
    constexpr int TILE = BN * RB;  // bytes of one V tile
    constexpr int NKS = D / 16, NDT = D / 32, CPW = D / 16;
    constexpr bool CVTV = __is_same(T, BF16);
    constexpr float kLazy = 8.0f;  // log2 headroom before the max is raised
    static_assert(D == 256, "split-K prefill serves head_dim 256");
    static_assert(32 * D * 4 <= 2 * TILE, "a wave's partial fits its two V stages");
    auto swz = [](int r) { return kv_swz<D>(r); };
    __shared__ __attribute__((aligned(1024))) char lds[4 * 2 * TILE];
    __shared__ float sm_ml[4][32][2];

    // Tasks are head-major (the heads of one kv head are adjacent and share
    // an XCD's L2: workgroup i runs on XCD i % 8), longest block first.
    const int total = n_head * nb;
    const int per_xcd = (total + 7) / 8;
    const int tsk = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (tsk >= total) return;
    const int head = tsk / nb, blk = nb - 1 - tsk % nb;
    const int kvh = head / kv_mul;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 31, h2 = lane >> 5;
    const int q0 = blk * 32;
    const int64_t q_dim = (int64_t)n_head * D;
    const int kv_len = start_pos + S;

    // Key tiles of the block, [lo, hi) in keys, split over the 4 waves.
    const int hi = start_pos + min(q0 + 32, S);
    int lo = 0;
    if (window > 0) lo = max(0, start_pos + q0 + 1 - window);
    lo = lo / BN * BN;
    const int nt = (hi - lo + BN - 1) / BN;
    const int ta = lo / BN + nt * wave / 4, tb = lo / BN + nt * (wave + 1) / 4;

    // Q rows of this wave as the B operand (d = s*16 + h2*8 + j).
    const int qrow = q0 + c;
    const bool row_ok = qrow < S;
    const int pos_row = start_pos + qrow;
    const int dlo = window > 0 ? -window : INT_MIN;
    u32x4 qreg[NKS];
    {
        const uint16_t *qp = q + (int64_t)(row_ok ? qrow : 0) * q_dim + (int64_t)head * D + h2 * 8;
#pragma unroll
        for (int s = 0; s < NKS; s++) qreg[s] = row_ok ? ld16(qp + s * 16) : u32x4{0, 0, 0, 0};
    }

    const int rbg = (int)(kv_stride * 2);
    const int range = (kv_len - 1) * rbg + D * 2;
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(kc + (int64_t)kvh * D * 2), 0, range, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(vc + (int64_t)kvh * D * 2), 0, range, kRsrcWord3);
    char *const vst = lds + wave * 2 * TILE;  // this wave's two V stages
    const int koff = c * rbg + h2 * 16;
    const int lr = lane / SLOTS, slot = lane % SLOTS;
    // Requests are issued unconditionally (fixed wait counts); a tile past
    // this wave's range is addressed past the buffer range, which reads
    // zero without touching memory, as do keys past the cache's end.
    auto tile_off = [&](int t) { return __builtin_amdgcn_readfirstlane(t < tb ? t * BN * rbg : range); };
    // Paged: the tile's page resources (a dead tile addresses the sequence
    // end, past every page's range).
    auto page_of = [&](int t, __amdgpu_buffer_rsrc_t &kp, __amdgpu_buffer_rsrc_t &vp, int &so) {
        page_tile<D>(pgs, kc, vc, kvh, rbg, kv_len, t < tb ? t * BN : kv_len, kp, vp, so);
    };
    auto issue_k = [&](u32x4(&kr)[NKS], int t) {
        __amdgpu_buffer_rsrc_t kp = krs, vp = vrs;
        int so;
        if (pgs.tab) page_of(t, kp, vp, so);
        else so = tile_off(t);
#pragma unroll
        for (int s = 0; s < NKS; s++)
            kr[s] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(kp, koff + s * 32 + so, 0, 0));
        __builtin_amdgcn_sched_barrier(0);  // keep the K loads ahead of later V requests
    };
    auto issue_v = [&](int st, int t) {
        __amdgpu_buffer_rsrc_t kp = krs, vp = vrs;
        int so;
        if (pgs.tab) page_of(t, kp, vp, so);
        else so = tile_off(t);
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int r = i * RPI + lr;
            dma16(vp, vst + st * TILE + i * 1024, r * rbg + ((slot ^ swz(r)) * 16) + so, 0);
        }
    };
    // bf16 -> f16 in place, for the chunks this lane's DMA wrote.
    auto widen = [&](int st) {
        if constexpr (CVTV) {
            const uint32_t vb = lds_addr(vst + st * TILE) + lane * 16;
#pragma unroll
            for (int i0 = 0; i0 < NI; i0 += 4) {
                u32x4 w[4];
#pragma unroll
                for (int i = 0; i < 4; i++) w[i] = lds_read_b128(vb + (i0 + i) * 1024);
                lds_wait_any();
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    tie(w[i]);
                    u32x4 o;
#pragma unroll
                    for (int e = 0; e < 4; e++) o[e] = pack_f16x2(bf16_lo(w[i][e]), bf16_hi(w[i][e]));
                    lds_write_b128(vb + (i0 + i) * 1024, o);
                }
            }
        }
    };

    // V^T operand addresses (stage 0, k-step 0): lane gets d = dt*32 + lane%32
    // ... as the transposing read delivers it, keys in the P^T order.
    const int g16 = lane >> 4, i16 = lane & 15;
    uint32_t va_addr[NDT][2];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int e0 = dt * 32 + (g16 & 1) * 16 + 4 * (i16 & 3);
            const int R = (g16 >> 1) * 4 + (i16 >> 2) + h * 8;
            va_addr[dt][h] = lds_addr(vst) + R * RB + (((e0 >> 3) ^ swz(R)) * 16) + (e0 & 7) * 2;
        }

    f32x16 oacc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; i++) oacc[i] = f32x16{};
    float m_run = -INFINITY, l_part = 0.f;

    u32x4 kreg[NKS];
    auto consume = [&](auto stc, int t) {
        constexpr int SOFF = decltype(stc)::value * TILE;
        // S^T = K . Q^T: lane = query row c, keys (i>>2)*8 + h2*4 + (i&3)
        f32x16 sacc = f32x16{};
#pragma unroll
        for (int s = 0; s < NKS; s++) sacc = mfma32<T>(kreg[s], qreg[s], sacc);
        issue_k(kreg, t + 1);  // the MFMAs above have read their K
        // Masked without branches: key - pos_row = kd + (i>>2)*8 + (i&3) must
        // lie in (dlo, 0] (dlo = -window, or below any offset with no window).
        const int kd = t * BN + h2 * 4 - pos_row;
        float mloc = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int dk = kd + (i >> 2) * 8 + (i & 3);
            const float sv = dk > 0 || dk <= dlo ? -INFINITY : sacc[i] * qscale;
            sacc[i] = sv;
            mloc = fmaxf(mloc, sv);
        }
        mloc = fmaxf(mloc, xor32(mloc));
        // Lazy max: raised only when a row's tile max passes it by 2^kLazy
        // (P = exp2(s - m) <= 256 stays exact in f16's range), so the O
        // rescale (128 accumulators) runs a few times per wave, not per tile.
        if (__any(mloc > m_run + kLazy)) {
            const float m_new = fmaxf(m_run, mloc);
            if (__any(m_run != -INFINITY)) {
                const float corr = __builtin_amdgcn_exp2f(m_run - (m_new == -INFINITY ? 0.f : m_new));
                l_part *= corr;
                // (pinned here, so the copies out of the accumulation
                // registers stay inside this rare branch)
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) asm volatile("" : "+a"(oacc[dt]));
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) oacc[dt] *= corr;
            }
            m_run = m_new;
        }
        const float mu = m_run == -INFINITY ? 0.f : m_run;
        u32x4 pk[2];
        float ls[4] = {0.f, 0.f, 0.f, 0.f};  // independent partial sums
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const float p0 = __builtin_amdgcn_exp2f(sacc[ks * 8 + 2 * jj] - mu);
                const float p1 = __builtin_amdgcn_exp2f(sacc[ks * 8 + 2 * jj + 1] - mu);
                ls[jj] += p0 + p1;
                pk[ks][jj] = pack_f16x2(p0, p1);
            }
        l_part += (ls[0] + ls[1]) + (ls[2] + ls[3]);
        // O^T += V^T . P^T, the V^T reads of d tile dt + 1 in flight during dt's MFMAs
        u32x2 vb[2][2][2];
        auto rd = [&](int dt, int buf) {
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                vb[buf][ks][0] = lds_read_tr16_b64(va_addr[dt][0] + SOFF + ks * 16 * RB);
                vb[buf][ks][1] = lds_read_tr16_b64(va_addr[dt][1] + SOFF + ks * 16 * RB);
            }
        };
        rd(0, 0);
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            if (dt + 1 < NDT) {
                rd(dt + 1, (dt + 1) & 1);
                asm volatile("s_waitcnt lgkmcnt(4)" ::: "memory");
            } else {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            }
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                tie(vb[dt & 1][ks][0]);
                tie(vb[dt & 1][ks][1]);
                const u32x2 a0 = vb[dt & 1][ks][0], a1 = vb[dt & 1][ks][1];
                oacc[dt] = mfma32<F16>(u32x4{a0[0], a0[1], a1[0], a1[1]}, pk[ks], oacc[dt]);
            }
        }
    };

    // ---- main loop ----
    // Request order: V(t) [tile t-2], K(t) [after QK(t-1)], V(t+1) [after
    // PV(t-1)]: entering tile t, V(t+1) stays in flight.
    issue_k(kreg, ta);
    issue_v(0, ta);
    issue_v(1, ta + 1);
    constexpr int kLgkm0 = vm_wait(63) & ~(15 << 8);
    for (int t = ta; t < tb; t += 2) {
        __builtin_amdgcn_s_waitcnt(vm_wait(NI));
        widen(0);
        consume(Int<0>{}, t);
        __builtin_amdgcn_s_waitcnt(kLgkm0);  // stage 0 read: refill it
        issue_v(0, t + 2);
        if (t + 1 >= tb) break;
        __builtin_amdgcn_s_waitcnt(vm_wait(NI));
        widen(1);
        consume(Int<1>{}, t + 1);
        __builtin_amdgcn_s_waitcnt(kLgkm0);
        issue_v(1, t + 3);
    }
    __builtin_amdgcn_s_waitcnt(vm_wait(0));

    // ---- merge the 4 partials through LDS (each wave's own stages) ----
    const float l_tot = l_part + xor32(l_part);
    if (h2 == 0) { sm_ml[wave][c][0] = m_run; sm_ml[wave][c][1] = l_tot; }
    // lane (c, h2) holds row c, d = dt*32 + g*8 + h2*4 + 0..3: chunk dt*8 + g*2 + h2,
    // stored at chunk ^ (row % 16) of a D-float row.
    const uint32_t pw = lds_addr(vst);
#pragma unroll
    for (int dt = 0; dt < NDT; dt++)
#pragma unroll
        for (int g = 0; g < 4; g++)
            lds_write_b128(pw + c * D * 4 + (((dt * 8 + g * 2 + h2) ^ (c & 15)) * 16),
                           __builtin_bit_cast(u32x4, f32x4{oacc[dt][g * 4], oacc[dt][g * 4 + 1],
                                                           oacc[dt][g * 4 + 2], oacc[dt][g * 4 + 3]}));
    __builtin_amdgcn_s_waitcnt(vm_wait(63) & ~(15 << 8));
    __syncthreads();
    // Wave w writes chunks [w*CPW, (w+1)*CPW) of every row, 64/CPW rows at a
    // time; every LDS read of the pass is issued before any is consumed.
    constexpr int RPS = 64 / CPW, NR = 32 / RPS;
    const int ch = wave * CPW + lane % CPW;
    u32x4 pv[NR][4];
    float2 ml[NR][4];
#pragma unroll
    for (int it = 0; it < NR; it++) {
        const int r = it * RPS + lane / CPW;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            pv[it][w] = lds_read_b128(lds_addr(lds + w * 2 * TILE) + r * D * 4 + ((ch ^ (r & 15)) * 16));
            ml[it][w] = *(const float2 *)sm_ml[w][r];
        }
    }
    lds_wait_any();
#pragma unroll
    for (int it = 0; it < NR; it++) {
        const int r = it * RPS + lane / CPW;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; w++) M = fmaxf(M, ml[it][w].x);
        const float mu = M == -INFINITY ? 0.f : M;
        float L = 0.f;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < 4; w++) {
            tie(pv[it][w]);
            const float a = __builtin_amdgcn_exp2f(ml[it][w].x - mu);
            L += ml[it][w].y * a;
            acc += __builtin_bit_cast(f32x4, pv[it][w]) * a;
        }
        const float inv = L > 0.f ? 1.0f / L : 0.f;
        if (q0 + r < S)
            __builtin_nontemporal_store(acc * inv, (f32x4 *)(out + (int64_t)(q0 + r) * q_dim +
                                                             (int64_t)head * D) + ch);
    }
}

// head_dim 256: prefill16_kernel (16-row waves, two per SIMD), or on request
// prefill_sk_kernel (split-K inside one-wave-per-SIMD workgroups).
template <class T, int D, bool V2 = (D <= 128)>
struct PrefillLaunch {
    static void run(const void *q, const void *kc, const void *vc, int64_t kvs, int S, int sp,
                    int win, int nh, int kv_mul, float qs, float *out, hipStream_t st,
                    KvPages pgs = KvPages{}) {
        // prefill16_kernel; ULLM_HIP_PREFILL256=1 selects prefill_sk_kernel
        // instead, for comparison.
        static const int pick = env_override("ULLM_HIP_PREFILL256");
        if (pick != 1) {
            launch_prefill16(__is_same(T, BF16) ? ULLM_DT_BF16 : ULLM_DT_F16, q, kc, vc, kvs, S, sp,
                             win, nh, kv_mul, qs, out, st, pgs);
            return;
        }
        const int nb = (S + 31) / 32;
        const int total = nh * nb;
        const int per_xcd = (total + 7) / 8;
        hipLaunchKernelGGL((prefill_sk_kernel<T, D>), dim3(per_xcd * 8), dim3(256), 0, st,
                           (const uint16_t *)q, (const char *)kc, (const char *)vc, kvs, S, sp,
                           win, nh, kv_mul, nb, qs, out, pgs);
    }
};
template <class T, int D>
struct PrefillLaunch<T, D, true> {
    static void run(const void *q, const void *kc, const void *vc, int64_t kvs, int S, int sp,
                    int win, int nh, int kv_mul, float qs, float *out, hipStream_t st,
                    KvPages pgs = KvPages{});
};

template <class T, int D>
void PrefillLaunch<T, D, true>::run(const void *q, const void *kc, const void *vc, int64_t kvs,
                                    int S, int sp, int win, int nh, int kv_mul, float qs,
                                    float *out, hipStream_t st, KvPages pgs) {
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
    // head_dim 128, short prompts: prefill16_kernel (16-row waves; K/V tiles
    // shared by the GQA group; two key streams when units are few) when
    // prefill4's causal pairs would cover half the CUs or fewer.  Measured
    // (us, prefill4 -> prefill16): 12/2 heads S=1024 26.2 -> 16.5, S=2048
    // 39.4 -> 29.6; 32/8 heads S=512 18.8 -> 12.0, S=1024 27.3 -> 23.7,
    // S=1536 (192 pairs) 39.7 -> 42.6, S=2048 (256) 51.8 -> 59.9.
    // ULLM_HIP_PREFILL128=16 / =4 forces either kernel (tuning override).
    static const int e128 = env_override("ULLM_HIP_PREFILL128");
    if (D == 128 && (e128 == 16 || (e128 != 4 && paired && total <= 128))) {
        launch_prefill16_128(__is_same(T, BF16) ? ULLM_DT_BF16 : ULLM_DT_F16, q, kc, vc, kvs, S, sp,
                             win, nh, kv_mul, qs, out, st, pgs);
        return;
    }
    if (D <= 128 && paired) {
        const int lhw = hw == 4 ? 2 : (hw == 2 ? 1 : 0);
        hipLaunchKernelGGL((prefill4_kernel<T, D>), dim3(per_xcd * 8), dim3(512), 0, st,
                           (const uint16_t *)q, (const char *)kc, (const char *)vc, kvs, S, sp,
                           nh, kv_mul, lhw, ng, np, qs, out, pgs);
        return;
    }
    hipLaunchKernelGGL((prefill2_kernel<T, D>), dim3(per_xcd * 8), dim3(512), 0, st,
                       (const uint16_t *)q, (const char *)kc, (const char *)vc, kvs, S, sp, win,
                       nh, kv_mul, hw, rw, n_units, ng, np, paired, qs, out, pgs);
}

template <class T, int D>
static int launch_prefill(const void *q, const void *kc, const void *vc, int64_t kvs, int S,
                          int sp, int win, int nh, int kv_mul, float qs, float *out,
                          hipStream_t st) {
    PrefillLaunch<T, D>::run(q, kc, vc, kvs, S, sp, win, nh, kv_mul, qs, out, st);
    return check_hip(hipGetLastError(), "prefill launch");
}

// ---------------------------------------------------------------------------
// Prefill over an f32 cache (the reference's own cache dtype,
// crates/ullm-metal/src/forward.rs:355-356), head_dim 64 or 128.
//
// The matrix cores take 16-bit inputs, so Q.K runs on bf16 hi + lo halves of
// both operands: x = hi + lo with hi = RNE(x), lo = RNE(x - hi), and
// S = Qhi.Khi + Qhi.Klo + Qlo.Khi (three MFMAs per k-step; the dropped
// Qlo.Klo term and the split residues are ~2^-16 of each product, far below
// the 1e-3 budget, where plain bf16 or f16 Q/K would cost it for scores above
// a few units).  V is rounded to f16 (2^-11, as P is), so P.V stays one f16
// MFMA per k-step; |V| must stay below 65504.
//
// Q is scaled by scale*log2(e) before its split, so the scores come out in
// the exp2 domain.
//
// The K/V tiles are shared by a workgroup's 4 waves.  A workgroup owns hw
// query heads of one kv head (hw = the largest power of two dividing kv_mul,
// at most 4) times 4/hw consecutive 32-row blocks: one "unit" of
// UR = 128/hw rows; wave w takes head hw0 + w % hw and rows (w / hw) * 32 ..
// +31 of the unit.  Units are taken in causal pairs, A = p and B = NU-1-p,
// so every workgroup attends about the same number of keys.  The workgroup
// walks the key tiles of A, then those of B, and each tile is loaded and
// converted once for all 4 waves:
//  * all 256 threads load the tile's f32 K and V rows (16-byte chunks, two
//    full rows per wave instruction) into registers, NRAW tiles ahead;
//  * they convert them into an LDS stage, a chunk at a time between the
//    k-steps of the previous tile's Q.K (the conversion's VALU work issues
//    while the MFMAs run): K as bf16 hi and lo rows (row pitch D*2 + 16
//    bytes, so the 16 rows one A-operand read touches lie on distinct
//    banks), V as f16 rows in the kv_swz layout the transposing reads expect;
//  * three stages: a stage is rewritten two tiles after it was read, so one
//    barrier per tile orders every rewrite after all reads of it.
// Each wave keeps (m, l, O) of its 32 rows over the whole key range, so it
// writes its rows of A (normalised) when A's tiles end and starts B afresh;
// no partials are merged.  A 32-row block of one head per workgroup with the
// 4 waves splitting its keys (each wave streaming and converting its own
// tiles) took 1.6x as long at the cfg3 shape.
template <int D, int NRAW = 2>
__global__ __launch_bounds__(256, 1) void prefill_f32_kernel(
    const float *__restrict__ q, const float *__restrict__ kc, const float *__restrict__ vc,
    int64_t kv_stride, int S, int start_pos, int window, int n_head, int kv_mul, int hw,
    int n_units, int n_pairs, float qscale, float *__restrict__ out, KvPages pgs) {
    constexpr int BN = 32, RB = D * 2, KP = D * 2 + 16;  // keys per tile; f16/bf16 row bytes; K pitch
    constexpr int NKS = D / 16, NDT = D / 32;
    constexpr int FPR = D / 4;              // 16-byte f32 chunks per cache row
    constexpr int NCH = BN * FPR / 256;     // chunks per thread per tile (K and V each)
    constexpr int KARR = BN * KP, VARR = BN * RB;
    constexpr int STAGE = 2 * KARR + VARR;  // K hi, K lo, V (f16)
    constexpr int NSTG = 3;
    constexpr float kLazy = 8.0f;
    static_assert(D == 64 || D == 128, "f32 prefill serves head_dim 64 and 128");
    auto swz = [](int r) { return kv_swz<D>(r); };
    constexpr int QB = 2 * NKS * 64 * 16;   // one wave's unit-B Q operands (hi, lo)
    __shared__ __attribute__((aligned(1024))) char lds[NSTG * STAGE];
    __shared__ __attribute__((aligned(16))) char qb_lds[4 * QB];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 31, h2 = lane >> 5;
    // Task: (head group, pair), pairs of one head group on one XCD's L2.
    const int n_hg = n_head / hw;
    const int total = n_hg * n_pairs;
    const int per_xcd = (total + 7) / 8;
    const int tsk = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (tsk >= total) return;
    const int hg = tsk / n_pairs, pr = tsk % n_pairs;
    const int rbw = 4 / hw, UR = 32 * rbw;
    const int head = hg * hw + wave % hw, kvh = head / kv_mul;
    const int roff = (wave / hw) * 32;  // this wave's rows within a unit
    const int64_t q_dim = (int64_t)n_head * D;
    const int kv_len = start_pos + S;
    const int ua = pr, ub = n_units - 1 - pr;  // ub == ua: the middle unit alone

    // Key tiles [first, end) of a unit: from the window start of its first
    // row to the causal end of its last row.
    auto tiles = [&](int u, int &t0, int &t1) {
        const int r0 = u * UR;
        const int hi = start_pos + min(r0 + UR, S);
        int lo = 0;
        if (window > 0) lo = max(0, start_pos + r0 + 1 - window);
        t0 = lo / BN;
        t1 = (hi + BN - 1) / BN;
    };
    int a0, a1, b0 = 0, b1 = 0;
    tiles(ua, a0, a1);
    if (ub != ua) tiles(ub, b0, b1);
    const int na = a1 - a0, nsteps = na + (b1 - b0);

    const int rbg = (int)(kv_stride * 4);
    const int range = (kv_len - 1) * rbg + D * 4;
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(kc + (int64_t)kvh * D), 0, range, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(vc + (int64_t)kvh * D), 0, range, kRsrcWord3);
    // Step j's tile; steps past the end address past the buffer (zeros,
    // no memory access), so every step issues the same requests.
    auto tile_of = [&](int j) { return j < na ? a0 + j : b0 + (j - na); };
    auto step_off = [&](int j) {
        return __builtin_amdgcn_readfirstlane(j < nsteps ? tile_of(j) * BN * rbg : range);
    };
    // Thread tid loads chunks ci = tid + 256 i: row ci / FPR, f32 chunk ci % FPR.
    u32x4 kraw[NRAW][NCH], vraw[NRAW][NCH];
    // Paged (pgs.tab): the tile's page gives the buffer resources (a tile
    // never crosses a page; keys past the sequence, or pages outside the
    // table or pool, read zeros).
    auto issue = [&](u32x4(&kr)[NCH], u32x4(&vr)[NCH], int j) {
        __amdgpu_buffer_rsrc_t kq = krs, vq = vrs;
        int so;
        if (pgs.tab) {
            const char *kcb = (const char *)kc, *vcb = (const char *)vc;
            page_tile<D, 4>(pgs, kcb, vcb, kvh, rbg, kv_len, j < nsteps ? tile_of(j) * BN : kv_len,
                            kq, vq, so);
        } else {
            so = step_off(j);
        }
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            const int ci = tid + 256 * i, off = (ci / FPR) * rbg + (ci % FPR) * 16 + so;
            kr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kq, off, 0, 0));
            vr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vq, off, 0, 0));
        }
    };
    const uint32_t lds0 = lds_addr(lds);
    // Chunk i of the thread's share (one K and one V chunk).
    auto convert1 = [&](const u32x4(&kr)[NCH], const u32x4(&vr)[NCH], int stg, int i) {
        const uint32_t sb = lds0 + stg * STAGE;
        {
            const int ci = tid + 256 * i, r = ci / FPR, f = ci % FPR;
            const f32x4 kv = __builtin_bit_cast(f32x4, kr[i]);
            const u32x2 p0 = split2<BF16>(kv[0], kv[1]), p1 = split2<BF16>(kv[2], kv[3]);
            lds_write_b64(sb + r * KP + f * 8, u32x2{p0[0], p1[0]});
            lds_write_b64(sb + KARR + r * KP + f * 8, u32x2{p0[1], p1[1]});
            const f32x4 vv = __builtin_bit_cast(f32x4, vr[i]);
            lds_write_b64(sb + 2 * KARR + r * RB + (((f >> 1) ^ swz(r)) * 16) + (f & 1) * 8,
                          u32x2{pack_f16x2(vv[0], vv[1]), pack_f16x2(vv[2], vv[3])});
        }
    };
    auto convert = [&](const u32x4(&kr)[NCH], const u32x4(&vr)[NCH], int stg) {
#pragma unroll
        for (int i = 0; i < NCH; i++) convert1(kr, vr, stg, i);
    };

    // Operand addresses within a stage: K (lane = key c, d = s*16 + h2*8 ..),
    // V^T (as prefill_sk_kernel).
    const uint32_t ka = c * KP + h2 * 16;
    const int g16 = lane >> 4, i16 = lane & 15;
    uint32_t va_addr[NDT][2];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int e0 = dt * 32 + (g16 & 1) * 16 + 4 * (i16 & 3);
            const int R = (g16 >> 1) * 4 + (i16 >> 2) + h * 8;
            va_addr[dt][h] = 2 * KARR + R * RB + (((e0 >> 3) ^ swz(R)) * 16) + (e0 & 7) * 2;
        }

    // Per-unit state of this wave: Q as hi/lo B operands (unit B's are
    // prepared at the start and parked in LDS, lane-major), row, (m, l, O).
    u32x4 qh[NKS], ql[NKS];
    const uint32_t qbw = lds_addr(qb_lds) + wave * QB + lane * 16;
    auto load_q = [&](int u, u32x4(&h)[NKS], u32x4(&l)[NKS]) {
        const int row = u * UR + roff + c;
        const bool ok = row < S;
        const float *qp = q + (int64_t)(ok ? row : 0) * q_dim + (int64_t)head * D + h2 * 8;
#pragma unroll
        for (int s = 0; s < NKS; s++) {
            // scaled before the split: the scores come out in the exp2 domain
            const f32x4 a = (ok ? *(const f32x4 *)(qp + s * 16) : f32x4{0.f, 0.f, 0.f, 0.f}) * qscale;
            const f32x4 b = (ok ? *(const f32x4 *)(qp + s * 16 + 4) : f32x4{0.f, 0.f, 0.f, 0.f}) * qscale;
            const u32x2 p0 = split2<BF16>(a[0], a[1]), p1 = split2<BF16>(a[2], a[3]);
            const u32x2 p2 = split2<BF16>(b[0], b[1]), p3 = split2<BF16>(b[2], b[3]);
            h[s] = u32x4{p0[0], p1[0], p2[0], p3[0]};
            l[s] = u32x4{p0[1], p1[1], p2[1], p3[1]};
        }
    };
    int qrow = 0, pos_row = 0;
    const int dlo = window > 0 ? -window : INT_MIN;
    f32x16 oacc[NDT];
    float m_run, l_part;
    auto begin_unit = [&](int u) {
        qrow = u * UR + roff + c;
        pos_row = start_pos + qrow;
#pragma unroll
        for (int i = 0; i < NDT; i++) oacc[i] = f32x16{};
        m_run = -INFINITY;
        l_part = 0.f;
    };
    // O^T in registers: lane (row c, h2) holds d = dt*32 + 8g + 4*h2 + 0..3.
    auto end_unit = [&]() {
        const float l_tot = l_part + xor32(l_part);
        const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
        if (qrow < S) {
            float *op = out + (int64_t)qrow * q_dim + (int64_t)head * D + h2 * 4;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                for (int g = 0; g < 4; g++)
                    __builtin_nontemporal_store(
                        f32x4{oacc[dt][g * 4], oacc[dt][g * 4 + 1], oacc[dt][g * 4 + 2],
                              oacc[dt][g * 4 + 3]} * inv,
                        (f32x4 *)(op + dt * 32 + g * 8));
        }
    };

    // mid(i) runs after k-step 2i+1 of Q.K (the next tile's conversion, one
    // chunk at a time, so its VALU work issues while the MFMAs run).
    auto compute = [&](int j, int stg, auto &&mid) {
        const uint32_t sb = lds0 + stg * STAGE;
        f32x16 sacc = f32x16{};
        // K operands of k-step s+1 are read while s's MFMAs run.
        u32x4 kh[2], kl[2];
        kh[0] = lds_read_b128(sb + ka);
        kl[0] = lds_read_b128(sb + KARR + ka);
#pragma unroll
        for (int s = 0; s < NKS; s++) {
            if (s + 1 < NKS) {
                kh[(s + 1) & 1] = lds_read_b128(sb + ka + (s + 1) * 32);
                kl[(s + 1) & 1] = lds_read_b128(sb + KARR + ka + (s + 1) * 32);
                asm volatile("s_waitcnt lgkmcnt(2)" ::: "memory");
            } else {
                lds_wait_any();
            }
            tie(kh[s & 1]);
            tie(kl[s & 1]);
            sacc = mfma32<BF16>(kh[s & 1], qh[s], sacc);
            sacc = mfma32<BF16>(kh[s & 1], ql[s], sacc);
            sacc = mfma32<BF16>(kl[s & 1], qh[s], sacc);
            if (s & 1) mid(s >> 1);
        }
        // V^T operands of d tile 0 go out before the softmax
        u32x2 vb[2][2][2];
        auto rd = [&](int dt, int buf) {
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                vb[buf][ks][0] = lds_read_tr16_b64(sb + va_addr[dt][0] + ks * 16 * RB);
                vb[buf][ks][1] = lds_read_tr16_b64(sb + va_addr[dt][1] + ks * 16 * RB);
            }
        };
        rd(0, 0);
        // Masked only where the tile reaches past the diagonal of the
        // wave's first row or before the window of its last (wave-uniform):
        // key - pos_row must lie in (dlo, 0].
        const int kb = tile_of(j) * BN, p_first = pos_row - c;
        float mloc = -INFINITY;
        if (kb + BN - 1 > p_first || (window > 0 && kb <= p_first + 31 - window)) {
            const int kd = kb + h2 * 4 - pos_row;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int dk = kd + (i >> 2) * 8 + (i & 3);
                const float sv = dk > 0 || dk <= dlo ? -INFINITY : sacc[i];
                sacc[i] = sv;
                mloc = fmaxf(mloc, sv);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++) mloc = fmaxf(mloc, sacc[i]);
        }
        mloc = max_xor32(mloc);
        if (__any(mloc > m_run + kLazy)) {
            const float m_new = fmaxf(m_run, mloc);
            if (__any(m_run != -INFINITY)) {
                const float corr = __builtin_amdgcn_exp2f(m_run - (m_new == -INFINITY ? 0.f : m_new));
                l_part *= corr;
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) oacc[dt] *= corr;
            }
            m_run = m_new;
        }
        const float mu = m_run == -INFINITY ? 0.f : m_run;
        u32x4 pk[2];
        float ls[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const float p0 = __builtin_amdgcn_exp2f(sacc[ks * 8 + 2 * jj] - mu);
                const float p1 = __builtin_amdgcn_exp2f(sacc[ks * 8 + 2 * jj + 1] - mu);
                ls[jj] += p0 + p1;
                pk[ks][jj] = pack_f16x2(p0, p1);
            }
        l_part += (ls[0] + ls[1]) + (ls[2] + ls[3]);
        // O^T += V^T.P^T, the reads of d tile dt+1 in flight during dt's MFMAs
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            if (dt + 1 < NDT) {
                rd(dt + 1, (dt + 1) & 1);
                asm volatile("s_waitcnt lgkmcnt(4)" ::: "memory");
            } else {
                lds_wait_any();
            }
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                tie(vb[dt & 1][ks][0]);
                tie(vb[dt & 1][ks][1]);
                const u32x2 a0 = vb[dt & 1][ks][0], a1 = vb[dt & 1][ks][1];
                oacc[dt] = mfma32<F16>(u32x4{a0[0], a0[1], a1[0], a1[1]}, pk[ks], oacc[dt]);
            }
        }
    };

    // ---- pipeline: raw tiles NRAW ahead in registers, 3 converted stages ----
    static_assert(NRAW == 2, "the step loop is unrolled for two raw register sets");
    issue(kraw[0], vraw[0], 0);
    issue(kraw[1], vraw[1], 1);
    if (ub != ua) {
        load_q(ub, qh, ql);
#pragma unroll
        for (int s = 0; s < NKS; s++) {
            lds_write_b128(qbw + (2 * s) * 1024, qh[s]);
            lds_write_b128(qbw + (2 * s + 1) * 1024, ql[s]);
        }
    }
    load_q(ua, qh, ql);
    begin_unit(ua);
    convert(kraw[0], vraw[0], 0);
    issue(kraw[0], vraw[0], 2);
    lds_wait_any();
    __syncthreads();
    // Step j: compute tile j from stage j%3 while converting tile j+1 (raw
    // set (j+1)%2) into stage (j+1)%3, request tile j+3 into that set, then
    // a barrier: tile j+1's stage is complete for every wave, and stage
    // (j+2)%3, read by compute(j-1), is free for the next conversion.
    int stg = 0;
    auto step = [&](auto rs, int j, bool live) {
        constexpr int R = decltype(rs)::value;  // raw set of tile j+1
        const int nstg = stg == NSTG - 1 ? 0 : stg + 1;
        if (live && j == na) {
            end_unit();
            begin_unit(ub);
#pragma unroll
            for (int s = 0; s < NKS; s++) {
                qh[s] = lds_read_b128(qbw + (2 * s) * 1024);
                ql[s] = lds_read_b128(qbw + (2 * s + 1) * 1024);
            }
            lds_wait_any();
#pragma unroll
            for (int s = 0; s < NKS; s++) { tie(qh[s]); tie(ql[s]); }
        }
        if (live) compute(j, stg, [&](int i) { convert1(kraw[R], vraw[R], nstg, i); });
        else convert(kraw[R], vraw[R], nstg);
        issue(kraw[R], vraw[R], j + 3);
        // LDS writes done, then a barrier that leaves the tile requests in
        // flight (a fence would wait for them); the clobber keeps LDS
        // accesses on their side of it.
        lds_wait_any();
        asm volatile("s_barrier" ::: "memory");
        stg = nstg;
    };
    // Both halves convert, request and synchronise unconditionally (a path
    // that skipped the second half's requests would make every wait at the
    // loop head drain all of them); only the compute of a step past the end
    // is skipped.
    for (int j = 0; j < nsteps; j += 2) {
        step(Int<1>{}, j, true);
        step(Int<0>{}, j + 1, j + 1 < nsteps);
    }
    end_unit();
}

template <int D>
static int launch_prefill_f32(const void *q, const void *kc, const void *vc, int64_t kvs, int S,
                              int sp, int win, int nh, int kv_mul, float qs, float *out,
                              hipStream_t st, KvPages pgs = KvPages{}) {
    int hw = 1;
    while (hw < 4 && kv_mul % (hw * 2) == 0) hw *= 2;
    const int n_units = (S + 128 / hw - 1) / (128 / hw);
    const int n_pairs = (n_units + 1) / 2;
    const int total = nh / hw * n_pairs;
    const int per_xcd = (total + 7) / 8;
    hipLaunchKernelGGL((prefill_f32_kernel<D>), dim3(per_xcd * 8), dim3(256), 0, st,
                       (const float *)q, (const float *)kc, (const float *)vc, kvs, S, sp, win,
                       nh, kv_mul, hw, n_units, n_pairs, qs, out, pgs);
    return check_hip(hipGetLastError(), "prefill (f32) launch");
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
    if (!dtype_ok(dtype))
        return set_error(ULLM_HIP_E_UNSUPPORTED, "prefill: dtype %d", dtype);
    if (n_head < 1 || n_kv_head < 1 || n_head % n_kv_head || S < 0 || start_pos < 0)
        return set_error(ULLM_HIP_E_INVALID, "prefill: bad shape S=%d start_pos=%d heads=%d/%d", S,
                         start_pos, n_head, n_kv_head);
    if (head_dim != 64 && head_dim != 128 && head_dim != 256)
        return set_error(ULLM_HIP_E_UNSUPPORTED, "prefill: head_dim %d not in {64,128,256}", head_dim);
    if (kv_stride < (int64_t)n_kv_head * head_dim || (kv_stride * dtype_bytes(dtype)) % 16)
        return set_error(ULLM_HIP_E_INVALID, "prefill: kv_stride must be >= n_kv_head*head_dim and 16-byte aligned");
    if ((int64_t)(start_pos + S) * kv_stride * dtype_bytes(dtype) > 0x7fff0000LL)
        return set_error(ULLM_HIP_E_INVALID, "prefill: a layer's cache exceeds 2 GiB");
    if ((int64_t)S * n_head * head_dim * dtype_bytes(dtype) > 0x7fff0000LL)  // q's buffer range
        return set_error(ULLM_HIP_E_INVALID, "prefill: q exceeds 2 GiB (split the prompt into chunks)");
    if (S == 0) return ULLM_HIP_OK;
    if (!q || !k_cache || !v_cache || !out)
        return set_error(ULLM_HIP_E_INVALID, "prefill: null tensor pointer");
    if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out) & 15)
        return set_error(ULLM_HIP_E_INVALID, "prefill: tensors must be 16-byte aligned");
    const float qs = scale * kLog2e;
    const int kv_mul = n_head / n_kv_head;
    hipStream_t st = (hipStream_t)stream;
    if (dtype == ULLM_DT_F32) {
        // head_dim 128: prefill16_kernel's f32 mode (faster at every measured
        // prompt, 128..4096 rows); ULLM_HIP_PREFILL_F32=4 keeps prefill_f32_kernel.
        static const int ef = env_override("ULLM_HIP_PREFILL_F32");
        if (head_dim == 256)
            return launch_prefill16(ULLM_DT_F32, q, k_cache, v_cache, kv_stride, S, start_pos, window,
                                    n_head, kv_mul, qs, out, st, KvPages{});
        if (head_dim == 128 && ef != 4)
            return launch_prefill16_128(ULLM_DT_F32, q, k_cache, v_cache, kv_stride, S, start_pos, window,
                                        n_head, kv_mul, qs, out, st, KvPages{});
        if (head_dim == 64)
            return launch_prefill_f32<64>(q, k_cache, v_cache, kv_stride, S, start_pos, window, n_head, kv_mul, qs, out, st);
        return launch_prefill_f32<128>(q, k_cache, v_cache, kv_stride, S, start_pos, window, n_head, kv_mul, qs, out, st);
    }
    if (dtype == ULLM_DT_BF16)
        return dispatch_prefill<BF16>(head_dim, q, k_cache, v_cache, kv_stride, S, start_pos, window, n_head, kv_mul, qs, out, st);
    return dispatch_prefill<F16>(head_dim, q, k_cache, v_cache, kv_stride, S, start_pos, window, n_head, kv_mul, qs, out, st);
}

extern "C" int ullm_hip_attn_prefill_paged(const void *q, const void *k_pages, const void *v_pages,
                                           int dtype, int64_t kv_stride, int page_size,
                                           int n_pages, const int32_t *block_table,
                                           int table_len, int S, int start_pos, int window,
                                           int n_head, int n_kv_head, int head_dim, float scale,
                                           float *out, void *stream) {
    if (!dtype_ok(dtype))
        return set_error(ULLM_HIP_E_UNSUPPORTED, "prefill_paged: dtype %d", dtype);
    if (head_dim != 64 && head_dim != 128 && head_dim != 256)
        return set_error(ULLM_HIP_E_UNSUPPORTED, "prefill_paged: head_dim %d not in {64,128,256}", head_dim);
    if (n_head < 1 || n_kv_head < 1 || n_head % n_kv_head || S < 0 || start_pos < 0)
        return set_error(ULLM_HIP_E_INVALID, "prefill_paged: bad shape S=%d start_pos=%d heads=%d/%d",
                         S, start_pos, n_head, n_kv_head);
    const int eb = dtype_bytes(dtype);
    if (kv_stride < (int64_t)n_kv_head * head_dim || (kv_stride * eb) % 16)
        return set_error(ULLM_HIP_E_INVALID,
                         "prefill_paged: kv_stride must be >= n_kv_head*head_dim and 16-byte aligned");
    if (page_size < 64 || (page_size & (page_size - 1)))
        return set_error(ULLM_HIP_E_INVALID, "prefill_paged: page_size %d must be a power of two >= 64",
                         page_size);
    if ((int64_t)page_size * kv_stride * eb > 0x7fff0000LL)
        return set_error(ULLM_HIP_E_INVALID, "prefill_paged: a page exceeds 2 GiB");
    if ((int64_t)S * n_head * head_dim * eb > 0x7fff0000LL)  // q's buffer range
        return set_error(ULLM_HIP_E_INVALID, "prefill_paged: q exceeds 2 GiB (split the prompt into chunks)");
    if (n_pages < 1) return set_error(ULLM_HIP_E_INVALID, "prefill_paged: n_pages %d < 1", n_pages);
    if ((int64_t)table_len * page_size < (int64_t)start_pos + S)
        return set_error(ULLM_HIP_E_INVALID, "prefill_paged: table of %d pages holds fewer than %d positions",
                         table_len, start_pos + S);
    if (S == 0) return ULLM_HIP_OK;
    if (!q || !k_pages || !v_pages || !block_table || !out)
        return set_error(ULLM_HIP_E_INVALID, "prefill_paged: null tensor pointer");
    if (((uintptr_t)q | (uintptr_t)k_pages | (uintptr_t)v_pages | (uintptr_t)out) & 15)
        return set_error(ULLM_HIP_E_INVALID, "prefill_paged: tensors must be 16-byte aligned");
    const KvPages pgs{block_table, table_len, __builtin_ctz(page_size), n_pages};
    const float qs = scale * kLog2e;
    const int kv_mul = n_head / n_kv_head;
    hipStream_t st = (hipStream_t)stream;
    if (dtype == ULLM_DT_F32) {  // f32 pages: prefill16_kernel's f32 mode, prefill_f32_kernel at 64
        if (head_dim == 64)
            return launch_prefill_f32<64>(q, k_pages, v_pages, kv_stride, S, start_pos, window, n_head,
                                          kv_mul, qs, out, st, pgs);
        if (head_dim == 256)
            return launch_prefill16(ULLM_DT_F32, q, k_pages, v_pages, kv_stride, S, start_pos, window,
                                    n_head, kv_mul, qs, out, st, pgs);
        return launch_prefill16_128(ULLM_DT_F32, q, k_pages, v_pages, kv_stride, S, start_pos, window,
                                    n_head, kv_mul, qs, out, st, pgs);
    }
    if (dtype == ULLM_DT_BF16) {
        if (head_dim == 64) PrefillLaunch<BF16, 64>::run(q, k_pages, v_pages, kv_stride, S, start_pos, window, n_head, kv_mul, qs, out, st, pgs);
        else if (head_dim == 128) PrefillLaunch<BF16, 128>::run(q, k_pages, v_pages, kv_stride, S, start_pos, window, n_head, kv_mul, qs, out, st, pgs);
        else PrefillLaunch<BF16, 256>::run(q, k_pages, v_pages, kv_stride, S, start_pos, window, n_head, kv_mul, qs, out, st, pgs);
    } else {
        if (head_dim == 64) PrefillLaunch<F16, 64>::run(q, k_pages, v_pages, kv_stride, S, start_pos, window, n_head, kv_mul, qs, out, st, pgs);
        else if (head_dim == 128) PrefillLaunch<F16, 128>::run(q, k_pages, v_pages, kv_stride, S, start_pos, window, n_head, kv_mul, qs, out, st, pgs);
        else PrefillLaunch<F16, 256>::run(q, k_pages, v_pages, kv_stride, S, start_pos, window, n_head, kv_mul, qs, out, st, pgs);
    }
    return check_hip(hipGetLastError(), "prefill_paged launch");
}

