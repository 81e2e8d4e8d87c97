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
//  * S^T[16 keys x 16 heads] = K . Q^T: K is the A operand, Q^T the B operand
//    held in registers for the whole call.  q (f32) is split into hi + lo
//    halves of the cache dtype, two MFMAs per step, so the product keeps
//    ~f32 accuracy.
//  * O^T[16 d x 16 heads] += V^T . P^T: V^T is the A operand, read from a
//    row-major LDS tile by the transposing ds_read_b64_tr_b16.  P^T (the B
//    operand) is exactly the S^T accumulator of two key tiles, exponentiated:
//    the key order inside a k-step is free, so P never moves between lanes.
//    f16 caches use P in f16 (2^-11); bf16 caches split P into hi + lo bf16
//    (two MFMAs) to stay inside a 1e-3 rel-L2 budget.
//  * In both accumulators a lane's column is one head, so the running max,
//    sum and rescale of a head live in the lanes that own its output.
//  * head_dim <= 128 streams K/V tiles global -> LDS by buffer_load ... lds
//    (decode_dma_kernel, 1 or 4 waves per workgroup); head_dim 256 stages
//    through registers (decode_mfma_kernel).
//  * The waves of a workgroup stream disjoint key blocks and combine through
//    LDS; the splits of a unit are combined by decode_merge_kernel.
#include <algorithm>
#include <cstdlib>
#include <type_traits>
#include "common.hpp"
#include "mfma_util.hpp"
#include "wave.hpp"

namespace ullm {

constexpr int kMW = 4;          // waves per workgroup
constexpr int kTok = 32;        // keys per wave iteration (two 16-key tiles)
constexpr int kMaxUnitHeads = 16;
constexpr int kMfmaTargetWG = 256;  // one 4-wave workgroup per CU (LDS-bound)

// Writes four columns (c*4 .. c*4+3) of head head0 + g for one split: the
// normalised output when the unit has one split, else the partial (O
// unnormalised; (m, l) once per head, by the thread of column group 0).
template <int D>
__device__ __forceinline__ void store_split(const f32x4 &num, float mx, float den, int c, int g,
                                            int b, int split, int splits, int gt, int n_head,
                                            int head0, int64_t u, int GD,
                                            float *__restrict__ out, float *__restrict__ ws_ml,
                                            float *__restrict__ ws_acc) {
    if (splits == 1) {
        f32x4 o;
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] = den > 0.f ? num[i] / den : 0.f;
        *(f32x4 *)(out + ((int64_t)b * n_head + head0 + g) * D + c * 4) = o;
    } else {
        *(f32x4 *)(ws_acc + (u * splits + split) * GD + g * D + c * 4) = num;
        if (c == 0)
            *(float2 *)(ws_ml + ((u * splits + split) * gt + g) * 2) = float2{mx, den};
    }
}

// Finishes one (sequence, unit) split after its waves have staged their
// (m, l, O) in LDS (sm_m, sm_l: [MW][16]; sm_o: [MW][16][D + 4]): combines
// the waves, four columns per thread; with one split writes `out`, otherwise
// writes the split's partial (O unnormalised, then m, l) for
// decode_merge_kernel.
template <int D, int MW = kMW>
__device__ void finish_unit(const float *sm_m, const float *sm_l, const float *sm_o, int b,
                            int unit, int split, int splits, int gt, int n_units, int n_head,
                            int head0, float *__restrict__ out, float *__restrict__ ws_ml,
                            float *__restrict__ ws_acc) {
    constexpr int NT = MW * 64, C4 = D / 4;
    const int tid = threadIdx.x;
    const int64_t u = (int64_t)b * n_units + unit;
    const int GD = gt * D;
    for (int idx = tid; idx < gt * C4; idx += NT) {
        const int g = idx / C4, c = idx % C4;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < MW; w++) mx = fmaxf(mx, sm_m[w * 16 + g]);
        const float mu = mx == -INFINITY ? 0.f : mx;
        f32x4 num = {0.f, 0.f, 0.f, 0.f};
        float den = 0.f;
#pragma unroll
        for (int w = 0; w < MW; w++) {
            const float cw = __builtin_amdgcn_exp2f(sm_m[w * 16 + g] - mu);
            num += *(const f32x4 *)&sm_o[(w * 16 + g) * (D + 4) + c * 4] * cw;
            den += sm_l[w * 16 + g] * cw;
        }
        store_split<D>(num, mx, den, c, g, b, split, splits, gt, n_head, head0, u, GD, out,
                       ws_ml, ws_acc);
    }
}

// PG: paged cache, addressed as in decode_dma_kernel below (a block's loads
// go through a buffer resource based at its page).
template <class T, int D, bool PG = false, int MW = kMW>
__global__ __launch_bounds__(MW * 64, D <= 128 ? 2 : 1) void decode_mfma_kernel(
    const float *__restrict__ q, const char *__restrict__ kc, const char *__restrict__ vc,
    int64_t kv_stride, int64_t seq_stride, const int32_t *__restrict__ seq_lens, int window,
    int fetch_len, int n_head, int kv_mul, int gt, int n_units, int chunk, int splits, float qscale,
    float *__restrict__ out, float *__restrict__ ws_ml, float *__restrict__ ws_acc,
    const int32_t *__restrict__ ptab, int ptab_stride, int page_shift, int n_pages) {
    constexpr int NS = D / 32;      // QK k-steps (32 d each)
    constexpr int NDT = D / 16;     // 16-wide d tiles of O^T
    constexpr int CPR = D / 8;      // 16-byte chunks per key row
    constexpr int VP = D + 16;      // LDS V row pitch (halves): conflict-free rows
    constexpr bool SPLITP = __is_same(T, BF16);

    const int split = blockIdx.x, unit = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int n16 = lane & 15, kg = lane >> 4;
    const int head0 = unit * gt, kvh = head0 / kv_mul;
    const bool head_ok = n16 < gt;

    // Raw q loads go out first (vmcnt retires in order, so q must precede
    // the K/V stream to be waited for on its own).
    f32x4 qa[NS][2];
    {
        const float *qp = q + ((int64_t)b * n_head + head0 + (head_ok ? n16 : 0)) * D;
#pragma unroll
        for (int s = 0; s < NS; s++) {
            qa[s][0] = *(const f32x4 *)(qp + (s * 4 + kg) * 8);
            qa[s][1] = *(const f32x4 *)(qp + (s * 4 + kg) * 8 + 4);
        }
    }

    // fetch_len > 0: the window cannot bind and keys 0..fetch_len-1 are
    // readable, so the first block is fetched before seq_lens[b] arrives
    // (keys past the length are masked (K) and zeroed (V) once it is known).
    const int len = __builtin_amdgcn_readfirstlane(seq_lens[b]);
    const int start = (fetch_len > 0 || window <= 0 || len <= window) ? 0 : len - window;
    const int c0 = (fetch_len > 0 ? 0 : (PG ? start & ~(kTok - 1) : start)) + split * chunk;
    const int c1 = min(c0 + chunk, len);
    const int cf = fetch_len > 0 ? min(c0 + chunk, fetch_len) : c1;

    __shared__ __attribute__((aligned(16))) uint16_t vt_all[MW][kTok * VP];
    uint16_t *vt = vt_all[wave];

    u32x4 qh[NS], ql[NS];  // Q^T operand (filled once the first block is in flight)
    f32x4 oacc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; i++) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_part = 0.f;

    const int rb = (int)(kv_stride * 2);  // bytes per key row
    // Buffer resources over this sequence's kv head, ending at key c1: loads
    // of keys >= c1 fall outside the range and return zero.
    const char *kb0 = kc + (int64_t)b * seq_stride * 2 + (int64_t)kvh * D * 2;
    const char *vb0 = vc + (int64_t)b * seq_stride * 2 + (int64_t)kvh * D * 2;
    const int range = cf > 0 ? (cf - 1) * rb + D * 2 : 0;
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(kb0), 0, range, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(vb0), 0, range, kRsrcWord3);

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
        __amdgpu_buffer_rsrc_t kr = krs, vr = vrs;
        int so;
        if constexpr (PG) {
            const int pg = __builtin_amdgcn_readfirstlane(tb >> page_shift);
            const int phys = pg < ptab_stride ? ptab[(int64_t)b * ptab_stride + pg] : -1;
            const bool ok = phys >= 0 && phys < n_pages;
            const int64_t pb = ((int64_t)(ok ? phys : 0) << page_shift) * rb + (int64_t)kvh * D * 2;
            const int prange = ok ? (rb << page_shift) : 0;
            kr = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(kc + pb), 0, prange, kRsrcWord3);
            vr = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(vc + pb), 0, prange, kRsrcWord3);
            so = __builtin_amdgcn_readfirstlane((tb & ((1 << page_shift) - 1)) * rb);
        } else {
            so = __builtin_amdgcn_readfirstlane(tb * rb);
        }
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int s = 0; s < NS; s++)
                T_.k[t][s] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, koffb[t] + s * 64 + so, 0, 2));
#pragma unroll
        for (int i = 0; i < VL; i++)
            T_.v[i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, voffb + i * KPI * rb + so, 0, 2));
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
        // V rows into the wave's LDS tile (row-major, padded pitch); fetched
        // rows at or past the length are zeroed (P is 0 there, 0 * NaN is not)
#pragma unroll
        for (int i = 0; i < VL; i++) {
            u32x4 vv = T_.v[i];
            if ((fetch_len > 0 || PG) && tb + vrow0 + i * KPI >= c1) vv = u32x4{0u, 0u, 0u, 0u};
            if (PG && tb + vrow0 + i * KPI < start) vv = u32x4{0u, 0u, 0u, 0u};
            *(u32x4 *)(vt + (vrow0 + i * KPI) * VP + vcol * 8) = vv;
        }
        // online softmax: lane = head n16, keys kg*4+i (tile 0) and 16+kg*4+i
        float sv[8];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) sv[t * 4 + i] = sacc[t][i];
        if (tb + kTok > c1) {  // partial block (wave-uniform branch)
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (tb + t * 16 + kg * 4 + i >= c1) sv[t * 4 + i] = -INFINITY;
        }
        if (PG && tb < start) {  // keys of the first block before the window start
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (tb + t * 16 + kg * 4 + i < start) sv[t * 4 + i] = -INFINITY;
        }
        float mt = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                         fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
        mt = rows_max(mt);
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
            if constexpr (SPLITP) {
                const u32x2 hl = split2<T>(p[2 * j], p[2 * j + 1]);
                ph[j] = hl[0];
                pl[j] = hl[1];
            } else {
                ph[j] = pack2<T>(p[2 * j], p[2 * j + 1]);
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
    constexpr int STEP = MW * kTok;
    int tb = c0 + wave * kTok;
    Tile A_;
    issue(A_, tb);  // first block in flight while q is prepared (past c1: zeros)

    // Q^T operand, hi/lo split: step s, lane (head n16, chunk c = s*4 + kg).
#pragma unroll
    for (int s = 0; s < NS; s++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float x0 = head_ok ? qa[s][j >> 1][(2 * j) & 3] * qscale : 0.f;
            const float x1 = head_ok ? qa[s][j >> 1][(2 * j + 1) & 3] * qscale : 0.f;
            const u32x2 hl = split2<T>(x0, x1);
            qh[s][j] = hl[0];
            ql[s][j] = hl[1];
        }

    if constexpr (D <= 128) {
        Tile B_;
        if (tb < c1) {
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
            consume(A_, tb);
            if (tb + STEP < c1) issue(A_, tb + STEP);
        }
    }

    // ---- wave result: head n16, d = dt*16 + kg*4 + i ----
    l_part = rows_sum(l_part);
    if constexpr (MW == 1) {
        // One wave: its registers are the split's result, written without an
        // LDS round trip (as decode_dma_kernel's one-wave path).
        if (head_ok) {
            const int64_t u = (int64_t)b * n_units + unit;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
                store_split<D>(oacc[dt], m_run, l_part, dt * 4 + kg, n16, b, split, splits, gt,
                               n_head, head0, u, gt * D, out, ws_ml, ws_acc);
        }
        return;
    }

    __syncthreads();  // all waves done with their V^T tiles: reuse the LDS
    float *sm = (float *)&vt_all[0][0];
    float *sm_m = sm;                                 // [MW][16]
    float *sm_l = sm + MW * 16;                      // [MW][16]
    float *sm_o = sm + 2 * MW * 16;                  // [MW][16][D + 4]
    if (kg == 0) { sm_m[wave * 16 + n16] = m_run; sm_l[wave * 16 + n16] = l_part; }
    // Row pitch D + 4 floats: the 16 heads of a lane group land on different
    // banks (a pitch of D would put them all on one).
#pragma unroll
    for (int dt = 0; dt < NDT; dt++)
        *(f32x4 *)&sm_o[(wave * 16 + n16) * (D + 4) + dt * 16 + kg * 4] = oacc[dt];
    __syncthreads();

    finish_unit<D, MW>(sm_m, sm_l, sm_o, b, unit, split, splits, gt, n_units, n_head, head0,
                       out, ws_ml, ws_acc);
}

}  // namespace ullm

namespace ullm {

// LDS-staged variant for head_dim <= 128: K and V tiles go global -> LDS by
// buffer_load ... lds (no staging registers), each instruction covering whole
// contiguous head rows of 4 (D=128) or 8 (D=64) keys.  A row of the tile is
// D*2 bytes in 16-byte slots; slot p of row r holds chunk p ^ (r % SLOTS), an
// XOR swizzle applied by permuting the global chunk each lane fetches, so the
// MFMA-operand reads below hit distinct banks.  K operands come from
// ds_read_b128, V^T operands from the transposing ds_read_b64_tr_b16.  Each
// wave owns two stages (double buffering); the wait for a stage leaves the
// other stage's transfers in flight.
//
// PG (paged cache): kc/vc are pools of pages of 2^page_shift token rows
// (kv_stride elements each); token t of sequence b lives in row t % P of
// page ptab[b * ptab_stride + t / P].  Every 32-key block lies inside one
// page (P is a multiple of 32), so a block's DMA goes through a buffer
// resource based at its page, whose range (one page; zero for a page index
// outside [0, n_pages)) bounds every read.  With a binding window the blocks
// start at the window start rounded down to 32 keys and the keys before it
// are masked.  Rows outside [start, length) hold whatever the page holds
// there: their V rows are zeroed in LDS (P is 0 for them, but 0 * NaN is
// NaN).

template <class T, int D, int MW, bool PG = false>
__global__ __launch_bounds__(MW * 64, 1) void decode_dma_kernel(
    const float *__restrict__ q, const char *__restrict__ kc, const char *__restrict__ vc,
    int64_t kv_stride, int64_t seq_stride, const int32_t *__restrict__ seq_lens, int window,
    int fetch_len, int n_head, int kv_mul, int gt, int n_units, int chunk, int splits, float qscale,
    float *__restrict__ out, float *__restrict__ ws_ml, float *__restrict__ ws_acc,
    const int32_t *__restrict__ ptab, int ptab_stride, int page_shift, int n_pages) {
    constexpr int NS = D / 32;          // QK k-steps (32 d each)
    constexpr int NDT = D / 16;         // 16-wide d tiles of O^T
    // An f32 cache (the reference's) arrives as f32 tiles; both contractions
    // then run on bf16 MFMAs over hi + lo halves, as in decode_block_kernel:
    // Q.K = Khi.Qhi + Khi.Qlo + Klo.Qhi, P.V = Vhi.Phi + Vhi.Plo + Vlo.Phi.
    constexpr bool F = __is_same(T, F32);
    using MT = typename std::conditional<F, BF16, T>::type;  // MFMA operand type
    constexpr int EB = T::bytes;        // cache element bytes
    constexpr int RB = D * EB;          // bytes per key row of one head
    constexpr int SLOTS = RB / 16;      // 16-byte slots per row
    constexpr int RPI = 1024 / RB;      // rows written by one DMA instruction
    constexpr int NI = kTok / RPI;      // DMA instructions per K (or V) tile
    constexpr int TILE = kTok * RB;     // bytes of one K (or V) tile
    constexpr int STAGE = 2 * TILE;     // K tile then V tile
    constexpr bool SPLITP = !__is_same(T, F16);
    static_assert(D == 64 || D == 128, "DMA decode path covers head_dim 64 and 128");
    static_assert(2 * MW * STAGE <= 160 * 1024, "two LDS stages per wave");

    const int split = blockIdx.x, unit = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n16 = lane & 15, kg = lane >> 4;
    const int head0 = unit * gt, kvh = head0 / kv_mul;
    const bool head_ok = n16 < gt;

    // One array per stage: the stage a read targets is then a distinct
    // object from the stage the DMA is filling, which keeps the compiler from
    // draining all DMA (vmcnt(0)) before every LDS read.
    __shared__ __attribute__((aligned(1024))) char lds0[MW * STAGE];
    __shared__ __attribute__((aligned(1024))) char lds1[MW * STAGE];
    char *const wb0 = lds0 + wave * STAGE;
    char *const wb1 = lds1 + wave * STAGE;

    // With fetch_len > 0 the window cannot bind (the split starts at
    // split * chunk whatever the length) and keys 0..fetch_len-1 are
    // readable: the K/V stream starts before seq_lens[b] arrives, over keys
    // c0..cf-1, and keys past the length are masked (K) and zeroed (V) once
    // it is known.  Otherwise the stream ends at the length (c1) and the
    // buffer range returns zero past it.
    // The length comes by a vector load (a scalar one would be waited for
    // together with the kernel arguments, before anything is issued).
    const __amdgpu_buffer_rsrc_t lrs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(seq_lens + b), 0, 4, kRsrcWord3);
    int lenv = __builtin_amdgcn_raw_buffer_load_b32(lrs, 0, 0, 0);
    int len, c1;
    auto take_len = [&] {
        asm volatile("" : "+v"(lenv));  // keeps the wait for it here
        len = __builtin_amdgcn_readfirstlane(lenv);
    };
    if (fetch_len <= 0) take_len();
    const int start = (fetch_len > 0 || window <= 0 || len <= window) ? 0 : len - window;
    const int c0 = (fetch_len > 0 ? 0 : (PG ? start & ~(kTok - 1) : start)) + split * chunk;
    const int cf = fetch_len > 0 ? min(c0 + chunk, fetch_len) : min(c0 + chunk, len);

    const int rb = (int)(kv_stride * EB);
    const char *kb0 = kc + (int64_t)b * seq_stride * EB + (int64_t)kvh * RB;
    const char *vb0 = vc + (int64_t)b * seq_stride * EB + (int64_t)kvh * RB;
    const int range = cf > 0 ? (cf - 1) * rb + RB : 0;
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(kb0), 0, range, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(vb0), 0, range, kRsrcWord3);

    // DMA lane map: instruction i writes rows i*RPI + lane/SLOTS, slot lane%SLOTS.
    const int drow = lane / SLOTS, dslot = lane % SLOTS;
    int dofs[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int r = i * RPI + drow;
        dofs[i] = r * rb + ((dslot ^ (r & (SLOTS - 1))) * 16);
    }
    auto issue = [&](char *kt, int tb) {
        char *vt = kt + TILE;
        if constexpr (PG) {
            const int pg = __builtin_amdgcn_readfirstlane(tb >> page_shift);
            // A table index past the row (a length above max_len) is an
            // invalid page too: never read past the caller's table.
            const int phys = pg < ptab_stride ? ptab[(int64_t)b * ptab_stride + pg] : -1;
            const bool ok = phys >= 0 && phys < n_pages;
            const int64_t pb = ((int64_t)(ok ? phys : 0) << page_shift) * rb + (int64_t)kvh * RB;
            const int prange = ok ? (rb << page_shift) : 0;
            const __amdgpu_buffer_rsrc_t kp =
                __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(kc + pb), 0, prange, kRsrcWord3);
            const __amdgpu_buffer_rsrc_t vp =
                __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(vc + pb), 0, prange, kRsrcWord3);
            const int so = __builtin_amdgcn_readfirstlane((tb & ((1 << page_shift) - 1)) * rb);
#pragma unroll
            for (int i = 0; i < NI; i++)
                dma16(kp, kt + i * 1024, dofs[i] + so, 0);
#pragma unroll
            for (int i = 0; i < NI; i++)
                dma16(vp, vt + i * 1024, dofs[i] + so, 0);
        } else {
            const int so = __builtin_amdgcn_readfirstlane(tb * rb);
#pragma unroll
            for (int i = 0; i < NI; i++)
                dma16(krs, kt + i * 1024, dofs[i] + so, 0);
#pragma unroll
            for (int i = 0; i < NI; i++)
                dma16(vrs, vt + i * 1024, dofs[i] + so, 0);
        }
    };

    // q goes out first: waiting for it then leaves the K/V stages in flight.
    f32x4 qa[NS][2];
    {
        const float *qp = q + ((int64_t)b * n_head + head0 + (head_ok ? n16 : 0)) * D;
#pragma unroll
        for (int s = 0; s < NS; s++) {
            qa[s][0] = *(const f32x4 *)(qp + (s * 4 + kg) * 8);
            qa[s][1] = *(const f32x4 *)(qp + (s * 4 + kg) * 8 + 4);
        }
    }
    // Stages are issued only for keys in the fetched range (a wave with one
    // block issues one stage); a stage is waited for with the other stage
    // still counted only when that one was issued, else with vmcnt(0).
    constexpr int STEP = MW * kTok;
    const int tb0 = c0 + wave * kTok;
    if (tb0 < cf) issue(wb0, tb0);
    if (tb0 + STEP < cf) issue(wb1, tb0 + STEP);
    if (fetch_len > 0) take_len();
    c1 = min(c0 + chunk, len);

    u32x4 qh[NS], ql[NS];
#pragma unroll
    for (int s = 0; s < NS; s++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float x0 = head_ok ? qa[s][j >> 1][(2 * j) & 3] * qscale : 0.f;
            const float x1 = head_ok ? qa[s][j >> 1][(2 * j + 1) & 3] * qscale : 0.f;
            const u32x2 hl = split2<MT>(x0, x1);
            qh[s][j] = hl[0];
            ql[s][j] = hl[1];
        }

    f32x4 oacc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; i++) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_part = 0.f;

    // more: the other stage is in flight behind this one.  The K tile is
    // waited for first and V stays in flight through Q.K and the softmax.
    auto consume = [&](const char *kt, int tb, bool more) {
        const char *vt = kt + TILE;
        if (more) __builtin_amdgcn_s_waitcnt(vm_wait(3 * NI));
        else __builtin_amdgcn_s_waitcnt(vm_wait(NI));
        // S^T = K . Q^T: lane (key t*16 + n16, chunk s*4 + kg)
        const uint32_t kbase = lds_addr(kt);
        constexpr int KR = F ? 2 : 1;  // 16-byte reads per operand
        u32x4 ka[2 * NS * KR];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int r = t * 16 + n16;
#pragma unroll
            for (int s = 0; s < NS; s++)
#pragma unroll
                for (int h = 0; h < KR; h++)
                    ka[(t * NS + s) * KR + h] =
                        lds_read_b128(kbase + r * RB + ((((s * 4 + kg) * KR + h) ^ (r & (SLOTS - 1))) * 16));
        }
        lds_wait(ka);
        f32x4 sacc[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            sacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < NS; s++) {
                if constexpr (F) {
                    const u32x4 a = ka[(t * NS + s) * 2], c = ka[(t * NS + s) * 2 + 1];
                    u32x4 kh, kl;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const u32x4 &src = j < 2 ? a : c;
                        const u32x2 hl = split2<BF16>(__uint_as_float(src[(2 * j) & 3]),
                                                      __uint_as_float(src[(2 * j + 1) & 3]));
                        kh[j] = hl[0];
                        kl[j] = hl[1];
                    }
                    sacc[t] = mfma16<BF16>(kh, qh[s], sacc[t]);
                    sacc[t] = mfma16<BF16>(kh, ql[s], sacc[t]);
                    sacc[t] = mfma16<BF16>(kl, qh[s], sacc[t]);
                } else {
                    sacc[t] = mfma16<T>(ka[t * NS + s], qh[s], sacc[t]);
                    sacc[t] = mfma16<T>(ka[t * NS + s], ql[s], sacc[t]);
                }
            }
        }
        float sv[8];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) sv[t * 4 + i] = sacc[t][i];
        if (tb + kTok > c1) {
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (tb + t * 16 + kg * 4 + i >= c1) sv[t * 4 + i] = -INFINITY;
        }
        if (PG && tb < start) {
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (tb + t * 16 + kg * 4 + i < start) sv[t * 4 + i] = -INFINITY;
        }
        float mt = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                         fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
        mt = rows_max(mt);
        const float m_new = fmaxf(m_run, mt);
        const float mu = m_new == -INFINITY ? 0.f : m_new;
        if (__any(m_new != m_run)) {
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
            if constexpr (SPLITP) {
                const u32x2 hl = split2<MT>(p[2 * j], p[2 * j + 1]);
                ph[j] = hl[0];
                pl[j] = hl[1];
            } else {
                ph[j] = pack2<T>(p[2 * j], p[2 * j + 1]);
            }
        }
        if (more) __builtin_amdgcn_s_waitcnt(vm_wait(2 * NI));
        else __builtin_amdgcn_s_waitcnt(vm_wait(0));
        if ((fetch_len > 0 || PG) && tb + kTok > c1) {
            // Fetched rows at or past the length hold whatever the cache
            // holds there (P is 0 for them, but 0 * NaN is NaN): zero them.
            const uint32_t vz = lds_addr(vt);
            const int nv = max(c1 - tb, 0);
            for (int i = nv * SLOTS + lane; i < kTok * SLOTS; i += 64)
                lds_write_b128(vz + i * 16, u32x4{0u, 0u, 0u, 0u});
        }
        if (PG && tb < start) {  // rows of the first block before the window start
            const uint32_t vz = lds_addr(vt);
            const int nz = min(start - tb, kTok);
            for (int i = lane; i < nz * SLOTS; i += 64)
                lds_write_b128(vz + i * 16, u32x4{0u, 0u, 0u, 0u});
        }
        // O^T += V^T . P^T; lane n16 of key group kg reads V rows kg*4 + n16/4
        // (+16), elements dt*16 + 4*(n16 % 4) .. +3, transposed by the read.
        if constexpr (F) {
            // V^T operand gathered from the f32 rows: lane (d = dt*16 + n16,
            // kg) takes rows kg*4 + j and 16 + kg*4 + j (j < 4) of column d,
            // then splits them into bf16 hi and lo halves.
            const uint32_t vbase = lds_addr(vt);
            float vv[NDT][8];
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                const int d = dt * 16 + n16;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const int r = (j >> 2) * 16 + kg * 4 + (j & 3);
                    vv[dt][j] = __uint_as_float(lds_read_b32(
                        vbase + r * RB + (((d >> 2) ^ (r & (SLOTS - 1))) * 16) + (d & 3) * 4));
                }
            }
            lds_wait_any();
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
#pragma unroll
                for (int j = 0; j < 8; j++) tie_f(vv[dt][j]);
                u32x4 vh, vl;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const u32x2 hl = split2<BF16>(vv[dt][2 * j], vv[dt][2 * j + 1]);
                    vh[j] = hl[0];
                    vl[j] = hl[1];
                }
                oacc[dt] = mfma16<BF16>(vh, ph, oacc[dt]);
                oacc[dt] = mfma16<BF16>(vh, pl, oacc[dt]);
                oacc[dt] = mfma16<BF16>(vl, ph, oacc[dt]);
            }
            return;
        }
        const int vr0 = kg * 4 + (n16 >> 2);
        const uint32_t vbase = lds_addr(vt);
        u32x4 va[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            const int ch = dt * 2 + ((n16 & 3) >> 1);
            const int bo = 8 * (n16 & 1);
            const u32x2 l2 = lds_read_tr16_b64(vbase + vr0 * RB + ((ch ^ (vr0 & (SLOTS - 1))) * 16) + bo);
            const u32x2 h2 = lds_read_tr16_b64(vbase + (vr0 + 16) * RB +
                                               ((ch ^ ((vr0 + 16) & (SLOTS - 1))) * 16) + bo);
            va[dt] = u32x4{l2[0], l2[1], h2[0], h2[1]};
        }
        lds_wait(va);
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            oacc[dt] = mfma16<T>(va[dt], ph, oacc[dt]);
            if constexpr (SPLITP) oacc[dt] = mfma16<T>(va[dt], pl, oacc[dt]);
        }
    };
    // Unrolled by the two stages; each stage is refilled once its LDS reads
    // have retired (lgkmcnt(0)), two blocks ahead.
    constexpr int kLgkm0 = vm_wait(63) & ~(15 << 8);
    // Past the first two stages only keys below the length are fetched, so
    // from there on "issued" is "below c1".
    for (int tb = tb0; tb < c1; tb += 2 * STEP) {
        const bool next1 = tb == tb0 ? tb + STEP < cf : tb + STEP < c1;
        consume(wb0, tb, next1);  // stage 1 in flight behind it when next1
        __builtin_amdgcn_s_waitcnt(kLgkm0);
        if (tb + 2 * STEP < c1) issue(wb0, tb + 2 * STEP);
        if (tb + STEP >= c1) break;
        consume(wb1, tb + STEP, tb + 2 * STEP < c1);
        __builtin_amdgcn_s_waitcnt(kLgkm0);
        if (tb + 3 * STEP < c1) issue(wb1, tb + 3 * STEP);
    }
    __builtin_amdgcn_s_waitcnt(vm_wait(0));  // drain DMA before the LDS is reused

    l_part = rows_sum(l_part);
    if constexpr (MW == 1) {
        // One wave: its registers are the split's result (lane: head n16,
        // columns dt*16 + kg*4 .. +3), written without an LDS round trip.
        if (head_ok) {
            const int64_t u = (int64_t)b * n_units + unit;
            if (splits == 1) {
#pragma unroll
                for (int dt = 0; dt < NDT; dt++)
                    store_split<D>(oacc[dt], m_run, l_part, dt * 4 + kg, n16, b, split, splits, gt,
                                   n_head, head0, u, gt * D, out, ws_ml, ws_acc);
            } else {
                // The split's partial: O unnormalised, then (m, l) once per head.
                float *ap = ws_acc + (u * splits + split) * (gt * D) + n16 * D + kg * 4;
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) *(f32x4 *)(ap + dt * 16) = oacc[dt];
                if (kg == 0)
                    *(float2 *)(ws_ml + ((u * splits + split) * gt + n16) * 2) = float2{m_run, l_part};
            }
        }
        return;
    }
    __syncthreads();
    float *sm = (float *)lds0;  // MW*16*(D+2) floats fit in one stage array
    float *sm_m = sm, *sm_l = sm + MW * 16, *sm_o = sm + 2 * MW * 16;
    if (kg == 0) { sm_m[wave * 16 + n16] = m_run; sm_l[wave * 16 + n16] = l_part; }
    // Row pitch D + 4 floats: the 16 heads of a lane group land on different
    // banks (a pitch of D would put them all on one).
#pragma unroll
    for (int dt = 0; dt < NDT; dt++)
        *(f32x4 *)&sm_o[(wave * 16 + n16) * (D + 4) + dt * 16 + kg * 4] = oacc[dt];
    __syncthreads();
    finish_unit<D, MW>(sm_m, sm_l, sm_o, b, unit, split, splits, gt, n_units, n_head, head0,
                       out, ws_ml, ws_acc);
}

// Splits of one or two blocks (short contexts: cfg2 cuts 4096 keys into 128
// one-block splits per kv head), on one-wave workgroups.  Straight-line code:
// q loads, the DMA of every block's K and V tiles at once, then per block
// S^T = K.Q^T and the softmax once its K has landed, O^T += V^T.P^T once its
// V has, and the split's store.  Measured at cfg2: 6.44 us per layer (graph
// of 28 layers) against 6.92 for the same splits on decode_dma_kernel's
// one-wave workgroups (its two-stage loop around the one block); sharing the
// block among 2, 4 or 8 waves measured 6.45, 6.65 and 7.31.  Same arguments,
// masks and partial layout as decode_dma_kernel (chunk = NB * KB).  KB = 16
// (head_dim 256): a block is one 16-key tile, so a short context spreads
// over twice the workgroups; the P^T operand's keys 16-31 are zero.
template <class T, int D, int NB, int KB = kTok>
__global__ __launch_bounds__(64, 1) void decode_block_kernel(
    const float *__restrict__ q, const char *__restrict__ kc, const char *__restrict__ vc,
    int64_t kv_stride, int64_t seq_stride, const int32_t *__restrict__ seq_lens, int window,
    int fetch_len, int n_head, int kv_mul, int gt, int n_units, int chunk, int splits, float qscale,
    float *__restrict__ out, float *__restrict__ ws_ml, float *__restrict__ ws_acc) {
    constexpr int NS = D / 32;          // QK k-steps (32 d each)
    constexpr int NDT = D / 16;         // 16-wide d tiles of O^T
    // An f32 cache (the reference's) runs both contractions on bf16 MFMAs
    // over hi + lo halves: Q.K = Khi.Qhi + Khi.Qlo + Klo.Qhi and
    // P.V = Vhi.Phi + Vhi.Plo + Vlo.Phi (about 2^-16 of each product).
    constexpr bool F = __is_same(T, F32);
    using MT = typename std::conditional<F, BF16, T>::type;  // MFMA operand type
    constexpr int RB = D * T::bytes;    // bytes per key row of one head
    constexpr int SLOTS = RB / 16;      // 16-byte slots per row
    constexpr int RPI = 1024 / RB;      // rows written by one DMA instruction
    constexpr int NI = KB / RPI;        // DMA instructions per K (or V) tile
    constexpr int TILE = KB * RB;
    constexpr int NT = KB / 16;         // 16-key tiles per block
    constexpr bool SPLITP = !__is_same(T, F16);
    static_assert(!F || KB == 32, "f32: 32-key blocks");
    static_assert(D == 64 || D == 128 || D == 256, "head_dim 64, 128, 256");
    static_assert(KB == 16 || KB == 32, "keys per block");

    const int split = blockIdx.x, unit = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63;
    const int n16 = lane & 15, kg = lane >> 4;
    const int head0 = unit * gt, kvh = head0 / kv_mul;
    const bool head_ok = n16 < gt;
    // Block i: K tile at 2i TILE, V tile at (2i + 1) TILE.
    __shared__ __attribute__((aligned(1024))) char lds[2 * NB * TILE];

    // Length, window start and fetched range exactly as decode_dma_kernel.
    const __amdgpu_buffer_rsrc_t lrs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(seq_lens + b), 0, 4, kRsrcWord3);
    int lenv = __builtin_amdgcn_raw_buffer_load_b32(lrs, 0, 0, 0);
    int len;
    auto take_len = [&] {
        asm volatile("" : "+v"(lenv));
        len = __builtin_amdgcn_readfirstlane(lenv);
    };
    if (fetch_len <= 0) take_len();
    const int start = (fetch_len > 0 || window <= 0 || len <= window) ? 0 : len - window;
    const int c0 = (fetch_len > 0 ? 0 : start) + split * chunk;
    const int cf = fetch_len > 0 ? min(c0 + chunk, fetch_len) : min(c0 + chunk, len);

    constexpr int EB = T::bytes;  // cache element bytes
    const int rb = (int)(kv_stride * EB);
    const char *kb0 = kc + (int64_t)b * seq_stride * EB + (int64_t)kvh * RB;
    const char *vb0 = vc + (int64_t)b * seq_stride * EB + (int64_t)kvh * RB;
    const int range = cf > 0 ? (cf - 1) * rb + RB : 0;
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(kb0), 0, range, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(vb0), 0, range, kRsrcWord3);

    // q first, then the DMA instructions of every block: K0, V0, K1, ...
    // (a block wholly past the fetched range is not requested).
    f32x4 qa[NS][2];
    {
        const float *qp = q + ((int64_t)b * n_head + head0 + (head_ok ? n16 : 0)) * D;
#pragma unroll
        for (int s = 0; s < NS; s++) {
            qa[s][0] = *(const f32x4 *)(qp + (s * 4 + kg) * 8);
            qa[s][1] = *(const f32x4 *)(qp + (s * 4 + kg) * 8 + 4);
        }
    }
    const int nfb = min(max((cf - c0 + KB - 1) / KB, 0), NB);  // blocks fetched (uniform)
    {
        const int drow = lane / SLOTS, dslot = lane % SLOTS;
        static_for<0, NB>([&](auto bc) {
            constexpr int bi = decltype(bc)::value;
            if (bi < nfb) {
                const int so = __builtin_amdgcn_readfirstlane((c0 + bi * KB) * rb);
#pragma unroll
                for (int i = 0; i < NI; i++) {
                    const int r = (i) * RPI + drow;
                    dma16(krs, lds + 2 * bi * TILE + (i) * 1024,
                          r * rb + ((dslot ^ (r & (SLOTS - 1))) * 16) + so, 0);
                }
#pragma unroll
                for (int i = 0; i < NI; i++) {
                    const int r = (i) * RPI + drow;
                    dma16(vrs, lds + (2 * bi + 1) * TILE + (i) * 1024,
                          r * rb + ((dslot ^ (r & (SLOTS - 1))) * 16) + so, 0);
                }
            }
        });
    }
    if (fetch_len > 0) take_len();
    const int c1 = min(c0 + chunk, len);

    u32x4 qh[NS], ql[NS];
#pragma unroll
    for (int s = 0; s < NS; s++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float x0 = head_ok ? qa[s][j >> 1][(2 * j) & 3] * qscale : 0.f;
            const float x1 = head_ok ? qa[s][j >> 1][(2 * j + 1) & 3] * qscale : 0.f;
            const u32x2 hl = split2<MT>(x0, x1);
            qh[s][j] = hl[0];
            ql[s][j] = hl[1];
        }

    f32x4 oacc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; i++) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_part = 0.f;
    // Block bi: its K is waited for with V bi and the later blocks still
    // counted; its V with the later blocks counted.  Those counts hold when
    // every block was fetched; a split with fewer (the end of a sequence)
    // waits for all of its DMA instead.
    static_for<0, NB>([&](auto bc) {
        constexpr int bi = decltype(bc)::value;
        const int tb = c0 + bi * KB;
        if (bi >= nfb) return;
        if (nfb == NB) __builtin_amdgcn_s_waitcnt(vm_wait((2 * (NB - bi) - 1) * NI));
        else __builtin_amdgcn_s_waitcnt(vm_wait(0));
        if (tb >= c1) {  // fetched but past the length: nothing to add
            __builtin_amdgcn_s_waitcnt(vm_wait(0));
            return;
        }
        const uint32_t kbase = lds_addr(lds + 2 * bi * TILE);
        // lane (key t*16 + n16, k-group kg): d = s*32 + kg*8 .. +7
        constexpr int KR = F ? 2 : 1;  // 16-byte reads per operand
        u32x4 ka[NT * NS * KR];
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int r = t * 16 + n16;
#pragma unroll
            for (int s = 0; s < NS; s++)
#pragma unroll
                for (int h = 0; h < KR; h++)
                    ka[(t * NS + s) * KR + h] =
                        lds_read_b128(kbase + r * RB + ((((s * 4 + kg) * KR + h) ^ (r & (SLOTS - 1))) * 16));
        }
        lds_wait(ka);
        f32x4 sacc[2];
        sacc[1] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};  // keys 16-31 of a 16-key block
#pragma unroll
        for (int t = 0; t < NT; t++) {
            sacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < NS; s++) {
                if constexpr (F) {
                    const u32x4 a = ka[(t * NS + s) * 2], c = ka[(t * NS + s) * 2 + 1];
                    u32x4 kh, kl;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const u32x4 &src = j < 2 ? a : c;
                        const u32x2 hl = split2<BF16>(__uint_as_float(src[(2 * j) & 3]),
                                                      __uint_as_float(src[(2 * j + 1) & 3]));
                        kh[j] = hl[0];
                        kl[j] = hl[1];
                    }
                    sacc[t] = mfma16<BF16>(kh, qh[s], sacc[t]);
                    sacc[t] = mfma16<BF16>(kh, ql[s], sacc[t]);
                    sacc[t] = mfma16<BF16>(kl, qh[s], sacc[t]);
                } else {
                    sacc[t] = mfma16<T>(ka[t * NS + s], qh[s], sacc[t]);
                    sacc[t] = mfma16<T>(ka[t * NS + s], ql[s], sacc[t]);
                }
            }
        }
        float sv[8];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) sv[t * 4 + i] = sacc[t][i];
        if (tb + KB > c1) {
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (tb + t * 16 + kg * 4 + i >= c1) sv[t * 4 + i] = -INFINITY;
        }
        float mt = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                         fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
        mt = rows_max(mt);
        const float m_new = fmaxf(m_run, mt);
        const float mu = m_new == -INFINITY ? 0.f : m_new;
        if (bi > 0 && __any(m_new != m_run)) {
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
            if constexpr (SPLITP) {
                const u32x2 hl = split2<MT>(p[2 * j], p[2 * j + 1]);
                ph[j] = hl[0];
                pl[j] = hl[1];
            } else {
                ph[j] = pack2<T>(p[2 * j], p[2 * j + 1]);
            }
        }
        if (nfb == NB) __builtin_amdgcn_s_waitcnt(vm_wait(2 * (NB - bi - 1) * NI));
        else __builtin_amdgcn_s_waitcnt(vm_wait(0));
        const uint32_t vbase = lds_addr(lds + (2 * bi + 1) * TILE);
        if (tb + KB > c1) {
            // Fetched rows at or past the length hold whatever the cache
            // holds there (P is 0 for them, but 0 * NaN is NaN): zero them.
            const int nv = max(c1 - tb, 0);
            for (int i = nv * SLOTS + lane; i < KB * SLOTS; i += 64)
                lds_write_b128(vbase + i * 16, u32x4{0u, 0u, 0u, 0u});
        }
        const int vr0 = kg * 4 + (n16 >> 2);
        u32x4 va[NDT];
        if constexpr (F) {
            // V^T operand gathered from the f32 rows: lane (d = dt*16 + n16,
            // kg) takes rows kg*4 + j and 16 + kg*4 + j (j < 4) of column d,
            // then splits them into bf16 hi (va) and lo (vl) halves.
            u32x4 vl[NDT];
            float vv[NDT][8];
#pragma unroll
            for (int i = 0; i < NDT; i++) {
                const int d = i * 16 + n16;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const int r = (j >> 2) * 16 + kg * 4 + (j & 3);
                    vv[i][j] = *(const float *)(lds + (2 * bi + 1) * TILE + r * RB +
                                                (((d >> 2) ^ (r & (SLOTS - 1))) * 16) + (d & 3) * 4);
                }
            }
#pragma unroll
            for (int i = 0; i < NDT; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const u32x2 hl = split2<BF16>(vv[i][2 * j], vv[i][2 * j + 1]);
                    va[i][j] = hl[0];
                    vl[i][j] = hl[1];
                }
#pragma unroll
            for (int i = 0; i < NDT; i++) {
                oacc[i] = mfma16<BF16>(va[i], ph, oacc[i]);
                oacc[i] = mfma16<BF16>(va[i], pl, oacc[i]);
                oacc[i] = mfma16<BF16>(vl[i], ph, oacc[i]);
            }
            return;
        } else {
#pragma unroll
        for (int i = 0; i < NDT; i++) {
            const int dt = i;
            const int ch = dt * 2 + ((n16 & 3) >> 1);
            const int bo = 8 * (n16 & 1);
            const u32x2 l2 = lds_read_tr16_b64(vbase + vr0 * RB + ((ch ^ (vr0 & (SLOTS - 1))) * 16) + bo);
            if constexpr (NT == 2) {
                const u32x2 h2 = lds_read_tr16_b64(vbase + (vr0 + 16) * RB +
                                                   ((ch ^ ((vr0 + 16) & (SLOTS - 1))) * 16) + bo);
                va[i] = u32x4{l2[0], l2[1], h2[0], h2[1]};
            } else {
                va[i] = u32x4{l2[0], l2[1], 0u, 0u};  // keys 16-31 absent (P is 0 there)
            }
        }
        lds_wait(va);
#pragma unroll
        for (int i = 0; i < NDT; i++) {
            oacc[i] = mfma16<T>(va[i], ph, oacc[i]);
            if constexpr (SPLITP) oacc[i] = mfma16<T>(va[i], pl, oacc[i]);
        }
        }
    });
    __builtin_amdgcn_s_waitcnt(vm_wait(0));  // no DMA may outlive the workgroup
    l_part = rows_sum(l_part);
    if (!head_ok) return;
    const int64_t u = (int64_t)b * n_units + unit;
    if (splits == 1) {
#pragma unroll
        for (int i = 0; i < NDT; i++)
            store_split<D>(oacc[i], m_run, l_part, i * 4 + kg, n16, b, split, splits,
                           gt, n_head, head0, u, gt * D, out, ws_ml, ws_acc);
    } else {
        float *ap = ws_acc + (u * splits + split) * (gt * D) + n16 * D + kg * 4;
#pragma unroll
        for (int i = 0; i < NDT; i++) *(f32x4 *)(ap + i * 16) = oacc[i];
        if (kg == 0)
            *(float2 *)(ws_ml + ((u * splits + split) * gt + n16) * 2) = float2{m_run, l_part};
    }
}

constexpr int kMaxSplits = 256;

// Combines the split partials of one (sequence, head) in one round trip.
// A workgroup takes D/4/kMergeGroups four-column groups of one head (the
// merge of a few heads then still spreads over many CUs).  Every load is
// issued branch-free before any is consumed: the split rows of this thread's
// column group with their m (indices clamped, weights of clamped duplicates
// zeroed), and the (m, l) of splits lane, lane + 64, ... from which every
// wave forms the maximum and the denominator by itself.  The only LDS round
// trip is the final sum of the R split residues across the waves.
// NL = partial rows per thread, ceil(splits / R).
// MT = threads: 64 (one wave, no LDS step, when NL <= 16 rows per lane
// cover the splits) or 256.
constexpr int kMergeGroups = 4;
// NML = (m, l) pairs per lane, ceil(splits / 64).
template <int D, int NL, int NML, int MT>
__global__ __launch_bounds__(MT) void decode_merge_kernel(
    const float *__restrict__ ws_ml, const float *__restrict__ ws_acc, int splits, int gt,
    int n_units, int n_head, float *__restrict__ out) {
    constexpr int kMergeThreads = MT;
    constexpr int NC = D / 4 / kMergeGroups, R = kMergeThreads / NC;
    static_assert(NML * 64 <= kMaxSplits, "merge reads at most kMaxSplits (m, l) pairs");
    const int g = blockIdx.x / kMergeGroups, cg = blockIdx.x % kMergeGroups;
    const int unit = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, col = tid % NC, r = tid / NC, lane = tid & 63;
    const int64_t u = (int64_t)b * n_units + unit;
    const int GD = gt * D;
    __shared__ f32x4 red[kMergeThreads / 64][NC];
    const int c4 = cg * NC + col;  // four-column group within the head
    const float *accp = ws_acc + u * splits * GD + g * D + c4 * 4;
    const float2 *mlu = (const float2 *)ws_ml + u * splits * gt + g;  // split sp at [sp * gt]
    f32x4 v[NL];
    float mt[NL];
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int sp = min(r + i * R, splits - 1);
        v[i] = *(const f32x4 *)(accp + (int64_t)sp * GD);
        mt[i] = mlu[(int64_t)sp * gt].x;
    }
    float2 ml[NML];
#pragma unroll
    for (int j = 0; j < NML; j++) {
        const int sp = lane + 64 * j;
        ml[j] = mlu[(int64_t)min(sp, splits - 1) * gt];
        if (sp >= splits) ml[j] = float2{-INFINITY, 0.f};
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NML; j++) mx = fmaxf(mx, ml[j].x);
    mx = wave_max(mx);
    const float mu = mx == -INFINITY ? 0.f : mx;
    f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const float w = r + i * R < splits ? __builtin_amdgcn_exp2f(mt[i] - mu) : 0.f;
        a += v[i] * w;
    }
    // Sum the split residues: across the lanes of a wave holding one column
    // group (lane bits above the column), then across the waves.
#pragma unroll
    for (int i = 0; i < 4; i++) a[i] = class_sum<NC>(a[i]);
    if constexpr (kMergeThreads == 64) {
        // One wave: every lane holds its column group's total.
        float den = 0.f;
#pragma unroll
        for (int j = 0; j < NML; j++) den += ml[j].y * __builtin_amdgcn_exp2f(ml[j].x - mu);
        den = wave_sum(den);
        const float inv = den > 0.f ? 1.0f / den : 0.f;
        if (lane < NC)
            *(f32x4 *)(out + ((int64_t)b * n_head + unit * gt + g) * D + c4 * 4) = a * inv;
        return;
    }
    if (lane < NC) red[tid >> 6][col] = a;
    __syncthreads();
    if (tid < 64) {  // wave 0: the denominator, then the NC output columns
        float den = 0.f;
#pragma unroll
        for (int j = 0; j < NML; j++) den += ml[j].y * __builtin_amdgcn_exp2f(ml[j].x - mu);
        den = wave_sum(den);
        const float inv = den > 0.f ? 1.0f / den : 0.f;
        for (int c = lane; c < NC; c += 64) {
            f32x4 t = red[0][c];
#pragma unroll
            for (int w = 1; w < kMergeThreads / 64; w++) t += red[w][c];
            *(f32x4 *)(out + ((int64_t)b * n_head + unit * gt + g) * D + (cg * NC + c) * 4) =
                t * inv;
        }
    }
}

}  // namespace ullm

namespace ullm {

struct MfmaPlan {
    int gt, n_units, chunk, splits, mw;
    int kb;  // 16: head_dim-256 splits of one 16-key block on decode_block_kernel (else 0)
    size_t off_ml, off_acc, bytes;
};

static const int kEnvMw = env_override("ULLM_HIP_DECODE_MW");
static const int kEnvSplitsM = env_override("ULLM_HIP_DECODE_SPLITS");
// Tuning override: ULLM_HIP_DECODE_NOBLOCK=1 runs one- and two-block splits
// on decode_dma_kernel instead of decode_block_kernel.
static const bool kNoBlock = env_override("ULLM_HIP_DECODE_NOBLOCK") == 1;

static MfmaPlan plan_mfma(int batch, int n_head, int n_kv_head, int D, int max_len, int window,
                          bool paged = false, int eb = 2) {
    MfmaPlan p{};
    const int kv_mul = n_head / n_kv_head;
    p.gt = kv_mul;
    if (p.gt > kMaxUnitHeads)
        for (p.gt = kMaxUnitHeads; kv_mul % p.gt; p.gt--) {}
    p.n_units = n_head / p.gt;
    const int visible = (window > 0 && max_len > window) ? window : max_len;
    const int units = batch * p.n_units;
    // Waves per workgroup: a short context spreads its blocks one wave per
    // workgroup over every CU (a CU's outstanding misses, not the waves,
    // bound how fast it streams).
    // A context of at most kMW * 4 blocks stays in one 4-wave workgroup per
    // unit (no partials, no merge kernel) only when the units alone fill the
    // chip; otherwise it is split like a long one.  Measured at 512 keys,
    // batch 1 (us per layer, one workgroup per unit -> 16 splits): 32/8 heads
    // D64 7.34 -> 5.46, 12/2 D128 9.81 -> 5.79, 8/4 D256 20.4 -> 6.26.
    // Long contexts use 2-wave workgroups, two per CU (64 KB of LDS stages
    // each): measured ~5 % faster at 32K than one 4-wave workgroup per CU.
    const int blocks = (visible + kTok - 1) / kTok;
    const bool whole = blocks <= kMW * 4 && units >= kMfmaTargetWG;  // one workgroup per unit
    if (D > 128 || whole) p.mw = kMW;
    else p.mw = (int64_t)units * blocks <= 1024 ? 1 : 2;
    if (D <= 128 && (kEnvMw == 1 || kEnvMw == 2 || kEnvMw == kMW)) p.mw = kEnvMw;  // tuning override
    // An f32 cache at head_dim 128: two 32 KB stages per wave, so at most two
    // waves per workgroup fit the LDS.
    if (eb == 4 && D == 128 && p.mw > 2) p.mw = 2;
    const int tile = p.mw * kTok;
    int splits = (visible + tile - 1) / tile;
    int want = (kMfmaTargetWG * (p.mw == kMW ? 1 : 2) + units - 1) / units;
    // Long-context batches: chunks of at most 22 blocks.  The sequences'
    // lengths are on the device, and a ragged batch leaves the splits past
    // each short sequence idle, so the busy ones must be small enough to
    // spread evenly.  cfg5 batch 8 ragged (us/layer): 16 splits 63.6, 32
    // 61.2, 44 56.0, 48 55.0, 52 58.0, 96 60.0; uniform batches lose 3-4 %
    // (8 x 16K keys: 49.4 at 16 splits, 51.3 at 48).
    if (batch > 1 && p.mw == 2) want = std::max(want, (visible + 22 * kTok - 1) / (22 * kTok));
    if (splits > want) splits = want;
    // head_dim 256 (4-wave workgroups): a short context would leave most CUs
    // idle at one tile per split, so splits go down to one 32-key block
    // (the waves past the split's keys contribute nothing).  Measured at
    // cfg4's 1024-key window: 32 splits per kv head 9.3 us, 8 splits 11.6 us.
    if (D > 128 && splits < want) splits = std::min(want, blocks);
    if (whole) splits = 1;
    const int cap = kMaxSplits;
    if (splits > cap) splits = cap;
    if (kEnvSplitsM >= 1) splits = kEnvSplitsM < cap ? kEnvSplitsM : cap;  // tuning override
    if (splits < 1) splits = 1;
    int chunk = (visible + splits - 1) / splits;
    chunk = (chunk + kTok - 1) / kTok * kTok;
    p.chunk = chunk;
    // head_dim 256 with one 32-key block per split: one-wave workgroups (the
    // other three waves of a 4-wave one would have no keys).
    if (D > 128 && p.mw == kMW && splits > 1 && (chunk == kTok || kEnvMw == 1)) p.mw = 1;
    p.splits = (visible + chunk - 1) / chunk;
    // head_dim 256, contiguous cache, one-block splits that leave CUs idle:
    // 16-key splits on decode_block_kernel, twice the workgroups (cfg4's
    // 1024-key window: 128 -> 256 workgroups).
    if (D > 128 && !paged && p.mw == 1 && chunk == kTok && p.splits > 1 &&
        units * p.splits < kMfmaTargetWG && 2 * p.splits <= kMaxSplits && !kNoBlock) {
        p.kb = 16;
        p.chunk = 16;
        p.splits = (visible + 15) / 16;
    }
    const size_t ml = ((size_t)units * p.splits * p.gt * 2 * 4 + 255) / 256 * 256;
    const size_t ac = (size_t)units * p.splits * p.gt * D * 4;
    p.off_ml = 0;
    p.off_acc = ml;
    p.bytes = p.splits > 1 ? ml + ac : 0;
    return p;
}

// Upper bound over every call with max_len' <= max_len (the planner's split
// count is not monotonic in the length: short contexts use more, smaller
// splits): every split holds at least one 32-key block (16 keys at
// head_dim 256), at most kMaxSplits exist, and contexts of at most kMW * 4
// blocks use one split when the units fill the chip.
size_t decode_mfma_workspace(int batch, int n_head, int n_kv_head, int D, int max_len,
                             int window) {
    const MfmaPlan p = plan_mfma(batch, n_head, n_kv_head, D, max_len, window);
    const int visible = (window > 0 && max_len > window) ? window : max_len;
    const int blocks = (visible + kTok - 1) / kTok;
    // head_dim 256 may split down to 16-key blocks.
    const size_t units = (size_t)batch * p.n_units;
    const bool whole = blocks <= kMW * 4 && units >= (size_t)kMfmaTargetWG;
    const int smax = whole ? 1 : std::min(kMaxSplits, D > 128 ? 2 * blocks : blocks);
    if (smax <= 1) return 0;
    const size_t ml = (units * smax * p.gt * 2 * 4 + 255) / 256 * 256;
    return ml + units * smax * p.gt * D * 4;
}

// head_dim <= 128 streams through LDS DMA; 256 keeps register staging.
template <class T, int D, bool DMA = (D <= 128)>
struct MainLaunch {
    template <class... A>
    static void run(int mw, dim3 g, hipStream_t st, A... a) {
        const int32_t *nt = nullptr;
        if (mw == 1) hipLaunchKernelGGL((decode_dma_kernel<T, D, 1>), g, dim3(64), 0, st, a..., nt, 0, 0, 0);
        else if (mw == 2 || (__is_same(T, F32) && D == 128))  // f32 at head_dim 128: at most 2 waves
            hipLaunchKernelGGL((decode_dma_kernel<T, D, 2>), g, dim3(128), 0, st, a..., nt, 0, 0, 0);
        else if constexpr (!(__is_same(T, F32) && D == 128))
            hipLaunchKernelGGL((decode_dma_kernel<T, D, kMW>), g, dim3(kMW * 64), 0, st, a..., nt, 0, 0, 0);
    }
};
template <class T, int D>
struct MainLaunch<T, D, false> {
    template <class... A>
    static void run(int mw, dim3 g, hipStream_t st, A... a) {
        const int32_t *nt = nullptr;
        if (mw == 1)
            hipLaunchKernelGGL((decode_mfma_kernel<T, D, false, 1>), g, dim3(64), 0, st, a..., nt, 0, 0, 0);
        else
            hipLaunchKernelGGL((decode_mfma_kernel<T, D>), g, dim3(kMW * 64), 0, st, a..., nt, 0, 0, 0);
    }
};

template <int D>
static void launch_merge(const MfmaPlan &p, int batch, int nh, float *out, char *ws, hipStream_t st) {
    constexpr int NC = D / 4 / kMergeGroups;
    const dim3 g(p.gt * kMergeGroups, p.n_units, batch);
    const float *ml = (const float *)(ws + p.off_ml), *ac = (const float *)(ws + p.off_acc);
    // (m, l) loads per lane: as many as the splits need, not kMaxSplits / 64.
    auto go = [&](auto nlc, auto mtc) {
        constexpr int NL = decltype(nlc)::value, MT = decltype(mtc)::value;
        if (p.splits <= 64)
            hipLaunchKernelGGL((decode_merge_kernel<D, NL, 1, MT>), g, dim3(MT), 0, st, ml, ac,
                               p.splits, p.gt, p.n_units, nh, out);
        else if (p.splits <= 128)
            hipLaunchKernelGGL((decode_merge_kernel<D, NL, 2, MT>), g, dim3(MT), 0, st, ml, ac,
                               p.splits, p.gt, p.n_units, nh, out);
        else
            hipLaunchKernelGGL((decode_merge_kernel<D, NL, kMaxSplits / 64, MT>), g, dim3(MT), 0,
                               st, ml, ac, p.splits, p.gt, p.n_units, nh, out);
    };
    // One wave (no LDS step) when 4 split rows per lane cover the splits;
    // with more, four waves keep the rows per lane, hence the serial loads,
    // low (one wave with 16 rows measured 0.25 us slower at cfg2's 128
    // splits; at cfg1's 16 it is 0.15 us faster).
    constexpr int R1 = 64 / NC, R4 = 256 / NC;
    const int nl1 = (p.splits + R1 - 1) / R1, nl4 = (p.splits + R4 - 1) / R4;
    if (nl1 <= 4) go(Int<4>{}, Int<64>{});
    else if (nl4 <= 1) go(Int<1>{}, Int<256>{});
    else if (nl4 <= 2) go(Int<2>{}, Int<256>{});
    else if (nl4 <= 4) go(Int<4>{}, Int<256>{});
    else if (nl4 <= 8) go(Int<8>{}, Int<256>{});
    else go(Int<16>{}, Int<256>{});
}

void decode_merge_launch(int D, const float *ws_ml, const float *ws_acc, int splits, int gt,
                         int n_units, int batch, int n_head, float *out, hipStream_t st) {
    MfmaPlan p{};
    p.splits = splits;
    p.gt = gt;
    p.n_units = n_units;
    p.off_ml = 0;
    p.off_acc = (size_t)((const char *)ws_acc - (const char *)ws_ml);
    char *ws = (char *)ws_ml;
    if (D == 64) launch_merge<64>(p, batch, n_head, out, ws, st);
    else if (D == 128) launch_merge<128>(p, batch, n_head, out, ws, st);
    else launch_merge<256>(p, batch, n_head, out, ws, st);
}

template <class T, int D>
static void launch_mfma(const MfmaPlan &p, const float *q, const void *kc, const void *vc,
                        int64_t kvs, int64_t ss, const int32_t *lens, int max_len, int win,
                        int batch, int nh, int kv_mul, float qs, float *out, char *ws,
                        hipStream_t st) {
    // Keys 0..max_len-1 of every sequence are readable (the cache holds them);
    // when the window cannot bind, the kernels fetch keys before the length.
    // Only for one sequence (whose length is normally max_len): in a ragged
    // batch the splits past a short sequence's length would fetch for nothing.
    const int fetch_len = batch == 1 && (win <= 0 || max_len <= win) ? max_len : 0;
    if constexpr (D > 128) {
        if (p.kb == 16) {
            hipLaunchKernelGGL((decode_block_kernel<T, D, 1, 16>), dim3(p.splits, p.n_units, batch),
                               dim3(64), 0, st, q, (const char *)kc, (const char *)vc, kvs, ss, lens,
                               win, fetch_len, nh, kv_mul, p.gt, p.n_units, p.chunk, p.splits, qs,
                               out, (float *)(ws + p.off_ml), (float *)(ws + p.off_acc));
            launch_merge<D>(p, batch, nh, out, ws, st);
            return;
        }
    } else {
        if (p.mw == 1 && (p.chunk == kTok || p.chunk == 2 * kTok) && p.splits > 1 && !kNoBlock) {
            auto go = [&](auto kern) {
                hipLaunchKernelGGL(kern, dim3(p.splits, p.n_units, batch), dim3(64), 0, st, q,
                                   (const char *)kc, (const char *)vc, kvs, ss, lens, win,
                                   fetch_len, nh, kv_mul, p.gt, p.n_units, p.chunk, p.splits, qs,
                                   out, (float *)(ws + p.off_ml), (float *)(ws + p.off_acc));
            };
            if (p.chunk == 2 * kTok) go(decode_block_kernel<T, D, 2>);
            else go(decode_block_kernel<T, D, 1>);
            launch_merge<D>(p, batch, nh, out, ws, st);
            return;
        }
    }
    if constexpr (__is_same(T, F32) && D > 128) return;  // f32 head_dim 256: decode.hip
    else {
    MainLaunch<T, D>::run(p.mw, dim3(p.splits, p.n_units, batch), st, q, (const char *)kc,
                          (const char *)vc, kvs, ss, lens, win, fetch_len, nh, kv_mul, p.gt,
                          p.n_units,
                          p.chunk, p.splits, qs, out, (float *)(ws + p.off_ml),
                          (float *)(ws + p.off_acc));
    if (p.splits > 1) launch_merge<D>(p, batch, nh, out, ws, st);
    }
}

size_t decode_mfma_plan_bytes(int batch, int n_head, int n_kv_head, int D, int max_len,
                              int window) {
    return plan_mfma(batch, n_head, n_kv_head, D, max_len, window).bytes;
}

// The reference's f32 cache at head_dim 64 and 128 runs on the MFMA kernels
// (decode_block_kernel for one- and two-block splits, decode_dma_kernel for
// longer ones); *bytes is that plan's workspace.  head_dim 256 stays on
// decode_split_kernel (decode.hip).
bool decode_f32_block_plan(int batch, int n_head, int n_kv_head, int D, int max_len, int window,
                           size_t *bytes) {
    if (D > 128) return false;
    *bytes = plan_mfma(batch, n_head, n_kv_head, D, max_len, window, false, 4).bytes;
    return true;
}

int decode_mfma(int dtype, const float *q, const void *kc, const void *vc, int64_t kvs,
                int64_t ss, const int32_t *lens, int max_len, int win, int batch, int nh,
                int nkv, int D, float qs, float *out, void *ws, size_t ws_bytes,
                hipStream_t st) {
    const MfmaPlan p = plan_mfma(batch, nh, nkv, D, max_len, win, false, dtype_bytes(dtype));
    if (p.bytes > 0 && (!ws || ws_bytes < p.bytes))
        return set_error(ULLM_HIP_E_WORKSPACE, "decode: workspace of %zu bytes needed, %zu given",
                         p.bytes, ws_bytes);
    const int kv_mul = nh / nkv;
    char *w = (char *)ws;
#define ULLM_MFMA_CASE(TT, DD) \
    launch_mfma<TT, DD>(p, q, kc, vc, kvs, ss, lens, max_len, win, batch, nh, kv_mul, qs, \
                        out, w, st)
    if (dtype == ULLM_DT_F32) {
        if (D == 64) ULLM_MFMA_CASE(F32, 64);
        else ULLM_MFMA_CASE(F32, 128);
    } else if (dtype == ULLM_DT_F16) {
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

// ---------------------------------------------------------------------------
// Paged KV cache (no counterpart in the reference, whose cache is one
// contiguous [n_ctx][kv_dim] array per layer, crates/ullm-model/src/lib.rs:
// 184-185; the reference's roadmap lists a paged cache for batching,
// docs/roadmap.md Phase 2).  Same split-KV kernels over a block table.
namespace ullm {

// Window used for planning: blocks start at the window start rounded down to
// 32 keys, so a binding window covers up to window + 31 keys.
static int paged_plan_window(int window) { return window > 0 ? window + kTok : 0; }

template <class T, int D>
static void launch_paged(const MfmaPlan &p, const float *q, const void *kp, const void *vp,
                         int64_t kvs, const int32_t *tab, int tab_stride, int shift, int n_pages,
                         const int32_t *lens, int win, int batch, int nh, int kv_mul, float qs,
                         float *out, char *ws, hipStream_t st) {
    const dim3 g(p.splits, p.n_units, batch);
    if constexpr (D > 128) {  // register-staged kernel, 4 waves
        if (p.mw == 1)
            hipLaunchKernelGGL((decode_mfma_kernel<T, D, true, 1>), g, dim3(64), 0, st, q,
                               (const char *)kp, (const char *)vp, kvs, (int64_t)0, lens, win, 0,
                               nh, kv_mul, p.gt, p.n_units, p.chunk, p.splits, qs, out,
                               (float *)(ws + p.off_ml), (float *)(ws + p.off_acc), tab,
                               tab_stride, shift, n_pages);
        else
            hipLaunchKernelGGL((decode_mfma_kernel<T, D, true>), g, dim3(kMW * 64), 0, st, q,
                               (const char *)kp, (const char *)vp, kvs, (int64_t)0, lens, win, 0,
                               nh, kv_mul, p.gt, p.n_units, p.chunk, p.splits, qs, out,
                               (float *)(ws + p.off_ml), (float *)(ws + p.off_acc), tab,
                               tab_stride, shift, n_pages);
    } else {
        auto go = [&](auto mwc) {
            constexpr int MW = decltype(mwc)::value;
            hipLaunchKernelGGL((decode_dma_kernel<T, D, MW, true>), g, dim3(MW * 64), 0, st, q,
                               (const char *)kp, (const char *)vp, kvs, (int64_t)0, lens, win, 0,
                               nh, kv_mul, p.gt, p.n_units, p.chunk, p.splits, qs, out,
                               (float *)(ws + p.off_ml), (float *)(ws + p.off_acc), tab,
                               tab_stride, shift, n_pages);
        };
        if (p.mw == 1) go(Int<1>{});
        else if (p.mw == 2) go(Int<2>{});
        else if constexpr (__is_same(T, F32) && D == 128) go(Int<2>{});
        else go(Int<kMW>{});
    }
    if (p.splits > 1) launch_merge<D>(p, batch, nh, out, ws, st);
}

}  // namespace ullm

using namespace ullm;

extern "C" size_t ullm_hip_paged_decode_workspace_bytes(int batch, int n_head, int n_kv_head,
                                                        int head_dim, int max_len, int window) {
    if (batch < 1 || n_head < 1 || n_kv_head < 1 || n_head % n_kv_head || max_len < 1) return 0;
    if (head_dim != 64 && head_dim != 128 && head_dim != 256) return 0;
    const size_t m = decode_mfma_workspace(batch, n_head, n_kv_head, head_dim, max_len,
                                           paged_plan_window(window));
    const size_t f = decode_f32_workspace(batch, n_head, n_kv_head, head_dim, max_len, window);
    return m > f ? m : f;
}

extern "C" int ullm_hip_attn_decode_paged(const float *q, const void *k_pages, const void *v_pages,
                                          int kv_dtype, int64_t kv_stride, int page_size,
                                          int n_pages, const int32_t *block_table,
                                          int table_stride, const int32_t *seq_lens, int max_len,
                                          int window, int batch, int n_head, int n_kv_head,
                                          int head_dim, float scale, float *out, void *workspace,
                                          size_t workspace_bytes, void *stream) {
    if (!dtype_ok(kv_dtype))
        return set_error(ULLM_HIP_E_UNSUPPORTED, "decode_paged: kv dtype %d", kv_dtype);
    if (head_dim != 64 && head_dim != 128 && head_dim != 256)
        return set_error(ULLM_HIP_E_UNSUPPORTED, "decode_paged: head_dim %d not in {64,128,256}", head_dim);
    if (batch < 1 || batch > 65535 || n_head < 1 || n_kv_head < 1 || n_head % n_kv_head)
        return set_error(ULLM_HIP_E_INVALID, "decode_paged: bad heads n_head=%d n_kv_head=%d batch=%d",
                         n_head, n_kv_head, batch);
    if (max_len < 1) return set_error(ULLM_HIP_E_INVALID, "decode_paged: max_len %d < 1", max_len);
    if (kv_stride < (int64_t)n_kv_head * head_dim || (kv_stride * dtype_bytes(kv_dtype)) % 16)
        return set_error(ULLM_HIP_E_INVALID,
                         "decode_paged: kv_stride %lld must be >= n_kv_head*head_dim and 16-byte aligned",
                         (long long)kv_stride);
    if (page_size < kTok || (page_size & (page_size - 1)))
        return set_error(ULLM_HIP_E_INVALID, "decode_paged: page_size %d must be a power of two >= %d",
                         page_size, kTok);
    if ((int64_t)page_size * kv_stride * dtype_bytes(kv_dtype) > 0x7fff0000LL)
        return set_error(ULLM_HIP_E_INVALID, "decode_paged: a page exceeds 2 GiB");
    if (n_pages < 1) return set_error(ULLM_HIP_E_INVALID, "decode_paged: n_pages %d < 1", n_pages);
    if (table_stride < (max_len + page_size - 1) / page_size)
        return set_error(ULLM_HIP_E_INVALID, "decode_paged: table_stride %d < %d pages of max_len",
                         table_stride, (max_len + page_size - 1) / page_size);
    if (!q || !k_pages || !v_pages || !block_table || !seq_lens || !out)
        return set_error(ULLM_HIP_E_INVALID, "decode_paged: null tensor pointer");
    if (((uintptr_t)k_pages | (uintptr_t)v_pages | (uintptr_t)q) & 15)
        return set_error(ULLM_HIP_E_INVALID, "decode_paged: q/k_pages/v_pages must be 16-byte aligned");
    // f32 pages at head_dim 256 run on the VALU split kernel (decode.hip);
    // every other shape on the MFMA kernels.
    if (kv_dtype == ULLM_DT_F32 && head_dim > 128)
        return decode_f32_paged(q, k_pages, v_pages, kv_stride, block_table, table_stride,
                                __builtin_ctz(page_size), n_pages, seq_lens, max_len, window,
                                batch, n_head, n_kv_head, head_dim, scale * kLog2e, out, workspace,
                                workspace_bytes, (hipStream_t)stream);
    const MfmaPlan p = plan_mfma(batch, n_head, n_kv_head, head_dim, max_len, paged_plan_window(window),
                                 true, dtype_bytes(kv_dtype));
    if (p.bytes > 0 && (!workspace || workspace_bytes < p.bytes))
        return set_error(ULLM_HIP_E_WORKSPACE, "decode_paged: workspace of %zu bytes needed, %zu given",
                         p.bytes, workspace_bytes);
    const int shift = __builtin_ctz(page_size);
    const float qs = scale * kLog2e;
    const int kv_mul = n_head / n_kv_head;
    char *w = (char *)workspace;
    hipStream_t st = (hipStream_t)stream;
#define ULLM_PAGED(TT, DD) \
    launch_paged<TT, DD>(p, q, k_pages, v_pages, kv_stride, block_table, table_stride, shift, n_pages, \
                         seq_lens, window, batch, n_head, kv_mul, qs, out, w, st)
    if (kv_dtype == ULLM_DT_F32) {
        if (head_dim == 64) ULLM_PAGED(F32, 64);
        else ULLM_PAGED(F32, 128);
    } else if (kv_dtype == ULLM_DT_F16) {
        if (head_dim == 64) ULLM_PAGED(F16, 64);
        else if (head_dim == 128) ULLM_PAGED(F16, 128);
        else ULLM_PAGED(F16, 256);
    } else {
        if (head_dim == 64) ULLM_PAGED(BF16, 64);
        else if (head_dim == 128) ULLM_PAGED(BF16, 128);
        else ULLM_PAGED(BF16, 256);
    }
#undef ULLM_PAGED
    return check_hip(hipGetLastError(), "decode_paged launch");
}
