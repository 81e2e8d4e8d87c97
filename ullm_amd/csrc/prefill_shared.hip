// Causal prefill at head_dim 256 with each K/V tile shared by a workgroup's
// 4 waves (gfx950), for prompts long enough to fill the chip with whole
// row blocks.
//
// Same arithmetic as prefill_sk_kernel (prefill.hip): S = Q.K^T on
// v_mfma_f32_32x32x16_{f16,bf16}, online softmax in the exp2 domain with a
// lazily raised max, P.V on v_mfma_f32_32x32x16_f16 with P and V in f16 (a
// bf16 cache's V is widened to f16 in LDS).  What differs is the work split:
//  * A workgroup owns hw query heads of one kv head (hw = the largest power
//    of two dividing kv_mul, at most 4) times 4/hw consecutive 32-row
//    blocks, a "unit" of UR = 128/hw rows; wave w takes head hw0 + w % hw
//    and rows (w / hw) * 32 .. +31 of the unit, over the unit's whole key
//    range (window start of its first row to the causal end of its last).
//  * Each 32-key K/V tile goes global -> LDS once (buffer_load ... lds,
//    kv_swz slot swizzle) into a 4-stage ring and serves all 4 waves: a
//    quarter of prefill_sk_kernel's L2 -> CU traffic per FLOP, where every
//    wave streams its own tiles.  A step (one tile for 4 waves) takes about
//    1.2 us against 2.4 us per wave tile there.
//  * The price is parallelism: the longest unit is one workgroup's serial
//    chain.  The host takes this kernel only when that chain is short next
//    to the total work per CU (prefill_shared_applies); splitting the long
//    units over workgroups was measured and rejected (the f32 partials and
//    their merge cost more than the split saved).
//  * Workgroup b takes the unit of rank b / n_hg (longest first) of head
//    group b % n_hg.  Dispatch deals blocks to the 8 XCDs round-robin, so
//    when n_hg divides 8 (or 8 divides n_hg) each XCD serves fixed head
//    groups and their K/V stays in one L2.
#include "common.hpp"
#include "mfma_util.hpp"
#include "wave.hpp"
#include <algorithm>
#include <vector>

namespace ullm {

constexpr int kSharedD = 256;

__device__ __forceinline__ int sk2_swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// Key tiles [t0, t1) of unit u: the window start of its first row to the
// causal end of its last.
__host__ __device__ inline void shared_unit_tiles(int u, int UR, int S, int start_pos, int window,
                                                 int &t0, int &t1) {
    const int r0 = u * UR;
    const int hi = start_pos + (r0 + UR < S ? r0 + UR : S);
    int lo = 0;
    if (window > 0) { lo = start_pos + r0 + 1 - window; if (lo < 0) lo = 0; }
    t0 = lo / 32;
    t1 = (hi + 31) / 32;
}

template <class T>
__global__ __launch_bounds__(256, 1) void prefill_shared_kernel(
    const uint16_t *__restrict__ q, const char *__restrict__ kc, const char *__restrict__ vc,
    int64_t kv_stride, int S, int start_pos, int window, int n_head, int kv_mul, int hw,
    int n_hg, int n_units, float qscale, float *__restrict__ out) {
    constexpr int D = kSharedD, BN = 32, RB = D * 2, TILE = BN * RB, STAGE = 2 * TILE;
    constexpr int NSTG = 4, NKS = D / 16, NDT = D / 32, NIW = TILE / 1024 / 4;  // DMA per wave per tile
    constexpr bool CVTV = __is_same(T, BF16);
    constexpr float kLazy = 8.0f;
    __shared__ __attribute__((aligned(1024))) char lds[NSTG * STAGE];

    const int hg = blockIdx.x % n_hg, u = n_units - 1 - (int)(blockIdx.x / n_hg);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 31, h2 = lane >> 5;
    const int UR = 128 / hw;
    const int head = hg * hw + wave % hw, kvh = head / kv_mul;
    const int qrow = u * UR + (wave / hw) * 32 + c;
    const int pos_row = start_pos + qrow;
    const int64_t q_dim = (int64_t)n_head * D;
    const int kv_len = start_pos + S;
    int t0, t1;
    shared_unit_tiles(u, UR, S, start_pos, window, t0, t1);
    const int ca = t0, n = t1 - t0;

    u32x4 qreg[NKS];  // Q rows of this wave (loaded after the first tile request)

    // K/V DMA: tile t's rows (wave*NIW + i)*2 + lane/32, slot lane%32 holding
    // chunk slot ^ swz(row); steps past the unit's range address past the buffer.
    const int rbg = (int)(kv_stride * 2);
    const int range = (kv_len - 1) * rbg + D * 2;
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(kc + (int64_t)kvh * D * 2), 0, range, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(vc + (int64_t)kvh * D * 2), 0, range, kRsrcWord3);
    int dofs[NIW];
#pragma unroll
    for (int i = 0; i < NIW; i++) {
        const int r = (wave * NIW + i) * 2 + (lane >> 5);
        dofs[i] = r * rbg + (((lane & 31) ^ sk2_swz(r)) * 16);
    }
    auto issue = [&](int j) {  // step j's tile into stage j % NSTG
        const int so = __builtin_amdgcn_readfirstlane(j < n ? (ca + j) * BN * rbg : range);
        char *st = lds + (j % NSTG) * STAGE + wave * NIW * 1024;
#pragma unroll
        for (int i = 0; i < NIW; i++) dma16(krs, st + i * 1024, dofs[i] + so, 0);
#pragma unroll
        for (int i = 0; i < NIW; i++) dma16(vrs, st + TILE + i * 1024, dofs[i] + so, 0);
    };
    // bf16 V -> f16 in place, for the chunks this wave's DMA wrote.
    auto widen = [&](int stg) {
        if constexpr (CVTV) {
            const uint32_t vb = lds_addr(lds + stg * STAGE + TILE + wave * NIW * 1024) + lane * 16;
            u32x4 w[NIW];
#pragma unroll
            for (int i = 0; i < NIW; i++) w[i] = lds_read_b128(vb + i * 1024);
            lds_wait_any();
#pragma unroll
            for (int i = 0; i < NIW; i++) {
                tie(w[i]);
                u32x4 o;
#pragma unroll
                for (int e = 0; e < 4; e++) o[e] = pack_f16x2(bf16_lo(w[i][e]), bf16_hi(w[i][e]));
                lds_write_b128(vb + i * 1024, o);
            }
        }
    };

    // Operand addresses within a stage.  K (A operand): lane = key row c,
    // chunk 2s + h2; the swizzle touches the low 4 chunk bits only, so
    // k-step s + 8 is k-step s's address + 256 bytes.  V^T: as prefill_sk.
    uint32_t ka[NKS / 2];
#pragma unroll
    for (int s = 0; s < NKS / 2; s++) ka[s] = c * RB + (((2 * s + h2) ^ sk2_swz(c)) * 16);
    const int g16 = lane >> 4, i16 = lane & 15;
    uint32_t va[NDT][2];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int e0 = dt * 32 + (g16 & 1) * 16 + 4 * (i16 & 3);
            const int R = (g16 >> 1) * 4 + (i16 >> 2) + h * 8;
            va[dt][h] = TILE + R * RB + (((e0 >> 3) ^ sk2_swz(R)) * 16) + (e0 & 7) * 2;
        }

    f32x16 oacc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; i++) oacc[i] = f32x16{};
    float m_run = -INFINITY, l_part = 0.f;
    const int dlo = window > 0 ? -window : INT_MIN;
    const int p_first = pos_row - c;
    const uint32_t lds0 = lds_addr(lds);

    auto compute = [&](int j) {
        const uint32_t sb = lds0 + (j % NSTG) * STAGE;
        f32x16 sacc = f32x16{};
        u32x4 kb[2][4];
        auto rdk = [&](int g, int buf) {  // K operands of k-steps 4g .. 4g+3
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int s = 4 * g + i;
                kb[buf][i] = lds_read_b128(sb + ka[s & 7] + (s >> 3) * 256);
            }
        };
        rdk(0, 0);
#pragma unroll
        for (int g = 0; g < NKS / 4; g++) {
            if (g + 1 < NKS / 4) {
                rdk(g + 1, (g + 1) & 1);
                asm volatile("s_waitcnt lgkmcnt(4)" ::: "memory");
            } else {
                lds_wait_any();
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                tie(kb[g & 1][i]);
                sacc = mfma32<T>(kb[g & 1][i], qreg[4 * g + i], sacc);
            }
        }
        // Scale, then mask where the tile reaches past the wave's first row
        // or before the window of its last (wave-uniform): key - pos_row
        // must lie in (dlo, 0].
        const int kbase = (ca + j) * BN;
        float mloc = -INFINITY;
        if (kbase + BN - 1 > p_first || (window > 0 && kbase <= p_first + 31 - window)) {
            const int kd = kbase + h2 * 4 - pos_row;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int dk = kd + (i >> 2) * 8 + (i & 3);
                const float sv = dk > 0 || dk <= dlo ? -INFINITY : sacc[i] * qscale;
                sacc[i] = sv;
                mloc = fmaxf(mloc, sv);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                sacc[i] *= qscale;
                mloc = fmaxf(mloc, sacc[i]);
            }
        }
        mloc = max_xor32(mloc);
        if (__any(mloc > m_run + kLazy)) {
            const float m_new = fmaxf(m_run, mloc);
            if (__any(m_run != -INFINITY)) {
                const float corr = __builtin_amdgcn_exp2f(m_run - (m_new == -INFINITY ? 0.f : m_new));
                l_part *= corr;
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) asm volatile("" : "+a"(oacc[dt]));
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
        u32x2 vb[2][2][2];
        auto rdv = [&](int dt, int buf) {
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                vb[buf][ks][0] = lds_read_tr16_b64(sb + va[dt][0] + ks * 16 * RB);
                vb[buf][ks][1] = lds_read_tr16_b64(sb + va[dt][1] + ks * 16 * RB);
            }
        };
        rdv(0, 0);
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            if (dt + 1 < NDT) {
                rdv(dt + 1, (dt + 1) & 1);
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
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) asm volatile("" : "+a"(oacc[dt]));
    };

    // ---- main loop: tiles three steps ahead in the 4-stage ring ----
    // Step j: this wave's DMA of step j has landed (steps j+1, j+2 stay in
    // flight), its bf16 V is widened, and the barrier makes every wave's
    // part visible and frees stage (j+3) % 4 (read in step j-1); then step
    // j+3 is requested and step j computed.
    // Q rows of this wave as the B operand (d = s*16 + h2*8 .. +7), requested
    // after the first tile and before the next two: the wait for Q then
    // leaves those in flight.
    // Untracked loads: the compiler does not count the DMA requests, so a
    // tracked Q would make it drain all of them before the first step.  The
    // loop's first wait (two tiles left in flight) covers Q, and the ties
    // keep every use after it.
    issue(0);
    {
        const i32x4 qrs = raw_rsrc(q, (int)((int64_t)S * q_dim * 2));
        const int qo = qrow < S ? (int)(((int64_t)qrow * q_dim + (int64_t)head * D + h2 * 8) * 2)
                                : 0x7ffffff0;  // past the range: zeros
#pragma unroll
        for (int s = 0; s < NKS; s++) qreg[s] = buffer_load_b128_untracked(qrs, qo + s * 32);
    }
    issue(1);
    issue(2);
    for (int j = 0; j < n; j++) {
        __builtin_amdgcn_s_waitcnt(vm_wait(4 * NIW));
#pragma unroll
        for (int s = 0; s < NKS; s++) tie(qreg[s]);
        widen(j % NSTG);
        lds_wait_any();
        asm volatile("s_barrier" ::: "memory");
        issue(j + 3);
        compute(j);
    }
    __builtin_amdgcn_s_waitcnt(vm_wait(0));

    // ---- result: lane (row c, h2) holds d = dt*32 + 8g + 4*h2 + 0..3 ----
    const float l_tot = l_part + xor32(l_part);
    if (qrow < S) {
        const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
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
}

static int shared_hw(int kv_mul) {
    int hw = 1;
    while (hw < 4 && kv_mul % (hw * 2) == 0) hw *= 2;
    return hw;
}

// True when the shared-tile kernel is expected to beat prefill_sk_kernel.
// Its step (one 32-key tile for a whole unit) costs about twice a
// prefill_sk wave tile but does four waves' work: about twice the
// throughput, and the longest unit is about twice as long a serial chain.
// It wins when that chain is at most ~3.5x the average tile steps per CU.
// Measured on MI355X (f16, us, shared vs prefill_sk; ratio in brackets):
// 8/4 heads S=1024 W=1024 [7.5] 43.2 vs 27.7; S=2048 global [3.9] 75.9 vs
// 61.2; S=1536 W=512 [3.2] 31.6 vs 36.7; S=2048 W=1024 [2.7] 48.3 vs 58.0;
// S=4096 W=1024 65.6 vs 114.1; S=8192 global 341 vs 747; 32/16 heads
// S=512 [3.6] 26.2 vs 31.2 and S=1024 [1.9] 45.7 vs 73.7.
bool prefill_shared_applies(int S, int start_pos, int window, int n_head, int kv_mul) {
    if ((int64_t)S * n_head * kSharedD * 2 >= 0x7fff0000LL) return false;  // 32-bit Q offsets
    const int hw = shared_hw(kv_mul), UR = 128 / hw;
    const int n_units = (S + UR - 1) / UR;
    int64_t total = 0;
    int max_nt = 0;
    for (int u = 0; u < n_units; u++) {
        int t0, t1;
        shared_unit_tiles(u, UR, S, start_pos, window, t0, t1);
        total += t1 - t0;
        max_nt = std::max(max_nt, t1 - t0);
    }
    total *= n_head / hw;
    return (int64_t)max_nt * 256 * 2 <= 7 * total;
}

int launch_prefill_shared(int dtype, const void *q, const void *kc, const void *vc, int64_t kvs,
                          int S, int start_pos, int window, int n_head, int kv_mul, float qs,
                          float *out, hipStream_t st) {
    const int hw = shared_hw(kv_mul), UR = 128 / hw;
    const int n_units = (S + UR - 1) / UR, n_hg = n_head / hw;
    const dim3 grid((unsigned)(n_units * n_hg));
    if (dtype == ULLM_DT_BF16)
        hipLaunchKernelGGL((prefill_shared_kernel<BF16>), grid, dim3(256), 0, st, (const uint16_t *)q,
                           (const char *)kc, (const char *)vc, kvs, S, start_pos, window, n_head,
                           kv_mul, hw, n_hg, n_units, qs, out);
    else
        hipLaunchKernelGGL((prefill_shared_kernel<F16>), grid, dim3(256), 0, st, (const uint16_t *)q,
                           (const char *)kc, (const char *)vc, kvs, S, start_pos, window, n_head,
                           kv_mul, hw, n_hg, n_units, qs, out);
    return check_hip(hipGetLastError(), "prefill (shared tiles) launch");
}

}  // namespace ullm
