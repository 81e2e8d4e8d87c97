// Batched projection Y[s, o] = sum_i W[o, i] * X[s, i] on CDNA4 MFMA (gfx950).
//
// The reference's batched prefill matmul (crates/ullm-metal/src/shader.metal:
// 519-566, encoded by forward.rs:675-726): bf16 weights W [out, in] row-major,
// f32 activations X [n_cols, in] token-major, f32 output Y [n_cols, out]
// token-major, f32 accumulation.  Every output equals the CPU reference's
// matvec of that token row (crates/ullm-model/src/math.rs:9-21) up to
// summation order.
//
// Precision: W is exact in bf16; X is split as X = Xhi + Xlo with both halves
// bf16 (Xhi = RNE(X), Xlo = RNE(X - Xhi)), which carries 16 significant bits
// of every activation (relative residual <= 2^-16), and both halves are
// multiplied on v_mfma_f32_32x32x16_bf16 into one f32 accumulator.  The
// products themselves are exact in the MFMA's f32 accumulate, so the result
// differs from an f32 dot product only by the residual of the split and the
// summation order.
//
// Tiling: a workgroup of 4 waves (2 x 2) computes a (64 SI) tokens x
// (64 OI) outputs tile of Y over in_dim in steps of 32; each wave owns a
// (32 SI) x (32 OI) block.  The large tile (SI 2, OI 4: 128 x 256, waves of
// 64 x 128) keeps LDS traffic per MFMA within the LDS's 128 bytes per clock
// (fragment reads 512 + DMA writes 256 bytes per 32-cycle MFMA); grids that
// it would leave below one tile per CU use SI 1, OI 2.  Both operands go
// global -> LDS by buffer_load ... lds (W as bf16 rows of 64 bytes, X as f32
// rows of 128 bytes) into a 4-stage ring, loaded three steps ahead.  The X
// fragments are split into bf16 hi/lo in registers after the LDS read.  The
// fragments of each k16 half-step are read two half-steps ahead and split in
// the shadow of the previous half-step's MFMAs.  With the MFMA computing
// Y^T = W . X^T, an accumulator lane holds one token (lane % 32) and 4
// consecutive outputs per register group, which become 16-byte row stores.
// 16-byte LDS slots are XOR-swizzled by row so that the ds_read_b128 of 16
// consecutive rows at one k offset hit 16 different bank groups.
#include "common.hpp"
#include "mfma_util.hpp"

namespace ullm {

constexpr int kMmK = 32;                  // in_dim per step
constexpr int kMmWRB = kMmK * 2;          // bytes of one W tile row (bf16)
constexpr int kMmXRB = kMmK * 4;          // bytes of one X tile row (f32)
constexpr int kMmNst = 4;                 // LDS ring stages
constexpr int kMmGroup = 8;               // token tiles per group of the tile order
constexpr int kMmOOB = 0x7ffffff0;        // buffer offset past every valid range: reads zero

// WS x WO waves, each owning SI x OI blocks of 32 x 32.
template <int SI, int OI, int WS, int WO>
struct MmCfg {
    static constexpr int NT = 64 * WS * WO;                  // threads
    static constexpr int BS = 32 * SI * WS, BO = 32 * OI * WO;  // tile tokens, tile outputs
    static constexpr int WT = BO * kMmWRB;                   // W bytes per stage
    static constexpr int STAGE = WT + BS * kMmXRB;           // W then X
    static constexpr int NWI = BO / 16, NXI = BS / 8;        // 1 KiB DMA instructions per stage
    static constexpr int NDMA = (NWI + NXI) / (WS * WO);     // ... per wave
    static_assert((NWI + NXI) % (WS * WO) == 0, "DMA split");
};

// Slot swizzles: 4 W rows (16 slots) or 2 X rows (8 slots each) share a
// 256-byte bank line; XOR the slot with the row's line index.
__device__ __forceinline__ int mm_wswz(int r) { return (r >> 2) & 3; }
__device__ __forceinline__ int mm_xswz(int r) { return (r >> 1) & 7; }

template <int SI, int OI, int WS, int WO>
__global__ __launch_bounds__(64 * WS * WO) void matmul_bf16_kernel(
    const char *__restrict__ w, const float *__restrict__ x, float *__restrict__ y, int in_dim,
    int out_dim, int n_cols, int mt, int nt) {
    using C = MmCfg<SI, OI, WS, WO>;
    constexpr int BS = C::BS, BO = C::BO, STAGE = C::STAGE, NDMA = C::NDMA;
    __shared__ __attribute__((aligned(1024))) char lds[kMmNst * STAGE];

    // Workgroup i runs on XCD i % 8; each XCD takes a contiguous run of tile
    // indices, and the indices run over groups of kMmGroup token tiles x all
    // output tiles, token tile fastest: the tiles an XCD holds at once form
    // a block that shares its X and W slices in that XCD's L2.
    const int total = mt * nt;
    const int per_xcd = (total + 7) / 8;
    const int t = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (t >= total) return;
    const int grp = t / (kMmGroup * nt), first = grp * kMmGroup;
    const int gm = min(mt - first, kMmGroup), r = t - grp * kMmGroup * nt;
    const int s0 = (first + r % gm) * BS, o0 = (r / gm) * BO;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c32 = lane & 31, h2 = lane >> 5;
    const int nk = (in_dim + kMmK - 1) / kMmK;

    const int wrange = (int)((int64_t)out_dim * in_dim * 2);
    const int xrange = (int)((int64_t)n_cols * in_dim * 4);
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(w), 0, wrange, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(x), 0, xrange, kRsrcWord3);

    // DMA plan: a stage is NWI one-KiB instructions of W (16 rows each) then
    // NXI of X (8 rows each); wave w issues instructions NDMA w .. NDMA w +
    // NDMA - 1.  Lane i of an instruction fills physical slot i of its KiB,
    // i.e. one row's slot p holding logical chunk p ^ swz(row).
    int dofs[NDMA], dk[NDMA];
#pragma unroll
    for (int c = 0; c < NDMA; c++) {
        const int ins = wave * NDMA + c;
        if (ins < C::NWI) {
            const int rr = ins * 16 + lane / 4;
            dk[c] = ((lane & 3) ^ mm_wswz(rr)) * 8;
            dofs[c] = o0 + rr < out_dim ? ((o0 + rr) * in_dim + dk[c]) * 2 : -1;
        } else {
            const int rr = (ins - C::NWI) * 8 + lane / 8;
            dk[c] = ((lane & 7) ^ mm_xswz(rr)) * 4;
            dofs[c] = s0 + rr < n_cols ? ((s0 + rr) * in_dim + dk[c]) * 4 : -1;
        }
    }
    // Loads of step k into its stage; steps past the end load zeros, so every
    // step issues the same count and one vmcnt value retires a step.
    auto issue = [&](int k) {
        char *dst = lds + (k % kMmNst) * STAGE + wave * NDMA * 1024;
        const int k0 = k * kMmK;
#pragma unroll
        for (int c = 0; c < NDMA; c++) {
            const bool isw = wave * NDMA + c < C::NWI;  // wave-uniform
            const int off = dofs[c] >= 0 && k0 + dk[c] < in_dim ? dofs[c] + k0 * (isw ? 2 : 4) : kMmOOB;
            dma16_cached(isw ? wrs : xrs, dst + c * 1024, off, 0);
        }
    };

    // Per-lane fragment addresses (stage 0): W rows wn*32*OI + c32 + 32 oi,
    // X rows wm*32*SI + c32 + 32 si.  Rows 32 apart share the swizzle, so oi,
    // si and the stage go into immediate offsets.
    const int wm = wave % WS, wn = wave / WS;
    const uint32_t lds0 = lds_addr(lds);
    uint32_t aw[2], ax[2][2];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
        aw[ks] = lds0 + (wn * 32 * OI + c32) * kMmWRB + (((2 * ks + h2) ^ mm_wswz(c32)) * 16);
#pragma unroll
        for (int hh = 0; hh < 2; hh++)
            ax[ks][hh] = lds0 + C::WT + (wm * 32 * SI + c32) * kMmXRB +
                         (((4 * ks + 2 * h2 + hh) ^ mm_xswz(c32)) * 16);
    }

    f32x16 acc[OI][SI];
#pragma unroll
    for (int i = 0; i < OI; i++)
#pragma unroll
        for (int j = 0; j < SI; j++) acc[i][j] = f32x16{};

    // Fragments of one k16 half-step: OI of W, SI x 2 of X as read (f32),
    // and the same operands ready for the matrix cores (X split hi/lo).
    struct Raw { u32x4 w[OI], x[SI][2]; };
    struct Ops { u32x4 w[OI], h[SI], l[SI]; };
    // Stages at or past 64 KiB are addressed from a second base (the
    // instruction offset field holds 16 bits).
    constexpr uint32_t kHi = 65536;
    auto read = [&](Raw &f, auto stc, auto ksc) {
        constexpr int SO0 = decltype(stc)::value * STAGE, KS = decltype(ksc)::value;
        constexpr int SO = SO0 >= (int)kHi ? SO0 - (int)kHi : SO0;
        constexpr uint32_t B = SO0 >= (int)kHi ? kHi : 0;
        static_for<0, OI>([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            f.w[i] = lds_read_b128_at<SO + i * 32 * kMmWRB>(aw[KS] + B);
        });
        static_for<0, SI>([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            f.x[i][0] = lds_read_b128_at<SO + i * 32 * kMmXRB>(ax[KS][0] + B);
            f.x[i][1] = lds_read_b128_at<SO + i * 32 * kMmXRB>(ax[KS][1] + B);
        });
    };
    auto convert = [&](Raw &f, Ops &o) {
#pragma unroll
        for (int i = 0; i < OI; i++) {
            tie(f.w[i]);
            o.w[i] = f.w[i];
        }
#pragma unroll
        for (int si = 0; si < SI; si++) {
            tie(f.x[si][0]);
            tie(f.x[si][1]);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const u32x4 &src = f.x[si][e >> 1];
                const u32x2 p = split2<BF16>(__uint_as_float(src[(e & 1) * 2]),
                                             __uint_as_float(src[(e & 1) * 2 + 1]));
                o.h[si][e] = p[0];
                o.l[si][e] = p[1];
            }
        }
    };
    // The MFMAs of one half-step (hi products, then lo products; the two
    // chains per accumulator are 2 OI SI MFMAs apart).
    auto mfma_at = [&](const Ops &o, int j) {
        const int lo = j / (OI * SI), oi = (j / SI) % OI, si = j % SI;
        acc[oi][si] = mfma32<BF16>(o.w[oi], lo ? o.l[si] : o.h[si], acc[oi][si]);
    };
    constexpr int NMF = 2 * OI * SI;
    constexpr int NRD = OI + 2 * SI;  // LDS reads per half-step
    // Half-step n: the MFMAs of `cur` (operands of half n), with half n+1's
    // fragments (read into `raw` a half-step earlier; the NRD reads of half
    // n+2 issued since may still be in flight) converted into `nxt` in their
    // shadow, MFMAs and conversion VALU alternating.
    auto half = [&](Ops &cur, Raw &raw, Ops &nxt) {
        lds_wait_n<NRD>();
        convert(raw, nxt);
#pragma unroll
        for (int j = 0; j < NMF; j++) mfma_at(cur, j);
        static_for<0, NMF>([&](auto) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // 3 VALU
        });
    };

    // Halves 2k (ks 0) and 2k+1 (ks 1) of step k use stage k % 4.  Step k
    // starts by retiring this wave's loads of step k+1 (k+2's stay in flight)
    // and meeting: everyone's step k+1 tiles have landed and everyone has
    // read (and converted) every fragment of step k-1, whose stage step k+3
    // refills.  Fragments are read two half-steps before their MFMAs.
    Raw ra, rb;
    Ops op[2];
    auto step = [&](auto stc, int k) {
        constexpr int NX = (decltype(stc)::value + 1) % kMmNst;
        __builtin_amdgcn_s_waitcnt(vm_wait(NDMA));
        wg_barrier();
        issue(k + 3);
        read(ra, Int<NX>{}, Int<0>{});  // half 2k+2
        half(op[0], rb, op[1]);         // MFMAs of 2k, convert 2k+1
        read(rb, Int<NX>{}, Int<1>{});  // half 2k+3
        half(op[1], ra, op[0]);         // MFMAs of 2k+1, convert 2k+2
    };

    issue(0);
    issue(1);
    issue(2);
    __builtin_amdgcn_s_waitcnt(vm_wait(NDMA));
    wg_barrier();
    read(ra, Int<0>{}, Int<0>{});
    read(rb, Int<0>{}, Int<1>{});
    lds_wait_n<NRD>();
    convert(ra, op[0]);
    for (int k = 0; k < nk; k += 4) {
        step(Int<0>{}, k);
        if (k + 1 < nk) step(Int<1>{}, k + 1);
        if (k + 2 < nk) step(Int<2>{}, k + 2);
        if (k + 3 < nk) step(Int<3>{}, k + 3);
    }
    // The zero-fill loads past the end and the last (unused) fragment reads.
    __builtin_amdgcn_s_waitcnt(vm_wait(0));
    lds_wait_any();

    // acc[oi][si][4 g + e] = Y[s, o] with s = s0 + wm*32*SI + si*32 + c32 and
    // o = o0 + wn*32*OI + oi*32 + 8 g + 4 h2 + e.
#pragma unroll
    for (int si = 0; si < SI; si++) {
        const int s = s0 + wm * 32 * SI + si * 32 + c32;
        if (s >= n_cols) continue;
        float *yr = y + (int64_t)s * out_dim;
#pragma unroll
        for (int oi = 0; oi < OI; oi++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int o = o0 + wn * 32 * OI + oi * 32 + 8 * g + 4 * h2;
                if (o < out_dim)
                    *(f32x4 *)(yr + o) = f32x4{acc[oi][si][4 * g], acc[oi][si][4 * g + 1],
                                               acc[oi][si][4 * g + 2], acc[oi][si][4 * g + 3]};
            }
    }
}

template <int SI, int OI, int WS, int WO>
static void launch_mm(const char *w, const float *x, float *y, int in_dim, int out_dim, int n,
                      hipStream_t st) {
    using C = MmCfg<SI, OI, WS, WO>;
    const int mt = (n + C::BS - 1) / C::BS, nt = (out_dim + C::BO - 1) / C::BO;
    const int per_xcd = (mt * nt + 7) / 8;
    hipLaunchKernelGGL((matmul_bf16_kernel<SI, OI, WS, WO>), dim3(per_xcd * 8), dim3(C::NT), 0, st,
                       w, x, y, in_dim, out_dim, n, mt, nt);
}

}  // namespace ullm

using namespace ullm;

extern "C" int ullm_hip_matmul(const void *w, int w_dtype, const float *x, float *y, int in_dim,
                               int out_dim, int n_cols, void *stream) {
    if (w_dtype != ULLM_DT_BF16)
        return set_error(ULLM_HIP_E_UNSUPPORTED, "matmul: weight dtype %d (bf16 only)", w_dtype);
    if (in_dim < 8 || in_dim % 8)
        return set_error(ULLM_HIP_E_INVALID, "matmul: in_dim %d must be a positive multiple of 8", in_dim);
    if (out_dim < 4 || out_dim % 4)
        return set_error(ULLM_HIP_E_INVALID, "matmul: out_dim %d must be a positive multiple of 4", out_dim);
    if (n_cols < 0) return set_error(ULLM_HIP_E_INVALID, "matmul: n_cols %d", n_cols);
    if ((int64_t)out_dim * in_dim * 2 > 0x7fff0000LL)
        return set_error(ULLM_HIP_E_INVALID, "matmul: weight of %lld bytes exceeds 2 GiB",
                         (long long)out_dim * in_dim * 2);
    if (n_cols == 0) return ULLM_HIP_OK;
    if (!w || !x || !y) return set_error(ULLM_HIP_E_INVALID, "matmul: null tensor pointer");
    if (((uintptr_t)w | (uintptr_t)x | (uintptr_t)y) & 15)
        return set_error(ULLM_HIP_E_INVALID, "matmul: w, x and y must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    // Token chunks whose X stays below 2 GiB (32-bit buffer offsets).
    const int chunk = (int)std::min<int64_t>(n_cols, (0x7fff0000LL / ((int64_t)in_dim * 4)) / 128 * 128);
    if (chunk < 1) return set_error(ULLM_HIP_E_INVALID, "matmul: in_dim %d too large", in_dim);
    for (int c0 = 0; c0 < n_cols; c0 += chunk) {
        const int n = std::min(chunk, n_cols - c0);
        const char *wp = (const char *)w;
        const float *xp = x + (int64_t)c0 * in_dim;
        float *yp = y + (int64_t)c0 * out_dim;
        // The large tile unless it leaves CUs idle (256 CUs, one workgroup each).
        const int64_t big = (int64_t)((n + 127) / 128) * ((out_dim + 255) / 256);
        if (big >= 256) launch_mm<2, 4, 2, 2>(wp, xp, yp, in_dim, out_dim, n, st);
        else launch_mm<1, 2, 2, 2>(wp, xp, yp, in_dim, out_dim, n, st);
    }
    return check_hip(hipGetLastError(), "matmul launch");
}
