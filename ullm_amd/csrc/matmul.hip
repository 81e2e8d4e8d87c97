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
// of every activation (relative residual <= 2^-17), and both halves are
// multiplied on v_mfma_f32_32x32x16_bf16 into one f32 accumulator.  The
// products themselves are exact in the MFMA's f32 accumulate, so the result
// differs from an f32 dot product only by the residual of the split and the
// summation order.
//
// Tiling: a workgroup of 4 waves computes a 128 (tokens) x 128 (outputs) tile
// of Y over in_dim in steps of 32.  Both operands go global -> LDS by
// buffer_load ... lds (W as bf16 rows of 64 bytes, X as f32 rows of 128
// bytes) into a 3-stage ring of 24 KiB stages, loaded two steps ahead, so a
// step waits on loads issued two steps earlier and two workgroups share a CU.
// The X fragments are split into bf16 hi/lo in registers after the LDS read.
// Each wave owns a 64 x 64 quadrant: with the MFMA computing Y^T = W . X^T, an
// accumulator lane holds one token (lane % 32) and 4 consecutive outputs per
// register group, which become 16-byte row stores.  16-byte LDS slots are
// XOR-swizzled by row so that the ds_read_b128 of 16 consecutive rows at one
// k offset hit 16 different bank groups.
#include "common.hpp"
#include "mfma_util.hpp"

namespace ullm {

constexpr int kMmB = 128;                 // tile rows (tokens) = tile columns (outputs)
constexpr int kMmK = 32;                  // in_dim per step
constexpr int kMmWRB = kMmK * 2;          // bytes of one W tile row (bf16)
constexpr int kMmXRB = kMmK * 4;          // bytes of one X tile row (f32)
constexpr int kMmWTile = kMmB * kMmWRB;   // 8 KiB
constexpr int kMmStage = kMmWTile + kMmB * kMmXRB;  // W then X: 24 KiB
constexpr int kMmNst = 3;
constexpr int kMmGroup = 8;              // token tiles per group of the tile order
constexpr int kMmThreads = 256;
constexpr int kMmDma = kMmStage / 1024 / 4;  // 1 KiB DMA instructions per wave per step
constexpr int kMmOOB = 0x7ffffff0;        // buffer offset past every valid range: reads zero

// Slot swizzles: 4 W rows (16 slots) or 2 X rows (8 slots each) share a
// 256-byte bank line; XOR the slot with the row's line index.
__device__ __forceinline__ int mm_wswz(int r) { return (r >> 2) & 3; }
__device__ __forceinline__ int mm_xswz(int r) { return (r >> 1) & 7; }

__global__ __launch_bounds__(kMmThreads, 2) void matmul_bf16_kernel(
    const char *__restrict__ w, const float *__restrict__ x, float *__restrict__ y, int in_dim,
    int out_dim, int n_cols, int mt, int nt) {
    __shared__ __attribute__((aligned(1024))) char lds[kMmNst * kMmStage];

    // Workgroup i runs on XCD i % 8; each XCD takes a contiguous run of tile
    // indices, and the indices run over groups of kMmGroup token tiles x all
    // output tiles, token tile fastest: the ~64 tiles an XCD holds at once
    // form an 8 x 8 block that shares its X and W slices in that XCD's L2.
    const int total = mt * nt;
    const int per_xcd = (total + 7) / 8;
    const int t = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (t >= total) return;
    const int grp = t / (kMmGroup * nt), first = grp * kMmGroup;
    const int gm = min(mt - first, kMmGroup), r = t - grp * kMmGroup * nt;
    const int s0 = (first + r % gm) * kMmB, o0 = (r / gm) * kMmB;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c32 = lane & 31, h2 = lane >> 5;
    const int nk = (in_dim + kMmK - 1) / kMmK;

    const int wrange = (int)((int64_t)out_dim * in_dim * 2);
    const int xrange = (int)((int64_t)n_cols * in_dim * 4);
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(w), 0, wrange, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(x), 0, xrange, kRsrcWord3);

    // DMA plan: a stage is 24 one-KiB instructions (8 of W: 16 rows each; 16
    // of X: 8 rows each); wave w issues instructions 6w .. 6w+5.  Lane i of an
    // instruction fills physical slot i of its KiB, i.e. one row's slot p
    // holding logical chunk p ^ swz(row).
    int dofs[kMmDma], dk[kMmDma];
#pragma unroll
    for (int c = 0; c < kMmDma; c++) {
        const int ins = wave * kMmDma + c;
        if (ins < 8) {
            const int r = ins * 16 + lane / 4;
            dk[c] = ((lane & 3) ^ mm_wswz(r)) * 8;
            dofs[c] = o0 + r < out_dim ? ((o0 + r) * in_dim + dk[c]) * 2 : -1;
        } else {
            const int r = (ins - 8) * 8 + lane / 8;
            dk[c] = ((lane & 7) ^ mm_xswz(r)) * 4;
            dofs[c] = s0 + r < n_cols ? ((s0 + r) * in_dim + dk[c]) * 4 : -1;
        }
    }
    // Loads of step k into its stage; steps past the end load zeros, so every
    // step issues the same count and one vmcnt value retires a step.
    auto issue = [&](int k) {
        char *dst = lds + (k % kMmNst) * kMmStage + wave * kMmDma * 1024;
        const int k0 = k * kMmK;
#pragma unroll
        for (int c = 0; c < kMmDma; c++) {
            const bool isw = wave * kMmDma + c < 8;  // wave-uniform
            const int off = dofs[c] >= 0 && k0 + dk[c] < in_dim ? dofs[c] + k0 * (isw ? 2 : 4) : kMmOOB;
            dma16_cached(isw ? wrs : xrs, dst + c * 1024, off, 0);
        }
    };

    // Per-lane fragment addresses: W rows wn*64 + c32 (+32), X rows
    // wm*64 + c32 (+32).  Rows 32 apart share the swizzle, so the +32 rows
    // and the stage go into immediate offsets.
    const int wm = wave & 1, wn = wave >> 1;
    const uint32_t lds0 = lds_addr(lds);
    uint32_t aw[2], ax[2][2];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
        aw[ks] = lds0 + (wn * 64 + c32) * kMmWRB + (((2 * ks + h2) ^ mm_wswz(c32)) * 16);
#pragma unroll
        for (int hh = 0; hh < 2; hh++)
            ax[ks][hh] = lds0 + kMmWTile + (wm * 64 + c32) * kMmXRB +
                         (((4 * ks + 2 * h2 + hh) ^ mm_xswz(c32)) * 16);
    }

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x16{};

    auto compute = [&](auto stc) {
        constexpr int SO = decltype(stc)::value * kMmStage;
        u32x4 fw[2][2], fx[2][2][2];  // [ks][tile](half)
        static_for<0, 2>([&](auto ksc) {
            constexpr int ks = decltype(ksc)::value;
            fw[ks][0] = lds_read_b128_at<SO>(aw[ks]);
            fw[ks][1] = lds_read_b128_at<SO + 32 * kMmWRB>(aw[ks]);
            static_for<0, 2>([&](auto hc) {
                constexpr int hh = decltype(hc)::value;
                fx[ks][0][hh] = lds_read_b128_at<SO>(ax[ks][hh]);
                fx[ks][1][hh] = lds_read_b128_at<SO + 32 * kMmXRB>(ax[ks][hh]);
            });
        });
        static_for<0, 2>([&](auto ksc) {
            constexpr int ks = decltype(ksc)::value;
            if constexpr (ks == 0) lds_wait_n<6>();
            else lds_wait_n<0>();
            u32x4 xh[2], xl[2];
#pragma unroll
            for (int si = 0; si < 2; si++) {
                tie(fw[ks][si]);
                tie(fx[ks][si][0]);
                tie(fx[ks][si][1]);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const u32x4 &src = fx[ks][si][e >> 1];
                    const u32x2 p = split2<BF16>(__uint_as_float(src[(e & 1) * 2]),
                                                 __uint_as_float(src[(e & 1) * 2 + 1]));
                    xh[si][e] = p[0];
                    xl[si][e] = p[1];
                }
            }
#pragma unroll
            for (int oi = 0; oi < 2; oi++)
#pragma unroll
                for (int si = 0; si < 2; si++) acc[oi][si] = mfma32<BF16>(fw[ks][oi], xh[si], acc[oi][si]);
#pragma unroll
            for (int oi = 0; oi < 2; oi++)
#pragma unroll
                for (int si = 0; si < 2; si++) acc[oi][si] = mfma32<BF16>(fw[ks][oi], xl[si], acc[oi][si]);
        });
    };
    // Step k: retire this wave's loads of step k (step k+1's stay in flight),
    // meet (everyone's step-k tiles landed; everyone done with step k-1, whose
    // stage step k+2 reuses), start step k+2, compute step k.
    auto step = [&](auto stc, int k) {
        __builtin_amdgcn_s_waitcnt(vm_wait(kMmDma));
        wg_barrier();
        issue(k + 2);
        compute(stc);
    };

    issue(0);
    issue(1);
    for (int k = 0; k < nk; k += 3) {
        step(Int<0>{}, k);
        if (k + 1 < nk) step(Int<1>{}, k + 1);
        if (k + 2 < nk) step(Int<2>{}, k + 2);
    }
    __builtin_amdgcn_s_waitcnt(vm_wait(0));  // the zero-fill loads past the end

    // acc[oi][si][4 g + e] = Y[s, o] with s = s0 + wm*64 + si*32 + c32 and
    // o = o0 + wn*64 + oi*32 + 8 g + 4 h2 + e.
#pragma unroll
    for (int si = 0; si < 2; si++) {
        const int s = s0 + wm * 64 + si * 32 + c32;
        if (s >= n_cols) continue;
        float *yr = y + (int64_t)s * out_dim;
#pragma unroll
        for (int oi = 0; oi < 2; oi++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int o = o0 + wn * 64 + oi * 32 + 8 * g + 4 * h2;
                if (o < out_dim)
                    *(f32x4 *)(yr + o) = f32x4{acc[oi][si][4 * g], acc[oi][si][4 * g + 1],
                                               acc[oi][si][4 * g + 2], acc[oi][si][4 * g + 3]};
            }
    }
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
    const int chunk = (int)std::min<int64_t>(n_cols, (0x7fff0000LL / ((int64_t)in_dim * 4)) / kMmB * kMmB);
    if (chunk < 1) return set_error(ULLM_HIP_E_INVALID, "matmul: in_dim %d too large", in_dim);
    for (int c0 = 0; c0 < n_cols; c0 += chunk) {
        const int n = std::min(chunk, n_cols - c0);
        const int mt = (n + kMmB - 1) / kMmB, nt = (out_dim + kMmB - 1) / kMmB;
        const int per_xcd = (mt * nt + 7) / 8;
        hipLaunchKernelGGL(matmul_bf16_kernel, dim3(per_xcd * 8), dim3(kMmThreads), 0, st,
                           (const char *)w, x + (int64_t)c0 * in_dim, y + (int64_t)c0 * out_dim,
                           in_dim, out_dim, n, mt, nt);
    }
    return check_hip(hipGetLastError(), "matmul launch");
}
