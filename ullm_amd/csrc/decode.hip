// Split-KV single-query GQA decode attention for gfx950.
//
// Computes, for every sequence b and query head h (kv head h / kv_mul),
//   out[b,h] = softmax_t(scale * q[b,h] . K[t]) . V[t],  t in start..len-1
// which is the CPU reference loop crates/ullm-model/src/lib.rs:916-938
// (windowed start: lib.rs:1183-1186).
//
// Design (HBM-bound stream):
//  * One workgroup owns (sequence b, a group of G query heads that share one
//    kv head, a chunk of keys).  Each K/V row is loaded ONCE, with 16-byte
//    loads, and serves all G heads from registers (the Metal path re-reads
//    K/V per query head, shader.metal:957-964, :1014-1020).
//  * A row of D elements is spread over LPT = D/EPL lanes (EPL elements per
//    16-byte load); a wave therefore covers TPW = 64/LPT consecutive keys per
//    load instruction.  Each such lane group runs its own online softmax over
//    its keys (tiles of TT keys, one max/rescale per tile), so the only
//    cross-lane traffic in the stream is the LPT-lane dot-product sum (DPP).
//  * Lane groups merge by shuffles, waves merge through LDS, and chunks
//    (splits) are combined by decode_merge_kernel (decode_mfma.hip) in a
//    second launch.  A merge inside this kernel by the last workgroup to
//    arrive costs more than that launch: one CU then reads every partial of
//    the unit, after a store-drain and a device-scope counter round trip.
//  * Softmax runs in the exp2 domain: q is pre-multiplied by scale*log2(e).
#include "common.hpp"
#include "wave.hpp"
#include "mfma_util.hpp"
#include <cstdlib>
#include <algorithm>
#include <mutex>

namespace ullm {

constexpr int kDecodeWaves = 8;
constexpr int kTargetWorkgroups = 256;  // about one per CU

template <class T, int D, int G>
struct DecodeCfg {
    static constexpr int EPL = Chunk<T>::n;
    static constexpr int LPT = D / EPL;
    static constexpr int TPW = 64 / LPT;
    static constexpr int NW = kDecodeWaves;
    static constexpr int NLG = NW * TPW;                 // lane groups per workgroup
    static constexpr int TT = (G * EPL <= 48) ? 8 : 4;   // keys per lane group per tile
    static_assert(LPT >= 1 && LPT <= 64 && (LPT & (LPT - 1)) == 0, "bad lanes per key");
};

// Paged K/V for the split-KV kernel (tab == nullptr: contiguous cache).
// Key t of sequence b is row t % P of page tab[b * stride + t / P]
// (P = 2^shift); a page index outside the table row or [0, n_pages) reads
// as zeros.
struct KeyPages {
    const int32_t *tab;
    int stride, shift, n_pages;
};

// TTK: keys per lane group per tile when the split is shorter than a full
// tile (1 or 2; 0 = the configuration's TT), so short splits do not compute
// masked key slots.
template <class T, int D, int G, int TTK = 0>
__global__ __launch_bounds__(kDecodeWaves * 64, 1) void decode_split_kernel(
    const float *__restrict__ q, const char *__restrict__ kc, const char *__restrict__ vc,
    int64_t kv_stride, int64_t seq_stride, const int32_t *__restrict__ seq_lens, int window,
    int n_head, int kv_mul, int n_groups, int chunk, int splits, float qscale,
    float *__restrict__ out, float *__restrict__ ws_ml, float *__restrict__ ws_acc, KeyPages kp) {
    using C = DecodeCfg<T, D, G>;
    constexpr int EPL = C::EPL, LPT = C::LPT, TPW = C::TPW, NW = C::NW, NLG = C::NLG;
    constexpr int TT = TTK > 0 && TTK < C::TT ? TTK : C::TT;
    constexpr int EB = T::bytes;

    const int split = blockIdx.x, grp = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sub = lane % LPT, lg = wave * TPW + lane / LPT;
    const int head0 = grp * G, kvh = head0 / kv_mul;

    const int len = seq_lens[b];
    const int start = (window > 0 && len > window) ? len - window : 0;
    const int c0 = start + split * chunk;
    const int c1 = min(c0 + chunk, len);

    // q slice of this lane, pre-scaled into the exp2 domain.
    float qf[G][EPL];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float *qp = q + ((int64_t)b * n_head + head0 + g) * D + sub * EPL;
#pragma unroll
        for (int e = 0; e < EPL; e += 4) {
            f32x4 v = *(const f32x4 *)(qp + e);
            qf[g][e] = v[0] * qscale; qf[g][e + 1] = v[1] * qscale;
            qf[g][e + 2] = v[2] * qscale; qf[g][e + 3] = v[3] * qscale;
        }
    }

    float m[G], l[G], acc[G][EPL];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -INFINITY; l[g] = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) acc[g][e] = 0.f;
    }

    const int64_t row_bytes = kv_stride * EB;
    const char *kbase = kc + (int64_t)b * seq_stride * EB + ((int64_t)kvh * D + sub * EPL) * EB;
    const char *vbase = vc + (int64_t)b * seq_stride * EB + ((int64_t)kvh * D + sub * EPL) * EB;

    // Cache row of key t: t itself, or its paged slot (-1: reads zeros).
    auto key_row = [&](int t) -> int64_t {
        if (!kp.tab) return t;
        const int pi = t >> kp.shift;
        const int phys = pi < kp.stride ? kp.tab[(int64_t)b * kp.stride + pi] : -1;
        if (phys < 0 || phys >= kp.n_pages) return -1;
        return ((int64_t)phys << kp.shift) + (t & ((1 << kp.shift) - 1));
    };
    for (int base = c0; base < c1; base += NLG * TT) {
        u32x4 kr[TT], vr[TT];
        bool ok[TT];
        int64_t rw[TT];
#pragma unroll
        for (int i = 0; i < TT; i++) {
            const int t = base + lg + NLG * i;
            ok[i] = t < c1;
            rw[i] = ok[i] ? key_row(t) : -1;
            kr[i] = rw[i] >= 0 ? ld16_stream(kbase + rw[i] * row_bytes) : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < TT; i++)
            vr[i] = rw[i] >= 0 ? ld16_stream(vbase + rw[i] * row_bytes) : u32x4{0, 0, 0, 0};
        float s[G][TT];
#pragma unroll
        for (int i = 0; i < TT; i++) {
            float kf[EPL];
            Chunk<T>::widen(kr[i], kf);
#pragma unroll
            for (int g = 0; g < G; g++) {
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < EPL; e++) d += qf[g][e] * kf[e];
                d = group_sum<LPT>(d);
                s[g][i] = ok[i] ? d : -INFINITY;
            }
        }
        float pv[G][TT], corr[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            float mt = s[g][0];
#pragma unroll
            for (int i = 1; i < TT; i++) mt = fmaxf(mt, s[g][i]);
            const float mn = fmaxf(m[g], mt);
            const float mu = (mn == -INFINITY) ? 0.f : mn;  // all masked so far
            corr[g] = exp2f(m[g] - mu);
            float ps = 0.f;
#pragma unroll
            for (int i = 0; i < TT; i++) { pv[g][i] = exp2f(s[g][i] - mu); ps += pv[g][i]; }
            l[g] = l[g] * corr[g] + ps;
            m[g] = mn;
#pragma unroll
            for (int e = 0; e < EPL; e++) acc[g][e] *= corr[g];
        }
#pragma unroll
        for (int i = 0; i < TT; i++) {
            float vf[EPL];
            Chunk<T>::widen(vr[i], vf);
#pragma unroll
            for (int g = 0; g < G; g++)
#pragma unroll
                for (int e = 0; e < EPL; e++) acc[g][e] += pv[g][i] * vf[e];
        }
    }

    // Merge the lane groups of this wave (lanes sub, sub+LPT, ...): a
    // butterfly over lane ^ LPT, .. lane ^ 32.  At 16 and 32 the row swaps
    // hand every lane both states of its pair in registers (the merge is
    // symmetric, so their order does not matter); below 16, shuffles.
    auto merge_pair = [&](int g, float m0, float l0, float m1, float l1, float &a, float &c) {
        const float mn = fmaxf(m0, m1);
        const float mu = (mn == -INFINITY) ? 0.f : mn;
        a = exp2f(m0 - mu);
        c = exp2f(m1 - mu);
        l[g] = l0 * a + l1 * c;
        m[g] = mn;
    };
    auto swap16 = [](float x) {
        return __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    };
    auto swap32 = [](float x) {
        return __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    };
    auto merge_rows = [&](auto swp) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            const auto mm = swp(m[g]), ll = swp(l[g]);
            float a, c;
            merge_pair(g, __uint_as_float(mm[0]), __uint_as_float(ll[0]), __uint_as_float(mm[1]),
                       __uint_as_float(ll[1]), a, c);
#pragma unroll
            for (int e = 0; e < EPL; e++) {
                const auto aa = swp(acc[g][e]);
                acc[g][e] = __uint_as_float(aa[0]) * a + __uint_as_float(aa[1]) * c;
            }
        }
    };
#pragma unroll
    for (int off = LPT; off < 16; off <<= 1) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float mo = __shfl_xor(m[g], off, 64), lo = __shfl_xor(l[g], off, 64);
            float a, c;
            merge_pair(g, m[g], l[g], mo, lo, a, c);
#pragma unroll
            for (int e = 0; e < EPL; e++) acc[g][e] = acc[g][e] * a + __shfl_xor(acc[g][e], off, 64) * c;
        }
    }
    if constexpr (LPT <= 16) merge_rows(swap16);
    if constexpr (LPT <= 32) merge_rows(swap32);

    // Merge the waves through LDS.
    constexpr int kAccFloats = NW * G * D;
    __shared__ float sm_ml[NW][G][2];
    __shared__ __attribute__((aligned(16))) float sm_acc[1][1][kAccFloats];
    if (lane < LPT) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            if (lane == 0) { sm_ml[wave][g][0] = m[g]; sm_ml[wave][g][1] = l[g]; }
#pragma unroll
            for (int e = 0; e < EPL; e++) sm_acc[0][0][(wave * G + g) * D + sub * EPL + e] = acc[g][e];
        }
    }
    __syncthreads();

    const int64_t unit = (int64_t)b * n_groups + grp;
    for (int idx = tid; idx < G * D; idx += NW * 64) {
        const int g = idx / D, d = idx % D;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) mx = fmaxf(mx, sm_ml[w][g][0]);
        const float mu = (mx == -INFINITY) ? 0.f : mx;
        float num = 0.f, den = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float c = exp2f(sm_ml[w][g][0] - mu);
            num += sm_acc[0][0][(w * G + g) * D + d] * c;
            den += sm_ml[w][g][1] * c;
        }
        if (splits == 1) {
            out[((int64_t)b * n_head + head0 + g) * D + d] = den > 0.f ? num / den : 0.f;
        } else {
            // The split's partial (O unnormalised, then m, l) for
            // decode_merge_kernel.
            ws_acc[(unit * splits + split) * (G * D) + idx] = num;
            if (d == 0)
                *(float2 *)(ws_ml + ((unit * splits + split) * G + g) * 2) = float2{mx, den};
        }
    }
}

// ---------------------------------------------------------------------------
// Host side: launch planning and dispatch.

struct DecodePlan {
    int G, n_groups, chunk, splits, nlg;
    size_t off_ml, off_acc, bytes;
};

static int pick_group(int kv_mul) {
    const int cands[] = {8, 6, 4, 2, 1};
    for (int g : cands)
        if (kv_mul % g == 0) return g;
    return 1;
}

static int lanes_per_key(int dtype, int D) { return D / (16 / dtype_bytes(dtype)); }

// Split-KV plan.  Chunks are multiples of the lane-group count so every lane
// group gets whole keys; the split count aims at a few workgroups per CU but is
// capped at the merge kernel's limit.
static const int kEnvSplits = env_override("ULLM_HIP_DECODE_SPLITS");

static DecodePlan plan_decode(int batch, int n_head, int n_kv_head, int D, int dtype, int max_len,
                              int window) {
    DecodePlan p{};
    const int kv_mul = n_head / n_kv_head;
    p.G = pick_group(kv_mul);
    p.n_groups = n_head / p.G;
    const int lpt = lanes_per_key(dtype, D);
    p.nlg = kDecodeWaves * (64 / lpt);
    const int visible = (window > 0 && max_len > window) ? window : max_len;
    const int units = batch * p.n_groups;
    // A context that one workgroup iteration covers (tile keys) is not
    // split.  Past that, every split holds at least one key per lane group,
    // so short contexts still spread over about one workgroup per CU
    // (measured: cfg1-shaped L = 512 over 16 splits 10.6 us per layer, over
    // 2 splits of one full tile each 12.1 us).
    const int epl = 16 / dtype_bytes(dtype);
    const int tile = p.nlg * ((p.G * epl <= 48) ? 8 : 4);
    int splits = visible <= tile ? 1 : (visible + p.nlg - 1) / p.nlg;
    const int want = (kTargetWorkgroups + units - 1) / units;
    if (splits > want) splits = want;
    const int merge_cap = 256 / p.G;                       // merge reads <= 256 partial rows
    if (splits > merge_cap) splits = merge_cap;
    if (kEnvSplits >= 1) splits = kEnvSplits < merge_cap ? kEnvSplits : merge_cap;  // tuning override
    if (splits < 1) splits = 1;
    int chunk = (visible + splits - 1) / splits;
    chunk = ((chunk + p.nlg - 1) / p.nlg) * p.nlg;
    p.chunk = chunk;
    p.splits = (visible + chunk - 1) / chunk;
    const size_t ml = ((size_t)units * p.splits * p.G * 2 * 4 + 255) / 256 * 256;
    const size_t ac = (size_t)units * p.splits * p.G * D * 4;
    p.off_ml = 0;
    p.off_acc = ml;
    p.bytes = p.splits > 1 ? ml + ac : 0;
    return p;
}

template <class T, int D, int G>
static void launch_decode(const DecodePlan &p, const float *q, const void *kc, const void *vc,
                          int64_t kv_stride, int64_t seq_stride, const int32_t *lens, int window,
                          int batch, int n_head, int kv_mul, float qscale, float *out, char *ws,
                          hipStream_t st, KeyPages kp) {
    dim3 grid(p.splits, p.n_groups, batch);
    const int kpl = (p.chunk + p.nlg - 1) / p.nlg;  // keys per lane group
#define ULLM_SPLIT(TTK)                                                                        \
    hipLaunchKernelGGL((decode_split_kernel<T, D, G, TTK>), grid, dim3(kDecodeWaves * 64), 0, st, \
                       q, (const char *)kc, (const char *)vc, kv_stride, seq_stride, lens,      \
                       window, n_head, kv_mul, p.n_groups, p.chunk, p.splits, qscale, out,      \
                       (float *)(ws + p.off_ml), (float *)(ws + p.off_acc), kp)
    if (kpl <= 1) ULLM_SPLIT(1);
    else if (kpl <= 2) ULLM_SPLIT(2);
    else ULLM_SPLIT(0);
#undef ULLM_SPLIT
    if (p.splits > 1)
        decode_merge_launch(D, (const float *)(ws + p.off_ml), (const float *)(ws + p.off_acc),
                            p.splits, G, p.n_groups, batch, n_head, out, st);
}

template <class T, int D>
static int dispatch_g(const DecodePlan &p, const float *q, const void *kc, const void *vc,
                      int64_t kvs, int64_t ss, const int32_t *lens, int win, int batch, int nh,
                      int kv_mul, float qs, float *out, char *ws, hipStream_t st, KeyPages kp) {
    switch (p.G) {
        case 1: launch_decode<T, D, 1>(p, q, kc, vc, kvs, ss, lens, win, batch, nh, kv_mul, qs, out, ws, st, kp); break;
        case 2: launch_decode<T, D, 2>(p, q, kc, vc, kvs, ss, lens, win, batch, nh, kv_mul, qs, out, ws, st, kp); break;
        case 4: launch_decode<T, D, 4>(p, q, kc, vc, kvs, ss, lens, win, batch, nh, kv_mul, qs, out, ws, st, kp); break;
        case 6: launch_decode<T, D, 6>(p, q, kc, vc, kvs, ss, lens, win, batch, nh, kv_mul, qs, out, ws, st, kp); break;
        case 8: launch_decode<T, D, 8>(p, q, kc, vc, kvs, ss, lens, win, batch, nh, kv_mul, qs, out, ws, st, kp); break;
        default: return set_error(ULLM_HIP_E_UNSUPPORTED, "decode: no kernel for head group %d", p.G);
    }
    return check_hip(hipGetLastError(), "decode launch");
}

template <class T>
static int dispatch_d(int D, const DecodePlan &p, const float *q, const void *kc, const void *vc,
                      int64_t kvs, int64_t ss, const int32_t *lens, int win, int batch, int nh,
                      int kv_mul, float qs, float *out, char *ws, hipStream_t st,
                      KeyPages kp = KeyPages{}) {
    switch (D) {
        case 64: return dispatch_g<T, 64>(p, q, kc, vc, kvs, ss, lens, win, batch, nh, kv_mul, qs, out, ws, st, kp);
        case 128: return dispatch_g<T, 128>(p, q, kc, vc, kvs, ss, lens, win, batch, nh, kv_mul, qs, out, ws, st, kp);
        case 256: return dispatch_g<T, 256>(p, q, kc, vc, kvs, ss, lens, win, batch, nh, kv_mul, qs, out, ws, st, kp);
        default: return set_error(ULLM_HIP_E_UNSUPPORTED, "decode: head_dim %d not in {64,128,256}", D);
    }
}

static int validate_decode(int kv_dtype, int64_t kv_stride, int max_len, int batch, int n_head,
                           int n_kv_head, int D) {
    if (!dtype_ok(kv_dtype)) return set_error(ULLM_HIP_E_UNSUPPORTED, "decode: kv dtype %d", kv_dtype);
    if (batch < 1 || n_head < 1 || n_kv_head < 1 || n_head % n_kv_head)
        return set_error(ULLM_HIP_E_INVALID, "decode: bad heads n_head=%d n_kv_head=%d batch=%d",
                         n_head, n_kv_head, batch);
    if (D != 64 && D != 128 && D != 256)
        return set_error(ULLM_HIP_E_UNSUPPORTED, "decode: head_dim %d not in {64,128,256}", D);
    if (max_len < 1) return set_error(ULLM_HIP_E_INVALID, "decode: max_len %d < 1", max_len);
    if (kv_stride < (int64_t)n_kv_head * D || (kv_stride * dtype_bytes(kv_dtype)) % 16)
        return set_error(ULLM_HIP_E_INVALID,
                         "decode: kv_stride %lld must be >= n_kv_head*head_dim and 16-byte aligned",
                         (long long)kv_stride);
    return ULLM_HIP_OK;
}

}  // namespace ullm

using namespace ullm;

extern "C" size_t ullm_hip_decode_workspace_bytes(int batch, int n_head, int n_kv_head,
                                                  int head_dim, int max_len, int window) {
    if (batch < 1 || n_head < 1 || n_kv_head < 1 || n_head % n_kv_head || max_len < 1) return 0;
    // The f32 cache has the most lanes per key and thus the smallest chunks:
    // size for the largest plan over the three dtypes.
    if (head_dim != 64 && head_dim != 128 && head_dim != 256) return 0;
    size_t best = decode_f32_workspace(batch, n_head, n_kv_head, head_dim, max_len, window);
    const size_t m = decode_mfma_workspace(batch, n_head, n_kv_head, head_dim, max_len, window);
    return m > best ? m : best;
}

extern "C" int ullm_hip_attn_decode(const float *q, const void *k_cache, const void *v_cache,
                                    int kv_dtype, int64_t kv_stride, int64_t seq_stride,
                                    const int32_t *seq_lens, int max_len, int window, int batch,
                                    int n_head, int n_kv_head, int head_dim, float scale,
                                    float *out, void *workspace, size_t workspace_bytes,
                                    void *stream) {
    int rc = validate_decode(kv_dtype, kv_stride, max_len, batch, n_head, n_kv_head, head_dim);
    if (rc) return rc;
    if (!q || !k_cache || !v_cache || !seq_lens || !out)
        return set_error(ULLM_HIP_E_INVALID, "decode: null tensor pointer");
    if (((uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)q) & 15)
        return set_error(ULLM_HIP_E_INVALID, "decode: q/k_cache/v_cache must be 16-byte aligned");
    if (batch > 1 && (seq_stride * dtype_bytes(kv_dtype)) % 16)
        return set_error(ULLM_HIP_E_INVALID, "decode: seq_stride must be 16-byte aligned");
    const float qscale = scale * kLog2e;
    hipStream_t st = (hipStream_t)stream;
    if (kv_dtype != ULLM_DT_F32)
        return decode_mfma(kv_dtype, q, k_cache, v_cache, kv_stride, seq_stride, seq_lens, max_len,
                           window, batch, n_head, n_kv_head, head_dim, qscale, out, workspace,
                           workspace_bytes, st);
    // Short splits of an f32 cache run on the MFMA block kernel (bf16 hi + lo
    // products); the rest on decode_split_kernel below.
    size_t fb = 0;
    if (decode_f32_block_plan(batch, n_head, n_kv_head, head_dim, max_len, window, &fb))
        return decode_mfma(kv_dtype, q, k_cache, v_cache, kv_stride, seq_stride, seq_lens, max_len,
                           window, batch, n_head, n_kv_head, head_dim, qscale, out, workspace,
                           workspace_bytes, st);
    DecodePlan p = plan_decode(batch, n_head, n_kv_head, head_dim, kv_dtype, max_len, window);
    if (p.bytes > 0 && (!workspace || workspace_bytes < p.bytes))
        return set_error(ULLM_HIP_E_WORKSPACE, "decode: workspace of %zu bytes needed, %zu given",
                         p.bytes, workspace_bytes);
    const int kv_mul = n_head / n_kv_head;
    return dispatch_d<F32>(head_dim, p, q, k_cache, v_cache, kv_stride, seq_stride, seq_lens,
                           window, batch, n_head, kv_mul, qscale, out, (char *)workspace, st);
}

namespace ullm {

// f32-cache decode over a paged cache (the paged entry point routes f32
// here; f16/bf16 go to the MFMA kernels).
// Upper bound over every call whose max_len' <= max_len.  plan_decode's
// split count is not monotonic in the length (its chunks round up to whole
// lane groups, so a longer context can plan fewer splits), but it never
// exceeds min(want, merge cap, ceil(visible / nlg)), and each of those grows
// with the length: size for that many splits.
size_t decode_f32_workspace(int batch, int n_head, int n_kv_head, int D, int max_len, int window) {
    const DecodePlan p = plan_decode(batch, n_head, n_kv_head, D, ULLM_DT_F32, max_len, window);
    const int visible = (window > 0 && max_len > window) ? window : max_len;
    const int epl = 16 / dtype_bytes(ULLM_DT_F32);
    const int tile = p.nlg * ((p.G * epl <= 48) ? 8 : 4);
    if (visible <= tile) return 0;  // every shorter call runs unsplit too
    const int units = batch * p.n_groups;
    const int want = (kTargetWorkgroups + units - 1) / units;
    const int merge_cap = 256 / p.G;
    int smax = (visible + p.nlg - 1) / p.nlg;
    if (smax > want) smax = want;
    if (smax > merge_cap) smax = merge_cap;
    if (kEnvSplits >= 1) smax = std::max(smax, std::min(kEnvSplits, merge_cap));
    if (smax <= 1) return 0;
    const size_t ml = ((size_t)units * smax * p.G * 2 * 4 + 255) / 256 * 256;
    return ml + (size_t)units * smax * p.G * D * 4;
}

int decode_f32_paged(const float *q, const void *kp, const void *vp, int64_t kvs,
                     const int32_t *tab, int tab_stride, int shift, int n_pages,
                     const int32_t *lens, int max_len, int win, int batch, int nh, int nkv, int D,
                     float qs, float *out, void *ws, size_t ws_bytes, hipStream_t st) {
    const DecodePlan p = plan_decode(batch, nh, nkv, D, ULLM_DT_F32, max_len, win);
    if (p.bytes > 0 && (!ws || ws_bytes < p.bytes))
        return set_error(ULLM_HIP_E_WORKSPACE, "decode_paged: workspace of %zu bytes needed, %zu given",
                         p.bytes, ws_bytes);
    return dispatch_d<F32>(D, p, q, kp, vp, kvs, 0, lens, win, batch, nh, nh / nkv, qs, out,
                           (char *)ws, st, KeyPages{tab, tab_stride, shift, n_pages});
}

}  // namespace ullm


// ---------------------------------------------------------------------------
// Decode without any allocation: the split partials live in a file-scope
// device array instead of a caller workspace.  No counterpart in the
// reference; for callers that cannot allocate (code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc).
namespace ullm {

constexpr size_t kScratchBytes = (size_t)4 << 20;
// One copy per GPU, held until the process ends.  In host code `scratch` is
// only a handle: its device address (per device) comes from
// hipGetSymbolAddress and is what kernels and copies receive.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static void *g_scratch_addr[kMaxDevices];
static std::once_flag g_scratch_once[kMaxDevices];
static hipError_t g_scratch_err[kMaxDevices];

// The device address of `scratch` on the current device, resolved once per
// device (with that device current) on its first call.
static int scratch_address(void **out) {
    int dev = -1;
    int rc = check_hip(hipGetDevice(&dev), "decode_noalloc: hipGetDevice");
    if (rc) return rc;
    if (dev < 0 || dev >= kMaxDevices)
        return set_error(ULLM_HIP_E_UNSUPPORTED, "decode_noalloc: device %d beyond %d", dev,
                         kMaxDevices);
    std::call_once(g_scratch_once[dev], [dev] {
        void *p = nullptr;
        g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch_addr[dev] = g_scratch_err[dev] == hipSuccess ? p : nullptr;
    });
    if (g_scratch_err[dev] != hipSuccess)
        return check_hip(g_scratch_err[dev], "decode_noalloc: hipGetSymbolAddress(scratch)");
    *out = g_scratch_addr[dev];
    return ULLM_HIP_OK;
}

}  // namespace ullm

extern "C" size_t ullm_hip_decode_noalloc_max_bytes(void) { return kScratchBytes; }

extern "C" int ullm_hip_attn_decode_noalloc(const float *q, const void *k_cache,
                                            const void *v_cache, int kv_dtype, int64_t kv_stride,
                                            int64_t seq_stride, const int32_t *seq_lens,
                                            int max_len, int window, int batch, int n_head,
                                            int n_kv_head, int head_dim, float scale, float *out,
                                            void *stream) {
    int rc = validate_decode(kv_dtype, kv_stride, max_len, batch, n_head, n_kv_head, head_dim);
    if (rc) return rc;
    // This call's partials (its own plan, not the bound over shorter calls).
    size_t need = 0;
    if (kv_dtype != ULLM_DT_F32)
        need = decode_mfma_plan_bytes(batch, n_head, n_kv_head, head_dim, max_len, window);
    else if (!decode_f32_block_plan(batch, n_head, n_kv_head, head_dim, max_len, window, &need))
        need = plan_decode(batch, n_head, n_kv_head, head_dim, kv_dtype, max_len, window).bytes;
    if (need > kScratchBytes)
        return set_error(ULLM_HIP_E_WORKSPACE,
                         "decode_noalloc: this shape needs %zu bytes of split partials, above the "
                         "%zu-byte static scratch; use ullm_hip_attn_decode with a workspace",
                         need, kScratchBytes);
    void *ws = nullptr;
    if (need > 0) {
        rc = scratch_address(&ws);
        if (rc) return rc;
    }
    return ullm_hip_attn_decode(q, k_cache, v_cache, kv_dtype, kv_stride, seq_stride, seq_lens,
                                max_len, window, batch, n_head, n_kv_head, head_dim, scale, out,
                                ws, need > 0 ? kScratchBytes : 0, stream);
}
