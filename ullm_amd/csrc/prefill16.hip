// Causal prefill with 16-row waves, two per SIMD (gfx950): head_dim 256, and
// head_dim 128 for short prompts (prefill.hip picks it where prefill4_kernel's
// causal pairs would leave half the CUs idle).  Over an f32 cache (T = F32,
// head_dim 128 and 256) it is the default prefill at those head dims: K and V
// arrive as f32 tiles and are split in LDS into bf16 hi/lo K and f16 V tiles,
// and Q.K runs as three bf16 products (Khi.Qhi + Khi.Qlo + Klo.Qhi).
//
// Computes, for query row s (pos = start_pos + s) of head h,
// out = softmax_t(scale q.K[t]) . V[t] over t in the window start .. pos: the
// CPU reference loop crates/ullm-model/src/lib.rs:1061-1087 with the window
// rule of lib.rs:1183-1186, as the Metal kernel applies it per row
// (shader.metal:1051).  Online softmax in the exp2 domain with f32
// statistics and a lazily raised running max (P <= 2^8, exact in f16); P.V
// on f16 operands (a bf16 cache's V is widened to f16 in LDS).
//
// Every contraction runs on v_mfma_f32_16x16x32_{f16,bf16}:
//  * S^T[16 keys x 16 rows] = K . Q^T: K (A operand) is read from LDS, one
//    16-byte read per MFMA; Q^T (B operand) stays in 32 registers.  A 32-key
//    tile is two such accumulators, 8 values per lane: lane (row l%16,
//    group g = l/16) holds keys 4g..4g+3 and 16+4g..16+4g+3.
//  * O^T[16 d x 16 rows] += V^T . P^T: P^T (B operand) is those 8 values
//    exponentiated and packed, in the same key order; V^T (A operand) comes
//    from ds_read_b64_tr_b16 on the row-major V tile, reading rows 4g..4g+3
//    and 16+4g..16+4g+3 so the key orders match.
//  * O for 16 rows x 256 d is 64 registers (128 at 32 rows), so a wave needs
//    ~214 registers (~130 at head_dim 128) and two waves share each SIMD: one wave's softmax VALU
//    work and LDS waits overlap the other's MFMAs, which a lone wave per
//    SIMD (the 32-row layout at D = 256) cannot arrange for itself.
//
// Work split.  A workgroup has 8 waves and KS key streams (1 or 2); the
// NWS = 8/KS waves of a stream cover hw query heads of one kv head (hw = the
// largest power of two dividing kv_mul, at most 4) times NWS/hw consecutive
// 16-row blocks: a unit of UR = 16*NWS/hw rows.  Each 32-key K/V tile goes
// global -> LDS once per stream (buffer_load ... lds, 16-byte slots XOR-
// swizzled by row) and serves all of the stream's waves.  With KS = 2 the
// unit's key range is cut in two halves, one per stream, and the two partial
// (m, l, O) of every row are merged through LDS at the end: twice the
// workgroups for a short prompt, where whole units would leave CUs idle.
// With DS = 2 two workgroups share a unit: each computes the full Q.K and
// softmax but P.V and the output for one half of the value columns, so its
// V tiles are half as large (a third ring stage fits) and its step a quarter
// shorter; a short prompt's time is its longest unit's chain of steps.
// Workgroup b takes unit n_units-1-b/n_hg (longest first) of head group
// b % n_hg; the dispatcher deals workgroups to the 8 XCDs round-robin, so
// when n_hg divides 8 each XCD serves fixed kv heads and their K/V stays in
// one L2.
#include "common.hpp"
#include "mfma_util.hpp"
#include "wave.hpp"
#include <algorithm>
#include <climits>

namespace ullm {

// Physical 16-byte slot of logical chunk c of key row r: c ^ p16_kswz(r) in
// a K tile, c ^ p16_vswz(r) in a V tile (the low four chunk bits only; a
// 512-byte row spans two 256-byte bank lines).  Measured on MI355X with 8
// waves per CU reading back to back (bytes per clock per CU):
//  * K operand, ds_read_b128, lanes (row l%16, chunk 4s + l/16): 208 with
//    c ^ (r & 15), 115-118 with p16_vswz or a 2-bit interleave -- the read
//    runs at full rate only when each 16-lane row group's slots are the
//    row-index permutation of a plain contiguous read;
//  * V^T operand, ds_read_b64_tr_b16, lanes reading rows 4(l/16) + (l%16)/4
//    (+16) at chunk pair {2dt, 2dt+1}: 177 with p16_vswz, 111-114 with
//    c ^ (r & 15) and other swizzles.
__device__ __forceinline__ int p16_kswz(int r) { return r & 15; }
__device__ __forceinline__ int p16_vswz(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }

// Ring stages per key stream: as many K/V stages as a workgroup's share of
// 160 KB holds (OCC workgroups per CU), at most 4.
template <int KS, int DS, int D, int OCC, int EB = 2>
constexpr int p16_stages() {
    constexpr int stage = EB == 4 ? 32 * D * 4 + 32 * D * 4 / DS : 32 * D * 2 + 32 * D * 2 / DS;
    // f32, one key stream, head_dim 128: two converted tiles beside the ring
    constexpr int conv = EB == 4 && KS == 1 && D == 128 ? 2 * (2 * 32 * D * 2 + 32 * D * 2 / DS) : 0;
    constexpr int st = (160 * 1024 / OCC - conv) / (KS * stage);
    return st > 4 ? 4 : st;
}

template <class T, int KS, int DS, int D = 256, int OCC = 1,
          int NSTG = p16_stages<KS, DS, D, OCC, T::bytes>()>
__global__ __launch_bounds__(512, OCC) void prefill16_kernel(
    const uint16_t *__restrict__ q, const char *__restrict__ kc, const char *__restrict__ vc,
    int64_t kv_stride, int S, int start_pos, int window, int n_head, int kv_mul, int hw,
    int n_hg, int n_units, float qscale, float *__restrict__ out, KvPages pgs) {
    // DS = 2: the workgroup computes the full Q.K and softmax of its rows but
    // P.V and the output for one half of the 256 value columns only; its V
    // tiles hold that half (256-byte rows).
    // T = F32 (the reference's cache dtype, head_dim 128): K and V tiles
    // arrive in f32 and each wave converts the chunks its own DMA wrote, in
    // place, into bf16 hi and lo K tiles and an f16 V tile laid out as the
    // 16-bit path's; Q.K = Khi.Qhi + Khi.Qlo + Klo.Qhi (about 2^-16 of each
    // product), P.V as for f16.
    constexpr bool F = __is_same(T, F32);
    using MT = typename std::conditional<F, BF16, T>::type;  // Q.K operand type
    constexpr int BN = 32, RB = D * 2, RBV = RB / DS;  // rows of the 16-bit tiles
    static_assert(D == 128 || D == 256, "head_dim");
    static_assert(!F || KS == 1 || D == 128, "f32 cache at head_dim 256: one key stream");
    constexpr int RBF = D * T::bytes;  // cache bytes per key row of one head
    constexpr int RBFV = RBF / DS;     // f32 V bytes fetched per key row
    constexpr int TILE = BN * RB, TILEV = BN * RBV;
    constexpr int DMAK = F ? BN * RBF : TILE, DMAV = F ? BN * RBFV : TILEV;  // bytes fetched
    constexpr int STAGE = DMAK + DMAV;
    constexpr int VOFF = F ? 2 * TILE : TILE;  // V tile in a stage (f32: after K hi, K lo)
    // f32 with one key stream at head_dim 128: the converted tiles go to two
    // buffers of their own beside the f32 ring (alternating steps), so the
    // conversion needs no barrier of its own: a wave's DMA and its reads of
    // the f32 ring touch only its own chunks.
    constexpr bool SEP = F && KS == 1 && D == 128;
    constexpr int CONV = VOFF + TILEV;  // converted K hi, K lo and V tiles
    constexpr int NW = 8, NWS = NW / KS;  // waves per stream
    constexpr int NIC = DMAK / 1024 / NWS;    // 1 KiB DMA chunks per wave, K
    constexpr int NICV = DMAV / 1024 / NWS;  // and V
    constexpr int NKS = D / 32, NDT = D / 16 / DS;  // Q k-steps; value d tiles of this workgroup
    constexpr bool CVTV = __is_same(T, BF16);
    constexpr float kLazy = 8.0f;
    static_assert(KS == 1 || KS == 2, "key streams");
    static_assert(DS == 1 || DS == 2, "value column split");
    static_assert(NSTG >= 2 && KS * NSTG * STAGE + (SEP ? 2 * CONV : 0) <= 160 * 1024 / OCC, "LDS ring");
    static_assert(NIC >= 1 && NICV >= 1, "DMA chunks per wave");
    // The V swizzle permutes the 16 slots of each 256-byte half of a row: V
    // rows of at least 256 bytes (no value split at head_dim 128).
    static_assert(RBV >= 256, "V rows of 256 bytes or more");
    __shared__ __attribute__((aligned(1024))) char lds[KS * NSTG * STAGE + (SEP ? 2 * CONV : 0)];

    const int dh = DS == 1 ? 0 : (int)(blockIdx.x % DS);  // value half
    const int bx = (int)(blockIdx.x / DS);
    const int hg = bx % n_hg, u = n_units - 1 - bx / n_hg;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ks = wave / NWS, ws = wave % NWS;  // key stream, wave within the stream
    const int r16 = lane & 15, g = lane >> 4;
    const int UR = 16 * NWS / hw;
    const int head = hg * hw + ws % hw, kvh = head / kv_mul;
    const int row0 = u * UR + (ws / hw) * 16;  // first query row of this wave
    const int qrow = row0 + r16;
    const int pos_row = start_pos + qrow;
    const int64_t q_dim = (int64_t)n_head * D;
    const int kv_len = start_pos + S;

    // Key tiles [t0, t1) of the unit: the window start of its first row to
    // the causal end of its last; stream ks takes [t0 + ks*nsteps, ..).
    int t0, t1;
    {
        const int hi = start_pos + min(u * UR + UR, S);
        int lo = 0;
        if (window > 0) lo = max(start_pos + u * UR + 1 - window, 0);
        t0 = lo / BN;
        t1 = (hi + BN - 1) / BN;
    }
    const int nsteps = (t1 - t0 + KS - 1) / KS;
    const int tbase = t0 + ks * nsteps;  // this stream's first tile

    // ---- K/V DMA: 1 KiB chunks = two key rows, lane -> (row, slot) ----
    const int rbg = (int)(kv_stride * T::bytes);
    // Contiguous cache: one resource over the layer (the entry point bounds it
    // below 2 GiB).  Paged: resources per tile from page_tile; a zero-range
    // resource for the steps past the unit's range.
    const int range = pgs.tab ? 0 : (kv_len - 1) * rbg + RBF;
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(kc + (int64_t)kvh * RBF), 0, range, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(vc + (int64_t)kvh * RBF), 0, range, kRsrcWord3);
    int kofs[NIC], vofs[NICV];
#pragma unroll
    for (int i = 0; i < NIC; i++) {
        if constexpr (F) {  // f32 staging: plain rows, read back by the lane that fetched them
            const int r = (ws * NIC + i) * (1024 / RBF) + lane / (RBF / 16);
            kofs[i] = r * rbg + (lane % (RBF / 16)) * 16;
        } else {
            constexpr int KSL = RB / 16;  // 16-byte slots per K row
            const int r = (ws * NIC + i) * (1024 / RB) + lane / KSL;
            kofs[i] = r * rbg + (((lane % KSL) ^ p16_kswz(r)) * 16);
        }
    }
    // A V chunk is 1024 / RBV rows; slot c of row r takes the row's value
    // chunk (c ^ p16_vswz(r)) of half dh.
    constexpr int VSL = RBV / 16;  // 16-byte slots per V row
#pragma unroll
    for (int i = 0; i < NICV; i++) {
        if constexpr (F) {
            const int r = (ws * NICV + i) * (1024 / RBFV) + lane / (RBFV / 16);
            vofs[i] = r * rbg + (lane % (RBFV / 16)) * 16 + dh * RBFV;
        } else {
            const int r = (ws * NICV + i) * (1024 / RBV) + lane / VSL;
            vofs[i] = r * rbg + ((((lane % VSL) ^ p16_vswz(r)) + dh * VSL) * 16);
        }
    }
    char *const ring = lds + ks * NSTG * STAGE;
    auto issue = [&](int j) {  // step j's tile of this stream into stage j % NSTG
        const int t = tbase + j;
        const bool live = j < nsteps && t < t1;
        __amdgpu_buffer_rsrc_t kr = krs, vr = vrs;
        int so;
        if (pgs.tab && live) page_tile<D, T::bytes>(pgs, kc, vc, kvh, rbg, kv_len, t * BN, kr, vr, so);
        else so = __builtin_amdgcn_readfirstlane(live ? t * BN * rbg : range);  // range 0 if paged
        char *st = ring + (j % NSTG) * STAGE;
#pragma unroll
        for (int i = 0; i < NIC; i++) dma16(kr, st + (ws * NIC + i) * 1024, kofs[i] + so, 0);
#pragma unroll
        for (int i = 0; i < NICV; i++)
            dma16(vr, st + DMAK + (ws * NICV + i) * 1024, vofs[i] + so, 0);
    };
    // bf16 V -> f16 in place, for the chunks this wave's DMA wrote; f32 K and
    // V -> bf16 hi/lo K and f16 V tiles (every wave reads its f32 chunks,
    // a barrier, then the converted writes: they land on other waves' rows).
    auto widen = [&](int j) {
        const int stg = j % NSTG;
        if constexpr (F) {
            const uint32_t base = lds_addr(ring + stg * STAGE);
            const uint32_t obase = SEP ? lds_addr(lds + NSTG * STAGE + (j & 1) * CONV) : base;
            u32x4 kx[NIC], vx[NICV];
#pragma unroll
            for (int i = 0; i < NIC; i++) kx[i] = lds_read_b128(base + (ws * NIC + i) * 1024 + lane * 16);
#pragma unroll
            for (int i = 0; i < NICV; i++)
                vx[i] = lds_read_b128(base + DMAK + (ws * NICV + i) * 1024 + lane * 16);
            lds_wait_any();
            if constexpr (!SEP) asm volatile("s_barrier" ::: "memory");
            constexpr int FSL = RBF / 16;  // f32 slots per row: four elements each
#pragma unroll
            for (int i = 0; i < NIC; i++) {
                tie(kx[i]);
                const int r = (ws * NIC + i) * (1024 / RBF) + lane / FSL, sl = lane % FSL;
                const u32x2 a = split2<BF16>(__uint_as_float(kx[i][0]), __uint_as_float(kx[i][1]));
                const u32x2 b = split2<BF16>(__uint_as_float(kx[i][2]), __uint_as_float(kx[i][3]));
                const uint32_t o = obase + r * RB + (((sl >> 1) ^ p16_kswz(r)) * 16) + (sl & 1) * 8;
                lds_write_b64(o, u32x2{a[0], b[0]});
                lds_write_b64(o + TILE, u32x2{a[1], b[1]});
            }
#pragma unroll
            for (int i = 0; i < NICV; i++) {
                tie(vx[i]);
                constexpr int FSLV = RBFV / 16;
                const int r = (ws * NICV + i) * (1024 / RBFV) + lane / FSLV, sl = lane % FSLV;
                const uint32_t o = obase + VOFF + r * RBV + (((sl >> 1) ^ p16_vswz(r)) * 16) + (sl & 1) * 8;
                lds_write_b64(o, u32x2{pack_f16x2(__uint_as_float(vx[i][0]), __uint_as_float(vx[i][1])),
                                       pack_f16x2(__uint_as_float(vx[i][2]), __uint_as_float(vx[i][3]))});
            }
        } else if constexpr (CVTV) {
            const uint32_t vb = lds_addr(ring + stg * STAGE + TILE + ws * NICV * 1024) + lane * 16;
            u32x4 w[NICV];
#pragma unroll
            for (int i = 0; i < NICV; i++) w[i] = lds_read_b128(vb + i * 1024);
            lds_wait_any();
#pragma unroll
            for (int i = 0; i < NICV; i++) {
                tie(w[i]);
                u32x4 o;
#pragma unroll
                for (int e = 0; e < 4; e++) o[e] = pack_f16x2(bf16_lo(w[i][e]), bf16_hi(w[i][e]));
                lds_write_b128(vb + i * 1024, o);
            }
        }
    };

    // ---- per-lane operand addresses within a stage ----
    // K (A operand of S^T): key row r16 (+16 for the second accumulator),
    // logical chunk 4s + g; chunks 16.. sit 256 bytes after chunks 0..15.
    uint32_t ka[4];
#pragma unroll
    for (int s = 0; s < 4; s++) ka[s] = r16 * RB + (((4 * s + g) ^ p16_kswz(r16)) * 16);
    // V^T (A operand of O^T): the 16 lanes of group g read rows 4g + r16/4
    // (+16), elements dt*16 + 4*(r16 % 4) .. +3; transposed, lane r16 gets
    // V[4g + 0..3][dt*16 + r16].  d tiles 8.. sit 256 bytes after 0..7 (DS 1).
    uint32_t va[8];
    {
        const int vr = 4 * g + (r16 >> 2);
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            const int ch = 2 * dt + ((r16 & 3) >> 1);
            va[dt] = VOFF + vr * RBV + ((ch ^ p16_vswz(vr)) * 16) + 8 * (r16 & 1);
        }
    }

    u32x4 qreg[NKS];  // Q^T operand: row r16, d = 32 s + 8 g .. +7
    u32x4 qlo[F ? NKS : 1];  // f32: the lo halves
    f32x4 oacc[NDT];
#pragma unroll
    for (int i = 0; i < NDT; i++) oacc[i] = f32x4{};
    float m_run = -INFINITY, l_part = 0.f;
    const int dlo = window > 0 ? -window : INT_MIN;
    const uint32_t ring0 = lds_addr(ring);

    auto compute = [&](int j) {
        const uint32_t sb = SEP ? lds_addr(lds + NSTG * STAGE + (j & 1) * CONV) : ring0 + (j % NSTG) * STAGE;
        // LDS operand reads in batches of eight, each batch issued as soon as
        // the one two ahead has been waited for, so the read queue stays
        // busy under the MFMAs and the softmax (reads retire in order; at
        // most 16 are outstanding):
        //   K 0-7, K 8-15 | QK on K 0-7, V d0-3 | QK on K 8-15, V d4-7 |
        //   softmax | PV d0-3, V d8-11 | PV d4-7, V d12-15 | PV d8-15.
        // S^T of the two 16-key halves alternate, so consecutive MFMAs are
        // independent.
        f32x4 sacc[2] = {f32x4{}, f32x4{}};
        // Per-step bases; the chunk-half, key-half and d-tile offsets ride in
        // the instructions' immediate fields.
        uint32_t kaddr[4], vaddr[8];
#pragma unroll
        for (int i = 0; i < 4; i++) kaddr[i] = sb + ka[i];
#pragma unroll
        for (int i = 0; i < 8; i++) vaddr[i] = sb + va[i];
        u32x4 kb[F ? 1 : 2 * NKS];
        if constexpr (!F)
            static_for<0, 2 * NKS>([&](auto ic) {
                constexpr int idx = decltype(ic)::value, s = idx >> 1, kt = idx & 1;
                kb[idx] = lds_read_b128_at<(s >> 2) * 256 + kt * 16 * RB>(kaddr[s & 3]);
            });
        u32x4 vb[NDT];
        auto rdv = [&](auto dtc) {
            constexpr int dt = decltype(dtc)::value;
            // (the reads of d tiles 8-15 are named only where NDT is 16)
            if constexpr (dt < NDT) {
                const u32x2 lo = lds_read_tr16_b64_at<(dt >> 3) * 256>(vaddr[dt & 7]);
                const u32x2 hi = lds_read_tr16_b64_at<(dt >> 3) * 256 + 16 * RBV>(vaddr[dt & 7]);
                vb[dt] = u32x4{lo[0], lo[1], hi[0], hi[1]};
            }
        };
        if constexpr (F) {
            // K hi and lo in batches of 8 operands each (head_dim 256: two
            // batches); the V^T reads go out with the last batch's MFMAs.
            static_assert(NDT == 8, "f32 mode: 8 value d tiles per workgroup");
            constexpr int CH = 2 * NKS > 8 ? 8 : 2 * NKS;
            static_for<0, 2 * NKS / CH>([&](auto hc) {
                constexpr int h = decltype(hc)::value;
                u32x4 kh[CH], kl[CH];
                static_for<0, CH>([&](auto ic) {
                    constexpr int idx = h * CH + decltype(ic)::value, s = idx >> 1, kt = idx & 1;
                    kh[idx - h * CH] = lds_read_b128_at<(s >> 2) * 256 + kt * 16 * RB>(kaddr[s & 3]);
                    kl[idx - h * CH] = lds_read_b128_at<TILE + (s >> 2) * 256 + kt * 16 * RB>(kaddr[s & 3]);
                });
                lds_wait_any();
                if constexpr (h == 2 * NKS / CH - 1) {
                    rdv(Int<0>{}); rdv(Int<1>{}); rdv(Int<2>{}); rdv(Int<3>{});
                    rdv(Int<4>{}); rdv(Int<5>{}); rdv(Int<6>{}); rdv(Int<7>{});
                }
                static_for<0, CH>([&](auto ic) {
                    constexpr int i = decltype(ic)::value, idx = h * CH + i, s = idx >> 1, kt = idx & 1;
                    tie(kh[i]);
                    tie(kl[i]);
                    sacc[kt] = mfma16<MT>(kh[i], qreg[s], sacc[kt]);
                    sacc[kt] = mfma16<MT>(kh[i], qlo[s], sacc[kt]);
                    sacc[kt] = mfma16<MT>(kl[i], qreg[s], sacc[kt]);
                });
            });
        } else {
        lds_wait_n<NKS>();  // the first half of the K reads
        static_for<0, 2 * NKS>([&](auto ic) {
            constexpr int idx = decltype(ic)::value, s = idx >> 1, kt = idx & 1;
            if constexpr (idx == NKS) asm volatile("s_waitcnt lgkmcnt(8)" ::: "memory");
            tie(kb[idx]);
            sacc[kt] = mfma16<T>(kb[idx], qreg[s], sacc[kt]);
            if constexpr (idx == 0) { rdv(Int<0>{}); rdv(Int<1>{}); rdv(Int<2>{}); rdv(Int<3>{}); }
            if constexpr (idx == NKS) { rdv(Int<4>{}); rdv(Int<5>{}); rdv(Int<6>{}); rdv(Int<7>{}); }
        });
        }
        // Mask where the tile reaches past the wave's first row or before the
        // window of its last (wave-uniform test): key - pos_row must lie in
        // (dlo, 0].  The scale is applied inside the exponent (qscale > 0, so
        // the row max of the raw scores scales with it).
        const int kbase = (tbase + j) * BN;
        float sv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) sv[i] = sacc[i >> 2][i & 3];
        const int p_first = start_pos + row0;
        if (kbase + BN - 1 > p_first || (window > 0 && kbase <= p_first + 15 - window)) {
            const int kd = kbase + 4 * g - pos_row;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int dk = kd + (i >> 2) * 16 + (i & 3);
                sv[i] = dk > 0 || dk <= dlo ? -INFINITY : sv[i];
            }
        }
        float mloc = __builtin_fmaxf(__builtin_fmaxf(__builtin_fmaxf(sv[0], sv[1]), sv[2]),
                                     __builtin_fmaxf(sv[3], sv[4]));
        mloc = __builtin_fmaxf(__builtin_fmaxf(mloc, sv[5]), __builtin_fmaxf(sv[6], sv[7]));
        mloc = rows_max(mloc) * qscale;  // lanes r16, +16, +32, +48 hold one row
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
        u32x4 ph;
        float ls[2] = {0.f, 0.f};
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[2 * jj], qscale, -mu));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[2 * jj + 1], qscale, -mu));
            ls[jj & 1] += p0 + p1;
            ph[jj] = pack_f16x2(p0, p1);
        }
        l_part += ls[0] + ls[1];
        // O^T += V^T.P^T.
        asm volatile("s_waitcnt lgkmcnt(8)" ::: "memory");
        static_for<0, NDT>([&](auto dc) {
            constexpr int dt = decltype(dc)::value;
            if constexpr (NDT == 16) {
                if constexpr (dt == 4 || dt == 8) asm volatile("s_waitcnt lgkmcnt(8)" ::: "memory");
                if constexpr (dt == 12) lds_wait_any();
            } else if constexpr (dt == 4) {
                lds_wait_any();
            }
            tie(vb[dt]);
            oacc[dt] = mfma16<F16>(vb[dt], ph, oacc[dt]);
            if constexpr (NDT == 16 && dt == 0) { rdv(Int<8>{}); rdv(Int<9>{}); rdv(Int<10>{}); rdv(Int<11>{}); }
            if constexpr (NDT == 16 && dt == 4) { rdv(Int<12>{}); rdv(Int<13>{}); rdv(Int<14>{}); rdv(Int<15>{}); }
        });
    };

    // ---- main loop: NSTG - 1 tiles in flight per stream ----
    // Step j: this wave's DMA of tile j has landed, its bf16 V is widened,
    // and the barrier makes every wave's part visible and frees the stage
    // read in step j-1, which then takes tile j + NSTG - 1.
    // Q goes out after the first tile, as untracked loads: the loop's first
    // wait (later tiles left in flight) covers it.
    issue(0);
    u32x4 qf[F ? 2 * NKS : 1];  // f32: raw q, split after it lands
    {
        const i32x4 qrs = raw_rsrc(q, (int)((int64_t)S * q_dim * T::bytes));
        const int qo = qrow < S ? (int)(((int64_t)qrow * q_dim + (int64_t)head * D + g * 8) * T::bytes)
                                : 0x7ffffff0;  // past the range: zeros
#pragma unroll
        for (int s = 0; s < NKS; s++) {
            if constexpr (F) {
                qf[2 * s] = buffer_load_b128_untracked(qrs, qo + s * 128);
                qf[2 * s + 1] = buffer_load_b128_untracked(qrs, qo + s * 128 + 16);
            } else {
                qreg[s] = buffer_load_b128_untracked(qrs, qo + s * 64);
            }
        }
    }
#pragma unroll
    for (int j = 1; j < NSTG - 1; j++) issue(j);
    if constexpr (F) {  // q landed with tile 0 (issued before tiles 1..): split it
        __builtin_amdgcn_s_waitcnt(vm_wait((NSTG - 2) * (NIC + NICV)));
#pragma unroll
        for (int s = 0; s < NKS; s++) {
            tie(qf[2 * s]);
            tie(qf[2 * s + 1]);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const u32x4 &src = e < 2 ? qf[2 * s] : qf[2 * s + 1];
                const u32x2 hl = split2<BF16>(__uint_as_float(src[(2 * e) & 3]),
                                              __uint_as_float(src[(2 * e + 1) & 3]));
                qreg[s][e] = hl[0];
                qlo[s][e] = hl[1];
            }
        }
    }
    for (int j = 0; j < nsteps; j++) {
        __builtin_amdgcn_s_waitcnt(vm_wait((NSTG - 2) * (NIC + NICV)));
#pragma unroll
        for (int s = 0; s < NKS; s++) {
            tie(qreg[s]);
            if constexpr (F) tie(qlo[s]);
        }
        widen(j);
        lds_wait_any();
        asm volatile("s_barrier" ::: "memory");
        issue(j + NSTG - 1);
        compute(j);
    }
    __builtin_amdgcn_s_waitcnt(vm_wait(0));

    // ---- result: lane (row r16, group g) holds d = dt*16 + 4g .. +3 ----
    float l_tot = rows_sum(l_part);
    if constexpr (KS == 2) {
        // Merge the two streams' partials of each row through the idle ring.
        asm volatile("s_barrier" ::: "memory");
        const uint32_t po = lds_addr(lds) + (ws * NDT * 64 + lane) * 16;
        const uint32_t pml = lds_addr(lds) + NWS * NDT * 64 * 16 + (ws * 64 + lane) * 8;
        if (ks == 1) {
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
                lds_write_b128(po + dt * 64 * 16, __builtin_bit_cast(u32x4, oacc[dt]));
            lds_write_b64(pml, u32x2{__float_as_uint(m_run), __float_as_uint(l_tot)});
        }
        lds_wait_any();
        asm volatile("s_barrier" ::: "memory");
        if (ks == 1) return;
        u32x4 o1[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) o1[dt] = lds_read_b128(po + dt * 64 * 16);
        u32x2 ml;
        asm volatile("ds_read_b64 %0, %1" : "=v"(ml) : "v"(pml));
        lds_wait_any();
        const float m1 = __uint_as_float(ml[0]), l1 = __uint_as_float(ml[1]);
        const float M = fmaxf(m_run, m1);
        const float mu = M == -INFINITY ? 0.f : M;
        const float a0 = __builtin_amdgcn_exp2f(m_run - mu), a1 = __builtin_amdgcn_exp2f(m1 - mu);
        l_tot = l_tot * a0 + l1 * a1;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            tie(o1[dt]);
            oacc[dt] = oacc[dt] * a0 + __builtin_bit_cast(f32x4, o1[dt]) * a1;
        }
    }
    if (qrow < S) {
        const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
        float *op = out + (int64_t)qrow * q_dim + (int64_t)head * D + dh * (D / DS) + 4 * g;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
            __builtin_nontemporal_store(oacc[dt] * inv, (f32x4 *)(op + dt * 16));
    }
}

static int p16_hw(int kv_mul, int nws) {
    int hw = 1;
    while (hw < nws && hw < 4 && kv_mul % (hw * 2) == 0) hw *= 2;
    return hw;
}

// Key streams and value-column split for a prompt.  Two key streams when
// whole units would leave CUs idle, or fill the chip exactly with causal
// (window-free) chains, whose longest unit then sets the time; the value
// split on top when the workgroups still fit one per CU.  Measured at 8/4
// heads, f16 (us; KS/DS): S=1024 KS2/DS2 23.9, KS2/DS1 27.1, KS1/DS2 34.5;
// S=2048 KS2/DS1 51.5, KS2/DS2 53.2; S=4096 causal KS2/DS1 122-130, KS1/DS1
// 134-137; S=4096 window 1024 KS1/DS1 57.9, KS2/DS1 76.6; 16/8 heads at
// S=1024 KS2/DS1 31.2, KS2/DS2 34.3.
static void prefill16_plan(int S, int start_pos, int window, int n_head, int kv_mul, int &ks,
                           int &ds) {
    static const int eks = env_override("ULLM_HIP_P16_KS");  // tuning overrides
    static const int eds = env_override("ULLM_HIP_P16_DS");
    const int hw = p16_hw(kv_mul, 8);
    const int64_t grid1 = (int64_t)((S + 128 / hw - 1) / (128 / hw)) * (n_head / hw);
    const bool binding = window > 0 && window < start_pos + S;
    ks = grid1 < 256 || (grid1 == 256 && !binding) ? 2 : 1;
    if (eks == 1 || eks == 2) ks = eks;
    const int hw2 = p16_hw(kv_mul, 8 / ks), ur = 16 * (8 / ks) / hw2;
    const int64_t grid = (int64_t)((S + ur - 1) / ur) * (n_head / hw2);
    ds = ks == 2 && grid * 2 <= 256 ? 2 : 1;
    if (eds == 1 || eds == 2) ds = eds;
}

int launch_prefill16(int dtype, const void *q, const void *kc, const void *vc, int64_t kvs, int S,
                     int start_pos, int window, int n_head, int kv_mul, float qs, float *out,
                     hipStream_t st, KvPages pgs) {
    int KS, DS;
    prefill16_plan(S, start_pos, window, n_head, kv_mul, KS, DS);
    const int hw = p16_hw(kv_mul, 8 / KS), UR = 16 * (8 / KS) / hw;
    const int n_units = (S + UR - 1) / UR, n_hg = n_head / hw;
    const dim3 grid((unsigned)(n_units * n_hg * DS));
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(512), 0, st, (const uint16_t *)q, (const char *)kc,
                           (const char *)vc, kvs, S, start_pos, window, n_head, kv_mul, hw, n_hg,
                           n_units, qs, out, pgs);
    };
    auto pick = [&](auto t) {
        using T = decltype(t);
        if (KS == 2) {
            if (DS == 2) go(prefill16_kernel<T, 2, 2>);
            else go(prefill16_kernel<T, 2, 1>);
        } else {
            if (DS == 2) go(prefill16_kernel<T, 1, 2>);
            else go(prefill16_kernel<T, 1, 1>);
        }
    };
    if (dtype == ULLM_DT_F32) {  // f32 cache: one key stream, value columns split
        const int hw1 = p16_hw(kv_mul, 8), UR1 = 16 * 8 / hw1;
        const int nu1 = (S + UR1 - 1) / UR1, nhg1 = n_head / hw1;
        hipLaunchKernelGGL((prefill16_kernel<F32, 1, 2>), dim3((unsigned)(nu1 * nhg1 * 2)), dim3(512), 0, st,
                           (const uint16_t *)q, (const char *)kc, (const char *)vc, kvs, S, start_pos,
                           window, n_head, kv_mul, hw1, nhg1, nu1, qs, out, pgs);
    } else if (dtype == ULLM_DT_BF16) pick(BF16{});
    else pick(F16{});
    return check_hip(hipGetLastError(), "prefill (16-row waves) launch");
}

// head_dim 128 on prefill16_kernel (short prompts; no value split), bf16,
// f16 or f32 cache, contiguous or paged.
int launch_prefill16_128(int dtype, const void *q, const void *kc, const void *vc, int64_t kvs,
                         int S, int start_pos, int window, int n_head, int kv_mul, float qs,
                         float *out, hipStream_t st, KvPages pgs) {
    int KS, DS;  // head_dim 128: no value split (V rows of 256 bytes)
    prefill16_plan(S, start_pos, window, n_head, kv_mul, KS, DS);
    const int hw = p16_hw(kv_mul, 8 / KS), UR = 16 * (8 / KS) / hw;
    const int n_units = (S + UR - 1) / UR, n_hg = n_head / hw;
    const dim3 grid((unsigned)(n_units * n_hg));
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(512), 0, st, (const uint16_t *)q, (const char *)kc,
                           (const char *)vc, kvs, S, start_pos, window, n_head, kv_mul, hw, n_hg,
                           n_units, qs, out, pgs);
    };
    auto pick = [&](auto t) {
        using T = decltype(t);
        if (KS == 2) go(prefill16_kernel<T, 2, 1, 128, 1>);
        else go(prefill16_kernel<T, 1, 1, 128, 1>);
    };
    if (dtype == ULLM_DT_BF16) pick(BF16{});
    else if (dtype == ULLM_DT_F32) pick(F32{});
    else pick(F16{});
    return check_hip(hipGetLastError(), "prefill (16-row waves, head_dim 128) launch");
}

}  // namespace ullm
