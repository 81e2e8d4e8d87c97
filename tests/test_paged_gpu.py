"""Paged KV-cache decode (ullm_hip_attn_decode_paged) on the GPU.

The paged cache is the reference's token-major cache (crates/ullm-model/src/
lib.rs:184-185) cut into fixed-size pages of a shared pool and addressed
through a block table; the attention itself is lib.rs:911-938 / :1180-1208.
Parity is pinned two ways: against the oracle on the gathered contiguous
cache, and -- without a binding window, where both paths cut the keys into
the same 32-key blocks and splits -- bit-for-bit against
ullm_hip_attn_decode on the contiguous cache holding the same values.
Unused slots and pages are filled with NaN, and table entries past a
sequence's pages with -1 or out-of-range indices, to show they are never
read into the result."""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as ora
from tests.helpers import assert_close
from ullm_amd import attention as A
from ullm_amd import synth
from ullm_amd import _lib as L

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def build(dev, lens, Hk, D, dt, page, pad=0, spare=3, seed=1):
    """Contiguous [B, max_len, kv_stride] caches and the same data paged
    over a shuffled pool; returns (kc, vc, kp, vp, table)."""
    B, L_ = len(lens), max(lens)
    kvs = Hk * D + pad
    kc = synth.randn(seed, 2, (B, L_, kvs), DT[dt]).to(dev)
    vc = synth.randn(seed, 3, (B, L_, kvs), DT[dt]).to(dev)
    need = [(n + page - 1) // page for n in lens]
    n_pages = sum(need) + spare
    rng = np.random.default_rng(seed)
    perm = rng.permutation(n_pages)
    kp = torch.full((n_pages, page, kvs), float("nan"), dtype=DT[dt], device=dev)
    vp = torch.full_like(kp, float("nan"))
    stride = (L_ + page - 1) // page + 1
    table = np.full((B, stride), -1, np.int32)
    table[:, -1] = n_pages + 5  # out of range: never addressed
    nxt = 0
    for b, n in enumerate(lens):
        for pg in range(need[b]):
            phys = int(perm[nxt]); nxt += 1
            table[b, pg] = phys
            rows = min(page, n - pg * page)
            kp[phys, :rows] = kc[b, pg * page:pg * page + rows]
            vp[phys, :rows] = vc[b, pg * page:pg * page + rows]
    return kc, vc, kp, vp, torch.from_numpy(table).to(dev)


def oracle_ref(q, kc, vc, lens, H, Hk, D, window, kvs):
    qn = q.cpu().numpy()
    out = []
    for b, n in enumerate(lens):
        out.append(ora.attn_decode(qn[b].reshape(-1).copy(), kc[b, :n].float().cpu().numpy(),
                                   vc[b, :n].float().cpu().numpy(), n - 1, H, Hk, D,
                                   1.0 / math.sqrt(D), window=window, kv_stride=kvs))
    return out


CASES = [
    # (lens, H, Hk, D, dtype, page, window, pad)
    ([1, 31, 32, 33, 100], 8, 2, 128, "f16", 32, 0, 0),
    ([4096, 700, 5000, 1], 12, 2, 128, "bf16", 64, 0, 8),
    ([9000, 3000], 32, 4, 128, "bf16", 256, 0, 0),
    ([2500, 65, 1200], 8, 8, 64, "f16", 32, 0, 0),
    ([777, 20000], 16, 4, 64, "bf16", 128, 0, 64),
    ([5000, 3000, 600], 12, 2, 128, "f16", 64, 1024, 0),
    ([5000, 4100, 40], 8, 4, 64, "bf16", 32, 37, 0),
    ([33000, 12000], 32, 4, 128, "bf16", 512, 4096, 0),
    ([8192, 3000, 1], 8, 4, 256, "f16", 64, 0, 0),       # head_dim 256 (register-staged kernel)
    ([512, 40, 1000], 32, 8, 64, "f32", 32, 0, 0),       # the reference's f32 cache (MFMA, f32 tiles)
    ([3000, 700], 12, 2, 128, "f32", 64, 333, 4),        # f32 with a binding window
    ([33000, 12000], 32, 4, 128, "f32", 512, 4096, 0),   # f32, long context, binding window
    ([9000, 20000, 3000, 1], 32, 4, 128, "f32", 256, 0, 0),  # f32, ragged batch
    ([6000, 800], 16, 16, 64, "f32", 64, 0, 8),          # f32, head_dim 64, padded rows
    ([3000, 1500], 8, 4, 256, "f32", 64, 0, 0),          # f32 at head_dim 256 (VALU kernel)
    ([9000, 2000], 16, 8, 256, "bf16", 256, 1024, 16),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_paged_vs_oracle(dev, case):
    lens, H, Hk, D, dt, page, window, pad = CASES[case]
    print(f"[paged] lens={lens} H{H} Hk{Hk} D{D} {dt} page{page} win{window} pad{pad}", flush=True)
    B, L_ = len(lens), max(lens)
    kc, vc, kp, vp, table = build(dev, lens, Hk, D, dt, page, pad, seed=case + 1)
    q = synth.randn(case, 1, (B, H, D)).to(dev)
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    out = A.attn_decode_paged(q, kp, vp, table, sl, L_, Hk, window=window)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    ref = oracle_ref(q, kc, vc, lens, H, Hk, D, window, Hk * D + pad)
    for b in range(B):
        assert_close(o[b].reshape(-1), ref[b], what=f"case {case} b={b}")
    if window == 0 and dt != "f32":
        # same blocks and splits as the contiguous path: identical bits (an
        # f32 cache's contiguous short splits run on the block kernel, its
        # pages on decode_dma_kernel: both checked against the oracle)
        ws = A.new_decode_workspace(B, H, Hk, D, L_, 0, dev)
        oc = A.attn_decode(q, kc, vc, sl, L_, Hk, kv_stride=Hk * D + pad, seq_stride=L_ * (Hk * D + pad),
                           workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(out, oc), f"case {case}: paged != contiguous bits"


def test_paged_graph_replay(dev):
    """A captured paged decode replayed with new lengths and tables between
    replays (the serving loop's pattern) matches eager calls every time."""
    H, Hk, D, page = 16, 4, 128, 64
    lens0 = [3000, 1500, 64]
    L_ = 4096
    kc, vc, kp, vp, table = build(dev, [L_] * 3, Hk, D, "bf16", page, seed=7)
    q = synth.randn(7, 1, (3, H, D)).to(dev)
    sl = torch.tensor(lens0, dtype=torch.int32, device=dev)
    out = torch.empty(3, H, D, device=dev)
    n = int(L.lib().ullm_hip_paged_decode_workspace_bytes(3, H, Hk, D, L_, 0))
    ws = torch.zeros(max(n, 256), dtype=torch.uint8, device=dev)
    A.attn_decode_paged(q, kp, vp, table, sl, L_, Hk, out=out, workspace=ws)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            A.attn_decode_paged(q, kp, vp, table, sl, L_, Hk, out=out, workspace=ws, stream=st)
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    for it, lens in enumerate(([3000, 1500, 64], [4096, 1, 2049], [100, 4000, 3333])):
        sl.copy_(torch.tensor(lens, dtype=torch.int32))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        want = A.attn_decode_paged(q, kp, vp, table, sl, L_, Hk)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {it}"


@pytest.mark.parametrize("D,kvdt,neox", [(128, "bf16", True), (64, "f16", False), (256, "f16", True)])
def test_paged_append(dev, D, kvdt, neox):
    """ullm_hip_qkv_append_paged: each row's K/V land in its own page slot
    with RoPE at its own position; matches the oracle's append (lib.rs:
    1021-1058) row by row within one storage ulp; rows with an invalid
    position or page write nothing."""
    print(f"[paged-append] D{D} kv={kvdt} neox={neox}", flush=True)
    H, Hk, page, theta = 8, 2, 64, 1e6
    pos = [0, 63, 64, 1500, 2999, -1, 700]   # row 5: invalid position
    rows = len(pos)
    n_ctx = 3000
    stride = n_ctx // page + 1
    rng = np.random.default_rng(D)
    n_pages = 40
    table = np.full((rows, stride), -1, np.int32)
    used = rng.permutation(n_pages)
    for r, p_ in enumerate(pos):
        if p_ >= 0:
            table[r, p_ // page] = used[r]
    table[6, 700 // page] = n_pages + 3          # row 6: page outside the pool
    q = synth.randn(D, 1, (rows, H * D))
    k = synth.randn(D, 2, (rows, Hk * D))
    v = synth.randn(D, 3, (rows, Hk * D))
    qn = synth.randn(D, 4, (D,)) * 0.2 + 1.0
    kn = synth.randn(D, 5, (D,)) * 0.2 + 1.0
    cs = A.rope_table(n_ctx, D, theta, device=dev)
    kp = torch.full((n_pages, page, Hk * D), float("nan"), dtype=DT[kvdt], device=dev)
    vp = torch.full_like(kp, float("nan"))
    qo = torch.full((rows, H * D), 7.0, device=dev)
    A.qkv_append_paged(q.to(dev), k.to(dev), v.to(dev), kp, vp, cs,
                       torch.tensor(pos, dtype=torch.int32, device=dev),
                       torch.from_numpy(table).to(dev), n_head=H, n_kv_head=Hk, head_dim=D,
                       neox=neox, q_norm=qn.to(dev), k_norm=kn.to(dev), eps=1e-6, q_out=qo)
    torch.cuda.synchronize()
    kp, vp, qo = kp.float().cpu().numpy(), vp.float().cpu().numpy(), qo.cpu().numpy()
    tol = {"f16": 2e-3, "bf16": 1.6e-2}[kvdt]
    written = set()
    for r, p_ in enumerate(pos):
        if r in (5, 6):
            assert np.all(qo[r] == 7.0), f"row {r}: skipped row wrote q"
            continue
        okc = np.zeros((p_ + 1, Hk * D), np.float32)
        ovc = np.zeros_like(okc)
        oq = ora.qkv_append(q[r:r + 1].numpy().copy(), k[r:r + 1].numpy().copy(),
                            v[r:r + 1].numpy().copy(), p_, H, Hk, D, D, theta, neox, okc, ovc,
                            q_norm=qn.numpy(), k_norm=kn.numpy(), eps=1e-6)
        assert np.abs(qo[r] - oq[0]).max() <= 2e-5 * max(1.0, np.abs(oq).max()), f"row {r} q"
        phys, slot = table[r, p_ // page], p_ % page
        written.add((phys, slot))
        for name, got, ref in (("k", kp[phys, slot], okc[p_]), ("v", vp[phys, slot], ovc[p_])):
            rr = torch.from_numpy(ref).to(DT[kvdt]).float().numpy()
            rel = np.abs(got - rr) / np.maximum(np.abs(rr), 1.0)
            assert rel.max() <= tol, f"row {r} {name}: max rel {rel.max():.3e}"
    # every other slot of the pool is untouched
    for p_i in range(n_pages):
        for sl in range(page):
            if (p_i, sl) not in written:
                assert np.all(np.isnan(kp[p_i, sl])) and np.all(np.isnan(vp[p_i, sl]))


def test_paged_serving_loop(dev):
    """A batched decode loop over the paged cache: each step appends one
    token per sequence (paged append) and attends (paged decode); every
    step's output matches the oracle on the rows the cache then holds."""
    H, Hk, D, page, n_ctx, theta = 16, 4, 128, 32, 512, 1e6
    lens = [5, 33, 200]
    B = len(lens)
    stride = n_ctx // page
    n_pages = B * stride
    perm = np.random.default_rng(3).permutation(n_pages)
    table = torch.from_numpy(perm.reshape(B, stride).astype(np.int32)).to(dev)
    kp = torch.full((n_pages, page, Hk * D), float("nan"), dtype=torch.float16, device=dev)
    vp = torch.full_like(kp, float("nan"))
    cs = A.rope_table(n_ctx, D, theta, device=dev)
    kn = (synth.randn(3, 9, (D,)) * 0.2 + 1.0).to(dev)
    # the prompts: positions 0..len-1 of each sequence, appended row by row
    for b, n in enumerate(lens):
        tb = table[b:b + 1].expand(n, stride).contiguous()
        A.qkv_append_paged(synth.randn(3, 10 + b, (n, H * D)).to(dev),
                           synth.randn(3, 20 + b, (n, Hk * D)).to(dev),
                           synth.randn(3, 30 + b, (n, Hk * D)).to(dev), kp, vp, cs,
                           torch.arange(n, dtype=torch.int32, device=dev), tb, n_head=H,
                           n_kv_head=Hk, head_dim=D, k_norm=kn)
    for step in range(4):
        pos = torch.tensor(lens, dtype=torch.int32, device=dev)
        qo = A.qkv_append_paged(synth.randn(4, 40 + step, (B, H * D)).to(dev),
                                synth.randn(4, 50 + step, (B, Hk * D)).to(dev),
                                synth.randn(4, 60 + step, (B, Hk * D)).to(dev), kp, vp, cs, pos,
                                table, n_head=H, n_kv_head=Hk, head_dim=D, k_norm=kn)
        lens = [n + 1 for n in lens]
        out = A.attn_decode_paged(qo.view(B, H, D), kp, vp, table,
                                  torch.tensor(lens, dtype=torch.int32, device=dev), n_ctx, Hk)
        torch.cuda.synchronize()
        kpc, vpc, tab = kp.float().cpu(), vp.float().cpu(), table.cpu().numpy()
        for b, n in enumerate(lens):
            rows = np.array([tab[b, t // page] * page + t % page for t in range(n)])
            kr = kpc.view(-1, Hk * D)[rows].numpy()
            vr = vpc.view(-1, Hk * D)[rows].numpy()
            assert np.all(np.isfinite(kr)) and np.all(np.isfinite(vr)), f"step {step} b={b}"
            ref = ora.attn_decode(qo[b].cpu().numpy().copy(), kr, vr, n - 1, H, Hk, D,
                                  1.0 / math.sqrt(D))
            assert_close(out[b].cpu().numpy().reshape(-1), ref, what=f"step {step} b={b}")


PREFILL_CASES = [
    # (S, start_pos, H, Hk, D, dtype, page, window)
    (300, 0, 8, 2, 128, "bf16", 64, 0),
    (200, 700, 32, 8, 128, "bf16", 128, 0),     # chunked prefill over earlier pages
    (150, 1000, 12, 2, 64, "f16", 64, 300),     # binding window (prefill2 path)
    (1, 63, 8, 8, 128, "f16", 64, 0),           # one row at a page edge
    (2048, 0, 32, 8, 128, "bf16", 256, 0),      # cfg3 shape
    (1024, 0, 8, 4, 256, "f16", 64, 0),         # head_dim 256 (split-K kernel), cfg4 shape
    (300, 900, 8, 4, 256, "bf16", 128, 500),    # head_dim 256, chunked, binding window
    (300, 0, 8, 2, 128, "f32", 64, 0),          # f32 pages (prefill16's f32 mode), two key streams
    (2048, 0, 32, 8, 128, "f32", 256, 0),       # f32, cfg3 shape, one key stream
    (200, 700, 12, 4, 128, "f32", 128, 250),    # f32, chunked, binding window, 1 head per workgroup
    (500, 300, 8, 4, 256, "f32", 64, 0),        # f32 at head_dim 256, chunked
    (700, 0, 32, 8, 64, "f32", 64, 0),          # f32 at head_dim 64 (prefill_f32_kernel)
    (300, 500, 16, 4, 64, "f32", 128, 200),     # f32 at head_dim 64, chunked, binding window
    (97, 31, 6, 2, 64, "f32", 64, 0),           # f32 at head_dim 64, ragged tail, 3:1 GQA
]


@pytest.mark.parametrize("case", range(len(PREFILL_CASES)))
def test_paged_prefill(dev, case):
    """ullm_hip_attn_prefill_paged equals ullm_hip_attn_prefill on the
    gathered cache bit for bit (same kernels and tiles; rows past the length
    read as zeros either way), and the oracle on sampled rows; unused slots
    hold NaN."""
    S, sp, H, Hk, D, dt, page, window = PREFILL_CASES[case]
    print(f"[paged-prefill] S{S} sp{sp} H{H} Hk{Hk} D{D} {dt} page{page} win{window}", flush=True)
    n = sp + S
    kvs = Hk * D
    kc = synth.randn(case, 2, (n, kvs), DT[dt]).to(dev)
    vc = synth.randn(case, 3, (n, kvs), DT[dt]).to(dev)
    q = synth.randn(case, 1, (S, H * D), DT[dt]).to(dev)
    n_used = (n + page - 1) // page
    n_pages = n_used + 3
    perm = np.random.default_rng(case).permutation(n_pages)[:n_used]
    kp = torch.full((n_pages, page, kvs), float("nan"), dtype=DT[dt], device=dev)
    vp = torch.full_like(kp, float("nan"))
    for pg in range(n_used):
        r = min(page, n - pg * page)
        kp[perm[pg], :r] = kc[pg * page:pg * page + r]
        vp[perm[pg], :r] = vc[pg * page:pg * page + r]
    table = torch.tensor(list(perm) + [-1], dtype=torch.int32, device=dev)
    out = A.attn_prefill_paged(q, kp, vp, table, H, Hk, D, start_pos=sp, window=window)
    ref_c = A.attn_prefill(q, kc, vc, H, Hk, D, start_pos=sp, window=window)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_c), f"case {case}: paged != contiguous bits"
    rows = sorted({0, S - 1, S // 2, min(31, S - 1), min(64, S - 1)})
    ref = ora.attn_prefill(q.float().cpu().numpy(), kc.float().cpu().numpy(),
                           vc.float().cpu().numpy(), S, sp, H, Hk, D, 1.0 / math.sqrt(D),
                           window=window, rows=rows)
    assert_close(out.cpu().numpy()[rows], ref[rows], what=f"case {case}")
