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

DT = {"f16": torch.float16, "bf16": torch.bfloat16}


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
    if window == 0:
        # same blocks and splits as the contiguous path: identical bits
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
