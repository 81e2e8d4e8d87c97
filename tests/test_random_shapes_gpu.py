"""Seeded random shapes for decode and prefill against the CPU oracle.

Each case draws head counts, GQA ratio, head_dim, dtype, lengths, start
position, window and cache padding from a fixed seed, so the sweep covers
combinations the hand-picked cases miss (odd GQA ratios at head_dim 128,
windows shorter than a tile with a start position, ragged batches with
padded rows) and every failure names its case and is reproducible.
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as ora
from tests.helpers import assert_close
from ullm_amd import attention as A
from ullm_amd import synth

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
GQA = [(4, 4), (8, 2), (6, 2), (6, 1), (12, 2), (15, 5), (16, 4), (24, 8), (20, 4), (14, 7)]


def _shape(rng):
    H, Hk = GQA[rng.integers(len(GQA))]
    D = int(rng.choice([64, 128, 256]))
    return int(H), int(Hk), D


def _decode_case(seed):
    rng = np.random.default_rng(1000 + seed)
    H, Hk, D = _shape(rng)
    dtype = str(rng.choice(["f32", "f16", "bf16"]))
    B = int(rng.integers(1, 5))
    lens = [int(x) for x in rng.integers(1, 6000, size=B)]
    window = int(rng.choice([0, 0, 1, 37, 512, 4096]))
    pad = int(rng.choice([0, 8, 64]))
    return dict(H=H, Hk=Hk, D=D, dtype=dtype, lens=lens, window=window, pad=pad)


def _prefill_case(seed):
    rng = np.random.default_rng(2000 + seed)
    H, Hk, D = _shape(rng)
    dtype = str(rng.choice(["f16", "bf16"]))
    S = int(rng.integers(1, 1500))
    start_pos = int(rng.choice([0, 0, 1, 77, 640]))
    window = int(rng.choice([0, 0, 0, 1, 100, 700]))
    return dict(H=H, Hk=Hk, D=D, dtype=dtype, S=S, start_pos=start_pos, window=window)


@pytest.mark.parametrize("seed", range(16))
def test_decode_random(dev, seed):
    c = _decode_case(seed)
    print(f"[decode-rand] seed={seed} {c}", flush=True)
    H, Hk, D, lens = c["H"], c["Hk"], c["D"], c["lens"]
    dt = DT[c["dtype"]]
    B, L = len(lens), max(lens)
    kv_stride = Hk * D + c["pad"]
    q = synth.randn(seed, 1, (B, H, D)).to(dev)
    k = synth.randn(seed, 2, (B, L, kv_stride), dt).to(dev)
    v = synth.randn(seed, 3, (B, L, kv_stride), dt).to(dev)
    lens_t = torch.tensor(lens, dtype=torch.int32, device=dev)
    scale = 1.0 / math.sqrt(D)
    out = A.attn_decode(q, k, v, lens_t, L, Hk, window=c["window"], scale=scale,
                        kv_stride=kv_stride, seq_stride=L * kv_stride)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    qn = q.cpu().numpy()
    for b in range(B):
        ref = ora.attn_decode(qn[b].reshape(-1).copy(), k[b].float().cpu().numpy(),
                              v[b].float().cpu().numpy(), lens[b] - 1, H, Hk, D, scale,
                              window=c["window"], kv_stride=kv_stride)
        assert_close(out[b].reshape(-1), ref, what=f"seed={seed} b={b}")


@pytest.mark.parametrize("seed", range(16))
def test_prefill_random(dev, seed):
    c = _prefill_case(seed)
    print(f"[prefill-rand] seed={seed} {c}", flush=True)
    H, Hk, D, S, sp = c["H"], c["Hk"], c["D"], c["S"], c["start_pos"]
    dt = DT[c["dtype"]]
    q = synth.randn(seed, 1, (S, H * D), dt).to(dev)
    k = synth.randn(seed, 2, (sp + S, Hk * D), dt).to(dev)
    v = synth.randn(seed, 3, (sp + S, Hk * D), dt).to(dev)
    scale = 1.0 / math.sqrt(D)
    out = A.attn_prefill(q, k, v, H, Hk, D, start_pos=sp, window=c["window"], scale=scale)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    rng = np.random.default_rng(seed)
    rows = sorted({0, S - 1, min(31, S - 1), min(32, S - 1)}
                  | set(int(x) for x in rng.integers(0, S, size=12)))
    ref = ora.attn_prefill(q.float().cpu().numpy(), k.float().cpu().numpy(),
                           v.float().cpu().numpy(), S, sp, H, Hk, D, scale,
                           window=c["window"], rows=rows)
    assert_close(out[rows], ref[rows], what=f"seed={seed} rows {rows[:6]}..")
