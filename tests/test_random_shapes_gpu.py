"""Seeded random shapes for decode, prefill and the fused append against the
CPU oracle.

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


def _prefill_case(seed, dtypes=("f16", "bf16"), base=2000):
    rng = np.random.default_rng(base + seed)
    H, Hk, D = _shape(rng)
    dtype = str(rng.choice(list(dtypes)))
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
    check_prefill(dev, seed, _prefill_case(seed))


@pytest.mark.parametrize("seed", range(10))
def test_prefill_random_f32_cache(dev, seed):
    """The reference's own f32 cache at every head_dim (64 on
    prefill_f32_kernel, 128 and 256 on prefill16_kernel's f32 mode)."""
    check_prefill(dev, seed, _prefill_case(seed, ("f32",), base=2500))


def check_prefill(dev, seed, c):
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


def _matmul_case(seed):
    rng = np.random.default_rng(3000 + seed)
    return dict(n=int(rng.integers(1, 1500)), i=8 * int(rng.integers(1, 400)),
                o=4 * int(rng.integers(1, 800)), xs=float(rng.choice([1.0, 1e-3, 1e3])))


@pytest.mark.parametrize("seed", range(8))
def test_matmul_random(dev, seed):
    """Projection GEMM at random shapes (tails in every dimension, both tile
    variants) against an f64 product of the same rounded inputs, with the
    bound of tests/test_matmul_gpu.py."""
    c = _matmul_case(seed)
    print(f"[matmul-rand] seed={seed} {c}", flush=True)
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(c["n"], c["i"], device=dev, generator=g) * c["xs"]
    w = (torch.randn(c["o"], c["i"], device=dev, generator=g) * 0.05).to(torch.bfloat16)
    y = A.matmul(w, x)
    torch.cuda.synchronize()
    x64, w64 = x.cpu().double().numpy(), w.cpu().double().numpy()
    ref = x64 @ w64.T
    bound = (2.0 ** -16 + c["i"] * 2.0 ** -24) * (np.abs(x64) @ np.abs(w64).T) + 1e-30
    worst = float(np.max(np.abs(y.cpu().double().numpy() - ref) / bound))
    assert worst <= 1.0, f"seed={seed}: error {worst:.3f} x the bound"


def _paged_case(seed):
    rng = np.random.default_rng(4000 + seed)
    H, Hk, D = _shape(rng)
    B = int(rng.integers(1, 6))
    return dict(H=H, Hk=Hk, D=D, dtype=str(rng.choice(["f16", "bf16"])), B=B,
                lens=[int(x) for x in rng.integers(1, 9000, size=B)],
                page=int(rng.choice([32, 64, 128, 256])),
                window=int(rng.choice([0, 0, 1, 100, 2000])))


@pytest.mark.parametrize("seed", range(8))
def test_paged_decode_random(dev, seed):
    """Paged decode at random shapes: pages shuffled over the pool, unused
    slots NaN, against the oracle on each sequence's gathered rows."""
    c = _paged_case(seed)
    print(f"[paged-rand] seed={seed} {c}", flush=True)
    H, Hk, D, P, lens = c["H"], c["Hk"], c["D"], c["page"], c["lens"]
    dt = DT[c["dtype"]]
    B, L_ = len(lens), max(lens)
    kvs = Hk * D
    need = [(n + P - 1) // P for n in lens]
    n_pages = sum(need) + 2
    perm = np.random.default_rng(seed).permutation(n_pages)
    kp = torch.full((n_pages, P, kvs), float("nan"), dtype=dt)
    vp = torch.full_like(kp, float("nan"))
    stride = (L_ + P - 1) // P
    table = np.full((B, stride), -1, np.int32)
    seqs = []
    i = 0
    for b, n in enumerate(lens):
        k = synth.randn(seed, 10 + b, (n, kvs), dt)
        v = synth.randn(seed, 20 + b, (n, kvs), dt)
        seqs.append((k, v))
        for pg in range(need[b]):
            phys = int(perm[i]); i += 1
            table[b, pg] = phys
            r = min(P, n - pg * P)
            kp[phys, :r] = k[pg * P:pg * P + r]
            vp[phys, :r] = v[pg * P:pg * P + r]
    q = synth.randn(seed, 1, (B, H, D)).to(dev)
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    out = A.attn_decode_paged(q, kp.to(dev), vp.to(dev), torch.from_numpy(table).to(dev), sl, L_,
                              Hk, window=c["window"])
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    qn = q.cpu().numpy()
    for b, n in enumerate(lens):
        k, v = seqs[b]
        ref = ora.attn_decode(qn[b].reshape(-1).copy(), k.float().numpy(), v.float().numpy(), n - 1,
                              H, Hk, D, 1.0 / math.sqrt(D), window=c["window"])
        assert_close(o[b].reshape(-1), ref, what=f"seed={seed} b={b}")


def _append_case(seed):
    rng = np.random.default_rng(5000 + seed)
    H, Hk, D = _shape(rng)
    if rng.integers(3) == 0:  # odd head counts leave partly empty head groups
        Hk = int(rng.choice([1, 3, 5]))
        H = Hk * int(rng.integers(1, 6))
    rows = int(rng.choice([1, 2, 7, 64, 255, 256, 300]))
    rd = D if rng.integers(2) else 2 * int(rng.integers(1, D // 2))
    return dict(rows=rows, start_pos=int(rng.choice([0, 5, 1000])), H=H, Hk=Hk, D=D, rd=rd,
                neox=bool(rng.integers(2)), norm=bool(rng.integers(2)), bias=bool(rng.integers(2)),
                qdt=str(rng.choice(["f32", "f16", "bf16"])), kvdt=str(rng.choice(["f32", "f16", "bf16"])))


@pytest.mark.parametrize("seed", range(12))
def test_append_random(dev, seed):
    """Fused bias + Q/K norm + RoPE + cache store on random head counts,
    head_dims, rotary widths, row counts (either side of the 256-row switch
    between one workgroup per row and a row spread over workgroups) and
    dtypes, against the oracle."""
    from tests.test_append_gpu import run_case

    c = _append_case(seed)
    print(f"[append-rand] seed={seed} {c}", flush=True)
    run_case(dev, c["rows"], c["start_pos"], c["H"], c["Hk"], c["D"], c["rd"], c["neox"],
             norm=c["norm"], bias=c["bias"], qdt=c["qdt"], kvdt=c["kvdt"], seed=seed + 1)
