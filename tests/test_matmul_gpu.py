"""Batched projection (ullm_hip_matmul) on the GPU against the CPU oracle.

The reference's prefill matmul (crates/ullm-metal/src/shader.metal:519-566)
computes, per token row, the same dot products as the CPU reference's
matvec (crates/ullm-model/src/math.rs:9-21).  Small shapes are checked
against the oracle's matvec row by row; full-size shapes against an f64
product of the same rounded inputs (the oracle's matvec is pinned to f64 in
test_oracle.py).  Bound: the activations enter the matrix cores as a bf16
hi + lo pair, residual <= 2^-16 |x|, and the f32 accumulation adds at most
in_dim * 2^-24 of sum |x w|, so |y - y64| <= (2^-16 + in_dim 2^-24) sum_i |x_i w_i|
elementwise, plus the attention path's tolerance (max-abs 2e-3, rel-L2 1e-3)."""
import numpy as np
import pytest
import torch

from oracle import oracle as ora
from tests.helpers import assert_close
from ullm_amd import attention as A
from ullm_amd import synth

pytestmark = pytest.mark.gpu


def _bits(w):
    return w.cpu().view(torch.int16).numpy().view(np.uint16)


def _check_bound(y, x64, w64, what):
    ref = x64 @ w64.T
    mag = np.abs(x64) @ np.abs(w64).T
    in_dim = x64.shape[1]
    bound = (2.0 ** -16 + in_dim * 2.0 ** -24) * mag + 1e-30
    d = np.abs(y.astype(np.float64) - ref)
    worst = float(np.max(d / bound))
    assert worst <= 1.0, f"{what}: error {worst:.3f} x the bound"
    assert_close(y, ref, what=what)


@pytest.mark.parametrize("n_cols,out_dim,in_dim", [
    (1, 4, 8), (3, 64, 40), (37, 132, 256), (130, 260, 264), (129, 128, 32), (64, 1000, 520),
])
def test_matmul_small_vs_oracle(dev, n_cols, out_dim, in_dim):
    print(f"[matmul] n{n_cols} out{out_dim} in{in_dim}", flush=True)
    x = synth.randn(11, 1, (n_cols, in_dim))
    w = (synth.randn(11, 2, (out_dim, in_dim)) * 0.05).to(torch.bfloat16)
    y = A.matmul(w.to(dev), x.to(dev))
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    xn = x.numpy()
    ref = np.stack([ora.matvec(_bits(w), 2, xn[s]) for s in range(n_cols)])
    assert_close(y, ref, what=f"n{n_cols} out{out_dim} in{in_dim}")
    _check_bound(y, xn.astype(np.float64), w.float().numpy().astype(np.float64),
                 f"n{n_cols} out{out_dim} in{in_dim}")


@pytest.mark.parametrize("n_cols,out_dim,in_dim", [
    (2048, 4096, 2560),   # Qwen3-4B q projection over a 2048-token prompt
    (2048, 1024, 2560),   # its k / v projection
    (777, 2304, 1544),    # ragged in every dimension
])
def test_matmul_full_vs_f64(dev, n_cols, out_dim, in_dim):
    print(f"[matmul-full] n{n_cols} out{out_dim} in{in_dim}", flush=True)
    g = torch.Generator(device=dev).manual_seed(n_cols + out_dim)
    x = torch.randn(n_cols, in_dim, device=dev, generator=g)
    w = (torch.randn(out_dim, in_dim, device=dev, generator=g) / in_dim ** 0.5).to(torch.bfloat16)
    y = A.matmul(w, x)
    torch.cuda.synchronize()
    _check_bound(y.cpu().numpy(), x.cpu().double().numpy(), w.cpu().double().numpy(),
                 f"n{n_cols} out{out_dim} in{in_dim}")


def test_matmul_dynamic_range(dev):
    """Activations over 2^-20 .. 2^20 (massive-activation rows): the hi/lo
    split is relative, so the bound still holds row by row."""
    print("[matmul-range]", flush=True)
    g = torch.Generator(device=dev).manual_seed(5)
    n, o, i = 256, 384, 1024
    x = torch.randn(n, i, device=dev, generator=g)
    x *= torch.exp2(torch.randint(-20, 21, (n, i), device=dev, generator=g).float())
    w = (torch.randn(o, i, device=dev, generator=g) * 0.03).to(torch.bfloat16)
    y = A.matmul(w, x)
    torch.cuda.synchronize()
    x64, w64 = x.cpu().double().numpy(), w.cpu().double().numpy()
    ref = x64 @ w64.T
    bound = (2.0 ** -16 + i * 2.0 ** -24) * (np.abs(x64) @ np.abs(w64).T)
    assert np.all(np.abs(y.cpu().numpy() - ref) <= bound)


def test_matmul_into_cache_view(dev):
    """forward.rs:800-801 writes K/V straight into the f32 cache at the
    layer offset: y is a view, and rows outside it stay untouched."""
    print("[matmul-view]", flush=True)
    n_ctx, kv_dim, in_dim, s = 300, 256, 512, 150
    cache = torch.full((2 * n_ctx, kv_dim), 7.0, device=dev)
    x = synth.randn(3, 1, (s, in_dim)).to(dev)
    w = (synth.randn(3, 2, (kv_dim, in_dim)) * 0.05).to(torch.bfloat16).to(dev)
    view = cache[n_ctx:n_ctx + s]
    A.matmul(w, x, view)
    torch.cuda.synchronize()
    c = cache.cpu()
    assert torch.all(c[:n_ctx] == 7.0) and torch.all(c[n_ctx + s:] == 7.0)
    _check_bound(c[n_ctx:n_ctx + s].numpy(), x.cpu().double().numpy(),
                 w.cpu().double().numpy(), "cache view")


def test_matmul_over_2gib_activations(dev):
    """X above 2 GiB goes in token chunks (32-bit buffer offsets): sampled
    rows on both sides of the chunk boundary."""
    in_dim, out_dim = 65536, 8
    n_cols = 8300  # chunk = 8064 rows at this in_dim
    print(f"[matmul-2gib] n{n_cols} in{in_dim}", flush=True)
    g = torch.Generator(device=dev).manual_seed(9)
    x = torch.randn(n_cols, in_dim, device=dev, generator=g)
    w = (torch.randn(out_dim, in_dim, device=dev, generator=g) * 0.004).to(torch.bfloat16)
    y = A.matmul(w, x)
    torch.cuda.synchronize()
    rows = [0, 1, 8063, 8064, 8065, n_cols - 1]
    _check_bound(y[rows].cpu().numpy(), x[rows].cpu().double().numpy(),
                 w.cpu().double().numpy(), "2 GiB chunks")
    del x
    torch.cuda.empty_cache()
