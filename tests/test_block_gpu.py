"""Attention blocks of GpuAttention from the normed hidden state, end to end
against the oracle: the projections (matvec_q, crates/ullm-model/src/math.rs:
9-21), the append (bias, Q/K norm, RoPE, cache store; lib.rs:857-914 and
:1021-1058) and the attention (lib.rs:911-938, :1061-1087), composed as the
reference's GPU forward composes them (forward.rs:415-466 for a decoded
token, :799-858 for a prompt).  The oracle runs on the same rounding: its
q (prefill) and cache rows are rounded to the cache dtype as the GPU path
stores them, but the GPU projections (f32 accumulation in another order,
bf16 hi + lo activations) differ from its f32 matvec by ~1e-5 relative, so
an isolated stored 16-bit value can round one ulp apart (2^-8 relative for
bf16).  With 16-bit storage the block is therefore held to rel-L2 <= 1e-3
and max-abs <= 2e-2 (one bf16 ulp of a |V| ~ 4 value carried at full
weight); with an f32 cache, to the attention path's own max-abs <= 2e-3."""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as ora
from tests.helpers import assert_close
from ullm_amd import attention as A
from ullm_amd import synth

pytestmark = pytest.mark.gpu


def _raw(w):
    if w.dtype == torch.float32:
        return w.cpu().numpy(), 0
    code = 1 if w.dtype == torch.float16 else 2
    return w.cpu().view(torch.int16).numpy().view(np.uint16), code


def _round(a, dt):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dt).float().numpy()


@pytest.mark.parametrize("wdt,kvdt,D,window", [
    (torch.bfloat16, torch.bfloat16, 128, 0),   # MFMA projections + MFMA prefill
    (torch.bfloat16, torch.float16, 64, 48),    # sliding window on layer 0
    (torch.float16, torch.float32, 128, 0),     # fused projection kernel + f32 cache
])
def test_prefill_then_decode_block(dev, wdt, kvdt, D, window):
    print(f"[block] w={wdt} kv={kvdt} D{D} window{window}", flush=True)
    n_embd, H, Hk, S, n_dec, theta = 512, 8, 2, 100, 3, 1e6
    p = A.AttnParams(n_layer=1, n_head=H, n_kv_head=Hk, head_dim=D, n_ctx=S + n_dec + 1,
                     rope_theta=theta, eps=1e-6, rope_neox=True, sliding_window=window,
                     kv_dtype=kvdt)
    ga = A.GpuAttention(p, device=dev)
    sd = 1.0 / math.sqrt(n_embd)
    wq = (synth.randn(9, 1, (H * D, n_embd)) * sd).to(wdt)
    wk = (synth.randn(9, 2, (Hk * D, n_embd)) * sd).to(wdt)
    wv = (synth.randn(9, 3, (Hk * D, n_embd)) * sd).to(wdt)
    qn = synth.randn(9, 4, (D,)) * 0.2 + 1.0
    kn = synth.randn(9, 5, (D,)) * 0.2 + 1.0
    xs = synth.randn(9, 6, (S + n_dec, n_embd))
    g = lambda t: t.to(dev)  # noqa: E731
    out_p = ga.forward_batch_proj(0, g(xs[:S]), g(wq), g(wk), g(wv), 0, q_norm=g(qn),
                                  k_norm=g(kn)).cpu().numpy()
    outs_d = [ga.forward_proj(0, g(xs[S + i]), S + i, g(wq), g(wk), g(wv), q_norm=g(qn),
                              k_norm=g(kn)).cpu().numpy() for i in range(n_dec)]
    torch.cuda.synchronize()

    # oracle
    T = S + n_dec
    xn = xs.numpy()
    mv = lambda w: np.stack([ora.matvec(*_raw(w), xn[r]) for r in range(T)])  # noqa: E731
    q, k, v = mv(wq), mv(wk), mv(wv)
    kc = np.zeros((p.n_ctx, Hk * D), np.float32)
    vc = np.zeros_like(kc)
    qp = ora.qkv_append(q, k, v, 0, H, Hk, D, D, theta, True, kc, vc, q_norm=qn.numpy(),
                        k_norm=kn.numpy(), eps=1e-6)
    kc, vc = _round(kc, kvdt), _round(vc, kvdt)
    scale = 1.0 / math.sqrt(D)
    qpp = qp[:S] if kvdt == torch.float32 else _round(qp[:S], kvdt)
    ref_p = ora.attn_prefill(qpp, kc[:S], vc[:S], S, 0, H, Hk, D, scale, window=window)
    tol = dict(max_abs=2e-3 if kvdt == torch.float32 else 2e-2, rel_l2=1e-3)
    assert_close(out_p, ref_p, what="prefill block", **tol)
    for i in range(n_dec):
        pos = S + i
        ref_d = ora.attn_decode(qp[pos].copy(), kc[:pos + 1], vc[:pos + 1], pos, H, Hk, D, scale,
                                window=window)
        assert_close(outs_d[i], ref_d, what=f"decode block pos {pos}", **tol)


def test_forward_debug_reports_every_op(dev):
    """GpuAttention.forward_debug (the attention half of the reference's
    GpuForward::forward_debug, forward.rs:530-635): one report line per op,
    all clean on finite inputs, the attention output and cache row of
    forward_proj (to f32 rounding / one bf16 ulp); a NaN in the hidden state shows up from the projections
    on."""
    n_embd, H, Hk, D, pos = 512, 8, 2, 128, 37
    p = A.AttnParams(n_layer=1, n_head=H, n_kv_head=Hk, head_dim=D, n_ctx=64, rope_theta=1e6,
                     kv_dtype=torch.bfloat16)
    sd = 1.0 / math.sqrt(n_embd)
    w = [(synth.randn(12, t, (n * D, n_embd)) * sd).to(torch.bfloat16).to(dev)
         for t, n in ((1, H), (2, Hk), (3, Hk))]
    qn = (synth.randn(12, 4, (D,)) * 0.2 + 1.0).to(dev)
    kn = (synth.randn(12, 5, (D,)) * 0.2 + 1.0).to(dev)
    qb = (synth.randn(12, 6, (H * D,)) * 0.1).to(dev)
    kb = (synth.randn(12, 7, (Hk * D,)) * 0.1).to(dev)
    vb = (synth.randn(12, 8, (Hk * D,)) * 0.1).to(dev)
    x = synth.randn(12, 9, (n_embd,)).to(dev)
    kw = dict(q_norm=qn, k_norm=kn, q_bias=qb, k_bias=kb, v_bias=vb)
    a, b = A.GpuAttention(p, device=dev), A.GpuAttention(p, device=dev)
    # earlier positions hold the same random rows in both caches
    a.key_cache.copy_(synth.randn(12, 10, tuple(a.key_cache.shape), torch.bfloat16))
    a.val_cache.copy_(synth.randn(12, 11, tuple(a.val_cache.shape), torch.bfloat16))
    b.key_cache.copy_(a.key_cache)
    b.val_cache.copy_(a.val_cache)
    out, rep = a.forward_debug(x, pos, *w, **kw, log=False)
    want = b.forward_proj(0, x, pos, *w, **kw)
    torch.cuda.synchronize()
    labels = [r[0] for r in rep]
    assert labels == ["attn_in", "wq", "wk", "wv", "bias_q", "bias_k", "bias_v", "q_norm",
                      "k_norm", "rope_q", "rope_k", "attn_out"], labels
    assert all(r[1] == 0 and r[2] == 0 and r[3] > 0 for r in rep), rep
    # The fused projection and the separate append compute the per-head RMS
    # sum in different lane orders: f32 rounding apart, not more.
    assert_close(out.cpu().numpy(), want.cpu().numpy(), max_abs=2e-5, rel_l2=1e-5,
                 what="debug vs forward_proj")
    kd = (a.key_cache[0, pos].float() - b.key_cache[0, pos].float()).abs()
    assert (kd <= 2.0**-7 * b.key_cache[0, pos].float().abs().clamp(min=1.0)).all()
    xn = x.clone()
    xn[3] = float("nan")
    _, rep = a.forward_debug(xn, pos, *w, **kw, log=False)
    nan = {r[0]: r[1] for r in rep}
    assert nan["attn_in"] == 1 and nan["wq"] == H * D and nan["wk"] == Hk * D
    assert nan["rope_q"] == H * D and nan["rope_k"] == Hk * D
    # attn_out: the split-KV kernels guard l > 0 when they normalise (as the
    # Metal kernels do, shader.metal:1070), so NaN scores leave zeros
    # there; the report has already named the first op that went bad.
