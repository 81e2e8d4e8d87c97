"""Q/K/V projection + fused append on the GPU vs the oracle: matvec_q
(crates/ullm-model/src/math.rs:9-21) per weight, then the append oracle
(lib.rs:857-914 for one decoded token, the same steps for several rows)."""
import numpy as np
import pytest
import torch

from oracle import oracle as ora
from tests.helpers import assert_close
from ullm_amd import attention as A
from ullm_amd import synth

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
ORA_DT = {"f32": 0, "f16": 1, "bf16": 2}


def raw16(t):
    """Host storage of a weight for the oracle: f32 array, or uint16 bits."""
    if t.dtype == torch.float32:
        return t.cpu().numpy()
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def run_case(dev, rows, start_pos, H, Hk, D, in_dim, wdt, rd, neox, norm, bias, qdt, kvdt,
             theta=1e6, seed=1):
    print(f"[proj] rows{rows} sp{start_pos} H{H} Hk{Hk} D{D} in{in_dim} w={wdt} rd{rd} "
          f"neox={neox} norm={norm} bias={bias} q={qdt} kv={kvdt}", flush=True)
    n_ctx = start_pos + rows + 2
    x = synth.randn(seed, 1, (rows, in_dim))
    sd = 1.0 / np.sqrt(in_dim)
    wq = (synth.randn(seed, 2, (H * D, in_dim)) * sd).to(DT[wdt])
    wk = (synth.randn(seed, 3, (Hk * D, in_dim)) * sd).to(DT[wdt])
    wv = (synth.randn(seed, 4, (Hk * D, in_dim)) * sd).to(DT[wdt])
    qn = (synth.randn(seed, 5, (D,)) * 0.2 + 1.0) if norm else None
    kn = (synth.randn(seed, 6, (D,)) * 0.2 + 1.0) if norm else None
    qb = synth.randn(seed, 7, (H * D,)) * 0.1 if bias else None
    kb = synth.randn(seed, 8, (Hk * D,)) * 0.1 if bias else None
    vb = synth.randn(seed, 9, (Hk * D,)) * 0.1 if bias else None
    cs = A.rope_table(n_ctx, rd, theta, device=dev)
    kc = torch.zeros(n_ctx, Hk * D, dtype=DT[kvdt], device=dev)
    vc = torch.zeros_like(kc)
    g = lambda t: None if t is None else t.to(dev)  # noqa: E731
    qo = A.qkv_proj_append(x.to(dev), g(wq), g(wk), g(wv), kc, vc, cs, start_pos=start_pos,
                           n_head=H, n_kv_head=Hk, head_dim=D, rotary_dim=rd, neox=neox,
                           q_norm=g(qn), k_norm=g(kn), eps=1e-6, q_bias=g(qb), k_bias=g(kb),
                           v_bias=g(vb), q_dtype=DT[qdt])
    torch.cuda.synchronize()
    # oracle: three matvecs per row, then the append steps
    xn = x.numpy()
    mv = lambda w: np.stack([ora.matvec(raw16(w), ORA_DT[wdt], xn[r]) for r in range(rows)])  # noqa: E731
    q, k, v = mv(wq), mv(wk), mv(wv)
    n = lambda t: None if t is None else t.numpy().copy()  # noqa: E731
    okc = np.zeros((n_ctx, Hk * D), np.float32)
    ovc = np.zeros_like(okc)
    oq = ora.qkv_append(q, k, v, start_pos, H, Hk, D, rd, theta, neox, okc, ovc, q_bias=n(qb),
                        k_bias=n(kb), v_bias=n(vb), q_norm=n(qn), k_norm=n(kn), eps=1e-6)
    # f32 sums in another order (per-lane partials + a wave tree): 1e-4
    # relative at these dot lengths; a 16-bit output adds its own rounding.
    tol = {"f32": 1e-4, "f16": 2e-3, "bf16": 1.6e-2}
    for name, got, ref, dt in (("q", qo, oq, qdt),
                               ("k", kc[start_pos:start_pos + rows], okc[start_pos:start_pos + rows], kvdt),
                               ("v", vc[start_pos:start_pos + rows], ovc[start_pos:start_pos + rows], kvdt)):
        got = got.float().cpu().numpy()
        assert_close(got, ref, max_abs=4 * tol[dt] * max(1.0, np.abs(ref).max()) + 1e-6,
                     rel_l2=tol[dt], what=name)
    assert torch.count_nonzero(kc[:start_pos]).item() == 0
    assert torch.count_nonzero(kc[start_pos + rows:]).item() == 0


def test_qwen3_4b_decode_token(dev):
    """Qwen3-4B-shaped decode step: hidden 2560, 32/8 heads, q/k norm, NeoX
    theta 1e6, bf16 weights, f32 q, bf16 cache."""
    run_case(dev, 1, 2047, 32, 8, 128, 2560, "bf16", 128, True, norm=True, bias=False,
             qdt="f32", kvdt="bf16", seed=2)


def test_qwen25_decode_token_bias(dev):
    """Qwen2.5-1.5B-shaped: hidden 1536, 12/2 heads, q/k/v biases, no norm."""
    run_case(dev, 1, 4095, 12, 2, 128, 1536, "bf16", 128, True, norm=False, bias=True,
             qdt="f32", kvdt="f16", seed=3)


@pytest.mark.parametrize("wdt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_weight_dtypes_head_dims(dev, wdt, D):
    run_case(dev, 2, 5, 8, 4, D, 512, wdt, D, True, norm=True, bias=True, qdt="f32",
             kvdt="f32", seed=4)


@pytest.mark.parametrize("neox", [True, False])
def test_interleaved_and_partial_rotary(dev, neox):
    run_case(dev, 3, 10, 4, 2, 128, 264, "f16", 64, neox, norm=False, bias=False, qdt="bf16",
             kvdt="bf16", theta=1e4, seed=5)


def test_many_rows_unsplit(dev):
    """rows * head vectors >= 256: one workgroup per head vector, no workspace."""
    assert A.proj_workspace(20, 8, 4, 128) is None
    run_case(dev, 20, 3, 8, 4, 128, 384, "bf16", 128, True, norm=True, bias=True, qdt="bf16",
             kvdt="bf16", seed=6)


def test_split_counters_reset_between_calls(dev):
    """The split path's arrival counters return to zero: three calls in a row on
    one workspace (different inputs) all match the oracle."""
    for seed in (7, 8, 9):
        run_case(dev, 1, 100, 12, 2, 128, 1536, "bf16", 128, True, norm=True, bias=False,
                 qdt="f32", kvdt="bf16", seed=seed)


def test_split_exchange_2000_calls_repeat_exactly(dev):
    """The split projection's cross-workgroup exchange under load: 2000
    back-to-back calls at the Qwen3-4B decode shape on one workspace, each
    call's q (written to its own row) and the final K/V row bit-identical to
    the first call's; a stale part reloaded by the last arriver would change
    a head.  All calls are queued first; the comparison afterwards reports
    the first mismatching call."""
    H, Hk, D, hidden, n = 32, 8, 128, 2560, 2000
    print(f"[proj] exchange repeat x{n}", flush=True)
    x = synth.randn(21, 1, (1, hidden)).to(dev)
    sd = 1.0 / np.sqrt(hidden)
    wq, wk, wv = ((synth.randn(21, t, (m * D, hidden)) * sd).to(torch.bfloat16).to(dev)
                  for t, m in ((2, H), (3, Hk), (4, Hk)))
    qn = (synth.randn(21, 5, (D,)) * 0.2 + 1.0).to(dev)
    kn = (synth.randn(21, 6, (D,)) * 0.2 + 1.0).to(dev)
    cs = A.rope_table(4096, D, 1e6, device=dev)
    kc = torch.zeros(4096, Hk * D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    ws = torch.zeros(int(A.L.lib().ullm_hip_qkv_proj_workspace_bytes(1, H, Hk, D)),
                     dtype=torch.uint8, device=dev)
    assert ws.numel() > 0, "the decode shape must take the split path"
    qs = torch.empty(n, 1, H * D, device=dev)
    kv0 = None
    for i in range(n):
        A.qkv_proj_append(x, wq, wk, wv, kc, vc, cs, start_pos=4095, n_head=H, n_kv_head=Hk,
                          head_dim=D, q_norm=qn, k_norm=kn, q_out=qs[i], workspace=ws)
        if i == 0:
            torch.cuda.synchronize()
            kv0 = (kc[4095].clone(), vc[4095].clone())
    torch.cuda.synchronize()
    same = (qs == qs[0]).all(dim=2).reshape(-1).cpu()
    bad = (~same).nonzero()
    assert bad.numel() == 0, f"call {int(bad[0])} differs from call 0"
    assert torch.equal(kc[4095], kv0[0]) and torch.equal(vc[4095], kv0[1])
    # the first call is right, too
    ref = qs[0].cpu().numpy()
    assert np.isfinite(ref).all() and np.abs(ref).max() > 0
