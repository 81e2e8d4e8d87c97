"""Fused bias + Q/K RMSNorm + RoPE + KV append on the GPU vs the oracle
(crates/ullm-model/src/lib.rs:1021-1058)."""
import numpy as np
import pytest
import torch

from oracle import oracle as ora
from tests.helpers import assert_close
from ullm_amd import attention as A
from ullm_amd import synth

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def run_case(dev, rows, start_pos, H, Hk, D, rd, neox, norm, bias, qdt, kvdt, theta=1e6,
             seed=1):
    print(f"[append] rows{rows} sp{start_pos} H{H} Hk{Hk} D{D} rd{rd} neox={neox} "
          f"norm={norm} bias={bias} q={qdt} kv={kvdt}", flush=True)
    n_ctx = start_pos + rows + 3
    q = synth.randn(seed, 1, (rows, H * D))
    k = synth.randn(seed, 2, (rows, Hk * D))
    v = synth.randn(seed, 3, (rows, Hk * D))
    qn = (synth.randn(seed, 4, (D,)) * 0.2 + 1.0) if norm else None
    kn = (synth.randn(seed, 5, (D,)) * 0.2 + 1.0) if norm else None
    qb = synth.randn(seed, 6, (H * D,)) if bias else None
    kb = synth.randn(seed, 7, (Hk * D,)) if bias else None
    vb = synth.randn(seed, 8, (Hk * D,)) if bias else None
    cs = A.rope_table(n_ctx, rd, theta, device=dev)
    kc = torch.zeros(n_ctx, Hk * D, dtype=DT[kvdt], device=dev)
    vc = torch.zeros_like(kc)
    g = lambda t: None if t is None else t.to(dev)  # noqa: E731
    qo = A.qkv_append(q.to(dev), k.to(dev), v.to(dev), kc, vc, cs, start_pos=start_pos,
                      n_head=H, n_kv_head=Hk, head_dim=D, rotary_dim=rd, neox=neox, q_norm=g(qn),
                      k_norm=g(kn), eps=1e-6, q_bias=g(qb), k_bias=g(kb), v_bias=g(vb),
                      q_dtype=DT[qdt])
    torch.cuda.synchronize()
    n = lambda t: None if t is None else t.numpy().copy()  # noqa: E731
    okc = np.zeros((n_ctx, Hk * D), np.float32)
    ovc = np.zeros_like(okc)
    oq = ora.qkv_append(q.numpy().copy(), k.numpy().copy(), v.numpy().copy(), start_pos, H, Hk,
                        D, rd, theta, neox, okc, ovc, q_bias=n(qb), k_bias=n(kb), v_bias=n(vb),
                        q_norm=n(qn), k_norm=n(kn), eps=1e-6)
    # The GPU rounds its outputs to the storage dtype; compare with the oracle
    # rounded the same way (round-to-nearest-even), allowing one ulp of that
    # dtype for the different summation order inside RMSNorm.
    def rounded(x, dt):
        return torch.from_numpy(x).to(dt).float().numpy()

    tol = {"f32": 2e-5, "f16": 2e-3, "bf16": 1.6e-2}
    for name, got, ref, dt in (("q", qo, oq, qdt),
                               ("k", kc[start_pos:start_pos + rows], okc[start_pos:start_pos + rows], kvdt),
                               ("v", vc[start_pos:start_pos + rows], ovc[start_pos:start_pos + rows], kvdt)):
        got = got.float().cpu().numpy()
        r = rounded(ref, DT[dt])
        rel = np.abs(got - r) / np.maximum(np.abs(r), 1.0)
        assert rel.max() <= tol[dt], f"{name}: max rel {rel.max():.3e}"
        assert_close(got, ref, max_abs=4 * tol[dt] * max(1.0, np.abs(ref).max()) + 1e-6,
                     rel_l2=tol[dt], what=name)
    # positions outside the written rows stay untouched
    assert torch.count_nonzero(kc[:start_pos]).item() == 0
    assert torch.count_nonzero(kc[start_pos + rows:]).item() == 0


@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_rope_modes_head_dims(dev, neox, D):
    run_case(dev, 5, 7, 4, 2, D, D, neox, norm=True, bias=False, qdt="f32", kvdt="f32")


@pytest.mark.parametrize("qdt,kvdt", [("f32", "f16"), ("bf16", "bf16"), ("f16", "f16"),
                                      ("f32", "bf16")])
def test_dtypes(dev, qdt, kvdt):
    run_case(dev, 16, 0, 8, 4, 128, 128, True, norm=True, bias=True, qdt=qdt, kvdt=kvdt)


@pytest.mark.parametrize("neox", [True, False])
def test_partial_rotary(dev, neox):
    run_case(dev, 3, 100, 4, 4, 128, 64, neox, norm=False, bias=True, qdt="f32", kvdt="f32",
             theta=1e4)


def test_cfg3_prefill_prep(dev):
    """cfg3 preparation: Qwen3 q/k-norm + NeoX RoPE theta 1e6 into a bf16 cache."""
    run_case(dev, 2048, 0, 32, 8, 128, 128, True, norm=True, bias=False, qdt="bf16",
             kvdt="bf16", seed=3)


def test_decode_single_row_far_position(dev):
    run_case(dev, 1, 32000, 32, 4, 128, 128, True, norm=True, bias=False, qdt="f32",
             kvdt="bf16")


@pytest.mark.parametrize("rows,H,Hk,D,rd,neox", [(4, 6, 3, 64, 64, True), (4, 5, 1, 128, 128, False),
                                                 (4, 3, 3, 256, 256, True), (4, 7, 7, 64, 32, False),
                                                 (4, 9, 3, 128, 96, True), (3, 42, 6, 64, 64, False),
                                                 (300, 5, 1, 128, 128, True)])
def test_partial_head_groups(dev, rows, H, Hk, D, rd, neox):
    """Head counts that leave a kind's last group of 256/D heads partly empty
    (the empty lanes must store nothing), with full and partial rotary; few
    rows spread a row's groups over several workgroups (42/6 heads at D 64:
    15 groups, a full part and a partial one), many rows keep one per row."""
    run_case(dev, rows, 3, H, Hk, D, rd, neox, norm=True, bias=True, qdt="f32", kvdt="bf16")
