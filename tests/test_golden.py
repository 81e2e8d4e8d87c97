"""Golden fixtures (tests/golden/*.npz, written by make_golden.py): the CPU
oracle must reproduce them bit for bit; the GPU path must match them within
the attention tolerance."""
import glob
import math
import os

import numpy as np
import pytest
import torch

from oracle import oracle as ora
from tests.helpers import assert_close

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FILES = sorted(glob.glob(os.path.join(HERE, "*.npz")))
TDT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
ODT = {"f32": 0, "f16": 1, "bf16": 2}


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def as_f32(a, dt):
    return a.astype(np.float32) if dt == "f32" else ora.widen(a, ODT[dt])


def as_tensor(a, dt, dev):
    if dt == "f32":
        return torch.from_numpy(a).to(dev)
    return torch.from_numpy(a.view(np.int16)).view(TDT[dt]).to(dev)


def test_fixture_set_present():
    kinds = {str(load(f)["kind"]) for f in FILES}
    assert kinds == {"decode", "prefill", "append"} and len(FILES) >= 8


@pytest.mark.parametrize("path", FILES, ids=os.path.basename)
def test_oracle_reproduces_fixture(path):
    z = load(path)
    kind = str(z["kind"])
    if kind == "decode":
        dt = str(z["dtype"])
        H, Hk, D, win = (int(x) for x in z["shape"])
        for b, ln in enumerate(z["lens"]):
            out = ora.attn_decode(z["q"][b].reshape(-1).copy(), as_f32(z["k"][b], dt),
                                  as_f32(z["v"][b], dt), int(ln) - 1, H, Hk, D,
                                  float(z["scale"]), window=win)
            np.testing.assert_array_equal(out, z["out"][b])
    elif kind == "prefill":
        dt = str(z["dtype"])
        S, sp, H, Hk, D, win = (int(x) for x in z["shape"])
        out = ora.attn_prefill(as_f32(z["q"], dt), as_f32(z["k"], dt), as_f32(z["v"], dt), S,
                               sp, H, Hk, D, float(z["scale"]), window=win)
        np.testing.assert_array_equal(out, z["out"])
    else:
        rows, sp, H, Hk, D, rd, neox = (int(x) for x in z["shape"])
        kc = np.zeros_like(z["k_cache"])
        vc = np.zeros_like(z["v_cache"])
        qo = ora.qkv_append(z["q"], z["k"], z["v"], sp, H, Hk, D, rd, float(z["theta"]),
                            bool(neox), kc, vc, k_bias=z["k_bias"], q_norm=z["q_norm"],
                            k_norm=z["k_norm"], eps=1e-6)
        np.testing.assert_array_equal(qo, z["q_out"])
        np.testing.assert_array_equal(kc, z["k_cache"])
        np.testing.assert_array_equal(vc, z["v_cache"])


@pytest.mark.gpu
@pytest.mark.parametrize("path", FILES, ids=os.path.basename)
def test_gpu_matches_fixture(dev, path):
    from ullm_amd import attention as A

    z = load(path)
    kind = str(z["kind"])
    print(f"[golden] {os.path.basename(path)}", flush=True)
    if kind == "decode":
        dt = str(z["dtype"])
        H, Hk, D, win = (int(x) for x in z["shape"])
        k, v = as_tensor(z["k"], dt, dev), as_tensor(z["v"], dt, dev)
        B, L = k.shape[0], k.shape[1]
        lens = torch.from_numpy(z["lens"]).to(dev)
        out = A.attn_decode(torch.from_numpy(z["q"]).to(dev), k, v, lens, L, Hk, window=win,
                            scale=float(z["scale"]), seq_stride=L * Hk * D)
        assert_close(out.view(B, -1).cpu().numpy(), z["out"], what="decode")
    elif kind == "prefill":
        dt = str(z["dtype"])
        S, sp, H, Hk, D, win = (int(x) for x in z["shape"])
        out = A.attn_prefill(as_tensor(z["q"], dt, dev), as_tensor(z["k"], dt, dev),
                             as_tensor(z["v"], dt, dev), H, Hk, D, start_pos=sp, window=win,
                             scale=float(z["scale"]))
        assert_close(out.cpu().numpy(), z["out"], what="prefill")
    else:
        rows, sp, H, Hk, D, rd, neox = (int(x) for x in z["shape"])
        cs = A.rope_table(sp + rows, rd, float(z["theta"]), device=dev)
        kc = torch.zeros(sp + rows, Hk * D, device=dev)
        vc = torch.zeros_like(kc)
        g = lambda n: torch.from_numpy(z[n]).to(dev)  # noqa: E731
        qo = A.qkv_append(g("q"), g("k"), g("v"), kc, vc, cs, start_pos=sp, n_head=H,
                          n_kv_head=Hk, head_dim=D, rotary_dim=rd, neox=bool(neox),
                          q_norm=g("q_norm"), k_norm=g("k_norm"), k_bias=g("k_bias"), eps=1e-6)
        for got, want in ((qo, z["q_out"]), (kc, z["k_cache"]), (vc, z["v_cache"])):
            np.testing.assert_allclose(got.cpu().numpy(), want, rtol=2e-5, atol=2e-5)
