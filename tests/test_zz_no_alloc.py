"""ullm_hip_attn_decode_noalloc (the allocation-free decode entry point)
through the C ABI, against ullm_hip_attn_decode with a caller workspace: the
same kernels and plan, so the outputs agree bit for bit.  Two calls in a
row, the second smaller, so the shared static scratch is reused."""
import ctypes as C
import math

import pytest
import torch

from ullm_amd import _lib as L
from ullm_amd import attention as A
from ullm_amd import synth

DT = {torch.float32: L.DT_F32, torch.float16: L.DT_F16, torch.bfloat16: L.DT_BF16}


def _p(t):
    return C.c_void_p(t.data_ptr())


def noalloc(q, kc, vc, lens, max_len, hk, window=0):
    B, H, D = q.shape
    out = torch.full((B, H, D), float("nan"), device=q.device)
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = L.lib().ullm_hip_attn_decode_noalloc(
        _p(q), _p(kc), _p(vc), DT[kc.dtype], hk * D, max_len * hk * D, _p(lens), max_len, window,
        B, H, hk, D, 1.0 / math.sqrt(D), _p(out), st)
    L.check(rc)
    return out


def case(dev, dt, B, H, Hk, D, lens, seed, window=0):
    L_ = max(lens)
    print(f"[noalloc] {dt} B{B} H{H} Hk{Hk} D{D} lens={lens} win={window}", flush=True)
    q = synth.randn(seed, 1, (B, H, D)).to(dev)
    kc = synth.randn(seed, 2, (B, L_, Hk * D), dt).to(dev)
    vc = synth.randn(seed, 3, (B, L_, Hk * D), dt).to(dev)
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    got = noalloc(q, kc, vc, sl, L_, Hk, window)
    want = A.attn_decode(q, kc, vc, sl, L_, Hk, window=window, seq_stride=L_ * Hk * D)
    torch.cuda.synchronize()
    assert torch.equal(got, want), (got - want).abs().max().item()


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_entry_two_calls(dev, dt):
    # cfg2-shaped at 4096 keys, then a smaller call reusing the scratch
    case(dev, dt, 1, 12, 2, 128, [4096], seed=41)
    case(dev, dt, 1, 12, 2, 128, [700], seed=42)


@pytest.mark.gpu
def test_noalloc_long_and_ragged(dev):
    case(dev, torch.bfloat16, 1, 32, 4, 128, [32768], seed=43)
    case(dev, torch.float16, 3, 8, 4, 256, [3000, 1200, 77], seed=44, window=1024)


def test_noalloc_rejects_shapes_past_the_scratch():
    """Checked before any device work: 16 query heads on one kv head at
    head_dim 256 and 32K keys (256 splits of 16 x 256 floats) need more than
    the static scratch and get ULLM_HIP_E_WORKSPACE with a clear message."""
    lib = L.lib()
    assert lib.ullm_hip_decode_noalloc_max_bytes() == 4 << 20
    fake = C.c_void_p(0x10000)
    rc = lib.ullm_hip_attn_decode_noalloc(fake, fake, fake, L.DT_BF16, 256, 0, fake, 32768, 0,
                                          1, 16, 1, 256, 0.1, fake, None)
    assert rc == L.E_WORKSPACE
    assert b"static scratch" in lib.ullm_hip_last_error()
