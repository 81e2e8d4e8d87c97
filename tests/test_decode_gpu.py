"""Decode attention on the GPU (libullm_hip.so) against the CPU oracle.

Cases follow the benchmark configurations (Llama-3.2-1B, Qwen2.5-1.5B,
Gemma-3 windowed, Qwen3-30B-A3B long context, ragged batch) plus the edges of
the split-KV planner: one key, lengths that are not a multiple of any chunk,
windows larger/smaller than the context, GQA ratios without a specialised
kernel, padded cache rows and back-to-back calls on one workspace.
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


def _inputs(seed, B, L, H, Hk, D, dt, kv_stride, device_rng):
    if device_rng:
        g = torch.Generator(device="cuda").manual_seed(seed)
        q = torch.randn(B, H, D, generator=g, device="cuda")
        k = torch.randn(B, L, kv_stride, generator=g, device="cuda").to(dt)
        v = torch.randn(B, L, kv_stride, generator=g, device="cuda").to(dt)
        return q, k, v
    q = synth.randn(seed, 1, (B, H, D))
    k = synth.randn(seed, 2, (B, L, kv_stride), dt)
    v = synth.randn(seed, 3, (B, L, kv_stride), dt)
    return q.cuda(), k.cuda(), v.cuda()


def run_case(dev, dtype, H, Hk, D, lens, window=0, seed=1, kv_pad=0, device_rng=False,
             workspace=None, check_heads=None):
    dt = DT[dtype]
    B, L = len(lens), max(lens)
    kv_stride = Hk * D + kv_pad
    print(f"[decode] {dtype} H{H} Hk{Hk} D{D} lens={lens[:4]}.. win={window} pad={kv_pad}",
          flush=True)
    q, k, v = _inputs(seed, B, L, H, Hk, D, dt, kv_stride, device_rng)
    lens_t = torch.tensor(lens, dtype=torch.int32, device=dev)
    scale = 1.0 / math.sqrt(D)
    out = A.attn_decode(q, k, v, lens_t, L, Hk, window=window, scale=scale,
                        kv_stride=kv_stride, seq_stride=L * kv_stride, workspace=workspace)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    qn = q.cpu().numpy()
    for b in range(B):
        kc = k[b].float().cpu().numpy()
        vc = v[b].float().cpu().numpy()
        ref = ora.attn_decode(qn[b].reshape(-1).copy(), kc, vc, lens[b] - 1, H, Hk, D, scale,
                              window=window, kv_stride=kv_stride)
        assert_close(out[b].reshape(-1), ref, what=f"b={b} len={lens[b]}")
    return out


def test_cfg1_llama_1b_f32(dev):
    run_case(dev, "f32", 32, 8, 64, [512])


def test_cfg2_qwen25_f16_4k(dev):
    run_case(dev, "f16", 12, 2, 128, [4096], seed=2)


@pytest.mark.parametrize("window", [0, 1024])
def test_cfg4_gemma3_f16_8k(dev, window):
    run_case(dev, "f16", 8, 4, 256, [8192], window=window, seed=4)


# Splits of one or two 32-key blocks, or of one 16-key block at head_dim 256
# (decode_block_kernel; f16, bf16 and the f32 cache): a last split that
# fetches only the first of its two blocks (8152), one whose second block
# ends inside the length (8100), binding windows that start off a block
# boundary, head_dim 64.
@pytest.mark.parametrize("dtype,H,Hk,D,L,window", [
    ("f16", 12, 2, 128, 8152, 0), ("bf16", 12, 2, 128, 8100, 0),
    ("f16", 12, 2, 128, 7000, 6000), ("bf16", 8, 4, 64, 2000, 1500),
    ("f16", 32, 8, 64, 2047, 0), ("bf16", 16, 2, 128, 4000, 3000),
    # head_dim 256 on 16-key splits: a binding window ending mid-block, and
    # a fetched range ending mid-block
    ("bf16", 8, 4, 256, 3000, 1000), ("f16", 16, 8, 256, 700, 0),
    # the reference's f32 cache on the block kernel (bf16 hi + lo products)
    ("f32", 12, 2, 128, 8152, 0), ("f32", 12, 2, 128, 8100, 0), ("f32", 8, 4, 64, 2000, 1500),
    ("f32", 32, 8, 64, 2047, 0), ("f32", 16, 2, 128, 4000, 3000), ("f32", 32, 8, 64, 100, 0)])
def test_block_splits(dev, dtype, H, Hk, D, L, window):
    run_case(dev, dtype, H, Hk, D, [L], window=window, seed=13)


# The reference's f32 cache past the one- and two-block splits: long
# contexts stream through decode_dma_kernel's f32 mode (f32 tiles by LDS DMA,
# bf16 hi + lo products), one split per unit when the units fill the chip
# (4-wave workgroups at head_dim 64, 2-wave at 128), windows and ragged
# batches.
@pytest.mark.parametrize("H,Hk,D,lens,window", [
    (32, 4, 128, [32768], 0),                       # cfg5's shape with an f32 cache
    (12, 2, 128, [20000], 0),
    (32, 8, 64, [16384], 0),
    (8, 4, 128, [5000], 333),
    (16, 4, 64, [9000], 4096),
    (32, 4, 128, [30000, 4100, 17000, 9000], 0),    # ragged batch, 2-wave workgroups
    (16, 8, 128, [400] * 32, 0),                    # units fill the chip: one split per unit
    (32, 8, 64, [300] * 64, 0),
])
def test_f32_cache_long(dev, H, Hk, D, lens, window):
    run_case(dev, "f32", H, Hk, D, lens, window=window, seed=14, device_rng=True)


def test_cfg5_qwen3_30b_bf16_32k(dev):
    run_case(dev, "bf16", 32, 4, 128, [32768], seed=5, device_rng=True)


def test_cfg5_ragged_batch8(dev):
    lens = synth.ragged_lengths(5, 8, 4096, 32768)
    run_case(dev, "bf16", 32, 4, 128, lens, seed=6, device_rng=True)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_dtypes_and_head_dims(dev, dtype, D):
    run_case(dev, dtype, 8, 2, D, [777], seed=7)


@pytest.mark.parametrize("L", [1, 2, 17, 63, 64, 65, 1000, 4097])
def test_lengths(dev, L):
    run_case(dev, "f16", 12, 2, 128, [L], seed=8)


@pytest.mark.parametrize("H,Hk", [(4, 4), (6, 2), (12, 4), (10, 2), (16, 1), (32, 2), (7, 7)])
def test_gqa_ratios(dev, H, Hk):
    run_case(dev, "bf16", H, Hk, 128, [300], seed=9)


@pytest.mark.parametrize("L,window", [(100, 1024), (1024, 1024), (1025, 1024), (5000, 1),
                                      (5000, 333)])
def test_windows(dev, L, window):
    run_case(dev, "f16", 8, 4, 128, [L], window=window, seed=10)


def test_padded_kv_stride(dev):
    run_case(dev, "f16", 8, 2, 128, [500], kv_pad=64, seed=11)


def test_ragged_small(dev):
    run_case(dev, "f32", 8, 2, 64, [1, 5, 300, 64, 1000], seed=12)


def test_workspace_reuse_back_to_back(dev):
    """Counters must be left at zero: repeated calls on one workspace agree."""
    ws = A.new_decode_workspace(1, 12, 2, 128, 4096)
    first = run_case(dev, "f16", 12, 2, 128, [4096], seed=13, workspace=ws)
    for _ in range(3):
        again = run_case(dev, "f16", 12, 2, 128, [4096], seed=13, workspace=ws)
        np.testing.assert_array_equal(first, again)
    run_case(dev, "f16", 12, 2, 128, [2000], seed=14, workspace=ws)


@pytest.mark.parametrize("dtype,H,Hk", [("f16", 12, 2), ("bf16", 32, 4)])
def test_workspace_sized_for_n_ctx_serves_shorter_calls(dev, dtype, H, Hk):
    """A workspace sized once for n_ctx must serve every call with a smaller
    max_len (decode passes max_len = pos + 1 each step), even where a short
    context plans more splits than a long one."""
    ws = A.new_decode_workspace(1, H, Hk, 128, 8192)
    for L in (600, 2048, 4096, 8192):
        run_case(dev, dtype, H, Hk, 128, [L], seed=15, workspace=ws)


def test_workspace_too_small_is_an_error(dev):
    q = torch.zeros(1, 12, 128, device=dev)
    k = torch.zeros(4096, 256, dtype=torch.float16, device=dev)
    lens = torch.tensor([4096], dtype=torch.int32, device=dev)
    ws = torch.zeros(16, dtype=torch.uint8, device=dev)
    with pytest.raises(A.L.UllmHipError) as e:
        A.attn_decode(q, k, k, lens, 4096, 2, workspace=ws)
    assert e.value.code == A.L.E_WORKSPACE
