"""Writes the golden fixtures of the attention path (tests/golden/*.npz).

Inputs come from the seeded generator (ullm_amd.synth); expected outputs come
from the CPU oracle (oracle/ref_attention.c) and each is checked here against
an independent f64 brute force before it is written.  The reference ships no
attention fixtures, so these are this build's own vectors: they pin the oracle
against regressions and give the GPU tests fixed cases.

    python tests/golden/make_golden.py
"""
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as ora  # noqa: E402
from ullm_amd import synth  # noqa: E402

DTS = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def raw(t):
    """Storage bits of a CPU tensor (f32 as float32, 16-bit types as uint16)."""
    if t.dtype == torch.float32:
        return t.numpy().copy()
    return t.view(torch.int16).numpy().view(np.uint16).copy()


def f64_rows(q, kc, vc, positions, window, H, Hk, D, scale):
    out = np.zeros((len(positions), H * D))
    for i, pos in enumerate(positions):
        st = ora.lib().ora_window_start(pos, window)
        for h in range(H):
            j = h // (H // Hk)
            s = kc[st:pos + 1, j * D:(j + 1) * D].astype(np.float64) @ q[i, h * D:(h + 1) * D]
            p = np.exp((s - s.max()) * scale)
            out[i, h * D:(h + 1) * D] = (p / p.sum()) @ vc[st:pos + 1, j * D:(j + 1) * D]
    return out


def decode_case(name, seed, dt, H, Hk, D, lens, window):
    B, L = len(lens), max(lens)
    q = synth.randn(seed, 1, (B, H, D))
    k = synth.randn(seed, 2, (B, L, Hk * D), DTS[dt])
    v = synth.randn(seed, 3, (B, L, Hk * D), DTS[dt])
    scale = 1 / math.sqrt(D)
    out = np.zeros((B, H * D), np.float32)
    for b in range(B):
        kc, vc = k[b].float().numpy(), v[b].float().numpy()
        out[b] = ora.attn_decode(q[b].reshape(-1).numpy().copy(), kc, vc, lens[b] - 1, H, Hk,
                                 D, scale, window=window)
        ref = f64_rows(q[b].reshape(1, -1).numpy().astype(np.float64), kc, vc, [lens[b] - 1],
                       window, H, Hk, D, scale)
        assert np.abs(out[b] - ref[0]).max() < 1e-5, name
    np.savez_compressed(os.path.join(HERE, name + ".npz"), kind="decode", dtype=dt, q=q.numpy(),
             k=raw(k), v=raw(v), lens=np.array(lens, np.int32),
             shape=np.array([H, Hk, D, window], np.int32), scale=np.float32(scale), out=out)


def prefill_case(name, seed, dt, S, sp, H, Hk, D, window):
    q = synth.randn(seed, 1, (S, H * D), DTS[dt])
    k = synth.randn(seed, 2, (sp + S, Hk * D), DTS[dt])
    v = synth.randn(seed, 3, (sp + S, Hk * D), DTS[dt])
    scale = 1 / math.sqrt(D)
    qf, kc, vc = q.float().numpy(), k.float().numpy(), v.float().numpy()
    out = ora.attn_prefill(qf, kc, vc, S, sp, H, Hk, D, scale, window=window)
    ref = f64_rows(qf.astype(np.float64), kc, vc, [sp + s for s in range(S)], window, H, Hk, D,
                   scale)
    assert np.abs(out - ref).max() < 1e-5, name
    np.savez_compressed(os.path.join(HERE, name + ".npz"), kind="prefill", dtype=dt, q=raw(q), k=raw(k),
             v=raw(v), shape=np.array([S, sp, H, Hk, D, window], np.int32),
             scale=np.float32(scale), out=out)


def append_case(name, seed, rows, sp, H, Hk, D, rd, neox, theta):
    q = synth.randn(seed, 1, (rows, H * D)).numpy()
    k = synth.randn(seed, 2, (rows, Hk * D)).numpy()
    v = synth.randn(seed, 3, (rows, Hk * D)).numpy()
    qn = (synth.randn(seed, 4, (D,)) * 0.2 + 1).numpy()
    kn = (synth.randn(seed, 5, (D,)) * 0.2 + 1).numpy()
    kb = synth.randn(seed, 6, (Hk * D,)).numpy()
    kc = np.zeros((sp + rows, Hk * D), np.float32)
    vc = np.zeros_like(kc)
    qo = ora.qkv_append(q, k, v, sp, H, Hk, D, rd, theta, neox, kc, vc, k_bias=kb, q_norm=qn,
                        k_norm=kn, eps=1e-6)
    # independent check of one head: bias, rmsnorm, rotation by complex phase
    x = (k[0, :D] + kb[:D]).astype(np.float64)
    x = x / math.sqrt((x * x).mean() + 1e-6) * kn
    ang = sp * theta ** (-2.0 * np.arange(rd // 2) / rd)
    if neox:
        z = (x[:rd // 2] + 1j * x[rd // 2:rd]) * np.exp(1j * ang)
        want = np.concatenate([z.real, z.imag, x[rd:]])
    else:
        z = (x[0:rd:2] + 1j * x[1:rd:2]) * np.exp(1j * ang)
        want = x.copy()
        want[0:rd:2], want[1:rd:2] = z.real, z.imag
    assert np.abs(kc[sp, :D] - want).max() < 1e-4, name
    np.savez_compressed(os.path.join(HERE, name + ".npz"), kind="append", q=q, k=k, v=v, q_norm=qn,
             k_norm=kn, k_bias=kb, shape=np.array([rows, sp, H, Hk, D, rd, int(neox)], np.int32),
             theta=np.float32(theta), q_out=qo, k_cache=kc, v_cache=vc)


def main():
    decode_case("decode_f32_h8k2d64", 101, "f32", 8, 2, 64, [64], 0)
    decode_case("decode_f16_h12k2d128", 102, "f16", 12, 2, 128, [100], 0)
    decode_case("decode_bf16_h4k1d256_win", 103, "bf16", 4, 1, 256, [96], 40)
    decode_case("decode_bf16_ragged_b3", 104, "bf16", 8, 1, 128, [1, 37, 90], 0)
    prefill_case("prefill_bf16_s64_sp16", 201, "bf16", 64, 16, 4, 2, 128, 0)
    prefill_case("prefill_f16_s48_win", 202, "f16", 48, 0, 4, 2, 64, 24)
    append_case("append_neox_d128", 301, 3, 9, 4, 2, 128, 128, True, 1e6)
    append_case("append_interleaved_partial_d64", 302, 2, 0, 2, 1, 64, 32, False, 1e4)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
