"""Seeded synthetic inputs: SplitMix64 -> Box-Muller N(0, 1) -> dtype.

SplitMix64 is the generator the reference's sampler uses
(crates/ullm-model/src/sample.rs:136-148); Box-Muller turns pairs of its
53-bit uniforms into normals.  Every tensor gets its own sub-stream
(seed, tag), so the same (seed, tag, shape) always yields the same values on
any machine.  Values are rounded to the target dtype (round-to-nearest-even)
before either the GPU path or the CPU oracle sees them.
"""
from __future__ import annotations

import numpy as np
import torch

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int) -> np.ndarray:
    """The first n outputs of SplitMix64 started from state `seed`."""
    with np.errstate(over="ignore"):
        i = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def normal(seed: int, n: int) -> np.ndarray:
    """n standard normals (f32) from one SplitMix64 stream."""
    m = (n + 1) // 2
    u = splitmix64(seed, 2 * m)
    u1 = ((u[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0**-53  # (0, 1]
    u2 = (u[1::2] >> np.uint64(11)).astype(np.float64) * 2.0**-53  # [0, 1)
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return z[:n].astype(np.float32)


def substream(seed: int, tag: int) -> int:
    """Seed of the independent stream `tag` under `seed`."""
    return int(splitmix64((seed << 16) ^ tag, 1)[0])


def randn(seed: int, tag: int, shape, dtype=torch.float32) -> torch.Tensor:
    """CPU tensor of N(0,1) values rounded to `dtype` (RNE)."""
    n = int(np.prod(shape)) if len(shape) else 1
    t = torch.from_numpy(normal(substream(seed, tag), n)).view(*shape)
    return t.to(dtype)


def ragged_lengths(seed: int, batch: int, lo: int, hi: int) -> list[int]:
    """Per-sequence lengths uniform in [lo, hi] (lo + u64 % (hi-lo+1))."""
    u = splitmix64(substream(seed, 99), batch)
    return [int(lo + int(x) % (hi - lo + 1)) for x in u]
