"""Shared checks for the parity tests."""
from __future__ import annotations

import numpy as np

# Tolerance of the attention path against the f32 CPU oracle on the same
# rounded inputs: max-abs <= 2e-3 and rel-L2 <= 1e-3.
MAX_ABS = 2e-3
REL_L2 = 1e-3


def errors(out, ref):
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    d = out - ref
    max_abs = float(np.max(np.abs(d))) if d.size else 0.0
    rel = float(np.linalg.norm(d) / max(np.linalg.norm(ref), 1e-30)) if d.size else 0.0
    return max_abs, rel


def assert_close(out, ref, max_abs=MAX_ABS, rel_l2=REL_L2, what=""):
    out = np.asarray(out)
    assert np.all(np.isfinite(out)), f"{what}: non-finite output"
    ma, rl = errors(out, ref)
    assert ma <= max_abs and rl <= rel_l2, f"{what}: max-abs {ma:.3e} rel-L2 {rl:.3e}"
    return ma, rl
