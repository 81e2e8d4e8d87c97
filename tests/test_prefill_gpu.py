"""Causal prefill attention (MFMA) on the GPU against the CPU oracle.

The oracle computes every query row where that stays within a few seconds
(S*S*H*D <= 2^32), else a sample (first rows, block and tile boundaries, the
last row, random rows), for every head; at full size the
GPU result is also checked row-wise against the GPU decode kernel, the
reference's own "batched prefill == per-token" invariant
(crates/ullm-model/src/lib.rs:1348-1382).
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

DT = {"f16": torch.float16, "bf16": torch.bfloat16}


def sample_rows(S, seed, extra=24):
    rows = {0, 1, 2, 31, 32, 63, 64, 127, 128, 129, S - 2, S - 1}
    rng = np.random.default_rng(seed)
    rows |= set(int(x) for x in rng.integers(0, S, size=extra))
    return sorted(r for r in rows if 0 <= r < S)


def run_case(dev, dtype, S, H, Hk, D, start_pos=0, window=0, seed=1, rows=None):
    dt = DT[dtype]
    kv_len = start_pos + S
    print(f"[prefill] {dtype} S{S} sp{start_pos} H{H} Hk{Hk} D{D} win={window}", flush=True)
    q = synth.randn(seed, 1, (S, H * D), dt).to(dev)
    k = synth.randn(seed, 2, (kv_len, Hk * D), dt).to(dev)
    v = synth.randn(seed, 3, (kv_len, Hk * D), dt).to(dev)
    scale = 1.0 / math.sqrt(D)
    out = A.attn_prefill(q, k, v, H, Hk, D, start_pos=start_pos, window=window, scale=scale)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    if rows is None:
        # every row where the oracle stays within a few seconds, else a sample
        rows = list(range(S)) if S * S * H * D <= (1 << 32) else sample_rows(S, seed)
    ref = ora.attn_prefill(q.float().cpu().numpy(), k.float().cpu().numpy(),
                           v.float().cpu().numpy(), S, start_pos, H, Hk, D, scale,
                           window=window, rows=rows)
    assert_close(out[rows], ref[rows], what=f"rows {rows[:6]}..")
    return q, k, v, out


def test_cfg3_qwen3_4b_bf16_2048(dev):
    run_case(dev, "bf16", 2048, 32, 8, 128, seed=3)


def test_cfg4_gemma3_f16_1024_window(dev):
    """cfg4's prefill at its full size, every one of the 1024 rows and 8
    heads against the oracle."""
    run_case(dev, "f16", 1024, 8, 4, 256, window=1024, seed=4, rows=list(range(1024)))


@pytest.mark.parametrize("S,window", [(1536, 512), (700, 100), (300, 1)])
def test_window_masking(dev, S, window):
    run_case(dev, "f16", S, 8, 4, 128, window=window, seed=5)


# cfg4's local layers with the prompt longer than the window (S > W), on the
# head_dim-256 kernel: masking at both ends of every row's key range.
@pytest.mark.parametrize("dtype,S,start_pos,window", [
    ("f16", 1536, 0, 1024), ("f16", 1536, 0, 512), ("bf16", 700, 300, 333)])
def test_head_dim_256_binding_window(dev, dtype, S, start_pos, window):
    run_case(dev, dtype, S, 8, 4, 256, start_pos=start_pos, window=window, seed=11)


def p16_geometry(S, H, Hk, start_pos=0, window=0):
    """(key streams, heads per workgroup, value split) of prefill16_kernel
    for a head_dim-256 prompt: the rule of prefill16_plan / p16_hw
    (prefill16.hip), restated to show which workgroup geometry a test case
    runs."""
    kv_mul = H // Hk

    def hw_of(nws):
        hw = 1
        while hw < nws and hw < 4 and kv_mul % (hw * 2) == 0:
            hw *= 2
        return hw
    hw1 = hw_of(8)
    grid1 = (S + 128 // hw1 - 1) // (128 // hw1) * (H // hw1)
    binding = 0 < window < start_pos + S
    ks = 2 if grid1 < 256 or (grid1 == 256 and not binding) else 1
    hw = hw_of(8 // ks)
    ur = 16 * (8 // ks) // hw
    ds = 2 if ks == 2 and (S + ur - 1) // ur * (H // hw) * 2 <= 256 else 1
    return ks, hw, ds


# head_dim 256 (prefill16_kernel): every workgroup geometry -- one or two key
# streams times 4, 2 or 1 heads per workgroup (kv_mul 8/4, 2, 3 and 1) --
# with windows, start_pos and lengths that end inside a unit.
P16_CASES = [
    ("f16", 4096, 8, 4, 0, 1024),    # cfg4's local layers at S=4096
    ("bf16", 4096, 8, 4, 0, 0),      # and its global layer
    ("f16", 1000, 16, 4, 37, 200),
    ("bf16", 777, 32, 4, 0, 0),
    ("bf16", 1024, 16, 16, 100, 128),
    ("f16", 2048, 12, 4, 0, 256),
    ("bf16", 3000, 16, 8, 500, 0),
    ("f16", 600, 32, 16, 0, 100),
    ("f16", 1024, 8, 4, 0, 1024),    # cfg4 as configured
    ("bf16", 333, 8, 1, 17, 0),
    ("f16", 257, 6, 2, 3, 40),
    ("bf16", 2500, 32, 8, 0, 0),
    ("f16", 1, 8, 4, 0, 0),
    ("bf16", 17, 16, 16, 5, 0),
    ("f16", 2100, 16, 16, 0, 0)]


@pytest.mark.parametrize("dtype,S,H,Hk,start_pos,window", P16_CASES)
def test_head_dim_256_geometries(dev, dtype, S, H, Hk, start_pos, window):
    run_case(dev, dtype, S, H, Hk, 256, start_pos=start_pos, window=window, seed=12)


def prefill128_kernel(S, H, Hk, start_pos=0, window=0):
    """Which kernel a head_dim-128 prompt runs: prefill16 when prefill4's
    causal pairs would be 128 or fewer (the rule in prefill.hip), restated."""
    kv_mul = H // Hk
    hw = 4 if kv_mul % 4 == 0 else (2 if kv_mul % 2 == 0 else 1)
    ng = (S + 32 * (4 // hw) - 1) // (32 * (4 // hw))
    pairs = (H // kv_mul) * (kv_mul // hw) * ((ng + 1) // 2)
    paired = not (0 < window < start_pos + S)
    return "prefill16" if paired and pairs <= 128 else ("prefill4" if paired else "prefill2")


# head_dim 128 on both sides of the prefill16 / prefill4 rule, with a
# chunk's start_pos and a GQA ratio that is not a power of two.
P128_CASES = [("bf16", 2048, 12, 2, 0), ("f16", 1024, 32, 8, 0), ("bf16", 1536, 32, 8, 0),
              ("f16", 777, 16, 2, 100), ("bf16", 300, 6, 2, 0), ("f16", 2048, 32, 8, 0)]


@pytest.mark.parametrize("dtype,S,H,Hk,start_pos", P128_CASES)
def test_head_dim_128_both_kernels(dev, dtype, S, H, Hk, start_pos):
    run_case(dev, dtype, S, H, Hk, 128, start_pos=start_pos, seed=21)


def test_head_dim_128_cases_cover_both_kernels():
    seen = {prefill128_kernel(S, H, Hk, sp) for (_, S, H, Hk, sp) in P128_CASES}
    assert {"prefill16", "prefill4"} <= seen, seen


def test_head_dim_256_geometries_covered():
    """The cases above reach both key-stream counts with 4, 2 and 1 heads per
    workgroup, and the value split with two key streams at each head count."""
    seen = {p16_geometry(S, H, Hk, sp, w) for (_, S, H, Hk, sp, w) in P16_CASES}
    assert {(1, 4, 1), (1, 2, 1), (1, 1, 1), (2, 4, 1), (2, 2, 1), (2, 1, 1),
            (2, 4, 2), (2, 2, 2), (2, 1, 2)} <= seen, seen


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_dtypes_head_dims(dev, dtype, D):
    run_case(dev, dtype, 200, 4, 2, D, seed=6, rows=list(range(200)))


@pytest.mark.parametrize("S", [1, 2, 31, 33, 127, 129, 257])
def test_ragged_lengths(dev, S):
    run_case(dev, "bf16", S, 8, 2, 128, seed=7, rows=list(range(S)))


@pytest.mark.parametrize("start_pos", [1, 100, 1000])
def test_chunked_prefill_start_pos(dev, start_pos):
    run_case(dev, "bf16", 300, 8, 4, 128, start_pos=start_pos, seed=8)


@pytest.mark.parametrize("H,Hk", [(6, 1), (12, 2), (8, 8), (10, 5)])
def test_gqa(dev, H, Hk):
    run_case(dev, "f16", 260, H, Hk, 64, seed=9, rows=list(range(260)))


def test_prefill_rows_match_decode_full_size(dev):
    """cfg3 at full size: every 97th row equals the decode kernel at that pos."""
    S, H, Hk, D = 2048, 32, 8, 128
    q, k, v, out = run_case(dev, "bf16", S, H, Hk, D, seed=10, rows=[0, S - 1])
    rows = list(range(0, S, 97)) + [S - 1]
    qd = q[rows].float().view(len(rows), H, D).contiguous()
    lens = torch.tensor([r + 1 for r in rows], dtype=torch.int32, device=dev)
    dec = A.attn_decode(qd, k, v, lens, S, Hk, seq_stride=0)
    torch.cuda.synchronize()
    assert_close(out[rows], dec.view(len(rows), -1).cpu().numpy(), what="prefill vs decode")


def run_f32(dev, S, H, Hk, D, start_pos=0, window=0, seed=1, rows=None, qk_scale=1.0):
    """The f32-cache prefill (Q.K on bf16 hi + lo halves, V and P in f16)
    against the f32 oracle on the same f32 inputs (no input rounding)."""
    kv_len = start_pos + S
    print(f"[prefill f32] S{S} sp{start_pos} H{H} Hk{Hk} D{D} win={window} x{qk_scale}", flush=True)
    q = synth.randn(seed, 1, (S, H * D)) * qk_scale
    k = synth.randn(seed, 2, (kv_len, Hk * D)) * qk_scale
    v = synth.randn(seed, 3, (kv_len, Hk * D))
    scale = 1.0 / math.sqrt(D)
    out = A.attn_prefill(q.to(dev), k.to(dev), v.to(dev), H, Hk, D, start_pos=start_pos,
                         window=window, scale=scale)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    if rows is None:
        # every row where the oracle stays within a few seconds, else a sample
        rows = list(range(S)) if S * S * H * D <= (1 << 32) else sample_rows(S, seed)
    ref = ora.attn_prefill(q.numpy(), k.numpy(), v.numpy(), S, start_pos, H, Hk, D, scale,
                           window=window, rows=rows)
    assert_close(out[rows], ref[rows], what=f"f32 rows {rows[:6]}..")


def test_f32_cache_cfg3_shape(dev):
    run_f32(dev, 2048, 32, 8, 128, seed=21)


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("S,start_pos,window", [(1, 0, 0), (33, 0, 0), (300, 0, 0),
                                                 (200, 100, 0), (700, 0, 100)])
def test_f32_cache_shapes(dev, D, S, start_pos, window):
    run_f32(dev, S, 8, 2, D, start_pos=start_pos, window=window, seed=22,
            rows=list(range(S)))


@pytest.mark.parametrize("D", [128, 256])
def test_f32_cache_sharp_scores(dev, D):
    """Scores three times sharper than N(0,1) Q/K give (std 9): Q.K in plain
    f16 or bf16 would miss the tolerance here; the hi + lo split does not."""
    run_f32(dev, 512, 8, 2, D, seed=23, rows=list(range(0, 512, 3)), qk_scale=3.0)


@pytest.mark.parametrize("H,Hk", [(6, 1), (8, 8), (10, 5)])
def test_f32_cache_gqa(dev, H, Hk):
    run_f32(dev, 130, H, Hk, 64, seed=24, rows=list(range(130)))


# Workgroup geometries of the f32 kernel: hw heads of one kv head x 4/hw row
# blocks per unit (8:1 -> two head groups per kv head; 3:1 -> one head over
# four row blocks, whose later rows start their windows later).
@pytest.mark.parametrize("H,Hk,D,S,start_pos,window", [
    (16, 2, 128, 257, 0, 0), (16, 2, 64, 190, 60, 70),
    (6, 2, 128, 300, 0, 90), (6, 2, 64, 129, 31, 0),
    (4, 2, 128, 250, 17, 45)])
def test_f32_cache_workgroup_geometries(dev, H, Hk, D, S, start_pos, window):
    run_f32(dev, S, H, Hk, D, start_pos=start_pos, window=window, seed=25,
            rows=list(range(S)))


# The f32 cache at head_dim 128 runs prefill16_kernel's f32 mode: its
# one- and two-stream geometries with 4, 2 and 1 heads per workgroup.
F32_P16_CASES = [(2048, 16, 8, 0, 0), (3000, 12, 4, 0, 0), (2048, 16, 8, 64, 500),
                 (1100, 32, 4, 0, 0), (400, 12, 4, 10, 0), (513, 8, 2, 0, 0)]


@pytest.mark.parametrize("S,H,Hk,start_pos,window", F32_P16_CASES)
def test_f32_cache_prefill16_geometries(dev, S, H, Hk, start_pos, window):
    run_f32(dev, S, H, Hk, 128, start_pos=start_pos, window=window, seed=26)


# head_dim 256 over an f32 cache: one key stream, the value columns split
# over two workgroups, 4, 2 and 1 heads per workgroup; cfg4's shape.
@pytest.mark.parametrize("S,H,Hk,start_pos,window", [
    (1024, 8, 4, 0, 1024), (700, 16, 4, 100, 300), (257, 6, 2, 3, 0), (130, 4, 4, 0, 0)])
def test_f32_cache_head_dim_256(dev, S, H, Hk, start_pos, window):
    run_f32(dev, S, H, Hk, 256, start_pos=start_pos, window=window, seed=27)


def test_f32_cache_geometries_covered():
    seen = {p16_geometry(S, H, Hk, sp, w)[:2] for (S, H, Hk, sp, w) in F32_P16_CASES}
    assert {(1, 4), (1, 2), (1, 1), (2, 4), (2, 2), (2, 1)} <= seen, seen


def test_cfg3_pipeline_norm_rope_all_rows(dev):
    """cfg3 as the benchmark configures it, end to end at full size: raw f32 Q/K/V
    ~ N(0,1) -> fused append (per-head RMSNorm with unit weights, eps 1e-6,
    NeoX RoPE theta 1e6, bf16 q and cache) -> causal prefill, every one of the
    2048 rows of all 32 heads against the oracle (lib.rs:1035-1058 then
    :1061-1087).

    Two comparisons:
     * the prefill kernel against the oracle's prefill on the very bf16
       values the GPU append produced (same inputs, the attention tolerance);
     * the whole GPU pipeline against the oracle's pipeline, whose prepared
       q/K/V are rounded to bf16 the same way (the RMS sums differ in order,
       so single values may round one bf16 ulp apart, and fewer than 1 %
       may differ at all; held to the same tolerance)."""
    S, H, Hk, D, theta = 2048, 32, 8, 128, 1e6
    print(f"[prefill] cfg3 pipeline S{S} H{H} Hk{Hk} D{D}", flush=True)
    q = synth.randn(31, 1, (S, H * D))
    k = synth.randn(31, 2, (S, Hk * D))
    v = synth.randn(31, 3, (S, Hk * D))
    ones = torch.ones(D)
    cs = A.rope_table(S, D, theta, device=dev)
    kc = torch.zeros(S, Hk * D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    qb = A.qkv_append(q.to(dev), k.to(dev), v.to(dev), kc, vc, cs, start_pos=0, n_head=H,
                      n_kv_head=Hk, head_dim=D, rotary_dim=D, neox=True, q_norm=ones.to(dev),
                      k_norm=ones.to(dev), eps=1e-6, q_dtype=torch.bfloat16)
    scale = 1.0 / math.sqrt(D)
    out = A.attn_prefill(qb, kc, vc, H, Hk, D, scale=scale)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    gq, gk, gv = (t.float().cpu().numpy() for t in (qb, kc, vc))
    ref = ora.attn_prefill(gq, gk, gv, S, 0, H, Hk, D, scale)
    assert_close(out, ref, what="cfg3 prefill on the GPU-prepared inputs")

    okc = np.zeros((S, Hk * D), np.float32)
    ovc = np.zeros_like(okc)
    on = ones.numpy().copy()
    oq = ora.qkv_append(q.numpy().copy(), k.numpy().copy(), v.numpy().copy(), 0, H, Hk, D, D,
                        theta, True, okc, ovc, q_norm=on, k_norm=on, eps=1e-6)
    r16 = lambda x: torch.from_numpy(x).to(torch.bfloat16).float().numpy()  # noqa: E731
    oq, okc, ovc = r16(oq), r16(okc), r16(ovc)
    # One bf16 ulp of a value in [1, 2) is 2^-7; below 1 the bound is absolute
    # (RoPE's a*cos - b*sin can cancel, so a one-ulp difference in the normed
    # input is no longer one ulp of a small output).
    for name, got, want in (("q", gq, oq), ("k", gk, okc), ("v", gv, ovc)):
        d = np.abs(got - want) / np.maximum(np.abs(want), 1.0)
        assert d.max() <= 2.0**-7, f"append {name}: {d.max():.3e} > one bf16 ulp"
        assert np.mean(got != want) < 0.01, f"append {name}: {np.mean(got != want):.3%} differ"
    ref2 = ora.attn_prefill(oq, okc, ovc, S, 0, H, Hk, D, scale)
    assert_close(out, ref2, what="cfg3 pipeline vs the oracle pipeline")


@pytest.mark.parametrize("dtype,D", [("bf16", 128), ("f16", 256)])
def test_q_past_the_call_limit_runs_in_chunks(dev, monkeypatch, dtype, D):
    """attn_prefill splits a q at or above PREFILL_Q_MAX_BYTES into row chunks
    at increasing start_pos (the limit is lowered here to 100 rows, so a
    300-row prompt at start_pos 50 runs as 100 + 100 + 100 rows): every row
    against the oracle, and against the one-call result within the
    attention tolerance (the chunks run other workgroup plans)."""
    S, sp, H, Hk = 300, 50, 8, 2
    dt = {"bf16": torch.bfloat16, "f16": torch.float16}[dtype]
    q = synth.randn(31, 1, (S, H * D), dt).to(dev)
    k = synth.randn(31, 2, (sp + S, Hk * D), dt).to(dev)
    v = synth.randn(31, 3, (sp + S, Hk * D), dt).to(dev)
    whole = A.attn_prefill(q, k, v, H, Hk, D, start_pos=sp, window=120)
    monkeypatch.setattr(A, "PREFILL_Q_MAX_BYTES", 100 * H * D * q.element_size())
    chunked = A.attn_prefill(q, k, v, H, Hk, D, start_pos=sp, window=120)
    torch.cuda.synchronize()
    rows = list(range(S))
    ref = ora.attn_prefill(q.float().cpu().numpy(), k.float().cpu().numpy(),
                           v.float().cpu().numpy(), S, sp, H, Hk, D, 1.0 / math.sqrt(D),
                           window=120, rows=rows)
    assert_close(chunked.cpu().numpy(), ref, what="chunked")
    assert_close(chunked.cpu().numpy(), whole.cpu().numpy(), what="chunked vs one call")


@pytest.mark.parametrize("dtype,S,H,Hk", [("bf16", 300, 8, 2), ("bf16", 2048, 32, 8), ("f32", 300, 8, 2)])
def test_v_beyond_f16_range_fails_loudly(dev, dtype, S, H, Hk):
    """P.V runs on f16 operands, so a bf16 or f32 cache holding |V| >= 65504
    is outside the kernels' range (include/ullm_hip.h).  Pinned here: V up
    to 6e4 stays within tolerance (relative to the output's scale), and one
    V element of 1e5 never yields a wrong finite value: every output equals
    the oracle or is non-finite (the overflowed element reaches the rows
    whose key tiles contain it as inf or NaN)."""
    D = 128
    dt = {"bf16": torch.bfloat16, "f32": torch.float32}[dtype]
    print(f"[prefill] |V| edge {dtype} S{S} H{H} Hk{Hk}", flush=True)
    q = synth.randn(31, 1, (S, H * D), dt).to(dev)
    k = synth.randn(31, 2, (S, Hk * D), dt).to(dev)
    v0 = synth.randn(31, 3, (S, Hk * D), torch.float32)
    scale = 1.0 / math.sqrt(D)
    rows = sample_rows(S, 31)
    for big, loud in ((6.0e4, False), (1.0e5, True)):
        v = v0.clone()
        v[S // 3, 5] = big          # kv head 0, column 5
        v[2 * S // 3, D + 17] = -big  # kv head 1, column 17
        v = v.to(dt).to(dev)
        out = A.attn_prefill(q, k, v, H, Hk, D, scale=scale)
        torch.cuda.synchronize()
        o = out.cpu().numpy()
        ref = ora.attn_prefill(q.float().cpu().numpy(), k.float().cpu().numpy(),
                               v.float().cpu().numpy(), S, 0, H, Hk, D, scale, rows=rows)
        o, ref = o[rows], ref[rows]
        if not loud:
            s = np.abs(ref).max()
            assert np.all(np.isfinite(o))
            assert np.abs(o - ref).max() <= 2e-3 * s
            assert np.linalg.norm(o - ref) <= 1e-3 * np.linalg.norm(ref)
        else:
            fin = np.isfinite(o)
            assert not fin.all(), "an element past f16's range must not vanish silently"
            err = np.abs(np.where(fin, o, 0.0) - np.where(fin, ref, 0.0))
            tol = 2e-3 * np.maximum(1.0, np.abs(ref))
            assert np.all(err <= tol), "a finite output differs from the oracle"
