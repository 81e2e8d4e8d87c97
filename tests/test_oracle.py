"""Pins of the CPU oracle (oracle/ref_attention.c) -- CPU only.

The reference ships no attention tests or fixtures, so each oracle function
is pinned by checks that a plausible mistake (dropped term, wrong sign or
index, transposed operand, wrong GQA grouping) would fail: library routines
(numpy/torch conversions, torch SDPA), closed forms, invariants and brute
force in f64.  Reference tests restated here: math.rs:175-181 (rmsnorm unit
RMS) and math.rs:184-189 (softmax is a distribution).
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as ora

RNG = np.random.default_rng(1234)


def f64_attention(q, k, v, scale):
    """Textbook softmax attention of one query in f64."""
    s = (k.astype(np.float64) @ q.astype(np.float64)) * scale
    s -= s.max()
    p = np.exp(s)
    p /= p.sum()
    return p @ v.astype(np.float64)


# --- dtype widening (crates/ullm-core/src/dequant.rs:15-31, :90-94) -------------

def test_f16_widening_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    got = ora.widen(bits, 1)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_bf16_widening_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    got = ora.widen(bits, 2)
    want = torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).float().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


# --- softmax / rmsnorm (math.rs:82-100) ---------------------------------------

def test_softmax_reference_case():
    y = ora.softmax(np.array([1.0, 2.0, 3.0], np.float32))
    assert abs(float(y.sum()) - 1.0) < 1e-6 and y[2] > y[1] > y[0]


def test_softmax_matches_f64_and_shift_invariance():
    # multiples of 1/64: x + 64 and x - max are exact in f32
    x = (np.round(RNG.standard_normal(257) * 5 * 64) / 64).astype(np.float32)
    y = ora.softmax(x)
    e = np.exp(x.astype(np.float64) - x.max())
    np.testing.assert_allclose(y, e / e.sum(), rtol=2e-5, atol=1e-12)
    # the max subtraction makes a constant shift exact when the shift is exact
    np.testing.assert_array_equal(ora.softmax(x + np.float32(64.0)), y)


def test_rmsnorm_reference_case():
    y = ora.rmsnorm(np.array([1, 2, 3, 4], np.float32), np.ones(4, np.float32), 0.0)
    assert abs(math.sqrt(float((y.astype(np.float64) ** 2).mean())) - 1.0) < 1e-5


def test_rmsnorm_weight_and_scale():
    x = RNG.standard_normal(128).astype(np.float32)
    w = RNG.standard_normal(128).astype(np.float32)
    one = ora.rmsnorm(x, np.ones(128, np.float32), 1e-6)
    # y = (x*inv)*w: the unit-weight result times w, bit for bit
    np.testing.assert_array_equal(ora.rmsnorm(x, w, 1e-6), one * w)
    np.testing.assert_allclose(ora.rmsnorm(x * 4, np.ones(128, np.float32), 0.0),
                               ora.rmsnorm(x, np.ones(128, np.float32), 0.0), rtol=1e-6)
    ms = float((x.astype(np.float64) ** 2).mean())
    np.testing.assert_allclose(one, x / math.sqrt(ms + 1e-6), rtol=2e-6)


# --- RoPE (math.rs:116-161) -----------------------------------------------------

@pytest.mark.parametrize("neox", [True, False])
def test_rope_position_zero_is_identity(neox):
    v = RNG.standard_normal(3 * 64).astype(np.float32)
    np.testing.assert_array_equal(ora.rope(v, 3, 64, 64, 0, 1e4, neox), v)


@pytest.mark.parametrize("neox", [True, False])
def test_rope_matches_complex_rotation(neox):
    hd, rd, pos, theta = 128, 96, 777, 1e6
    v = RNG.standard_normal(hd).astype(np.float32)
    y = ora.rope(v, 1, hd, rd, pos, theta, neox)
    half = rd // 2
    i = np.arange(half)
    ang = pos * theta ** (-2.0 * i / rd)
    if neox:
        z = (v[:half] + 1j * v[half:rd]) * np.exp(1j * ang)
        want = np.concatenate([z.real, z.imag, v[rd:]])
    else:
        z = (v[0:rd:2] + 1j * v[1:rd:2]) * np.exp(1j * ang)
        want = v.astype(np.float64).copy()
        want[0:rd:2], want[1:rd:2] = z.real, z.imag
    np.testing.assert_allclose(y, want, rtol=0, atol=5e-4)  # f32 angles at pos 777
    np.testing.assert_array_equal(y[rd:], v[rd:])  # partial rotary passes through


def test_rope_neox_is_interleaved_on_permuted_dims():
    hd = 64
    v = RNG.standard_normal(hd).astype(np.float32)
    perm = np.empty(hd, np.int64)
    perm[0::2], perm[1::2] = np.arange(hd // 2), np.arange(hd // 2) + hd // 2
    a = ora.rope(v, 1, hd, hd, 513, 1e4, True)[perm]
    b = ora.rope(v[perm].copy(), 1, hd, hd, 513, 1e4, False)
    np.testing.assert_array_equal(a, b)


def test_rope_relative_position():
    hd, theta = 64, 1e4
    q = RNG.standard_normal(hd).astype(np.float32)
    k = RNG.standard_normal(hd).astype(np.float32)
    d1 = float(ora.rope(q, 1, hd, hd, 40, theta, True) @ ora.rope(k, 1, hd, hd, 30, theta, True))
    d2 = float(ora.rope(q, 1, hd, hd, 110, theta, True) @ ora.rope(k, 1, hd, hd, 100, theta, True))
    assert abs(d1 - d2) < 1e-3 * (1 + abs(d1))
    n0 = np.linalg.norm(q)
    assert abs(np.linalg.norm(ora.rope(q, 1, hd, hd, 12345, theta, True)) - n0) < 1e-4 * n0


# --- attention (lib.rs:911-938, :1061-1087, :1180-1208) ---------------------------

def _cache(L, Hk, D, seed):
    r = np.random.default_rng(seed)
    return (r.standard_normal((L, Hk * D)).astype(np.float32),
            r.standard_normal((L, Hk * D)).astype(np.float32))


@pytest.mark.parametrize("H,Hk,D,L", [(4, 2, 16, 9), (6, 3, 8, 33), (8, 8, 32, 100)])
def test_decode_matches_f64_brute_force(H, Hk, D, L):
    kc, vc = _cache(L, Hk, D, H * L)
    q = RNG.standard_normal(H * D).astype(np.float32)
    scale = 1 / math.sqrt(D)
    out = ora.attn_decode(q, kc, vc, L - 1, H, Hk, D, scale)
    kv_mul = H // Hk
    for h in range(H):
        j = h // kv_mul
        want = f64_attention(q[h * D:(h + 1) * D], kc[:, j * D:(j + 1) * D],
                             vc[:, j * D:(j + 1) * D], scale)
        np.testing.assert_allclose(out[h * D:(h + 1) * D], want, rtol=1e-5, atol=1e-6)


def test_decode_matches_torch_sdpa_gqa_grouping():
    H, Hk, D, L = 12, 2, 64, 70
    kc, vc = _cache(L, Hk, D, 5)
    q = RNG.standard_normal(H * D).astype(np.float32)
    out = ora.attn_decode(q, kc, vc, L - 1, H, Hk, D, 1 / math.sqrt(D))
    # contiguous groups: head h uses kv head h // (H/Hk)  -> repeat_interleave
    K = torch.from_numpy(kc).view(L, Hk, D).transpose(0, 1).repeat_interleave(H // Hk, 0)
    V = torch.from_numpy(vc).view(L, Hk, D).transpose(0, 1).repeat_interleave(H // Hk, 0)
    Q = torch.from_numpy(q).view(H, 1, D)
    ref = torch.nn.functional.scaled_dot_product_attention(Q.double(), K.double(), V.double())
    np.testing.assert_allclose(out, ref.reshape(-1).numpy(), rtol=1e-5, atol=1e-6)


def test_decode_closed_forms():
    D, Hk, H = 16, 2, 4
    kc, vc = _cache(50, Hk, D, 9)
    q = RNG.standard_normal(H * D).astype(np.float32)
    # a single key: softmax is exactly 1 -> out = V[0]
    out = ora.attn_decode(q, kc, vc, 0, H, Hk, D, 0.25)
    for h in range(H):
        j = h // 2
        np.testing.assert_array_equal(out[h * D:(h + 1) * D], vc[0, j * D:(j + 1) * D])
    # q = 0 -> uniform weights -> mean of the visible V rows
    out = ora.attn_decode(np.zeros(H * D, np.float32), kc, vc, 49, H, Hk, D, 0.25, window=20)
    want = vc[30:50].astype(np.float64).mean(0)
    for h in range(H):
        j = h // 2
        np.testing.assert_allclose(out[h * D:(h + 1) * D], want[j * D:(j + 1) * D], atol=1e-6)


def test_window_equals_truncated_cache():
    H, Hk, D, L, W = 4, 2, 32, 300, 64
    kc, vc = _cache(L, Hk, D, 11)
    q = RNG.standard_normal(H * D).astype(np.float32)
    a = ora.attn_decode(q, kc, vc, L - 1, H, Hk, D, 0.17, window=W)
    b = ora.attn_decode(q, kc[L - W:].copy(), vc[L - W:].copy(), W - 1, H, Hk, D, 0.17)
    np.testing.assert_array_equal(a, b)
    assert ora.lib().ora_window_start(99, 100) == 0 and ora.lib().ora_window_start(100, 100) == 1


@pytest.mark.parametrize("window", [0, 37])
def test_prefill_row_equals_decode(window):
    """The reference's prefill-check invariant (lib.rs:1348-1382): batched
    prefill row s equals per-token decode at pos = start_pos + s."""
    H, Hk, D, S, sp = 6, 2, 32, 50, 13
    kc, vc = _cache(sp + S, Hk, D, 3)
    q = RNG.standard_normal((S, H * D)).astype(np.float32)
    out = ora.attn_prefill(q, kc, vc, S, sp, H, Hk, D, 0.2, window=window)
    for s in (0, 1, 17, S - 1):
        d = ora.attn_decode(q[s].copy(), kc, vc, sp + s, H, Hk, D, 0.2, window=window)
        np.testing.assert_array_equal(out[s], d)
    part = ora.attn_prefill(q, kc, vc, S, sp, H, Hk, D, 0.2, window=window, rows=[3, 40])
    np.testing.assert_array_equal(part[[3, 40]], out[[3, 40]])
    assert np.isnan(part[0]).all()


def test_qkv_append_composition():
    H, Hk, D, rows, sp = 4, 2, 64, 3, 5
    q = RNG.standard_normal((rows, H * D)).astype(np.float32)
    k = RNG.standard_normal((rows, Hk * D)).astype(np.float32)
    v = RNG.standard_normal((rows, Hk * D)).astype(np.float32)
    kc = np.zeros((10, Hk * D), np.float32)
    vc = np.zeros_like(kc)
    qo = ora.qkv_append(q, k, v, sp, H, Hk, D, D, 1e4, True, kc, vc)
    for r in range(rows):
        np.testing.assert_array_equal(qo[r], ora.rope(q[r], H, D, D, sp + r, 1e4, True))
        np.testing.assert_array_equal(kc[sp + r], ora.rope(k[r], Hk, D, D, sp + r, 1e4, True))
        np.testing.assert_array_equal(vc[sp + r], v[r])
    assert not kc[:sp].any() and not kc[sp + rows:].any()
    # with per-head norm: norm then rope
    w = (RNG.standard_normal(D) * 0.1 + 1).astype(np.float32)
    kc2 = np.zeros_like(kc)
    qo2 = ora.qkv_append(q, k, v, sp, H, Hk, D, D, 1e4, False, kc2, vc.copy(), q_norm=w,
                         k_norm=w, eps=1e-6)
    h0 = ora.rmsnorm(q[0, :D].copy(), w, 1e-6)
    np.testing.assert_array_equal(qo2[0, :D], ora.rope(h0, 1, D, D, sp, 1e4, False))


def test_qkv_append_bias_closed_form():
    """Bias terms (lib.rs:1021-1034): with norm off and pos 0 (RoPE is the
    identity there), q_out = q + b_q, K = k + b_k and V = v + b_v bit for bit
    (one f32 add each).  At pos > 0 the bias goes in before the rotation:
    the biased append equals the unbiased append of (q + b_q, k + b_k,
    v + b_v); a bias added after RoPE, or only to some rows or heads, or the
    wrong bias vector on a tensor, fails one of the two checks."""
    H, Hk, D, rows = 4, 2, 64, 3
    q = RNG.standard_normal((rows, H * D)).astype(np.float32)
    k = RNG.standard_normal((rows, Hk * D)).astype(np.float32)
    v = RNG.standard_normal((rows, Hk * D)).astype(np.float32)
    qb = RNG.standard_normal(H * D).astype(np.float32)
    kb = RNG.standard_normal(Hk * D).astype(np.float32)
    vb = RNG.standard_normal(Hk * D).astype(np.float32)
    for neox in (True, False):
        kc = np.zeros((rows, Hk * D), np.float32)
        vc = np.zeros_like(kc)
        qo = ora.qkv_append(q[:1].copy(), k[:1].copy(), v[:1].copy(), 0, H, Hk, D, D, 1e6, neox,
                            kc, vc, q_bias=qb, k_bias=kb, v_bias=vb)
        np.testing.assert_array_equal(qo[0], q[0] + qb)
        np.testing.assert_array_equal(kc[0], k[0] + kb)
        np.testing.assert_array_equal(vc[0], v[0] + vb)
        sp = 7
        kc1 = np.zeros((sp + rows, Hk * D), np.float32)
        vc1 = np.zeros_like(kc1)
        kc2, vc2 = kc1.copy(), vc1.copy()
        qo1 = ora.qkv_append(q, k, v, sp, H, Hk, D, D, 1e6, neox, kc1, vc1, q_bias=qb,
                             k_bias=kb, v_bias=vb)
        qo2 = ora.qkv_append(q + qb, k + kb, v + vb, sp, H, Hk, D, D, 1e6, neox, kc2, vc2)
        np.testing.assert_array_equal(qo1, qo2)
        np.testing.assert_array_equal(kc1, kc2)
        np.testing.assert_array_equal(vc1, vc2)
        assert not np.array_equal(qo1, ora.qkv_append(q, k, v, sp, H, Hk, D, D, 1e6, neox,
                                                      kc2.copy(), vc2.copy()) + qb)


def test_split_kv_merge_math():
    """The (m, l, acc) log-sum-exp merge the GPU kernels use equals one softmax."""
    L, D = 200, 16
    k = RNG.standard_normal((L, D))
    v = RNG.standard_normal((L, D))
    q = RNG.standard_normal(D)
    s = k @ q
    parts = []
    for a, b in ((0, 37), (37, 120), (120, 200)):
        m = s[a:b].max()
        p = np.exp(s[a:b] - m)
        parts.append((m, p.sum(), p @ v[a:b]))
    M = max(m for m, _, _ in parts)
    num = sum(acc * np.exp(m - M) for m, _, acc in parts)
    den = sum(l * np.exp(m - M) for m, l, _ in parts)
    np.testing.assert_allclose(num / den, f64_attention(q, k, v, 1.0), rtol=1e-12)


# --- matvec (math.rs:9-21) --------------------------------------------------------

def test_matvec_reference_cases():
    # math.rs:192-205 matvec_q_f32_identity
    eye = np.array([[1.0, 0.0], [0.0, 1.0]], dtype=np.float32)
    np.testing.assert_array_equal(ora.matvec(eye, 0, np.array([3.0, 5.0], np.float32)), [3.0, 5.0])
    # math.rs:208-233: the stacked per-token matvecs of a 3x2 weight
    w = np.array([[1.0, 2.0], [3.0, 4.0], [-1.0, 0.5]], dtype=np.float32)
    xs = np.array([[1.0, 0.0], [0.5, -2.0], [3.0, 3.0]], dtype=np.float32)
    want = [[1.0, 3.0, -1.0], [-3.5, -6.5, -1.5], [9.0, 21.0, -1.5]]
    for x, y in zip(xs, want):
        np.testing.assert_array_equal(ora.matvec(w, 0, x), y)


def test_matvec_left_fold_order():
    # A sequential f32 sum drops the 1 next to 1e8 before the cancellation;
    # any reordering (pairwise, tree, f64) returns 1.
    w = np.array([[1e8, 1.0, -1e8]], dtype=np.float32)
    assert ora.matvec(w, 0, np.ones(3, np.float32))[0] == 0.0


@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_matvec_matches_f64(dtype):
    out, cols = 37, 300
    wf = (0.05 * RNG.standard_normal((out, cols))).astype(np.float32)
    if dtype == 0:
        raw, wexact = wf, wf.astype(np.float64)
    elif dtype == 1:
        raw = wf.astype(np.float16).view(np.uint16)
        wexact = raw.view(np.float16).astype(np.float64)
    else:
        raw = (torch.from_numpy(wf).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
        wexact = torch.from_numpy(raw.view(np.int16)).view(torch.bfloat16).double().numpy()
    x = RNG.standard_normal(cols).astype(np.float32)
    y = ora.matvec(raw, dtype, x)
    ref = wexact @ x.astype(np.float64)
    bound = cols * np.finfo(np.float32).eps * (np.abs(wexact) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(y - ref) <= bound)
    # transposed operand or a row offset would fail this
    assert np.abs(y - ref).max() < 1e-4
