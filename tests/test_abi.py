"""C ABI of libullm_hip.so without a GPU: loading, exported symbols, the host
RoPE table, and argument validation (all return before touching the device)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from oracle import oracle as ora
from ullm_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    src = open(os.path.join(ROOT, "include", "ullm_hip.h")).read()
    return sorted(set(re.findall(r"\b(ullm_hip_\w+)\s*\(", src)))


def test_library_exports_every_declared_function():
    lib = L.lib()
    names = header_functions()
    assert len(names) >= 7
    for n in names:
        assert hasattr(lib, n), n
        assert n in L.SIGNATURES, f"{n} has no ctypes signature"


def test_version():
    assert L.lib().ullm_hip_version().decode().startswith("ullm-hip ")


@pytest.mark.parametrize("neox", [True, False])
def test_rope_table_reproduces_reference_rope_exactly(neox):
    """The host table gives the CPU reference's rotation bit for bit
    (same f32 angle, same libm)."""
    hd, n_pos = 128, 4096
    cs = np.empty((n_pos, hd // 2, 2), np.float32)
    L.check(L.lib().ullm_hip_rope_table(C.c_void_p(cs.ctypes.data), n_pos, hd, 1e6))
    rng = np.random.default_rng(0)
    for pos in (0, 1, 77, 4095):
        v = rng.standard_normal(hd).astype(np.float32)
        want = ora.rope(v, 1, hd, hd, pos, 1e6, neox)
        c, s = cs[pos, :, 0], cs[pos, :, 1]
        if neox:
            a, b = v[: hd // 2], v[hd // 2:]
            got = np.concatenate([a * c - b * s, a * s + b * c])
        else:
            a, b = v[0::2], v[1::2]
            got = np.empty_like(v)
            got[0::2], got[1::2] = a * c - b * s, a * s + b * c
        np.testing.assert_array_equal(got, want)


def _decode(**kw):
    args = dict(q=None, k=None, v=None, dt=L.DT_F16, kvs=256, ss=0, lens=None, max_len=100,
                win=0, b=1, h=12, hk=2, d=128, scale=0.1, out=None, ws=None, wsb=0, st=None)
    args.update(kw)
    a = args
    return L.lib().ullm_hip_attn_decode(a["q"], a["k"], a["v"], a["dt"], a["kvs"], a["ss"],
                                         a["lens"], a["max_len"], a["win"], a["b"], a["h"],
                                         a["hk"], a["d"], a["scale"], a["out"], a["ws"],
                                         a["wsb"], a["st"])


def test_decode_argument_validation():
    assert _decode(d=96) == L.E_UNSUPPORTED
    assert _decode(dt=7) == L.E_UNSUPPORTED
    assert _decode(h=12, hk=5) == L.E_INVALID
    assert _decode(max_len=0) == L.E_INVALID
    assert _decode(kvs=100) == L.E_INVALID
    assert _decode() == L.E_INVALID  # null tensors
    assert b"null" in L.lib().ullm_hip_last_error()


def test_prefill_and_append_validation():
    lib = L.lib()
    # every dtype takes head_dim 64/128/256: an f32 cache at 256 passes the
    # dtype checks and stops at the null pointers; head_dim 96 is unsupported
    assert lib.ullm_hip_attn_prefill(None, None, None, L.DT_F32, 1024, 16, 0, 0, 8, 2, 256, 0.1,
                                     None, None) == L.E_INVALID
    assert b"null" in lib.ullm_hip_last_error()
    assert lib.ullm_hip_attn_prefill(None, None, None, L.DT_F32, 512, 16, 0, 0, 8, 2, 96, 0.1,
                                     None, None) == L.E_UNSUPPORTED
    # q of 32768 rows x 128 heads x 256 (4 GiB) over a 32 MB one-kv-head cache
    assert lib.ullm_hip_attn_prefill(None, None, None, L.DT_F32, 256, 32768, 0, 0, 128, 1, 256,
                                     0.1, None, None) == L.E_INVALID
    assert b"q exceeds 2 GiB" in lib.ullm_hip_last_error()
    assert lib.ullm_hip_attn_prefill(None, None, None, 7, 256, 16, 0, 0, 8, 2, 128, 0.1,
                                     None, None) == L.E_UNSUPPORTED
    assert lib.ullm_hip_attn_prefill(None, None, None, L.DT_BF16, 256, 16, 0, 0, 8, 3, 128,
                                     0.1, None, None) == L.E_INVALID
    assert lib.ullm_hip_attn_prefill(None, None, None, L.DT_BF16, 256, 0, 0, 0, 8, 2, 128, 0.1,
                                     None, None) == L.OK  # S == 0 is a no-op
    rc = lib.ullm_hip_qkv_append(None, None, None, None, None, None, None, None, 1e-6, None, 10,
                                 1, 128, 4, 8, 8, 2, 128, None, L.DT_F32, None, None, L.DT_F16,
                                 256, None)
    assert rc == L.E_INVALID  # rope table shorter than start_pos + rows
    assert lib.ullm_hip_rope_table(None, 10, 128, 1e4) == L.E_INVALID


def test_workspace_size_planning():
    ws = L.lib().ullm_hip_decode_workspace_bytes
    assert ws(1, 12, 2, 128, 4096, 0) > 0
    assert ws(1, 12, 2, 128, 64, 0) > 0  # a short context still splits over the CUs
    assert ws(128, 12, 2, 128, 64, 0) == 0  # 256 units fill the chip: one split each
    assert ws(1, 32, 4, 128, 32768, 0) >= ws(1, 32, 4, 128, 4096, 0)
    assert ws(1, 12, 5, 128, 4096, 0) == 0  # invalid shape


def test_proj_append_validation():
    f = L.lib().ullm_hip_qkv_proj_append

    def call(**kw):
        a = dict(x=None, in_dim=1536, wq=None, wk=None, wv=None, wdt=L.DT_BF16, qb=None, kb=None,
                 vb=None, qn=None, kn=None, eps=1e-6, cs=None, npos=10, neox=1, rd=128, rows=1,
                 sp=0, h=12, hk=2, d=128, qo=None, qdt=L.DT_F32, kc=None, vc=None,
                 kvdt=L.DT_F16, kvs=256, ws=None, wsb=0, st=None)
        a.update(kw)
        return f(*a.values())

    assert call(wdt=7) == L.E_UNSUPPORTED
    assert call(d=96) == L.E_UNSUPPORTED
    assert call(hk=5) == L.E_INVALID
    assert call(in_dim=1540) == L.E_INVALID  # not a multiple of 8
    assert call(rd=3) == L.E_INVALID
    assert call(kvs=100) == L.E_INVALID
    assert call(rows=0) == L.OK  # nothing to do
    assert call() == L.E_INVALID  # null pointers
    wsz = L.lib().ullm_hip_qkv_proj_workspace_bytes
    assert wsz(1, 32, 8, 128) == 48 * 128 * 4 + 256  # decode: split, y + counters
    assert wsz(2048, 32, 8, 128) == 0  # prefill rows: no split


def test_matmul_validation():
    f = L.lib().ullm_hip_matmul

    def call(**kw):
        a = dict(w=None, wdt=L.DT_BF16, x=None, y=None, i=2560, o=4096, n=16, st=None)
        a.update(kw)
        return f(*a.values())

    assert call(wdt=L.DT_F32) == L.E_UNSUPPORTED  # batched path is bf16, as forward.rs:710-714
    assert call(wdt=L.DT_F16) == L.E_UNSUPPORTED
    assert call(i=2564) == L.E_INVALID  # in_dim % 8
    assert call(o=4098) == L.E_INVALID  # out_dim % 4
    assert call(n=-1) == L.E_INVALID
    assert call(i=1 << 20, o=1 << 11) == L.E_INVALID  # 4 GiB weight
    assert call(n=0) == L.OK  # nothing to do
    assert call() == L.E_INVALID  # null pointers


def test_paged_decode_validation():
    f = L.lib().ullm_hip_attn_decode_paged

    def call(**kw):
        a = dict(q=None, kp=None, vp=None, dt=L.DT_BF16, kvs=512, page=64, npages=10, tab=None,
                 ts=64, sl=None, ml=4096, win=0, b=1, h=16, hk=4, d=128, sc=0.1, out=None,
                 ws=None, wsb=0, st=None)
        a.update(kw)
        return f(*a.values())

    assert call(dt=9) == L.E_UNSUPPORTED
    assert call(d=96) == L.E_UNSUPPORTED
    assert call(page=48) == L.E_INVALID  # not a power of two
    assert call(page=16) == L.E_INVALID  # below one 32-key block
    assert call(ts=63) == L.E_INVALID   # table too short for max_len
    assert call(hk=3) == L.E_INVALID
    assert call(kvs=500) == L.E_INVALID
    assert call(npages=0) == L.E_INVALID
    assert call() == L.E_INVALID  # null pointers


def test_paged_append_validation():
    f = L.lib().ullm_hip_qkv_append_paged

    def call(**kw):
        a = dict(q=None, k=None, v=None, qb=None, kb=None, vb=None, qn=None, kn=None, eps=1e-6,
                 cs=None, npos=4096, neox=1, rd=128, rows=4, pos=None, h=16, hk=4, d=128,
                 qo=None, qdt=L.DT_F32, kp=None, vp=None, kvdt=L.DT_BF16, kvs=512, page=64,
                 npages=10, tab=None, ts=64, st=None)
        a.update(kw)
        return f(*a.values())

    assert call(kvdt=9) == L.E_UNSUPPORTED
    assert call(d=96) == L.E_UNSUPPORTED
    assert call(page=48) == L.E_INVALID
    assert call(hk=3) == L.E_INVALID
    assert call(kvs=100) == L.E_INVALID
    assert call(npages=0) == L.E_INVALID
    assert call(rows=0) == L.OK
    assert call() == L.E_INVALID  # null pointers


def test_paged_prefill_validation():
    f = L.lib().ullm_hip_attn_prefill_paged

    def call(**kw):
        a = dict(q=None, kp=None, vp=None, dt=L.DT_BF16, kvs=1024, page=64, npages=10, tab=None,
                 tl=40, s=512, sp=0, win=0, h=32, hk=8, d=128, sc=0.1, out=None, st=None)
        a.update(kw)
        return f(*a.values())

    assert call(dt=L.DT_F32, d=64) == L.E_INVALID       # f32 pages at every head_dim; null pointers
    assert call(dt=L.DT_F32) == L.E_INVALID              # accepted; then the null pointers
    assert call(dt=L.DT_F16, kvs=1028) == L.E_INVALID    # 2056-byte rows: not
    assert call(d=96) == L.E_UNSUPPORTED
    # q of 32768 rows x 128 heads x 256 f32 = 4 GiB over a 1-kv-head cache
    assert call(dt=L.DT_F32, kvs=256, s=32768, tl=600, h=128, hk=1, d=256) == L.E_INVALID
    assert b"q exceeds 2 GiB" in L.lib().ullm_hip_last_error()
    assert call(page=32) == L.E_INVALID   # below one 64-key tile
    assert call(page=96) == L.E_INVALID
    assert call(tl=7) == L.E_INVALID      # 7 pages < 512 positions
    assert call(hk=3) == L.E_INVALID
    assert call(s=0) == L.OK
    assert call() == L.E_INVALID  # null pointers


def test_stream_read_validation():
    """The calibration read rejects null, unaligned and empty arguments
    before any HIP call."""
    lib = L.lib()
    sink = C.c_void_p(64)
    assert lib.ullm_hip_stream_read(None, 1024, 4, sink, None) == L.E_INVALID
    assert lib.ullm_hip_stream_read(C.c_void_p(4096 + 8), 1024, 4, sink, None) == L.E_INVALID
    assert lib.ullm_hip_stream_read(C.c_void_p(4096), 8, 4, sink, None) == L.E_INVALID
    assert lib.ullm_hip_stream_read(C.c_void_p(4096), 1024, 0, sink, None) == L.E_INVALID


def _gpu_visible():
    try:
        import torch

        return torch.cuda.device_count() > 0
    except Exception:
        return False


def _needed_ws(dt, h, hk, d, n, win, paged=False):
    """Workspace bytes one decode call of max_len n asks for, read from the
    E_WORKSPACE message (the call stops there, before any device work; a
    call that needs none gets as far as the launch and fails without a GPU).
    Only ever called with no GPU visible: on a GPU machine such a call would
    launch kernels on the fake addresses below."""
    assert not _gpu_visible(), "_needed_ws reaches a kernel launch on a GPU machine"
    lib = L.lib()
    fake = C.c_void_p(0x10000)
    kvs = hk * d
    if paged:
        rc = lib.ullm_hip_attn_decode_paged(fake, fake, fake, dt, kvs, 32, 1 << 20, fake,
                                            (n + 31) // 32, fake, n, win, 1, h, hk, d, 0.1,
                                            fake, None, 0, None)
    else:
        rc = lib.ullm_hip_attn_decode(fake, fake, fake, dt, kvs, 0, fake, n, win, 1, h, hk, d,
                                      0.1, fake, None, 0, None)
    if rc == L.E_WORKSPACE:
        m = re.search(rb"workspace of (\d+) bytes needed", lib.ullm_hip_last_error())
        return int(m.group(1))
    assert rc in (L.OK, L.E_HIP), (rc, lib.ullm_hip_last_error())
    return 0


@pytest.mark.parametrize("dt", [L.DT_F32, L.DT_F16, L.DT_BF16])
@pytest.mark.parametrize("shape", [(12, 2, 128), (32, 8, 64), (8, 4, 256)])
@pytest.mark.parametrize("n_ctx,win", [(1024, 0), (700, 0), (1024, 300), (2048, 1000)])
@pytest.mark.parametrize("paged", [False, True])
def test_workspace_for_n_ctx_bounds_every_shorter_call(dt, shape, n_ctx, win, paged):
    """A workspace sized for max_len = n_ctx serves every call with a smaller
    max_len (the header's promise), for every cache dtype, including the f32
    path whose split count is not monotonic in the length.  CPU only: a call
    that needs no workspace passes validation and reaches a kernel launch,
    which must not happen with the fake pointers on a machine with a GPU."""
    if _gpu_visible():
        pytest.skip("launches kernels on fake pointers when a GPU is visible; runs on CPU-only hosts")
    h, hk, d = shape
    fn = (L.lib().ullm_hip_paged_decode_workspace_bytes if paged
          else L.lib().ullm_hip_decode_workspace_bytes)
    bound = fn(1, h, hk, d, n_ctx, win)
    for n in range(1, n_ctx + 1):
        need = _needed_ws(dt, h, hk, d, n, win, paged)
        assert need <= bound, f"max_len {n}: needs {need} > {bound} sized for {n_ctx}"
