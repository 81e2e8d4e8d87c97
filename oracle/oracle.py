"""Python view of the CPU oracle (liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker or the timed CPU baseline.  Each wrapper
names the reference lines its C function restates (see ref_attention.c).
All arrays are numpy f32, C-contiguous.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_f = C.POINTER(C.c_float)
_lib = None


def build() -> str:
    """Compile ref_attention.c with the oracle's float-exact flags."""
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        h = C.CDLL(LIB_PATH)
        h.ora_f16_to_f32.restype = C.c_float
        h.ora_f16_to_f32.argtypes = [C.c_uint16]
        h.ora_bf16_to_f32.restype = C.c_float
        h.ora_bf16_to_f32.argtypes = [C.c_uint16]
        h.ora_widen.argtypes = [C.c_void_p, C.c_int, C.c_size_t, _f]
        h.ora_rmsnorm.argtypes = [_f, _f, C.c_int, C.c_float, _f]
        h.ora_softmax.argtypes = [_f, C.c_int]
        for n in ("ora_rope", "ora_rope_neox"):
            getattr(h, n).argtypes = [_f, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]
        h.ora_window_start.argtypes = [C.c_int, C.c_int]
        h.ora_attn_decode.argtypes = [_f, _f, _f, C.c_size_t, C.c_int, C.c_int, C.c_int, C.c_int,
                                      C.c_int, C.c_float, _f]
        h.ora_attn_prefill.argtypes = [_f, _f, _f, C.c_size_t, C.c_int, C.c_int, C.c_int,
                                       C.c_int, C.c_int, C.c_int, C.c_float,
                                       C.POINTER(C.c_int), C.c_int, _f]
        h.ora_qkv_append.argtypes = [_f, _f, _f, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                     C.c_int, _f, _f, _f, _f, _f, C.c_float, C.c_int, C.c_float,
                                     _f, _f, C.c_size_t]
        h.ora_matvec.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, _f, _f]
        _lib = h
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags.c_contiguous, "oracle takes C-contiguous f32"
    return a.ctypes.data_as(_f)


def _rc(rc):
    if rc != 0:
        raise RuntimeError(f"oracle error {rc}")


def widen(raw: np.ndarray, dtype: int) -> np.ndarray:
    """dequant.rs:61-94 for f32/f16/bf16; raw is the uint16 (or f32) storage."""
    raw = np.ascontiguousarray(raw)
    out = np.empty(raw.size, dtype=np.float32)
    lib().ora_widen(raw.ctypes.data_as(C.c_void_p), dtype, raw.size, _p(out))
    return out.reshape(raw.shape)


def rmsnorm(x, w, eps):
    """math.rs:82-86."""
    y = np.empty_like(x)
    lib().ora_rmsnorm(_p(x), _p(w), x.size, eps, _p(y))
    return y


def softmax(x):
    """math.rs:89-100 (returns a new array)."""
    y = np.array(x, dtype=np.float32, copy=True)
    lib().ora_softmax(_p(y), y.size)
    return y


def rope(v, n_heads, head_dim, rotary_dim, pos, theta, neox):
    """math.rs:116-136 (interleaved) or :140-161 (NeoX); returns a new array."""
    y = np.array(v, dtype=np.float32, copy=True)
    fn = lib().ora_rope_neox if neox else lib().ora_rope
    fn(_p(y), n_heads, head_dim, rotary_dim, pos, theta)
    return y


def attn_decode(q, kc, vc, pos, n_head, n_kv_head, head_dim, scale, window=0, kv_stride=None):
    """lib.rs:911-938 (window>0: lib.rs:1180-1208).  kc/vc: f32 layer cache."""
    if kv_stride is None:
        kv_stride = n_kv_head * head_dim
    out = np.empty(n_head * head_dim, dtype=np.float32)
    _rc(lib().ora_attn_decode(_p(q), _p(kc), _p(vc), kv_stride, pos, window, n_head, n_kv_head,
                              head_dim, scale, _p(out)))
    return out


def attn_prefill(q, kc, vc, S, start_pos, n_head, n_kv_head, head_dim, scale, window=0,
                 rows=None, kv_stride=None):
    """lib.rs:1061-1087 for the listed rows (all if None); other rows are NaN."""
    if kv_stride is None:
        kv_stride = n_kv_head * head_dim
    out = np.full((S, n_head * head_dim), np.nan, dtype=np.float32)
    if rows is None:
        rp, nr = None, 0
    else:
        ra = np.ascontiguousarray(np.asarray(rows, dtype=np.int32))
        rp, nr = ra.ctypes.data_as(C.POINTER(C.c_int)), ra.size
    _rc(lib().ora_attn_prefill(_p(q), _p(kc), _p(vc), kv_stride, S, start_pos, window, n_head,
                               n_kv_head, head_dim, scale, rp, nr, _p(out)))
    return out


def qkv_append(q, k, v, start_pos, n_head, n_kv_head, head_dim, rotary_dim, theta, neox,
               kc, vc, q_bias=None, k_bias=None, v_bias=None, q_norm=None, k_norm=None,
               eps=1e-6, kv_stride=None):
    """lib.rs:1021-1058: returns the prepared q; writes K/V rows into kc/vc."""
    if kv_stride is None:
        kv_stride = n_kv_head * head_dim
    qo = np.array(q, dtype=np.float32, copy=True)
    _rc(lib().ora_qkv_append(_p(qo), _p(k), _p(v), q.shape[0], start_pos, n_head, n_kv_head,
                             head_dim, rotary_dim, _p(q_bias), _p(k_bias), _p(v_bias),
                             _p(q_norm), _p(k_norm), eps, int(bool(neox)), theta, _p(kc), _p(vc),
                             kv_stride))
    return qo


def matvec(w_raw: np.ndarray, dtype: int, x: np.ndarray) -> np.ndarray:
    """math.rs:9-21 (matvec_q): y = W x with W [out][cols] in f32 (dtype 0)
    or raw uint16 f16 (1) / bf16 (2) storage; sequential f32 sums."""
    w_raw = np.ascontiguousarray(w_raw)
    out, cols = w_raw.shape
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.size == cols
    y = np.empty(out, dtype=np.float32)
    _rc(lib().ora_matvec(w_raw.ctypes.data_as(C.c_void_p), dtype, out, cols, _p(x), _p(y)))
    return y
