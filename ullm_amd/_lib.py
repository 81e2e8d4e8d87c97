"""ctypes binding of libullm_hip.so -- the C ABI declared in include/ullm_hip.h.

Loading fails loudly: there is no fallback path.  If the library is missing
the caller gets an ImportError telling it to build (python -m ullm_amd.build).
"""
from __future__ import annotations

import ctypes as C
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libullm_hip.so")

OK, E_INVALID, E_UNSUPPORTED, E_HIP, E_WORKSPACE = 0, -1, -2, -3, -4
DT_F32, DT_F16, DT_BF16 = 0, 1, 2

# name -> (restype, argtypes); mirrors include/ullm_hip.h one to one.
_vp, _i, _i64, _f, _sz = C.c_void_p, C.c_int, C.c_int64, C.c_float, C.c_size_t
SIGNATURES = {
    "ullm_hip_version": (C.c_char_p, []),
    "ullm_hip_last_error": (C.c_char_p, []),
    "ullm_hip_decode_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i]),
    "ullm_hip_attn_decode": (
        _i,
        [_vp, _vp, _vp, _i, _i64, _i64, _vp, _i, _i, _i, _i, _i, _i, _f, _vp, _vp, _sz, _vp],
    ),
    "ullm_hip_attn_decode_noalloc": (
        _i, [_vp, _vp, _vp, _i, _i64, _i64, _vp, _i, _i, _i, _i, _i, _i, _f, _vp, _vp],
    ),
    "ullm_hip_decode_noalloc_max_bytes": (_sz, []),
    "ullm_hip_attn_prefill": (
        _i, [_vp, _vp, _vp, _i, _i64, _i, _i, _i, _i, _i, _i, _f, _vp, _vp]
    ),
    "ullm_hip_rope_table": (_i, [_vp, _i, _i, _f]),
    "ullm_hip_stream_read": (_i, [_vp, _sz, _i, _vp, _vp]),
    "ullm_hip_qkv_append": (
        _i,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f, _vp, _i, _i, _i, _i, _i, _i, _i, _i,
         _vp, _i, _vp, _vp, _i, _i64, _vp],
    ),
    "ullm_hip_qkv_proj_append": (
        _i,
        [_vp, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _f, _vp, _i, _i, _i, _i, _i, _i,
         _i, _i, _vp, _i, _vp, _vp, _i, _i64, _vp, _sz, _vp],
    ),
    "ullm_hip_qkv_proj_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "ullm_hip_matmul": (_i, [_vp, _i, _vp, _vp, _i, _i, _i, _vp]),
    "ullm_hip_attn_prefill_paged": (
        _i, [_vp, _vp, _vp, _i, _i64, _i, _i, _vp, _i, _i, _i, _i, _i, _i, _i, _f, _vp, _vp]
    ),
    "ullm_hip_qkv_append_paged": (
        _i,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f, _vp, _i, _i, _i, _i, _vp, _i, _i, _i, _vp,
         _i, _vp, _vp, _i, _i64, _i, _i, _vp, _i, _vp],
    ),
    "ullm_hip_paged_decode_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i]),
    "ullm_hip_attn_decode_paged": (
        _i,
        [_vp, _vp, _vp, _i, _i64, _i, _i, _vp, _i, _vp, _i, _i, _i, _i, _i, _i, _f, _vp, _vp, _sz,
         _vp],
    ),
}


class UllmHipError(RuntimeError):
    """A non-zero status from the C ABI (code + the library's message)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"ullm_hip error {code}: {msg}")
        self.code = code


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m ullm_amd.build` "
                "(there is no CPU fallback)"
            )
        h = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype, fn.argtypes = res, args
        _lib = h
    return _lib


def check(rc: int) -> None:
    if rc != OK:
        raise UllmHipError(rc, lib().ullm_hip_last_error().decode())
