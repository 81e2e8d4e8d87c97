"""ullm_amd -- MI355X (gfx950) attention path for uLLM.

Hand-written HIP kernels behind the C ABI of include/ullm_hip.h:
single-query GQA decode attention (split-KV), causal prefill attention
(MFMA), and the fused Q/K-norm + RoPE + KV-cache append.  The Python layer
here only binds that ABI (ctypes) and uses torch for device memory.
"""
from ._lib import UllmHipError, lib  # noqa: F401
from .attention import (  # noqa: F401
    GpuAttention,
    attn_decode,
    attn_prefill,
    decode_workspace_bytes,
    qkv_append,
    rope_table,
)

__version__ = "0.1.0"
