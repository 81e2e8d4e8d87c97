"""Torch-tensor front end of the C ABI, and `GpuAttention`, the attention
part of the reference's `GpuForward` (crates/ullm-metal/src/forward.rs).

Every op here is a thin call into libullm_hip.so; torch supplies device
memory and the current HIP stream and nothing else.  There is no CPU or
PyTorch fallback: without the library or a GPU the calls raise.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib as L

_DT = {torch.float32: L.DT_F32, torch.float16: L.DT_F16, torch.bfloat16: L.DT_BF16}


def _dt(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise L.UllmHipError(L.E_UNSUPPORTED, f"dtype {t.dtype} not supported") from None


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(stream=None):
    s = torch.cuda.current_stream() if stream is None else stream
    return C.c_void_p(s.cuda_stream)


def _need_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise L.UllmHipError(L.E_INVALID, "tensors must live on the GPU")


def decode_workspace_bytes(batch, n_head, n_kv_head, head_dim, max_len, window=0) -> int:
    return int(L.lib().ullm_hip_decode_workspace_bytes(batch, n_head, n_kv_head, head_dim,
                                                       max_len, window))


def new_decode_workspace(batch, n_head, n_kv_head, head_dim, max_len, window=0, device="cuda"):
    """Workspace for attn_decode (split partials; zeroed only for determinism of
    unused bytes, the kernels write every partial before reading it)."""
    n = max(decode_workspace_bytes(batch, n_head, n_kv_head, head_dim, max_len, window), 256)
    return torch.zeros(n, dtype=torch.uint8, device=device)


def attn_decode(q, k_cache, v_cache, seq_lens, max_len, n_kv_head, *, window=0, scale=None,
                kv_stride=None, seq_stride=0, out=None, workspace=None, stream=None):
    """Single-query GQA decode attention (lib.rs:911-938 / :1180-1208).

    q: [B, n_head, D] f32.  k_cache/v_cache: layer base (f32/f16/bf16) with
    `kv_stride` elements per position (default n_kv_head*D) and `seq_stride`
    between sequences.  seq_lens: int32 [B] on the GPU (= pos + 1).
    """
    B, H, D = q.shape
    _need_cuda(q, k_cache, v_cache, seq_lens)
    if q.dtype != torch.float32 or not q.is_contiguous():
        raise L.UllmHipError(L.E_INVALID, "q must be contiguous f32 [B, n_head, head_dim]")
    if seq_lens.dtype != torch.int32 or seq_lens.numel() != B:
        raise L.UllmHipError(L.E_INVALID, "seq_lens must be int32 [B]")
    if kv_stride is None:
        kv_stride = n_kv_head * D
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty(B, H, D, dtype=torch.float32, device=q.device)
    if workspace is None:
        workspace = new_decode_workspace(B, H, n_kv_head, D, max_len, window, q.device)
    rc = L.lib().ullm_hip_attn_decode(
        _ptr(q), _ptr(k_cache), _ptr(v_cache), _dt(k_cache), kv_stride, seq_stride,
        _ptr(seq_lens), max_len, window, B, H, n_kv_head, D, float(scale), _ptr(out),
        _ptr(workspace), workspace.numel(), _stream(stream))
    L.check(rc)
    return out


def attn_decode_paged(q, k_pages, v_pages, block_table, seq_lens, max_len, n_kv_head, *,
                      window=0, scale=None, out=None, workspace=None, stream=None):
    """Decode attention over a paged KV cache (same result as attn_decode).

    q: [B, n_head, D] f32.  k_pages/v_pages: [n_pages, page_size, kv_stride]
    f16/bf16.  block_table: int32 [B, table_stride] (page of position t of
    sequence b = block_table[b, t // page_size]).  seq_lens: int32 [B].
    """
    B, H, D = q.shape
    _need_cuda(q, k_pages, v_pages, block_table, seq_lens)
    if q.dtype != torch.float32 or not q.is_contiguous():
        raise L.UllmHipError(L.E_INVALID, "q must be contiguous f32 [B, n_head, head_dim]")
    if k_pages.dim() != 3 or k_pages.shape != v_pages.shape or not k_pages.is_contiguous() \
            or not v_pages.is_contiguous():
        raise L.UllmHipError(L.E_INVALID, "k_pages/v_pages must be contiguous [n_pages, page_size, kv_stride]")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.shape[0] != B \
            or not block_table.is_contiguous():
        raise L.UllmHipError(L.E_INVALID, "block_table must be contiguous int32 [B, table_stride]")
    if seq_lens.dtype != torch.int32 or seq_lens.numel() != B:
        raise L.UllmHipError(L.E_INVALID, "seq_lens must be int32 [B]")
    n_pages, page_size, kv_stride = k_pages.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty(B, H, D, dtype=torch.float32, device=q.device)
    if workspace is None:
        n = int(L.lib().ullm_hip_paged_decode_workspace_bytes(B, H, n_kv_head, D, max_len, window))
        workspace = torch.zeros(max(n, 256), dtype=torch.uint8, device=q.device)
    rc = L.lib().ullm_hip_attn_decode_paged(
        _ptr(q), _ptr(k_pages), _ptr(v_pages), _dt(k_pages), kv_stride, page_size, n_pages,
        _ptr(block_table), block_table.shape[1], _ptr(seq_lens), max_len, window, B, H, n_kv_head,
        D, float(scale), _ptr(out), _ptr(workspace), workspace.numel(), _stream(stream))
    L.check(rc)
    return out


def qkv_append_paged(q, k, v, k_pages, v_pages, rope_cs, positions, block_table, *, n_head,
                     n_kv_head, head_dim, rotary_dim=None, neox=True, q_norm=None, k_norm=None,
                     eps=1e-6, q_bias=None, k_bias=None, v_bias=None, q_out=None, q_dtype=None,
                     stream=None):
    """Append one token per sequence into a paged cache: row r of q/k/v [rows,
    *] f32 is sequence r's token at positions[r] (int32 [rows] on the GPU);
    its K/V rows land in block_table[r, pos // page_size].  Returns q_out."""
    rows = q.shape[0]
    _need_cuda(q, k, v, k_pages, v_pages, rope_cs, positions, block_table)
    for t in (q, k, v):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise L.UllmHipError(L.E_INVALID, "q/k/v must be contiguous f32")
    if k_pages.dim() != 3 or k_pages.shape != v_pages.shape:
        raise L.UllmHipError(L.E_INVALID, "k_pages/v_pages must be [n_pages, page_size, kv_stride]")
    if positions.dtype != torch.int32 or positions.numel() != rows:
        raise L.UllmHipError(L.E_INVALID, "positions must be int32 [rows]")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.shape[0] != rows \
            or not block_table.is_contiguous():
        raise L.UllmHipError(L.E_INVALID, "block_table must be contiguous int32 [rows, table_stride]")
    n_pages, page_size, kv_stride = k_pages.shape
    if rotary_dim is None:
        rotary_dim = head_dim
    if q_dtype is None:
        q_dtype = torch.float32
    if q_out is None:
        q_out = torch.empty(rows, n_head * head_dim, dtype=q_dtype, device=q.device)
    rc = L.lib().ullm_hip_qkv_append_paged(
        _ptr(q), _ptr(k), _ptr(v), _ptr(q_bias), _ptr(k_bias), _ptr(v_bias), _ptr(q_norm),
        _ptr(k_norm), float(eps), _ptr(rope_cs), rope_cs.shape[0], int(bool(neox)), rotary_dim,
        rows, _ptr(positions), n_head, n_kv_head, head_dim, _ptr(q_out), _DT[q_out.dtype],
        _ptr(k_pages), _ptr(v_pages), _dt(k_pages), kv_stride, page_size, n_pages,
        _ptr(block_table), block_table.shape[1], _stream(stream))
    L.check(rc)
    return q_out


def attn_prefill_paged(q, k_pages, v_pages, block_table, n_head, n_kv_head, head_dim, *,
                       start_pos=0, window=0, scale=None, out=None, stream=None):
    """Causal prefill of S rows (positions start_pos..) of one sequence whose
    keys live in pages: block_table int32 [table_len] (page of key t =
    block_table[t // page_size]).  q: [S, n_head*head_dim] f16/bf16, or f32
    with f32 pages (head_dim 64, 128 or 256)."""
    S = q.shape[0]
    _need_cuda(q, k_pages, v_pages, block_table)
    if not q.is_contiguous() or q.numel() != S * n_head * head_dim:
        raise L.UllmHipError(L.E_INVALID, "q must be contiguous [S, n_head*head_dim]")
    if k_pages.dim() != 3 or k_pages.shape != v_pages.shape or q.dtype != k_pages.dtype:
        raise L.UllmHipError(L.E_INVALID, "k_pages/v_pages must be [n_pages, page_size, kv_stride] of q's dtype")
    if block_table.dtype != torch.int32 or block_table.dim() != 1:
        raise L.UllmHipError(L.E_INVALID, "block_table must be int32 [table_len]")
    n_pages, page_size, kv_stride = k_pages.shape
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    if out is None:
        out = torch.empty(S, n_head * head_dim, dtype=torch.float32, device=q.device)
    rc = L.lib().ullm_hip_attn_prefill_paged(
        _ptr(q), _ptr(k_pages), _ptr(v_pages), _dt(q), kv_stride, page_size, n_pages,
        _ptr(block_table), block_table.numel(), S, start_pos, window, n_head, n_kv_head, head_dim,
        float(scale), _ptr(out), _stream(stream))
    L.check(rc)
    return out


# Largest q the prefill entry points take in one call (below 2 GiB, and a
# multiple of 16 bytes so every chunk stays 16-byte aligned).
PREFILL_Q_MAX_BYTES = 0x7fff0000


def attn_prefill(q, k_cache, v_cache, n_head, n_kv_head, head_dim, *, start_pos=0, window=0,
                 scale=None, kv_stride=None, out=None, stream=None):
    """Causal prefill attention on MFMA (lib.rs:1061-1087).

    q: [S, n_head*head_dim] in the cache dtype (f16, bf16 or f32); the cache
    already holds positions 0..start_pos+S-1.  Returns [S, n_head*head_dim]
    f32.  A q of PREFILL_Q_MAX_BYTES or more (the kernels address it through
    a 32-bit buffer range) runs as row chunks at increasing start_pos: the
    cache already holds every position, so each chunk's rows see the same
    keys.
    """
    S = q.shape[0]
    _need_cuda(q, k_cache, v_cache)
    if not q.is_contiguous() or q.numel() != S * n_head * head_dim:
        raise L.UllmHipError(L.E_INVALID, "q must be contiguous [S, n_head*head_dim]")
    if q.dtype != k_cache.dtype or q.dtype != v_cache.dtype:
        raise L.UllmHipError(L.E_INVALID, "q and cache dtypes differ")
    if kv_stride is None:
        kv_stride = n_kv_head * head_dim
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    if out is None:
        out = torch.empty(S, n_head * head_dim, dtype=torch.float32, device=q.device)
    row_bytes = n_head * head_dim * q.element_size()
    rows = max(1, PREFILL_Q_MAX_BYTES // row_bytes)
    for r0 in range(0, max(S, 1), rows):
        n = min(rows, S - r0)
        rc = L.lib().ullm_hip_attn_prefill(
            _ptr(q[r0:r0 + n]), _ptr(k_cache), _ptr(v_cache), _dt(q), kv_stride, n,
            start_pos + r0, window, n_head, n_kv_head, head_dim, float(scale),
            _ptr(out[r0:r0 + n]), _stream(stream))
        L.check(rc)
    return out


def rope_table(n_pos: int, rotary_dim: int, theta: float, device="cuda") -> torch.Tensor:
    """(cos, sin) table [n_pos, rotary_dim/2, 2] with the reference formula,
    computed on the host by the library and uploaded."""
    host = torch.empty(n_pos, rotary_dim // 2, 2, dtype=torch.float32)
    L.check(L.lib().ullm_hip_rope_table(C.c_void_p(host.data_ptr()), n_pos, rotary_dim,
                                        float(theta)))
    return host.to(device) if device != "cpu" else host


def qkv_append(q, k, v, k_cache, v_cache, rope_cs, *, start_pos, n_head, n_kv_head, head_dim,
               rotary_dim=None, neox=True, q_norm=None, k_norm=None, eps=1e-6, q_bias=None,
               k_bias=None, v_bias=None, q_out=None, q_dtype=None, kv_stride=None, stream=None):
    """Fused bias + Q/K RMSNorm + RoPE + KV append (lib.rs:1021-1058).

    q: [rows, n_head*D] f32, k/v: [rows, n_kv_head*D] f32.  K/V land in the
    cache at positions start_pos..; returns q_out ([rows, n_head*D], q_dtype).
    """
    rows = q.shape[0]
    _need_cuda(q, k, v, k_cache, v_cache, rope_cs)
    for t in (q, k, v):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise L.UllmHipError(L.E_INVALID, "q/k/v must be contiguous f32")
    if rotary_dim is None:
        rotary_dim = head_dim
    if q_dtype is None:
        q_dtype = torch.float32
    if q_out is None:
        q_out = torch.empty(rows, n_head * head_dim, dtype=q_dtype, device=q.device)
    if kv_stride is None:
        kv_stride = n_kv_head * head_dim
    rc = L.lib().ullm_hip_qkv_append(
        _ptr(q), _ptr(k), _ptr(v), _ptr(q_bias), _ptr(k_bias), _ptr(v_bias), _ptr(q_norm),
        _ptr(k_norm), float(eps), _ptr(rope_cs), rope_cs.shape[0], int(bool(neox)), rotary_dim,
        rows, start_pos, n_head, n_kv_head, head_dim, _ptr(q_out), _DT[q_out.dtype],
        _ptr(k_cache), _ptr(v_cache), _dt(k_cache), kv_stride, _stream(stream))
    L.check(rc)
    return q_out


_proj_ws = {}


def proj_workspace(rows, n_head, n_kv_head, head_dim, device="cuda"):
    """The (zeroed once, reusable) workspace ullm_hip_qkv_proj_append needs for
    this shape, or None; cached per shape and device."""
    n = int(L.lib().ullm_hip_qkv_proj_workspace_bytes(rows, n_head, n_kv_head, head_dim))
    if n == 0:
        return None
    key = (str(torch.device(device)), rows, n_head, n_kv_head, head_dim)
    if key not in _proj_ws:
        _proj_ws[key] = torch.zeros(n, dtype=torch.uint8, device=device)
    return _proj_ws[key]


def qkv_proj_append(x, w_q, w_k, w_v, k_cache, v_cache, rope_cs, *, start_pos, n_head,
                    n_kv_head, head_dim, rotary_dim=None, neox=True, q_norm=None, k_norm=None,
                    eps=1e-6, q_bias=None, k_bias=None, v_bias=None, q_out=None, q_dtype=None,
                    kv_stride=None, workspace=None, stream=None):
    """Q/K/V projection (matvec_q, math.rs:9-21) with the append fused in
    (lib.rs:857-914).  x: [rows, in_dim] f32; w_*: [out, in_dim] f32/f16/bf16.
    Returns q_out ([rows, n_head*D], q_dtype); K/V land in the cache.  The
    workspace defaults to a cached one per shape (one caller at a time, as for
    GpuForward)."""
    rows, in_dim = x.shape
    _need_cuda(x, w_q, w_k, w_v, k_cache, v_cache, rope_cs)
    if x.dtype != torch.float32 or not x.is_contiguous():
        raise L.UllmHipError(L.E_INVALID, "x must be contiguous f32")
    if not (w_q.dtype == w_k.dtype == w_v.dtype):
        raise L.UllmHipError(L.E_INVALID, "w_q/w_k/w_v must share one dtype")
    for w, n in ((w_q, n_head), (w_k, n_kv_head), (w_v, n_kv_head)):
        if tuple(w.shape) != (n * head_dim, in_dim) or not w.is_contiguous():
            raise L.UllmHipError(L.E_INVALID, f"weight shape {tuple(w.shape)} != ({n * head_dim}, {in_dim})")
    if rotary_dim is None:
        rotary_dim = head_dim
    if q_dtype is None:
        q_dtype = torch.float32
    if q_out is None:
        q_out = torch.empty(rows, n_head * head_dim, dtype=q_dtype, device=x.device)
    if kv_stride is None:
        kv_stride = n_kv_head * head_dim
    if workspace is None:
        workspace = proj_workspace(rows, n_head, n_kv_head, head_dim, x.device)
    wsb = 0 if workspace is None else workspace.numel() * workspace.element_size()
    rc = L.lib().ullm_hip_qkv_proj_append(
        _ptr(x), in_dim, _ptr(w_q), _ptr(w_k), _ptr(w_v), _dt(w_q), _ptr(q_bias), _ptr(k_bias),
        _ptr(v_bias), _ptr(q_norm), _ptr(k_norm), float(eps), _ptr(rope_cs), rope_cs.shape[0],
        int(bool(neox)), rotary_dim, rows, start_pos, n_head, n_kv_head, head_dim, _ptr(q_out),
        _DT[q_out.dtype], _ptr(k_cache), _ptr(v_cache), _dt(k_cache), kv_stride, _ptr(workspace),
        wsb, _stream(stream))
    L.check(rc)
    return q_out


def matmul(w, x, y=None, *, stream=None):
    """Batched projection y = x . w^T (forward.rs:675-726, shader.metal:519-566).
    w: [out, in] bf16; x: [n_cols, in] f32; y: [n_cols, out] f32 (allocated if
    None, else written in place, e.g. a view into an f32 KV cache)."""
    _need_cuda(w, x)
    if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1]:
        raise L.UllmHipError(L.E_INVALID, f"shapes w {tuple(w.shape)} x {tuple(x.shape)}")
    if x.dtype != torch.float32 or not x.is_contiguous() or not w.is_contiguous():
        raise L.UllmHipError(L.E_INVALID, "x must be contiguous f32 and w contiguous")
    n_cols, in_dim = x.shape
    out_dim = w.shape[0]
    if y is None:
        y = torch.empty(n_cols, out_dim, dtype=torch.float32, device=x.device)
    elif y.dtype != torch.float32 or tuple(y.shape) != (n_cols, out_dim) or not y.is_contiguous():
        raise L.UllmHipError(L.E_INVALID, "y must be contiguous f32 [n_cols, out]")
    L.check(L.lib().ullm_hip_matmul(_ptr(w), _dt(w), _ptr(x), _ptr(y), in_dim, out_dim, n_cols,
                                    _stream(stream)))
    return y


@dataclass
class AttnParams:
    """The attention fields of the reference's GpuParams (forward.rs:23-51)."""

    n_layer: int
    n_head: int
    n_kv_head: int
    head_dim: int
    n_ctx: int
    rope_theta: float = 10000.0
    eps: float = 1e-6
    rope_neox: bool = True
    rotary_dim: Optional[int] = None
    sliding_window: int = 0
    kv_dtype: torch.dtype = torch.float16


class GpuAttention:
    """Resident KV cache + the attention ops of one model, on one GPU.

    Mirrors what `GpuForward` owns and does for attention: the cache is
    `[n_layer][n_ctx][n_kv_head*head_dim]` (forward.rs:355-356), per-token
    decode appends then attends (forward.rs:414-466), batched prefill
    appends all rows then runs one causal attention (forward.rs:799-858),
    and Gemma-style local layers (`l % 6 != 5`) use the sliding window
    (forward.rs:450-454, :857).  Like GpuForward it is not thread-safe:
    one caller at a time (forward.rs:221-225).
    """

    def __init__(self, p: AttnParams, device="cuda"):
        if p.n_head % p.n_kv_head:
            raise L.UllmHipError(L.E_INVALID, "n_head must be a multiple of n_kv_head")
        self.p = p
        self.device = torch.device(device)
        self.rotary_dim = p.rotary_dim or p.head_dim
        self.kv_dim = p.n_kv_head * p.head_dim
        self.scale = 1.0 / math.sqrt(p.head_dim)
        shape = (p.n_layer, p.n_ctx, self.kv_dim)
        self.key_cache = torch.zeros(shape, dtype=p.kv_dtype, device=self.device)
        self.val_cache = torch.zeros(shape, dtype=p.kv_dtype, device=self.device)
        self.rope_cs = rope_table(p.n_ctx, self.rotary_dim, p.rope_theta, device=self.device)
        self.workspace = new_decode_workspace(1, p.n_head, p.n_kv_head, p.head_dim, p.n_ctx,
                                              0, self.device)
        # seq_lens for every position, uploaded once: decoding at pos passes
        # the device slice holding pos + 1 (no per-token copy or fill, nothing
        # for a captured graph to replay but kernels).
        self._lens = torch.arange(1, p.n_ctx + 1, dtype=torch.int32, device=self.device)

    def supports_batched_prefill(self) -> bool:
        """Prefill runs on MFMA for every cache dtype and head_dim (an f32
        cache with Q.K on bf16 hi + lo halves)."""
        return True

    def _window(self, layer: int) -> int:
        p = self.p
        return p.sliding_window if (p.sliding_window > 0 and layer % 6 != 5) else 0

    def _append(self, layer, q, k, v, start_pos, q_dtype, norms, biases):
        p = self.p
        qn, kn = norms
        qb, kb, vb = biases
        return qkv_append(q, k, v, self.key_cache[layer], self.val_cache[layer], self.rope_cs,
                          start_pos=start_pos, n_head=p.n_head, n_kv_head=p.n_kv_head,
                          head_dim=p.head_dim, rotary_dim=self.rotary_dim, neox=p.rope_neox,
                          q_norm=qn, k_norm=kn, eps=p.eps, q_bias=qb, k_bias=kb, v_bias=vb,
                          q_dtype=q_dtype)

    def forward(self, layer: int, q, k, v, pos: int, q_norm=None, k_norm=None, q_bias=None,
                k_bias=None, v_bias=None):
        """Decode one token: q [n_head*D], k/v [n_kv_head*D] f32 projections.
        Returns the attention output [n_head*D] f32."""
        p = self.p
        if not 0 <= pos < p.n_ctx:
            raise L.UllmHipError(L.E_INVALID, f"pos {pos} outside the context")
        qr = self._append(layer, q.view(1, -1), k.view(1, -1), v.view(1, -1), pos,
                          torch.float32, (q_norm, k_norm), (q_bias, k_bias, v_bias))
        out = attn_decode(qr.view(1, p.n_head, p.head_dim), self.key_cache[layer],
                          self.val_cache[layer], self._lens[pos:pos + 1], pos + 1, p.n_kv_head,
                          window=self._window(layer), scale=self.scale,
                          workspace=self.workspace)
        return out.view(-1)

    def forward_batch(self, layer: int, q, k, v, start_pos: int = 0, q_norm=None, k_norm=None,
                      q_bias=None, k_bias=None, v_bias=None):
        """Prefill S tokens at start_pos..: q [S, n_head*D], k/v [S, kv_dim] f32.
        Returns the attention output [S, n_head*D] f32."""
        p = self.p
        S = q.shape[0]
        if start_pos + S > p.n_ctx:
            raise L.UllmHipError(L.E_INVALID, "prompt exceeds the context")
        qr = self._append(layer, q, k, v, start_pos, p.kv_dtype, (q_norm, k_norm),
                          (q_bias, k_bias, v_bias))
        return attn_prefill(qr, self.key_cache[layer], self.val_cache[layer], p.n_head,
                            p.n_kv_head, p.head_dim, start_pos=start_pos,
                            window=self._window(layer), scale=self.scale)

    # ---- attention blocks from the normed hidden state ----

    def forward_proj(self, layer: int, xb, pos: int, wq, wk, wv, q_norm=None, k_norm=None,
                     q_bias=None, k_bias=None, v_bias=None):
        """Decode one token from the attention-normed hidden state xb [n_embd]
        f32 (forward.rs:415-466): the Q/K/V matvecs with bias, norm, RoPE and
        the cache store fused into one launch, then decode attention."""
        p = self.p
        if not 0 <= pos < p.n_ctx:
            raise L.UllmHipError(L.E_INVALID, f"pos {pos} outside the context")
        qr = qkv_proj_append(xb.view(1, -1), wq, wk, wv, self.key_cache[layer],
                             self.val_cache[layer], self.rope_cs, start_pos=pos,
                             n_head=p.n_head, n_kv_head=p.n_kv_head, head_dim=p.head_dim,
                             rotary_dim=self.rotary_dim, neox=p.rope_neox, q_norm=q_norm,
                             k_norm=k_norm, eps=p.eps, q_bias=q_bias, k_bias=k_bias,
                             v_bias=v_bias, q_dtype=torch.float32)
        out = attn_decode(qr.view(1, p.n_head, p.head_dim), self.key_cache[layer],
                          self.val_cache[layer], self._lens[pos:pos + 1], pos + 1, p.n_kv_head,
                          window=self._window(layer), scale=self.scale,
                          workspace=self.workspace)
        return out.view(-1)

    def forward_batch_proj(self, layer: int, xbs, wq, wk, wv, start_pos: int = 0, q_norm=None,
                           k_norm=None, q_bias=None, k_bias=None, v_bias=None):
        """Prefill S tokens from the attention-normed hidden states xbs
        [S, n_embd] f32 (forward.rs:799-858): with bf16 weights the three
        projections run as MFMA matmuls (forward.rs:799-801), then the fused
        append and causal prefill attention; other weight dtypes use the
        fused projection kernel over the S rows."""
        p = self.p
        S = xbs.shape[0]
        if start_pos + S > p.n_ctx:
            raise L.UllmHipError(L.E_INVALID, "prompt exceeds the context")
        if wq.dtype == torch.bfloat16:
            q = matmul(wq, xbs)
            k = matmul(wk, xbs)
            v = matmul(wv, xbs)
            return self.forward_batch(layer, q, k, v, start_pos, q_norm, k_norm, q_bias, k_bias,
                                      v_bias)
        q_dtype = torch.float32 if p.kv_dtype == torch.float32 else p.kv_dtype
        qr = qkv_proj_append(xbs, wq, wk, wv, self.key_cache[layer], self.val_cache[layer],
                             self.rope_cs, start_pos=start_pos, n_head=p.n_head,
                             n_kv_head=p.n_kv_head, head_dim=p.head_dim,
                             rotary_dim=self.rotary_dim, neox=p.rope_neox, q_norm=q_norm,
                             k_norm=k_norm, eps=p.eps, q_bias=q_bias, k_bias=k_bias,
                             v_bias=v_bias, q_dtype=q_dtype)
        return attn_prefill(qr, self.key_cache[layer], self.val_cache[layer], p.n_head,
                            p.n_kv_head, p.head_dim, start_pos=start_pos,
                            window=self._window(layer), scale=self.scale)


    # ---- numerical debugging ----

    def forward_debug(self, xb, pos: int, wq, wk, wv, q_norm=None, k_norm=None, q_bias=None,
                      k_bias=None, v_bias=None, layer: int = 0, log=True):
        """The attention half of GpuForward::forward_debug (forward.rs:530-635):
        layer 0's attention one op at a time from the normed hidden state xb,
        each op its own launch followed by a synchronisation, reporting the
        NaN count, inf count and largest finite |value| of every intermediate
        (printed as `[dbg posP] label nan=.. inf=.. maxabs=..` when `log`, as
        the reference prints them).  The fused kernels are run with their
        later stages switched off to expose the intermediates: the raw
        projections come from the fused projection at position 0 with no
        norm or bias (RoPE at position 0 is the identity), then the bias,
        the Q/K norms and RoPE follow as appends into scratch rows, and the
        last append writes the cache row exactly as forward_proj does.  The
        attention scores are never materialised by this path, so the report
        goes from rope_k to attn_out.  Returns (attention output, report:
        a list of (label, nan, inf, maxabs))."""
        p = self.p
        if not 0 <= pos < p.n_ctx:
            raise L.UllmHipError(L.E_INVALID, f"pos {pos} outside the context")
        report = []

        def check(t, label):
            torch.cuda.synchronize()
            v = t.detach().float().reshape(-1).cpu()
            nan = int(torch.isnan(v).sum())
            inf = int(torch.isinf(v).sum())
            fin = v[torch.isfinite(v)]
            mx = float(fin.abs().max()) if fin.numel() else 0.0
            report.append((label, nan, inf, mx))
            if log:
                import sys

                print(f"[dbg pos{pos}] {label:<14} nan={nan} inf={inf} maxabs={mx:.4f}",
                      file=sys.stderr)

        dev, kd = self.device, self.kv_dim
        x = xb.view(1, -1)
        check(x, "attn_in")
        # raw projections: scratch f32 K/V row 0, identity RoPE, no norm/bias
        sk = torch.zeros(1, kd, device=dev)
        sv = torch.zeros_like(sk)
        q_raw = qkv_proj_append(x, wq, wk, wv, sk, sv, self.rope_cs, start_pos=0,
                                n_head=p.n_head, n_kv_head=p.n_kv_head, head_dim=p.head_dim,
                                rotary_dim=self.rotary_dim, neox=p.rope_neox,
                                q_dtype=torch.float32)
        k_raw, v_raw = sk.clone(), sv.clone()
        check(q_raw, "wq")
        check(k_raw, "wk")
        check(v_raw, "wv")

        def scratch_append(norms, biases, at):
            ck = torch.zeros(at + 1, kd, device=dev)
            cv = torch.zeros_like(ck)
            qo = qkv_append(q_raw, k_raw, v_raw, ck, cv, self.rope_cs, start_pos=at,
                            n_head=p.n_head, n_kv_head=p.n_kv_head, head_dim=p.head_dim,
                            rotary_dim=self.rotary_dim, neox=p.rope_neox, q_norm=norms[0],
                            k_norm=norms[1], eps=p.eps, q_bias=biases[0], k_bias=biases[1],
                            v_bias=biases[2], q_dtype=torch.float32)
            return qo, ck[at], cv[at]

        biases = (q_bias, k_bias, v_bias)
        if any(b is not None for b in biases):
            qb_, kb_, vb_ = scratch_append((None, None), biases, 0)
            check(qb_, "bias_q")
            check(kb_, "bias_k")
            check(vb_, "bias_v")
        if q_norm is not None or k_norm is not None:
            qn_, kn_, _ = scratch_append((q_norm, k_norm), biases, 0)
            if q_norm is not None:
                check(qn_, "q_norm")
            if k_norm is not None:
                check(kn_, "k_norm")
        # the real append: RoPE at pos, K/V into the cache (as forward_proj)
        qr = self._append(layer, q_raw, k_raw, v_raw, pos, torch.float32, (q_norm, k_norm),
                          biases)
        check(qr, "rope_q")
        check(self.key_cache[layer, pos], "rope_k")
        out = attn_decode(qr.view(1, p.n_head, p.head_dim), self.key_cache[layer],
                          self.val_cache[layer], self._lens[pos:pos + 1], pos + 1, p.n_kv_head,
                          window=self._window(layer), scale=self.scale,
                          workspace=self.workspace)
        check(out, "attn_out")
        return out.view(-1), report
