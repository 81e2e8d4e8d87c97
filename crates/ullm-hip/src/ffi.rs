//! extern "C" view of include/ullm_hip.h (one declaration per entry point).
//! Not compiled here (no cargo in the build image); checked against the
//! header by eye and by tests/test_rust_crate.py, which matches every
//! declared name and its argument count.
use std::os::raw::{c_char, c_int, c_void};

pub const ULLM_HIP_OK: c_int = 0;
pub const ULLM_HIP_E_INVALID: c_int = -1;
pub const ULLM_HIP_E_UNSUPPORTED: c_int = -2;
pub const ULLM_HIP_E_HIP: c_int = -3;
pub const ULLM_HIP_E_WORKSPACE: c_int = -4;
pub const ULLM_DT_F32: c_int = 0;
pub const ULLM_DT_F16: c_int = 1;
pub const ULLM_DT_BF16: c_int = 2;

// `unsafe extern`: required by edition 2024 (the workspace edition).
#[link(name = "ullm_hip")]
unsafe extern "C" {
    pub fn ullm_hip_version() -> *const c_char;
    pub fn ullm_hip_last_error() -> *const c_char;
    /// Measurement only (no GpuForward call site): one read-only pass over
    /// `bytes` of device memory, the floor the decode op is compared with.
    pub fn ullm_hip_stream_read(src: *const c_void, bytes: usize, workgroups: c_int,
        sink: *mut u32, stream: *mut c_void) -> c_int;
    pub fn ullm_hip_decode_workspace_bytes(batch: c_int, n_head: c_int, n_kv_head: c_int,
        head_dim: c_int, max_len: c_int, window: c_int) -> usize;
    pub fn ullm_hip_attn_decode(q: *const f32, k_cache: *const c_void, v_cache: *const c_void,
        kv_dtype: c_int, kv_stride: i64, seq_stride: i64, seq_lens: *const i32, max_len: c_int,
        window: c_int, batch: c_int, n_head: c_int, n_kv_head: c_int, head_dim: c_int,
        scale: f32, out: *mut f32, workspace: *mut c_void, workspace_bytes: usize,
        stream: *mut c_void) -> c_int;
    /// ullm_hip_attn_decode without a workspace (static per-GPU scratch);
    /// calls overlapping on one GPU race.
    pub fn ullm_hip_attn_decode_noalloc(q: *const f32, k_cache: *const c_void,
        v_cache: *const c_void, kv_dtype: c_int, kv_stride: i64, seq_stride: i64,
        seq_lens: *const i32, max_len: c_int, window: c_int, batch: c_int, n_head: c_int,
        n_kv_head: c_int, head_dim: c_int, scale: f32, out: *mut f32,
        stream: *mut c_void) -> c_int;
    pub fn ullm_hip_decode_noalloc_max_bytes() -> usize;
    pub fn ullm_hip_attn_prefill(q: *const c_void, k_cache: *const c_void,
        v_cache: *const c_void, dtype: c_int, kv_stride: i64, s: c_int, start_pos: c_int,
        window: c_int, n_head: c_int, n_kv_head: c_int, head_dim: c_int, scale: f32,
        out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn ullm_hip_rope_table(cs: *mut f32, n_pos: c_int, rotary_dim: c_int, theta: f32) -> c_int;
    pub fn ullm_hip_qkv_append(q_in: *const f32, k_in: *const f32, v_in: *const f32,
        q_bias: *const f32, k_bias: *const f32, v_bias: *const f32, q_norm: *const f32,
        k_norm: *const f32, eps: f32, rope_cs: *const f32, rope_n_pos: c_int, rope_neox: c_int,
        rotary_dim: c_int, rows: c_int, start_pos: c_int, n_head: c_int, n_kv_head: c_int,
        head_dim: c_int, q_out: *mut c_void, q_dtype: c_int, k_cache: *mut c_void,
        v_cache: *mut c_void, kv_dtype: c_int, kv_stride: i64, stream: *mut c_void) -> c_int;
    pub fn ullm_hip_qkv_proj_append(x: *const f32, in_dim: c_int, w_q: *const c_void,
        w_k: *const c_void, w_v: *const c_void, w_dtype: c_int, q_bias: *const f32,
        k_bias: *const f32, v_bias: *const f32, q_norm: *const f32, k_norm: *const f32,
        eps: f32, rope_cs: *const f32, rope_n_pos: c_int, rope_neox: c_int, rotary_dim: c_int,
        rows: c_int, start_pos: c_int, n_head: c_int, n_kv_head: c_int, head_dim: c_int,
        q_out: *mut c_void, q_dtype: c_int, k_cache: *mut c_void, v_cache: *mut c_void,
        kv_dtype: c_int, kv_stride: i64, workspace: *mut c_void, workspace_bytes: usize,
        stream: *mut c_void) -> c_int;
    pub fn ullm_hip_qkv_proj_workspace_bytes(rows: c_int, n_head: c_int, n_kv_head: c_int,
        head_dim: c_int) -> usize;
    pub fn ullm_hip_paged_decode_workspace_bytes(batch: c_int, n_head: c_int, n_kv_head: c_int,
        head_dim: c_int, max_len: c_int, window: c_int) -> usize;
    pub fn ullm_hip_attn_decode_paged(q: *const f32, k_pages: *const c_void,
        v_pages: *const c_void, kv_dtype: c_int, kv_stride: i64, page_size: c_int,
        n_pages: c_int, block_table: *const i32, table_stride: c_int, seq_lens: *const i32,
        max_len: c_int, window: c_int, batch: c_int, n_head: c_int, n_kv_head: c_int,
        head_dim: c_int, scale: f32, out: *mut f32, workspace: *mut c_void,
        workspace_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn ullm_hip_qkv_append_paged(q_in: *const f32, k_in: *const f32, v_in: *const f32,
        q_bias: *const f32, k_bias: *const f32, v_bias: *const f32, q_norm: *const f32,
        k_norm: *const f32, eps: f32, rope_cs: *const f32, rope_n_pos: c_int, rope_neox: c_int,
        rotary_dim: c_int, rows: c_int, positions: *const i32, n_head: c_int, n_kv_head: c_int,
        head_dim: c_int, q_out: *mut c_void, q_dtype: c_int, k_pages: *mut c_void,
        v_pages: *mut c_void, kv_dtype: c_int, kv_stride: i64, page_size: c_int, n_pages: c_int,
        block_table: *const i32, table_stride: c_int, stream: *mut c_void) -> c_int;
    pub fn ullm_hip_attn_prefill_paged(q: *const c_void, k_pages: *const c_void,
        v_pages: *const c_void, dtype: c_int, kv_stride: i64, page_size: c_int, n_pages: c_int,
        block_table: *const i32, table_len: c_int, s: c_int, start_pos: c_int, window: c_int,
        n_head: c_int, n_kv_head: c_int, head_dim: c_int, scale: f32, out: *mut f32,
        stream: *mut c_void) -> c_int;
    pub fn ullm_hip_matmul(w: *const c_void, w_dtype: c_int, x: *const f32, y: *mut f32,
        in_dim: c_int, out_dim: c_int, n_cols: c_int, stream: *mut c_void) -> c_int;
}

/// Status -> ullm_core::Error, as forward.rs:369-380 reports unsupported dtypes.
pub fn check(rc: c_int) -> ullm_core::Result<()> {
    if rc == ULLM_HIP_OK { return Ok(()); }
    let msg = unsafe { std::ffi::CStr::from_ptr(ullm_hip_last_error()) }
        .to_string_lossy().into_owned();
    Err(match rc {
        ULLM_HIP_E_UNSUPPORTED => ullm_core::Error::Unsupported(msg),
        _ => ullm_core::Error::Format(msg),
    })
}
