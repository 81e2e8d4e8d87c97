//! HIP attention for uLLM on MI355X: the attention half of the reference's
//! `GpuForward` (crates/ullm-metal/src/forward.rs:22-366), over the C ABI of
//! libullm_hip.so (include/ullm_hip.h).
//!
//! `HipAttention` owns what `GpuForward` owns for attention -- the KV cache
//! `[n_layer][n_ctx][n_kv_head * head_dim]` (forward.rs:355-356), the RoPE
//! table and the workspaces -- and keeps its surface: `new`, per-token
//! `forward` (forward.rs:384, attention part :415-466), batched
//! `forward_batch` (forward.rs:757, attention part :799-858) and
//! `supports_batched_prefill` (forward.rs:744).  Like `GpuForward` it is
//! `Send` but not `Sync`: one caller at a time (forward.rs:221-225).
//!
//! Not compiled here: the build image of this repository has no cargo.
//! Every call it makes is one the repository's tests drive through ctypes.
use std::os::raw::{c_int, c_void};

use ullm_core::{Error, Result};

pub mod ffi;

mod hip {
    use std::os::raw::{c_int, c_void};
    #[link(name = "amdhip64")]
    unsafe extern "C" {
        pub fn hipMalloc(p: *mut *mut c_void, bytes: usize) -> c_int;
        pub fn hipFree(p: *mut c_void) -> c_int;
        pub fn hipMemset(p: *mut c_void, v: c_int, bytes: usize) -> c_int;
        pub fn hipMemcpy(dst: *mut c_void, src: *const c_void, bytes: usize, kind: c_int) -> c_int;
    }
    pub const H2D: c_int = 1;
    pub const D2H: c_int = 2;
}

/// One device allocation, zeroed, freed on drop.
pub struct DevBuf {
    ptr: *mut c_void,
    bytes: usize,
}

impl DevBuf {
    pub fn zeroed(bytes: usize) -> Result<Self> {
        let mut ptr = std::ptr::null_mut();
        let n = bytes.max(256);
        if unsafe { hip::hipMalloc(&mut ptr, n) } != 0 {
            return Err(Error::Format(format!("hipMalloc of {n} bytes failed")));
        }
        let buf = Self { ptr, bytes: n };
        if unsafe { hip::hipMemset(ptr, 0, n) } != 0 {
            return Err(Error::Format("hipMemset failed".into()));
        }
        Ok(buf)
    }
    pub fn from_slice<T: Copy>(src: &[T]) -> Result<Self> {
        let b = Self::zeroed(std::mem::size_of_val(src))?;
        b.upload(src, 0)?;
        Ok(b)
    }
    /// Copy `src` to byte offset `off` (synchronous).
    pub fn upload<T: Copy>(&self, src: &[T], off: usize) -> Result<()> {
        let n = std::mem::size_of_val(src);
        if off + n > self.bytes {
            return Err(Error::Format(format!("upload of {n} bytes at {off} past {}", self.bytes)));
        }
        let rc = unsafe { hip::hipMemcpy(self.at(off), src.as_ptr().cast(), n, hip::H2D) };
        (rc == 0).then_some(()).ok_or_else(|| Error::Format("hipMemcpy H2D failed".into()))
    }
    /// Copy to host from the start of the buffer (synchronous: this is the
    /// one synchronisation point of a step, as commit + wait is in Metal).
    pub fn download(&self, dst: &mut [f32]) -> Result<()> {
        let n = std::mem::size_of_val(dst);
        if n > self.bytes {
            return Err(Error::Format(format!("download of {n} bytes past {}", self.bytes)));
        }
        let rc = unsafe { hip::hipMemcpy(dst.as_mut_ptr().cast(), self.ptr, n, hip::D2H) };
        (rc == 0).then_some(()).ok_or_else(|| Error::Format("hipMemcpy D2H failed".into()))
    }
    pub fn ptr(&self) -> *mut c_void {
        self.ptr
    }
    pub fn at(&self, byte_off: usize) -> *mut c_void {
        unsafe { self.ptr.cast::<u8>().add(byte_off).cast() }
    }
}

impl Drop for DevBuf {
    fn drop(&mut self) {
        unsafe { hip::hipFree(self.ptr) };
    }
}

/// The attention fields of GpuParams (forward.rs:23-51), plus the cache
/// dtype (ffi::ULLM_DT_*; the reference's cache is f32).
#[derive(Debug, Clone, Copy)]
pub struct AttnParams {
    pub n_layer: usize,
    pub n_head: usize,
    pub n_kv_head: usize,
    pub head_dim: usize,
    pub n_ctx: usize,
    pub rope_theta: f32,
    pub eps: f32,
    pub rope_neox: bool,
    /// Rotated dims per head (math.rs:116-161); 0 means head_dim.  Dims past
    /// it pass through unrotated.
    pub rotary_dim: usize,
    pub sliding_window: usize,
    pub kv_dtype: c_int,
}

/// Per-layer Q/K RMSNorm weights and Q/K/V biases, already on the device
/// (uploaded with the weights, as GpuForward::new does).
#[derive(Default, Clone, Copy)]
pub struct HeadParams<'a> {
    pub q_norm: Option<&'a DevBuf>,
    pub k_norm: Option<&'a DevBuf>,
    pub q_bias: Option<&'a DevBuf>,
    pub k_bias: Option<&'a DevBuf>,
    pub v_bias: Option<&'a DevBuf>,
}

fn dev_f32(b: Option<&DevBuf>) -> *const f32 {
    b.map_or(std::ptr::null(), |b| b.ptr as *const f32)
}

pub struct HipAttention {
    p: AttnParams,
    rd: usize,
    kv_dim: usize,
    elt: usize,
    key_cache: DevBuf,
    val_cache: DevBuf,
    rope_cs: DevBuf,
    /// 1..=n_ctx as i32, uploaded once: the decode at `pos` passes the device
    /// address of entry `pos` (= pos + 1) as its seq_lens, so no step
    /// uploads a length (and a captured step replays kernels only).
    lens: DevBuf,
    ws: DevBuf,
    ws_bytes: usize,
    q: DevBuf,
    kv: DevBuf,
    out: DevBuf,
}

unsafe impl Send for HipAttention {}

impl HipAttention {
    pub fn new(p: AttnParams) -> Result<Self> {
        if p.n_kv_head == 0 || p.n_head % p.n_kv_head != 0 {
            return Err(Error::Format("n_head must be a multiple of n_kv_head".into()));
        }
        let rd = if p.rotary_dim == 0 { p.head_dim } else { p.rotary_dim };
        let kv_dim = p.n_kv_head * p.head_dim;
        let q_dim = p.n_head * p.head_dim;
        let elt = if p.kv_dtype == ffi::ULLM_DT_F32 { 4 } else { 2 };
        let cache = p.n_layer * p.n_ctx * kv_dim * elt;
        let mut cs = vec![0f32; p.n_ctx * rd];
        ffi::check(unsafe {
            ffi::ullm_hip_rope_table(cs.as_mut_ptr(), p.n_ctx as c_int, rd as c_int, p.rope_theta)
        })?;
        let lens: Vec<i32> = (1..=p.n_ctx as i32).collect();
        let ws_bytes = unsafe {
            ffi::ullm_hip_decode_workspace_bytes(1, p.n_head as c_int, p.n_kv_head as c_int,
                                                 p.head_dim as c_int, p.n_ctx as c_int, 0)
        };
        Ok(Self {
            p,
            rd,
            kv_dim,
            elt,
            key_cache: DevBuf::zeroed(cache)?,
            val_cache: DevBuf::zeroed(cache)?,
            rope_cs: DevBuf::from_slice(&cs)?,
            lens: DevBuf::from_slice(&lens)?,
            ws: DevBuf::zeroed(ws_bytes)?,
            ws_bytes,
            q: DevBuf::zeroed(p.n_ctx * q_dim * 4)?,
            kv: DevBuf::zeroed(2 * p.n_ctx * kv_dim * 4)?,
            out: DevBuf::zeroed(p.n_ctx * q_dim * 4)?,
        })
    }

    pub fn supports_batched_prefill(&self) -> bool {
        true
    }

    /// Gemma-style local layers (forward.rs:450-454): every layer but each
    /// sixth uses the sliding window.
    fn window(&self, layer: usize) -> c_int {
        if self.p.sliding_window > 0 && layer % 6 != 5 {
            self.p.sliding_window as c_int
        } else {
            0
        }
    }
    fn layer_off(&self, layer: usize) -> usize {
        layer * self.p.n_ctx * self.kv_dim * self.elt
    }
    fn scale(&self) -> f32 {
        (self.p.head_dim as f32).sqrt().recip() // forward.rs:399
    }

    /// Bias, Q/K norm, RoPE and the cache store of `rows` token rows at
    /// positions start.. (lib.rs:1021-1058): f32 q/k/v in the `q`/`kv`
    /// scratch, q out in `q_dtype` into `q_out`.
    fn append(&self, layer: usize, rows: usize, start: usize, hp: HeadParams,
              q_out: *mut c_void, q_dtype: c_int) -> Result<()> {
        let (p, kd) = (&self.p, self.kv_dim);
        let off = self.layer_off(layer);
        ffi::check(unsafe {
            ffi::ullm_hip_qkv_append(
                self.q.ptr.cast(), self.kv.ptr.cast(), self.kv.at(rows * kd * 4).cast(),
                dev_f32(hp.q_bias), dev_f32(hp.k_bias), dev_f32(hp.v_bias),
                dev_f32(hp.q_norm), dev_f32(hp.k_norm), p.eps, self.rope_cs.ptr.cast(),
                p.n_ctx as c_int, p.rope_neox as c_int, self.rd as c_int, rows as c_int,
                start as c_int, p.n_head as c_int, p.n_kv_head as c_int, p.head_dim as c_int,
                q_out, q_dtype, self.key_cache.at(off), self.val_cache.at(off), p.kv_dtype,
                kd as i64, std::ptr::null_mut())
        })
    }

    /// Decode one token at `pos` from its f32 projections q [n_head*D] and
    /// k/v [kv_dim] (before bias, norm and RoPE): append, then attend
    /// (forward.rs:415-466; lib.rs:857-938).  Returns [n_head*D] f32.
    pub fn forward(&self, layer: usize, q: &[f32], k: &[f32], v: &[f32], pos: usize,
                   hp: HeadParams) -> Result<Vec<f32>> {
        let (p, kd) = (&self.p, self.kv_dim);
        if pos >= p.n_ctx {
            return Err(Error::Format(format!("pos {pos} >= n_ctx {}", p.n_ctx)));
        }
        self.q.upload(q, 0)?;
        self.kv.upload(k, 0)?;
        self.kv.upload(v, kd * 4)?;
        self.append(layer, 1, pos, hp, self.q.ptr, ffi::ULLM_DT_F32)?;
        let off = self.layer_off(layer);
        ffi::check(unsafe {
            ffi::ullm_hip_attn_decode(
                self.q.ptr.cast(), self.key_cache.at(off), self.val_cache.at(off), p.kv_dtype,
                kd as i64, 0, self.lens.at(pos * 4).cast(), (pos + 1) as c_int,
                self.window(layer), 1, p.n_head as c_int, p.n_kv_head as c_int,
                p.head_dim as c_int, self.scale(), self.out.ptr.cast(), self.ws.ptr,
                self.ws_bytes, std::ptr::null_mut())
        })?;
        let mut o = vec![0f32; p.n_head * p.head_dim];
        self.out.download(&mut o)?;
        Ok(o)
    }

    /// Prefill s tokens at positions 0..s from their f32 projections qs
    /// [s][n_head*D] and ks/vs [s][kv_dim] (forward.rs:799-858;
    /// lib.rs:1021-1087).  Returns [s][n_head*D] f32.
    ///  * f16/bf16 cache: q goes out in the cache dtype, then one causal
    ///    prefill launch on the matrix cores.
    ///  * f32 cache (the reference's own): q stays f32 and the prefill
    ///    kernel runs Q.K on bf16 hi + lo halves.
    pub fn forward_batch(&self, layer: usize, qs: &[f32], ks: &[f32], vs: &[f32], s: usize,
                         hp: HeadParams) -> Result<Vec<f32>> {
        let (p, kd) = (&self.p, self.kv_dim);
        if s == 0 || s > p.n_ctx {
            return Err(Error::Format(format!("prompt of {s} tokens for n_ctx {}", p.n_ctx)));
        }
        self.q.upload(qs, 0)?;
        self.kv.upload(ks, 0)?;
        self.kv.upload(vs, s * kd * 4)?;
        let off = self.layer_off(layer);
        // 16-bit caches: q in the cache dtype goes to `out` and the
        // attention writes its f32 rows to `q`.  An f32 cache: q is prepared
        // in place in `q` and the attention writes `out`.
        let q_prep = if p.kv_dtype == ffi::ULLM_DT_F32 { self.q.ptr } else { self.out.ptr };
        let o_dst = if p.kv_dtype == ffi::ULLM_DT_F32 { self.out.ptr } else { self.q.ptr };
        self.append(layer, s, 0, hp, q_prep, p.kv_dtype)?;
        ffi::check(unsafe {
            ffi::ullm_hip_attn_prefill(
                q_prep, self.key_cache.at(off), self.val_cache.at(off), p.kv_dtype,
                kd as i64, s as c_int, 0, self.window(layer), p.n_head as c_int,
                p.n_kv_head as c_int, p.head_dim as c_int, self.scale(), o_dst.cast(),
                std::ptr::null_mut())
        })?;
        if p.kv_dtype != ffi::ULLM_DT_F32 {
            let mut o = vec![0f32; s * p.n_head * p.head_dim];
            self.q.download(&mut o)?;
            return Ok(o);
        }
        let mut o = vec![0f32; s * p.n_head * p.head_dim];
        self.out.download(&mut o)?;
        Ok(o)
    }
}
