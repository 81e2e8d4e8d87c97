//! HIP attention for uLLM on MI355X: the attention half of the reference's
//! `GpuForward` (crates/ullm-metal/src/forward.rs:22-366), over the C ABI of
//! libullm_hip.so (include/ullm_hip.h).
//!
//! `HipAttention` owns what `GpuForward` owns for attention -- the KV cache
//! `[n_layer][n_ctx][n_kv_head * head_dim]` (forward.rs:355-356), the RoPE
//! table and the workspaces -- and keeps its surface: `new`, per-token
//! `forward` (forward.rs:384, attention part :415-466), batched
//! `forward_batch` (forward.rs:757, attention part :799-858),
//! `supports_batched_prefill` (forward.rs:744) and `forward_debug`
//! (forward.rs:530-635).  Like `GpuForward` it is `Send` but not `Sync`: one
//! caller at a time (forward.rs:221-225).
//!
//! Device-resident path: `forward_dev` / `forward_batch_dev` take device
//! views (`DevSlice`) of the f32 projections and the output, queue the fused
//! append and the attention on one stream, and neither copy nor wait, so a
//! whole token's layers run back to back and the caller synchronises once
//! (`synchronize`), as GpuForward commits one command buffer and waits once
//! (forward.rs:406-509).  `forward` / `forward_batch` are host-slice
//! conveniences over them (upload, run, read back).
//!
//! Unverified: the build image of this repository has no cargo, so this
//! crate has never been compiled or run.  Every C entry point it calls is
//! one the repository's tests drive through ctypes.
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
        pub fn hipStreamSynchronize(stream: *mut c_void) -> c_int;
    }
    pub const H2D: c_int = 1;
    pub const D2H: c_int = 2;
}

/// One device allocation, zeroed, freed on drop.
pub struct DevBuf {
    ptr: *mut c_void,
    bytes: usize,
}

/// A borrowed byte range of device memory: what the `*_dev` calls take for
/// their inputs and outputs, so a step's tensors stay on the device
/// (GpuForward keeps q, the K/V rows and the attention output in its own
/// Metal buffers, forward.rs:384-515).
#[derive(Clone, Copy, Debug)]
pub struct DevSlice {
    ptr: *mut c_void,
    bytes: usize,
}

impl DevSlice {
    /// A view of raw device memory the caller owns (e.g. its projection
    /// outputs).  Safety: `ptr` must address `bytes` of device memory that
    /// outlives every call given this view.
    pub unsafe fn from_raw(ptr: *mut c_void, bytes: usize) -> Self {
        Self { ptr, bytes }
    }
    pub fn ptr(&self) -> *mut c_void {
        self.ptr
    }
    pub fn bytes(&self) -> usize {
        self.bytes
    }
    fn need_f32(&self, n: usize, what: &str) -> Result<*mut f32> {
        if self.bytes < n * 4 {
            return Err(Error::Format(format!("{what}: {} bytes for {n} f32", self.bytes)));
        }
        Ok(self.ptr.cast())
    }
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
    /// Copy `dst.len()` elements from byte offset `off` to host
    /// (synchronous: it waits for the work queued before it, as commit +
    /// wait does in Metal).
    pub fn download_at<T: Copy>(&self, dst: &mut [T], off: usize) -> Result<()> {
        let n = std::mem::size_of_val(dst);
        if off + n > self.bytes {
            return Err(Error::Format(format!("download of {n} bytes at {off} past {}", self.bytes)));
        }
        let rc = unsafe { hip::hipMemcpy(dst.as_mut_ptr().cast(), self.at(off), n, hip::D2H) };
        (rc == 0).then_some(()).ok_or_else(|| Error::Format("hipMemcpy D2H failed".into()))
    }
    pub fn download(&self, dst: &mut [f32]) -> Result<()> {
        self.download_at(dst, 0)
    }
    pub fn ptr(&self) -> *mut c_void {
        self.ptr
    }
    pub fn at(&self, byte_off: usize) -> *mut c_void {
        unsafe { self.ptr.cast::<u8>().add(byte_off).cast() }
    }
    /// The whole buffer as a device view.
    pub fn view(&self) -> DevSlice {
        DevSlice { ptr: self.ptr, bytes: self.bytes }
    }
    /// `bytes` from byte offset `off` as a device view.
    pub fn slice(&self, off: usize, bytes: usize) -> Result<DevSlice> {
        if off + bytes > self.bytes {
            return Err(Error::Format(format!("view of {bytes} bytes at {off} past {}", self.bytes)));
        }
        Ok(DevSlice { ptr: self.at(off), bytes })
    }
}

impl Drop for DevBuf {
    fn drop(&mut self) {
        unsafe { hip::hipFree(self.ptr) };
    }
}

/// NaN count, inf count and largest finite |value|: one line of
/// `forward_debug`'s report (forward.rs:558-569).
#[derive(Debug, Clone)]
pub struct DebugStat {
    pub label: &'static str,
    pub nan: usize,
    pub inf: usize,
    pub maxabs: f32,
}

fn stat(label: &'static str, v: &[f32]) -> DebugStat {
    let nan = v.iter().filter(|x| x.is_nan()).count();
    let inf = v.iter().filter(|x| x.is_infinite()).count();
    let maxabs = v.iter().copied().filter(|x| x.is_finite()).fold(0f32, |a, b| a.max(b.abs()));
    DebugStat { label, nan, inf, maxabs }
}

/// 16-bit cache element -> f32 (the cache dtype's own bits).
fn half_to_f32(h: u16, dtype: c_int) -> f32 {
    if dtype == ffi::ULLM_DT_BF16 {
        return f32::from_bits((h as u32) << 16);
    }
    let neg = h >> 15 != 0;
    let exp = ((h >> 10) & 0x1f) as i32;
    let man = (h & 0x3ff) as u32;
    let mag = if exp == 0x1f {
        f32::from_bits(0x7f80_0000 | (man << 13))
    } else if exp == 0 {
        man as f32 * (2f32).powi(-24) // zero or subnormal
    } else {
        f32::from_bits((((exp - 15 + 127) as u32) << 23) | (man << 13))
    };
    if neg { -mag } else { mag }
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
    /// Prepared q (bias, norm, RoPE applied) in the dtype the attention
    /// reads: f32 for the decode and the f32-cache prefill, the cache dtype
    /// for a 16-bit prefill.  [n_ctx][n_head*D] f32 bytes.
    qprep: DevBuf,
    /// Staging for the host-slice wrappers only: q, k and v rows uploaded
    /// before the device path runs, and the output read back after it.
    host_in: DevBuf,
    host_out: DevBuf,
    /// The HIP stream every launch goes to (null: the default stream).
    stream: *mut c_void,
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
            qprep: DevBuf::zeroed(p.n_ctx * q_dim * 4)?,
            host_in: DevBuf::zeroed(p.n_ctx * (q_dim + 2 * kv_dim) * 4)?,
            host_out: DevBuf::zeroed(p.n_ctx * q_dim * 4)?,
            stream: std::ptr::null_mut(),
        })
    }

    pub fn supports_batched_prefill(&self) -> bool {
        true
    }

    /// Launch on `stream` (a hipStream_t; null = the default stream) from
    /// now on.  Safety: the stream must outlive this object's use of it.
    pub unsafe fn set_stream(&mut self, stream: *mut c_void) {
        self.stream = stream;
    }

    /// Wait for everything queued on this object's stream: the one
    /// synchronisation of a token, as commit + wait_until_completed ends
    /// GpuForward::forward (forward.rs:507-509).
    pub fn synchronize(&self) -> Result<()> {
        let rc = unsafe { hip::hipStreamSynchronize(self.stream) };
        (rc == 0).then_some(()).ok_or_else(|| Error::Format("hipStreamSynchronize failed".into()))
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
    fn q_dim(&self) -> usize {
        self.p.n_head * self.p.head_dim
    }
    fn check_layer(&self, layer: usize) -> Result<()> {
        if layer >= self.p.n_layer {
            return Err(Error::Format(format!("layer {layer} >= n_layer {}", self.p.n_layer)));
        }
        Ok(())
    }

    /// Bias, Q/K norm, RoPE and the cache store of `rows` token rows at
    /// positions start.. (lib.rs:1021-1058): f32 q/k/v rows on the device,
    /// q out in `q_dtype` into `q_out`.  Queued, not waited for.
    #[allow(clippy::too_many_arguments)]
    fn append(&self, layer: usize, rows: usize, start: usize, hp: HeadParams, q: *const f32,
              k: *const f32, v: *const f32, q_out: *mut c_void, q_dtype: c_int) -> Result<()> {
        let (p, kd) = (&self.p, self.kv_dim);
        let off = self.layer_off(layer);
        ffi::check(unsafe {
            ffi::ullm_hip_qkv_append(
                q, k, v, dev_f32(hp.q_bias), dev_f32(hp.k_bias), dev_f32(hp.v_bias),
                dev_f32(hp.q_norm), dev_f32(hp.k_norm), p.eps, self.rope_cs.ptr as *const f32,
                p.n_ctx as c_int, p.rope_neox as c_int, self.rd as c_int, rows as c_int,
                start as c_int, p.n_head as c_int, p.n_kv_head as c_int, p.head_dim as c_int,
                q_out, q_dtype, self.key_cache.at(off), self.val_cache.at(off), p.kv_dtype,
                kd as i64, self.stream)
        })
    }

    /// The decode attention of layer `layer` at `pos` over the prepared q in
    /// `qprep`, into `out`.  Queued, not waited for.
    fn decode(&self, layer: usize, pos: usize, out: *mut f32) -> Result<()> {
        let (p, kd) = (&self.p, self.kv_dim);
        let off = self.layer_off(layer);
        ffi::check(unsafe {
            ffi::ullm_hip_attn_decode(
                self.qprep.ptr as *const f32, self.key_cache.at(off), self.val_cache.at(off),
                p.kv_dtype, kd as i64, 0, self.lens.at(pos * 4) as *const i32, (pos + 1) as c_int,
                self.window(layer), 1, p.n_head as c_int, p.n_kv_head as c_int,
                p.head_dim as c_int, self.scale(), out, self.ws.ptr, self.ws_bytes, self.stream)
        })
    }

    /// Decode one token at `pos` with every tensor on the device: q
    /// [n_head*D] and k/v [kv_dim] f32 projections (before bias, norm and
    /// RoPE) in, [n_head*D] f32 attention output out.  Appends the K/V row to
    /// layer `layer`'s cache, then attends (forward.rs:415-466;
    /// lib.rs:857-938).  Two launches are queued on the stream and nothing
    /// is copied or waited for: the caller runs its other layers and calls
    /// `synchronize` once per token.
    pub fn forward_dev(&self, layer: usize, q: DevSlice, k: DevSlice, v: DevSlice, pos: usize,
                       hp: HeadParams, out: DevSlice) -> Result<()> {
        let (p, kd, qd) = (&self.p, self.kv_dim, self.q_dim());
        self.check_layer(layer)?;
        if pos >= p.n_ctx {
            return Err(Error::Format(format!("pos {pos} >= n_ctx {}", p.n_ctx)));
        }
        let (qp, kp, vp) = (q.need_f32(qd, "q")?, k.need_f32(kd, "k")?, v.need_f32(kd, "v")?);
        let op = out.need_f32(qd, "out")?;
        self.append(layer, 1, pos, hp, qp, kp, vp, self.qprep.ptr, ffi::ULLM_DT_F32)?;
        self.decode(layer, pos, op)
    }

    /// Prefill s tokens at positions 0..s with every tensor on the device:
    /// qs [s][n_head*D] and ks/vs [s][kv_dim] f32 projections in, [s][n_head*D]
    /// f32 out (forward.rs:799-858; lib.rs:1021-1087).  Queued, not waited for.
    ///  * f16/bf16 cache: q is prepared in the cache dtype, then one causal
    ///    prefill launch on the matrix cores.
    ///  * f32 cache (the reference's own): q stays f32 and the prefill
    ///    kernel runs Q.K on bf16 hi + lo halves.
    #[allow(clippy::too_many_arguments)]
    pub fn forward_batch_dev(&self, layer: usize, qs: DevSlice, ks: DevSlice, vs: DevSlice,
                             s: usize, hp: HeadParams, out: DevSlice) -> Result<()> {
        let (p, kd, qd) = (&self.p, self.kv_dim, self.q_dim());
        self.check_layer(layer)?;
        if s == 0 || s > p.n_ctx {
            return Err(Error::Format(format!("prompt of {s} tokens for n_ctx {}", p.n_ctx)));
        }
        let qp = qs.need_f32(s * qd, "qs")?;
        let (kp, vp) = (ks.need_f32(s * kd, "ks")?, vs.need_f32(s * kd, "vs")?);
        let op = out.need_f32(s * qd, "out")?;
        self.append(layer, s, 0, hp, qp, kp, vp, self.qprep.ptr, p.kv_dtype)?;
        let off = self.layer_off(layer);
        ffi::check(unsafe {
            ffi::ullm_hip_attn_prefill(
                self.qprep.ptr, self.key_cache.at(off), self.val_cache.at(off), p.kv_dtype,
                kd as i64, s as c_int, 0, self.window(layer), p.n_head as c_int,
                p.n_kv_head as c_int, p.head_dim as c_int, self.scale(), op, self.stream)
        })
    }

    /// Host-slice form of `forward_dev` for callers whose projections live in
    /// host memory: checks the slice lengths, uploads them, runs the device
    /// path and reads the output back (the read is the step's one wait).
    pub fn forward(&self, layer: usize, q: &[f32], k: &[f32], v: &[f32], pos: usize,
                   hp: HeadParams) -> Result<Vec<f32>> {
        let (kd, qd) = (self.kv_dim, self.q_dim());
        if q.len() != qd || k.len() != kd || v.len() != kd {
            return Err(Error::Format(format!(
                "q/k/v of {}/{}/{} floats, expected {qd}/{kd}/{kd}", q.len(), k.len(), v.len())));
        }
        let (qv, kv, vv) = self.stage(q, k, v, 1)?;
        self.forward_dev(layer, qv, kv, vv, pos, hp, self.host_out.view())?;
        let mut o = vec![0f32; qd];
        self.host_out.download(&mut o)?;
        Ok(o)
    }

    /// Host-slice form of `forward_batch_dev` (lengths checked against s).
    pub fn forward_batch(&self, layer: usize, qs: &[f32], ks: &[f32], vs: &[f32], s: usize,
                         hp: HeadParams) -> Result<Vec<f32>> {
        let (p, kd, qd) = (&self.p, self.kv_dim, self.q_dim());
        if s == 0 || s > p.n_ctx {
            return Err(Error::Format(format!("prompt of {s} tokens for n_ctx {}", p.n_ctx)));
        }
        if qs.len() != s * qd || ks.len() != s * kd || vs.len() != s * kd {
            return Err(Error::Format(format!(
                "qs/ks/vs of {}/{}/{} floats, expected {}/{}/{} for {s} tokens",
                qs.len(), ks.len(), vs.len(), s * qd, s * kd, s * kd)));
        }
        let (qv, kv, vv) = self.stage(qs, ks, vs, s)?;
        self.forward_batch_dev(layer, qv, kv, vv, s, hp, self.host_out.view())?;
        let mut o = vec![0f32; s * qd];
        self.host_out.download(&mut o)?;
        Ok(o)
    }

    /// Upload host q/k/v rows into `host_in` and return device views of them.
    fn stage(&self, q: &[f32], k: &[f32], v: &[f32], rows: usize)
             -> Result<(DevSlice, DevSlice, DevSlice)> {
        let (kd, qd) = (self.kv_dim, self.q_dim());
        let (qb, kb) = (rows * qd * 4, rows * kd * 4);
        self.host_in.upload(q, 0)?;
        self.host_in.upload(k, qb)?;
        self.host_in.upload(v, qb + kb)?;
        Ok((self.host_in.slice(0, qb)?, self.host_in.slice(qb, kb)?,
            self.host_in.slice(qb + kb, kb)?))
    }

    /// The attention half of GpuForward::forward_debug (forward.rs:530-635):
    /// one decode step of layer `layer` at `pos`, one op at a time with a
    /// wait after each, reporting NaN count, inf count and largest finite
    /// |value| of every intermediate, printed as the reference prints them
    /// (`[dbg posP] label nan=.. inf=.. maxabs=..`): the raw projections,
    /// then q and the cache's K and V rows after the fused append (bias,
    /// norm, RoPE, store), then the attention output.  The fused decode
    /// never materialises the scores, so the report goes from rope_k to
    /// attn_out.  Unlike the device path it synchronises after every op.
    pub fn forward_debug(&self, layer: usize, q: &[f32], k: &[f32], v: &[f32], pos: usize,
                         hp: HeadParams) -> Result<Vec<DebugStat>> {
        let (p, kd, qd) = (&self.p, self.kv_dim, self.q_dim());
        self.check_layer(layer)?;
        if pos >= p.n_ctx {
            return Err(Error::Format(format!("pos {pos} >= n_ctx {}", p.n_ctx)));
        }
        if q.len() != qd || k.len() != kd || v.len() != kd {
            return Err(Error::Format(format!(
                "q/k/v of {}/{}/{} floats, expected {qd}/{kd}/{kd}", q.len(), k.len(), v.len())));
        }
        let mut rep = Vec::new();
        let mut log = |st: DebugStat| {
            eprintln!("[dbg pos{pos}] {:<14} nan={} inf={} maxabs={:.4}", st.label, st.nan,
                      st.inf, st.maxabs);
            rep.push(st);
        };
        log(stat("wq", q));
        log(stat("wk", k));
        log(stat("wv", v));
        let (qv, kv, vv) = self.stage(q, k, v, 1)?;
        self.append(layer, 1, pos, hp, qv.ptr as *const f32, kv.ptr as *const f32, vv.ptr as *const f32,
                    self.qprep.ptr, ffi::ULLM_DT_F32)?;
        self.synchronize()?;
        let mut buf = vec![0f32; qd];
        self.qprep.download(&mut buf)?;
        log(stat("rope_q", &buf));
        let row = self.layer_off(layer) + pos * kd * self.elt;
        for (cache, label) in [(&self.key_cache, "rope_k"), (&self.val_cache, "v_row")] {
            let vals = if p.kv_dtype == ffi::ULLM_DT_F32 {
                let mut r = vec![0f32; kd];
                cache.download_at(&mut r, row)?;
                r
            } else {
                let mut r = vec![0u16; kd];
                cache.download_at(&mut r, row)?;
                r.iter().map(|&h| half_to_f32(h, p.kv_dtype)).collect()
            };
            log(stat(label, &vals));
        }
        self.decode(layer, pos, self.host_out.ptr as *mut f32)?;
        self.synchronize()?;
        self.host_out.download(&mut buf)?;
        log(stat("attn_out", &buf));
        Ok(rep)
    }
}
