/*
 * ullm_hip.h -- C ABI of the MI355X (gfx950) attention path for uLLM.
 *
 * These entry points replace the attention ops that the reference's Metal
 * backend encodes inside `GpuForward` (crates/ullm-metal/src/forward.rs).
 * A Rust `ullm-hip` crate binds them with `extern "C"` and keeps the
 * `GpuForward::{new, forward, forward_batch}` surface unchanged.
 *
 * Conventions shared by every entry point:
 *  - All tensor pointers are DEVICE pointers owned by the caller.
 *  - `stream` is a hipStream_t (NULL = the default stream).  Calls are
 *    asynchronous on that stream; nothing synchronises the device.
 *  - The return value is a status: ULLM_HIP_OK (0) or a negative code.  The
 *    thread-local message of the last failure is ullm_hip_last_error().
 *    The Rust side maps ULLM_HIP_E_INVALID to `Error::Format` and
 *    ULLM_HIP_E_UNSUPPORTED to `Error::Unsupported`
 *    (crates/ullm-core/src/error.rs:11-18), as forward.rs:369-380 does for
 *    dtypes it cannot encode.
 *  - KV cache layout is the reference's, token-major per layer
 *    (crates/ullm-model/src/lib.rs:184-185, forward.rs:355-356):
 *    position t of kv head j starts at element  t*kv_stride + j*head_dim
 *    from the layer base, kv_stride = n_kv_head*head_dim for a dense cache.
 *    Element type is f32, f16 or bf16 (ullm_hip_dtype).
 *  - The library keeps no global mutable state besides the error string;
 *    calls on different streams may overlap if their buffers do not.
 */
#ifndef ULLM_HIP_H
#define ULLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ULLM_HIP_OK = 0,
    ULLM_HIP_E_INVALID = -1,     /* bad shape / argument                */
    ULLM_HIP_E_UNSUPPORTED = -2, /* dtype / head_dim combination absent */
    ULLM_HIP_E_HIP = -3,         /* HIP runtime error                   */
    ULLM_HIP_E_WORKSPACE = -4    /* workspace missing or too small      */
};

typedef enum { ULLM_DT_F32 = 0, ULLM_DT_F16 = 1, ULLM_DT_BF16 = 2 } ullm_hip_dtype;

/* Library version string, e.g. "ullm-hip 0.1.0 gfx950". */
const char *ullm_hip_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char *ullm_hip_last_error(void);

/* Bytes of device workspace ullm_hip_attn_decode needs for this shape.
 * max_len is the largest seq_len the calls will see; a workspace sized for
 * max_len serves every call whose own max_len is smaller.  The workspace holds
 * the split-KV partials; every call writes before it reads, so it needs no
 * initialisation.  One workspace serves one stream at a time. */
size_t ullm_hip_decode_workspace_bytes(int batch, int n_head, int n_kv_head, int head_dim,
                                       int max_len, int window);

/* Single-query GQA decode attention over the resident KV cache.
 * Replaces attn_scores/attn_softmax/attn_output
 * (crates/ullm-metal/src/forward.rs:449-466, shader.metal:944-1021) and
 * computes what the CPU reference computes at
 * crates/ullm-model/src/lib.rs:911-938 (full) and :1180-1208 (windowed):
 *   for each sequence b and query head h, kv head j = h / (n_head/n_kv_head):
 *     keys  start..len-1,  len = seq_lens[b] (= pos+1),
 *     start = (window > 0 && len > window) ? len - window : 0
 *     out[b,h,:] = softmax_t(scale * q[b,h,:].K[t,j,:]) . V[t,j,:]
 * q:        [batch][n_head][head_dim] f32 (after bias, Q-norm and RoPE)
 * k_cache,
 * v_cache:  layer base of sequence 0; sequence b starts seq_stride elements
 *           after sequence b-1 (ignored when batch == 1)
 * seq_lens: DEVICE int32[batch], each in 1..max_len
 * max_len:  host-side upper bound of seq_lens (sizes the split-KV grid);
 *           keys 0..max_len-1 of every sequence must be readable memory
 *           (keys from seq_lens[b] on may be fetched, never used)
 * out:      [batch][n_head][head_dim] f32
 * head_dim in {64, 128, 256}; n_head % n_kv_head == 0. */
int ullm_hip_attn_decode(const float *q, const void *k_cache, const void *v_cache, int kv_dtype,
                         int64_t kv_stride, int64_t seq_stride, const int32_t *seq_lens,
                         int max_len, int window, int batch, int n_head, int n_kv_head,
                         int head_dim, float scale, float *out, void *workspace,
                         size_t workspace_bytes, void *stream);

/* ullm_hip_attn_decode without a workspace and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and result as
 * ullm_hip_attn_decode, minus the workspace: the split-KV partials live in a
 * static device array of ullm_hip_decode_noalloc_max_bytes() bytes per GPU
 * (4 MiB), held by every GPU the library runs on until the process ends.
 * A shape whose partials exceed it returns ULLM_HIP_E_WORKSPACE (batch 1
 * covers every config up to 32 query heads at head_dim 128 and 32K keys).
 * The first call on a device resolves the array's address (no allocation).
 * All calls on one GPU share that array: calls that overlap on one GPU
 * (different streams, or host threads) race and must be serialised by the
 * caller.  Nothing needs clearing between calls (every partial is written
 * before it is read). */
int ullm_hip_attn_decode_noalloc(const float *q, const void *k_cache, const void *v_cache,
                                 int kv_dtype, int64_t kv_stride, int64_t seq_stride,
                                 const int32_t *seq_lens, int max_len, int window, int batch,
                                 int n_head, int n_kv_head, int head_dim, float scale, float *out,
                                 void *stream);

/* Bytes of the static scratch behind ullm_hip_attn_decode_noalloc. */
size_t ullm_hip_decode_noalloc_max_bytes(void);

/* Causal multi-token prefill attention on MFMA.
 * Replaces attn_flash_batch (crates/ullm-metal/src/forward.rs:855-858,
 * :1116-1147; shader.metal:1030-1074) and computes what the CPU reference
 * computes at crates/ullm-model/src/lib.rs:1061-1087: query row s sits at
 * pos = start_pos + s and attends keys start..pos, where start is 0, or
 * pos+1-window when window > 0 and pos+1 > window (a sliding-window layer,
 * shader.metal:1051).  The cache must already hold positions
 * 0..start_pos+S-1 (lib.rs:1056-1058).
 * q:     [S][n_head*head_dim] in `dtype` (after Q-norm and RoPE)
 * cache: `dtype` (f16, bf16 or f32; the same dtype as q)
 * out:   [S][n_head*head_dim] f32
 * head_dim in {64, 128, 256}, for every dtype.  With an f32 cache (the
 * reference's own cache dtype) Q.K runs on bf16 hi + lo halves of Q and K (~2^-16 per product) and
 * V is rounded to f16.  For bf16 and f32 caches P.V runs in f16 (V is
 * converted to f16 on chip), so |V| must stay below 65504 (beyond it the
 * affected rows come out inf or NaN, never as wrong finite values).  A layer's cache
 * and q must each stay below 2 GiB (a longer prompt runs as chunks at
 * increasing start_pos). */
int ullm_hip_attn_prefill(const void *q, const void *k_cache, const void *v_cache, int dtype,
                          int64_t kv_stride, int S, int start_pos, int window, int n_head,
                          int n_kv_head, int head_dim, float scale, float *out, void *stream);

/* Fills host memory `cs` ([n_pos][rotary_dim/2][2] f32, (cos, sin)) with the
 * RoPE angles of the CPU reference: freq_i = theta.powf(2i/rd).recip() and
 * (sin, cos) = (pos*freq_i).sin_cos() in f32
 * (crates/ullm-model/src/math.rs:116-161).  The same table serves NeoX and
 * interleaved RoPE.  Upload it once per model, like GpuForward::new uploads
 * weights. */
int ullm_hip_rope_table(float *cs, int n_pos, int rotary_dim, float theta);

/* Fused Q/K/V preparation and KV-cache append for `rows` tokens at positions
 * start_pos..start_pos+rows-1.  Replaces the bias / rmsnorm_heads / rope
 * dispatches (forward.rs:416-447 decode, :799-853 prefill;
 * shader.metal:828-941) and computes lib.rs:1021-1058 (:877-914 for one row):
 *   q += q_bias; k += k_bias; v += v_bias          (each optional)
 *   per-head RMSNorm of q with q_norm, of k with k_norm (optional, eps)
 *   RoPE of q and k (rope_neox != 0: rotate-half, else interleaved) over the
 *   first rotary_dim dims of each head, using the table from
 *   ullm_hip_rope_table (rope_cs: DEVICE, rope_n_pos >= start_pos+rows)
 *   q_out = q (q_dtype), K/V rows stored into the cache (kv_dtype).
 * q_in/k_in/v_in: [rows][n_head*head_dim] / [rows][n_kv_head*head_dim] f32.
 * q_out may alias q_in when q_dtype is f32. */
int ullm_hip_qkv_append(const float *q_in, const float *k_in, const float *v_in,
                        const float *q_bias, const float *k_bias, const float *v_bias,
                        const float *q_norm, const float *k_norm, float eps,
                        const float *rope_cs, int rope_n_pos, int rope_neox, int rotary_dim,
                        int rows, int start_pos, int n_head, int n_kv_head, int head_dim,
                        void *q_out, int q_dtype, void *k_cache, void *v_cache, int kv_dtype,
                        int64_t kv_stride, void *stream);

/* Decode-side Q/K/V projection with the append fused into its epilogue, for
 * `rows` tokens at positions start_pos..: computes lib.rs:857-914 (the
 * non-gated attention path) and replaces the Metal forward's wq/wk/wv matvecs
 * into q and the cache slot plus the bias / rmsnorm_heads / rope dispatches
 * (forward.rs:415-447):
 *   q = W_q x, k = W_k x, v = W_v x      (math.rs:9-21 matvec_q, f32 sums)
 * followed by exactly what ullm_hip_qkv_append does to q, k and v.
 * x:   [rows][in_dim] f32 (the attention-normed hidden state), DEVICE
 * w_q: [n_head*head_dim][in_dim], w_k / w_v: [n_kv_head*head_dim][in_dim],
 *      row-major, w_dtype f32, f16 or bf16 (other weight formats: unsupported)
 * in_dim a multiple of 8; x and the weights 16-byte aligned; rows <= 65535.
 * HBM-bound on the weights.  With few head vectors (rows * (n_head +
 * 2*n_kv_head) < 256, i.e. decode) each is split over 4 workgroups that
 * meet in `workspace`: size it with ullm_hip_qkv_proj_workspace_bytes and
 * ZERO it once after allocating it (its counters return to zero after every
 * call); calls sharing a workspace must not overlap.  With more head vectors
 * the workspace is not used (0 bytes needed; may be NULL). */
int ullm_hip_qkv_proj_append(const float *x, int in_dim, const void *w_q, const void *w_k,
                             const void *w_v, int w_dtype, const float *q_bias,
                             const float *k_bias, const float *v_bias, const float *q_norm,
                             const float *k_norm, float eps, const float *rope_cs,
                             int rope_n_pos, int rope_neox, int rotary_dim, int rows,
                             int start_pos, int n_head, int n_kv_head, int head_dim, void *q_out,
                             int q_dtype, void *k_cache, void *v_cache, int kv_dtype,
                             int64_t kv_stride, void *workspace, size_t workspace_bytes,
                             void *stream);

/* Workspace bytes ullm_hip_qkv_proj_append needs for this many rows (0 when
 * it does not split head vectors). */
size_t ullm_hip_qkv_proj_workspace_bytes(int rows, int n_head, int n_kv_head, int head_dim);

/* Batched projection for prefill: y[s*out_dim + o] = sum_i w[o*in_dim + i] *
 * x[s*in_dim + i] for s < n_cols, o < out_dim.  Replaces the reference's
 * batched matmul (crates/ullm-metal/src/forward.rs:675-726, kernel
 * matmul_bf16_tiled at shader.metal:519-566), same argument meaning: w is
 * [out_dim, in_dim] row-major, x [n_cols, in_dim] and y [n_cols, out_dim]
 * token-major f32; the caller offsets y (y_off) as forward.rs does when K/V
 * land in the cache.  Weights bf16 only (w_dtype = ULLM_DT_BF16, as the
 * reference's batched path; other dtypes -> ULLM_HIP_E_UNSUPPORTED).  The
 * activations enter the matrix cores as a bf16 hi + lo pair (16 significant
 * bits), accumulation is f32.  in_dim % 8 == 0, out_dim % 4 == 0, w/x/y
 * 16-byte aligned, weight below 2 GiB.  n_cols == 0 is a no-op. */
int ullm_hip_matmul(const void *w, int w_dtype, const float *x, float *y, int in_dim,
                    int out_dim, int n_cols, void *stream);

/* Bytes of workspace ullm_hip_attn_decode_paged needs (same meaning as
 * ullm_hip_decode_workspace_bytes). */
size_t ullm_hip_paged_decode_workspace_bytes(int batch, int n_head, int n_kv_head, int head_dim,
                                             int max_len, int window);

/* Decode attention over a PAGED KV cache: the same result as
 * ullm_hip_attn_decode for batch > 1 with sequences of different lengths
 * whose positions live in fixed-size pages of a shared pool.  No
 * counterpart in the reference (its cache is one contiguous [n_ctx][kv_dim]
 * array per layer, crates/ullm-model/src/lib.rs:184-185, capped at 8192
 * positions, lib.rs:236); it is the paged/batched cache the reference's
 * roadmap names (docs/roadmap.md, Phase 2).
 * k_pages,
 * v_pages:     pools of n_pages pages; page p holds page_size positions of
 *              kv_stride elements: element (slot i, kv head j, d) at
 *              (p*page_size + i)*kv_stride + j*head_dim + d
 * block_table: DEVICE int32[batch][table_stride]; position t of sequence b
 *              is slot t % page_size of page block_table[b][t / page_size].
 *              Entries for pages holding positions in the attended range
 *              must lie in [0, n_pages) (others are read as zeros)
 * page_size:   a power of two >= 32; table_stride >= ceil(max_len/page_size)
 * Other arguments as for ullm_hip_attn_decode.  Slots past a sequence's
 * length may hold anything (they are masked and their V rows zeroed).
 * kv_dtype f32, f16 or bf16; head_dim 64, 128 or 256 (else ULLM_HIP_E_UNSUPPORTED). */
int ullm_hip_attn_decode_paged(const float *q, const void *k_pages, const void *v_pages,
                               int kv_dtype, int64_t kv_stride, int page_size, int n_pages,
                               const int32_t *block_table, int table_stride,
                               const int32_t *seq_lens, int max_len, int window, int batch,
                               int n_head, int n_kv_head, int head_dim, float scale, float *out,
                               void *workspace, size_t workspace_bytes, void *stream);

/* Batched append into a PAGED cache: row r is the new token of sequence r at
 * position positions[r] (DEVICE int32[rows]); it gets the same bias, Q/K
 * norm and RoPE (at its own position) as ullm_hip_qkv_append, q goes to row r
 * of q_out, and the K/V rows go to slot pos % page_size of page
 * block_table[r][pos / page_size] (the layout of ullm_hip_attn_decode_paged).
 * No counterpart in the reference (its cache is contiguous and it decodes
 * one sequence at a time, crates/ullm-model/src/lib.rs:857-914); it is the
 * append step of a batched decode over the paged cache.  A row whose
 * position is outside [0, rope_n_pos) or whose page index is outside the
 * table or [0, n_pages) writes nothing.  page_size: a power of two. */
int ullm_hip_qkv_append_paged(const float *q_in, const float *k_in, const float *v_in,
                              const float *q_bias, const float *k_bias, const float *v_bias,
                              const float *q_norm, const float *k_norm, float eps,
                              const float *rope_cs, int rope_n_pos, int rope_neox, int rotary_dim,
                              int rows, const int32_t *positions, int n_head, int n_kv_head,
                              int head_dim, void *q_out, int q_dtype, void *k_pages, void *v_pages,
                              int kv_dtype, int64_t kv_stride, int page_size, int n_pages,
                              const int32_t *block_table, int table_stride, void *stream);

/* Causal prefill attention whose keys live in a PAGED cache: the S query
 * rows are positions start_pos..start_pos+S-1 of one sequence, and key t of
 * that sequence is slot t % page_size of page block_table[t / page_size]
 * (the layout of ullm_hip_attn_decode_paged; DEVICE int32[table_len],
 * table_len * page_size >= start_pos + S).  Same result as
 * ullm_hip_attn_prefill on the gathered cache: chunked prefill of a
 * sequence whose earlier positions are already in pages.  No counterpart in
 * the reference (contiguous cache, lib.rs:184-185).  page_size: a power of
 * two >= 64; head_dim 64, 128 or 256 with f16, bf16 or f32 pages (q in the
 * pages' dtype; else ULLM_HIP_E_UNSUPPORTED).
 * Pages outside [0, n_pages) read as zeros. */
int ullm_hip_attn_prefill_paged(const void *q, const void *k_pages, const void *v_pages,
                                int dtype, int64_t kv_stride, int page_size, int n_pages,
                                const int32_t *block_table, int table_len, int s, int start_pos,
                                int window, int n_head, int n_kv_head, int head_dim, float scale,
                                float *out, void *stream);

/* Measurement calibration (no counterpart in the reference): reads `bytes`
 * bytes of DEVICE memory at `src` (16-byte aligned) once, with 16-byte loads
 * split over `workgroups` 256-thread workgroups, and writes at most one word
 * per workgroup into `sink` (DEVICE uint32[workgroups]).  It is the floor a
 * read-only stream of that size reaches in one launch, against which the
 * decode op (a read-only stream of its K/V bytes) is compared. */
int ullm_hip_stream_read(const void *src, size_t bytes, int workgroups, uint32_t *sink,
                         void *stream);

#ifdef __cplusplus
}
#endif
#endif /* ULLM_HIP_H */
