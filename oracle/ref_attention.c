/*
 * CPU oracle for the uLLM attention path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C, single-threaded restatement of the reference CPU attention in
 * nobottomline/ullm (Rust).  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load this library, always as the checker.
 * The product path (ullm_amd/, libullm_hip.so) never links or calls it.
 *
 * Built with `-O2 -ffp-contract=off` and without fast-math so that every
 * float operation happens in the order and precision the Rust source states:
 * Rust neither contracts a*b+c into an FMA nor reassociates, and
 * `Iterator::sum::<f32>()` is a left fold.  expf/powf/sinf/cosf come from the
 * platform libm, as Rust's f32 methods do on Linux.
 *
 * Every function cites the reference lines it restates (paths relative to the
 * reference repository root).  Parity pins (what checks each function beyond
 * a restatement) live in tests/test_oracle.py.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

#define ORA_F32 0
#define ORA_F16 1
#define ORA_BF16 2

/* crates/ullm-core/src/dequant.rs:15-31 -- IEEE half -> f32, written the same
 * way (subnormals via mant * 2^-24, normals via (1 + mant/1024) * 2^(e-15)). */
float ora_f16_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u;
    uint32_t ex = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    float v;
    if (ex == 0) {
        v = (float)mant * ldexpf(1.0f, -24);
    } else if (ex == 0x1f) {
        v = mant == 0 ? INFINITY : NAN;
    } else {
        v = (1.0f + (float)mant / 1024.0f) * ldexpf(1.0f, (int)ex - 15);
    }
    return sign ? -v : v;
}

/* crates/ullm-core/src/dequant.rs:90-94 (and bf16_to_f32 :286-289):
 * bf16 bits are the high half of the f32 bits. */
float ora_bf16_to_f32(uint16_t h) {
    uint32_t b = (uint32_t)h << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* Widen n elements of dtype (0 f32, 1 f16, 2 bf16) to f32 -- the reference's
 * dequantize_into for those three dtypes (dequant.rs:61-94). */
void ora_widen(const void *src, int dtype, size_t n, float *dst) {
    if (dtype == ORA_F32) {
        memcpy(dst, src, n * 4);
        return;
    }
    const uint16_t *s = (const uint16_t *)src;
    for (size_t i = 0; i < n; i++)
        dst[i] = dtype == ORA_F16 ? ora_f16_to_f32(s[i]) : ora_bf16_to_f32(s[i]);
}

/* crates/ullm-model/src/math.rs:82-86 -- rmsnorm:
 *   ms  = (sum of x*x, left fold) / n + eps
 *   inv = ms.sqrt().recip()
 *   y   = x * inv * w                                                     */
void ora_rmsnorm(const float *x, const float *w, int n, float eps, float *y) {
    float s = 0.0f;
    for (int i = 0; i < n; i++) s += x[i] * x[i];
    float ms = s / (float)n + eps;
    float inv = 1.0f / sqrtf(ms);
    for (int i = 0; i < n; i++) y[i] = x[i] * inv * w[i];
}

/* crates/ullm-model/src/math.rs:89-100 -- softmax in place: max fold from
 * -inf, v = exp(v - max) with a running sum, then v *= sum.recip(). */
void ora_softmax(float *x, int n) {
    float mx = -INFINITY;
    for (int i = 0; i < n; i++) mx = fmaxf(mx, x[i]);
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    float inv = 1.0f / sum;
    for (int i = 0; i < n; i++) x[i] *= inv;
}

/* crates/ullm-model/src/math.rs:116-136 -- interleaved ("NORM") RoPE: for
 * even i < rotary_dim, freq = theta.powf(i/rd).recip(), rotate (x_i, x_i+1). */
void ora_rope(float *v, int n_heads, int head_dim, int rotary_dim, int pos, float theta) {
    for (int h = 0; h < n_heads; h++) {
        size_t off = (size_t)h * head_dim;
        for (int i = 0; i + 1 < rotary_dim; i += 2) {
            float freq = 1.0f / powf(theta, (float)i / (float)rotary_dim);
            float ang = (float)pos * freq;
            float sn = sinf(ang), cs = cosf(ang);
            float a = v[off + i], b = v[off + i + 1];
            v[off + i] = a * cs - b * sn;
            v[off + i + 1] = a * sn + b * cs;
        }
    }
}

/* crates/ullm-model/src/math.rs:140-161 -- NeoX (rotate-half) RoPE with
 * partial rotary: for i < rd/2, freq = theta.powf(2i/rd).recip(), rotate
 * (x_i, x_{i+rd/2}); dims past rotary_dim pass through. */
void ora_rope_neox(float *v, int n_heads, int head_dim, int rotary_dim, int pos, float theta) {
    int half = rotary_dim / 2;
    for (int h = 0; h < n_heads; h++) {
        size_t off = (size_t)h * head_dim;
        for (int i = 0; i < half; i++) {
            float freq = 1.0f / powf(theta, 2.0f * (float)i / (float)rotary_dim);
            float ang = (float)pos * freq;
            float sn = sinf(ang), cs = cosf(ang);
            float a = v[off + i], b = v[off + i + half];
            v[off + i] = a * cs - b * sn;
            v[off + i + half] = a * sn + b * cs;
        }
    }
}

/* One query head against keys start..=pos of one kv head: the body of the
 * per-head loop at crates/ullm-model/src/lib.rs:917-938 (forward_llama) and
 * :1187-1208 (forward_gemma, where start is the sliding-window start).
 *   score_t = (sum_d q_d * K[t,d], left fold) * scale
 *   softmax(scores)
 *   out[d] += a_t * V[t,d]  in t order (out starts at zero)
 * kc/vc point at the layer base; row t of kv head kvh is at
 * t*kv_stride + kvh*head_dim.  `scores` is caller scratch of pos+1 floats. */
static void attend_one(const float *qh, const float *kc, const float *vc, size_t kv_stride,
                       int kvh, int head_dim, int start, int pos, float scale, float *scores,
                       float *oh) {
    int n = pos - start + 1;
    for (int idx = 0; idx < n; idx++) {
        size_t ko = (size_t)(start + idx) * kv_stride + (size_t)kvh * head_dim;
        float s = 0.0f;
        for (int d = 0; d < head_dim; d++) s += qh[d] * kc[ko + d];
        scores[idx] = s * scale;
    }
    ora_softmax(scores, n);
    for (int d = 0; d < head_dim; d++) oh[d] = 0.0f;
    for (int idx = 0; idx < n; idx++) {
        size_t vo = (size_t)(start + idx) * kv_stride + (size_t)kvh * head_dim;
        float a = scores[idx];
        for (int d = 0; d < head_dim; d++) oh[d] += a * vc[vo + d];
    }
}

/* Sliding-window start, crates/ullm-model/src/lib.rs:1183-1186:
 * start = pos + 1 - W when W > 0 and pos + 1 > W (the caller decides whether
 * the layer is local; window <= 0 means full attention). */
int ora_window_start(int pos, int window) {
    return (window > 0 && pos + 1 > window) ? pos + 1 - window : 0;
}

/* Single-query GQA decode attention (lib.rs:911-938; windowed :1180-1208).
 * q: [n_head*head_dim] f32; kc/vc: the layer's f32 cache, token stride
 * kv_stride floats; the query sits at position pos and sees start..=pos with
 * start = ora_window_start(pos, window).  kv head = h / (n_head/n_kv_head)
 * (lib.rs:918).  out: [n_head*head_dim]. */
int ora_attn_decode(const float *q, const float *kc, const float *vc, size_t kv_stride, int pos,
                    int window, int n_head, int n_kv_head, int head_dim, float scale, float *out) {
    if (n_kv_head <= 0 || n_head % n_kv_head != 0 || pos < 0) return -1;
    int kv_mul = n_head / n_kv_head;
    int start = ora_window_start(pos, window);
    float *scores = (float *)malloc(sizeof(float) * (size_t)(pos + 1));
    if (!scores) return -2;
    for (int h = 0; h < n_head; h++)
        attend_one(q + (size_t)h * head_dim, kc, vc, kv_stride, h / kv_mul, head_dim, start, pos,
                   scale, scores, out + (size_t)h * head_dim);
    free(scores);
    return 0;
}

/* Causal multi-token prefill attention (lib.rs:1061-1087): query row s sits
 * at pos = start_pos + s and attends to keys 0..=pos, all K/V rows having
 * been appended first (:1056-1058).  With window > 0 each row uses the
 * sliding-window start of lib.rs:1183-1186 (the row-wise semantics of the
 * windowed GPU prefill, crates/ullm-metal/src/shader.metal:1051).
 * q/out: token-major [S, n_head*head_dim].  Only the rows listed in `rows`
 * (n_rows of them; NULL = all S rows) are computed, so a test can check a
 * sample of a long prompt; other output rows are left untouched. */
int ora_attn_prefill(const float *q, const float *kc, const float *vc, size_t kv_stride, int S,
                     int start_pos, int window, int n_head, int n_kv_head, int head_dim,
                     float scale, const int *rows, int n_rows, float *out) {
    if (n_kv_head <= 0 || n_head % n_kv_head != 0) return -1;
    int kv_mul = n_head / n_kv_head;
    size_t q_dim = (size_t)n_head * head_dim;
    float *scores = (float *)malloc(sizeof(float) * (size_t)(start_pos + S));
    if (!scores) return -2;
    int cnt = rows ? n_rows : S;
    for (int r = 0; r < cnt; r++) {
        int s = rows ? rows[r] : r;
        if (s < 0 || s >= S) { free(scores); return -3; }
        int pos = start_pos + s;
        int start = ora_window_start(pos, window);
        for (int h = 0; h < n_head; h++)
            attend_one(q + (size_t)s * q_dim + (size_t)h * head_dim, kc, vc, kv_stride,
                       h / kv_mul, head_dim, start, pos, scale, scores,
                       out + (size_t)s * q_dim + (size_t)h * head_dim);
    }
    free(scores);
    return 0;
}

/* Per-row Q/K/V preparation and KV append, lib.rs:1021-1058 (prefill) and
 * :877-914 (decode, one row):
 *   q += q_bias, k += k_bias, v += v_bias            (optional, :1027-1035)
 *   per-head rmsnorm of q with q_norm, of k with k_norm (optional, :1036-1049)
 *   RoPE of q and k at pos = start_pos + s            (:1050-1055)
 *   key_cache[pos] = k, val_cache[pos] = v            (:1056-1058)
 * q is modified in place ([rows, n_head*head_dim]); k/v ([rows, kv_dim]) are
 * read and written into kc/vc (layer base, token stride kv_stride).
 * neox != 0 selects rope_neox. */
int ora_qkv_append(float *q, const float *k, const float *v, int rows, int start_pos, int n_head,
                   int n_kv_head, int head_dim, int rotary_dim, const float *q_bias,
                   const float *k_bias, const float *v_bias, const float *q_norm,
                   const float *k_norm, float eps, int neox, float theta, float *kc, float *vc,
                   size_t kv_stride) {
    size_t q_dim = (size_t)n_head * head_dim, kv_dim = (size_t)n_kv_head * head_dim;
    float *kb = (float *)malloc(sizeof(float) * kv_dim);
    float *vb = (float *)malloc(sizeof(float) * kv_dim);
    float *tmp = (float *)malloc(sizeof(float) * (size_t)head_dim);
    if (!kb || !vb || !tmp) { free(kb); free(vb); free(tmp); return -2; }
    for (int s = 0; s < rows; s++) {
        int pos = start_pos + s;
        float *qs = q + (size_t)s * q_dim;
        memcpy(kb, k + (size_t)s * kv_dim, kv_dim * 4);
        memcpy(vb, v + (size_t)s * kv_dim, kv_dim * 4);
        if (q_bias) for (size_t i = 0; i < q_dim; i++) qs[i] += q_bias[i];
        if (k_bias) for (size_t i = 0; i < kv_dim; i++) kb[i] += k_bias[i];
        if (v_bias) for (size_t i = 0; i < kv_dim; i++) vb[i] += v_bias[i];
        if (q_norm)
            for (int h = 0; h < n_head; h++) {
                ora_rmsnorm(qs + (size_t)h * head_dim, q_norm, head_dim, eps, tmp);
                memcpy(qs + (size_t)h * head_dim, tmp, (size_t)head_dim * 4);
            }
        if (k_norm)
            for (int h = 0; h < n_kv_head; h++) {
                ora_rmsnorm(kb + (size_t)h * head_dim, k_norm, head_dim, eps, tmp);
                memcpy(kb + (size_t)h * head_dim, tmp, (size_t)head_dim * 4);
            }
        if (neox) {
            ora_rope_neox(qs, n_head, head_dim, rotary_dim, pos, theta);
            ora_rope_neox(kb, n_kv_head, head_dim, rotary_dim, pos, theta);
        } else {
            ora_rope(qs, n_head, head_dim, rotary_dim, pos, theta);
            ora_rope(kb, n_kv_head, head_dim, rotary_dim, pos, theta);
        }
        memcpy(kc + (size_t)pos * kv_stride, kb, kv_dim * 4);
        memcpy(vc + (size_t)pos * kv_stride, vb, kv_dim * 4);
    }
    free(kb); free(vb); free(tmp);
    return 0;
}

/* crates/ullm-model/src/math.rs:9-21 -- matvec_q for an f32/f16/bf16 weight:
 * for every output row o, dequantize row o (dequant.rs:61-94) and
 *   y[o] = sum_i w[o][i] * x[i]      (a left fold from 0.0, one rounding per
 *                                      product and per add: Rust's `.sum()`)
 * w: [out][cols] raw storage (f32 or 16-bit), x: [cols], y: [out]. */
int ora_matvec(const void *w, int dtype, int out, int cols, const float *x, float *y) {
    float *row = (float *)malloc(sizeof(float) * (size_t)cols);
    if (!row) return -2;
    const size_t esz = dtype == ORA_F32 ? 4 : 2;
    for (int o = 0; o < out; o++) {
        ora_widen((const char *)w + (size_t)o * cols * esz, dtype, (size_t)cols, row);
        float acc = 0.0f;
        for (int i = 0; i < cols; i++) {
            const float p = row[i] * x[i];
            acc = acc + p;
        }
        y[o] = acc;
    }
    free(row);
    return 0;
}
