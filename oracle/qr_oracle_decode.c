/*
 * qr_oracle_decode.c -- TEST INFRASTRUCTURE: CPU restatement of quantr-in-c's
 * single-token decode step (forward_runtime, src/runtime.c:94-288) for the
 * parity checks of the device decoder.  Same arithmetic, same order, compiled
 * -std=c99 -ffp-contract=off; glibc powf / cosf / sinf / expf / sqrtf as the
 * reference calls them.
 *
 * Generalisations of the reference, each checked where the reference can run:
 *   - head_dim is a parameter (the reference fixes it at dim / n_heads,
 *     src/runtime.c:102), q has n_heads * head_dim elements and RoPE is
 *     apply_rope over that whole vector (src/runtime.c:19-41, its `dim`
 *     argument being the q length, as in the reference where q_dim == dim);
 *   - the KV cache holds fp32 rows (the reference's type 0), fp16 rows (its
 *     type 1: kv_store_row's truncating fp32_to_fp16 and kv_get_element's
 *     fp16_to_fp32, src/runtime.c:74-92) or Q8_0 rows (quantize_row_q8_0 of
 *     each position's kv_dim values; an element reads as qs * d like
 *     dequantize_row, src/quant.c:169-176): the reference's own type 2 is
 *     unimplemented (src/runtime.c:74-84 writes fp32 into a buffer sized at
 *     one byte per element, src/model.c:82-88).
 * With head_dim = dim / n_heads and an fp32 or fp16 cache, qro_forward is
 * pinned bit for bit to the reference's forward_runtime by golden logits
 * (tests/golden/decode.npz).  Matrices of llama.cpp's K-quant layouts
 * (QRO_GGML) take ggml's Q8_K dot (qr_oracle_ggml.c), the embedding row its
 * dequantization: that composition has no reference counterpart.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "qr_oracle.h"

#define QK8 32
#define Q8_BYTES 34

/* rmsnorm_ref (src/kernels.c:170-180). */
void qro_rmsnorm(float* o, const float* x, const float* w, int n) {
    float ss = 0.0f, scale;
    int i;
    for (i = 0; i < n; i++) ss += x[i] * x[i];
    ss = ss / (float)n + 1e-5f;
    scale = 1.0f / sqrtf(ss);
    for (i = 0; i < n; i++) o[i] = w[i] * (x[i] * scale);
}

/* apply_rope (src/runtime.c:19-41) with `dim` = qlen. */
void qro_rope(float* q, float* k, int qlen, int head_dim, int n_kv_heads, int pos, float base) {
    int kv_dim = n_kv_heads * head_dim, i;
    if (kv_dim > qlen) kv_dim = qlen;
    if (!(base > 0.0f)) base = 10000.0f;
    for (i = 0; i < qlen; i += 2) {
        float freq = powf(base, -((float)i / (float)head_dim));
        float theta = (float)pos * freq;
        float c = cosf(theta), s = sinf(theta);
        float q0 = q[i], q1 = q[i + 1];
        q[i] = q0 * c - q1 * s;
        q[i + 1] = q0 * s + q1 * c;
        if (i < kv_dim) {
            float k0 = k[i], k1 = k[i + 1];
            k[i] = k0 * c - k1 * s;
            k[i + 1] = k0 * s + k1 * c;
        }
    }
}

/* The cos / sin of apply_rope for one position, as the device decoder's
 * tables hold them: cs[2 p] = cosf(theta_p), cs[2 p + 1] = sinf(theta_p) for
 * pair p = i / 2. */
void qro_rope_table(float* cs, int qlen, int head_dim, int pos, float base) {
    int i;
    if (!(base > 0.0f)) base = 10000.0f;
    for (i = 0; i < qlen; i += 2) {
        float freq = powf(base, -((float)i / (float)head_dim));
        float theta = (float)pos * freq;
        cs[i] = cosf(theta);
        cs[i + 1] = sinf(theta);
    }
}

static float kv_elem(const uint8_t* row, int kv_type, int i) {
    if (kv_type == QRO_KV_Q8_0) {
        const uint8_t* b = row + (size_t)(i / QK8) * Q8_BYTES;
        return (float)(int8_t)b[2 + i % QK8] * qro_h2f((uint16_t)(b[0] | (b[1] << 8)));
    }
    if (kv_type == QRO_KV_F16) /* kv_get_element, src/runtime.c:87-92 */
        return qro_h2f((uint16_t)(row[2 * i] | (row[2 * i + 1] << 8)));
    return ((const float*)row)[i];
}

size_t qro_kv_row_bytes(int kv_type, int kv_dim) {
    if (kv_type == QRO_KV_Q8_0) return (size_t)(kv_dim / QK8) * Q8_BYTES;
    return (size_t)kv_dim * (kv_type == QRO_KV_F16 ? 2 : 4);
}

/* One position's K or V row into the cache: fp32 copy, truncated halves
 * (kv_store_row, src/runtime.c:74-79), or quantize_row_q8_0. */
void qro_kv_store(void* row, const float* src, int kv_dim, int kv_type) {
    int i;
    if (kv_type == QRO_KV_Q8_0) {
        qro_quantize_row_q8_0(src, row, kv_dim);
    } else if (kv_type == QRO_KV_F16) {
        uint8_t* r = (uint8_t*)row;
        for (i = 0; i < kv_dim; i++) {
            uint16_t h = qro_f2h(src[i]);
            r[2 * i] = (uint8_t)(h & 0xFF);
            r[2 * i + 1] = (uint8_t)(h >> 8);
        }
    } else {
        memcpy(row, src, (size_t)kv_dim * sizeof(float));
    }
}

/* The attention of forward_runtime (src/runtime.c:136-193) at position pos:
 * kc / vc hold rows for positions 0..pos (row t at t * row_stride bytes, kv
 * head h's elements at h * head_dim of the row).  Scores with dot_ref
 * (src/kernels.c:162-168) times 1 / sqrtf(head_dim), softmax_ref, then each
 * output element accumulated over the positions in order.  att: scratch of
 * n_heads * (pos + 1) floats (optional: the normalised weights). */
static void attention_head(float* out, const float* q, const uint8_t* K, const uint8_t* V,
                           size_t row_stride, int kv_type, int pos, int h, int kv_mul,
                           int head_dim, float* att, float* kb) {
    int kvh = h / kv_mul, t, i;
    float inv_sqrt = 1.0f / sqrtf((float)head_dim);
    const float* qh = q + (size_t)h * head_dim;
    float* a = att + (size_t)h * (pos + 1);
    float* o = out + (size_t)h * head_dim;
    for (t = 0; t <= pos; t++) {
        const uint8_t* row = K + (size_t)t * row_stride;
        float s = 0.0f;
        for (i = 0; i < head_dim; i++) kb[i] = kv_elem(row, kv_type, kvh * head_dim + i);
        for (i = 0; i < head_dim; i++) s += qh[i] * kb[i];
        a[t] = s * inv_sqrt;
    }
    qro_softmax(a, pos + 1);
    memset(o, 0, (size_t)head_dim * sizeof(float));
    for (t = 0; t <= pos; t++) {
        const uint8_t* row = V + (size_t)t * row_stride;
        for (i = 0; i < head_dim; i++) o[i] += a[t] * kv_elem(row, kv_type, kvh * head_dim + i);
    }
}

/* Each head's scores, softmax and value sums depend on that head alone (the
 * reference's two head loops, src/runtime.c:136-193, share nothing between
 * heads), so heads run in parallel with the same bits at any width. */
void qro_attention_mt(float* out, const float* q, const void* kc, const void* vc,
                      size_t row_stride, int kv_type, int pos, int n_heads, int n_kv_heads,
                      int head_dim, float* att, int threads) {
    int kv_mul = n_heads / (n_kv_heads > 0 ? n_kv_heads : 1), h;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
    {
        float* kb = (float*)malloc((size_t)head_dim * sizeof(float));
#pragma omp for schedule(static)
        for (h = 0; h < n_heads; h++)
            if (kb)
                attention_head(out, q, (const uint8_t*)kc, (const uint8_t*)vc, row_stride,
                               kv_type, pos, h, kv_mul, head_dim, att, kb);
        free(kb);
    }
}

void qro_attention(float* out, const float* q, const void* kc, const void* vc, size_t row_stride,
                   int kv_type, int pos, int n_heads, int n_kv_heads, int head_dim, float* att) {
    qro_attention_mt(out, q, kc, vc, row_stride, kv_type, pos, n_heads, n_kv_heads, head_dim, att,
                     1);
}

/* matmul_q (src/runtime.c:58-70). */
static void mq(float* out, const float* x, const void* w, uint32_t type, int n, int d, int order,
               int threads) {
    if (w == NULL) memset(out, 0, (size_t)n * sizeof(float));
    else if (type == QRO_TYPE_F32) qro_matmul_f32(out, x, (const float*)w, n, d, order);
    else if (type & QRO_GGML) qro_ggml_matmul_mt(out, x, w, (int)(type & ~QRO_GGML), n, d, 1, threads);
    else qro_matmul_q_fused(out, x, w, type, n, d, threads, order);
}

/* forward_runtime (src/runtime.c:94-288) for one token at position pos.  kc / vc:
 * the cache, layer l's row for position t at ((l * seq_len) + t) * row_stride
 * bytes.  x: the residual [dim] (written); logits [vocab].  order: the
 * reference build (router / F32 matmul order and Q8_0 dot order). */
void qro_forward(const qro_model* m, void* kc, void* vc, int token, int pos, int order, float* x,
                 float* logits) {
    const int dim = m->dim, hd = m->head_dim, qd = m->n_heads * hd, kvd = m->n_kv_heads * hd;
    const size_t rs = qro_kv_row_bytes(m->kv_type, kvd);
    float *xb = (float*)calloc((size_t)dim, sizeof(float)), *xb2 = (float*)calloc((size_t)dim, 4);
    float *q = (float*)calloc((size_t)qd, 4), *k = (float*)calloc((size_t)qd, 4);
    float *v = (float*)calloc((size_t)qd, 4), *ao = (float*)calloc((size_t)qd, 4);
    float* att = (float*)calloc((size_t)m->n_heads * (size_t)(pos + 1), 4);
    int l, i;
    if (!xb || !xb2 || !q || !k || !v || !ao || !att) goto done;
    if (m->tok_type & QRO_GGML)
        qro_ggml_dequantize_row((int)(m->tok_type & ~QRO_GGML),
                                (const uint8_t*)m->tok_embd + (size_t)token * m->tok_row_bytes, x,
                                dim);
    else
        qro_dequantize_row(x, (const uint8_t*)m->tok_embd + (size_t)token * m->tok_row_bytes,
                           m->tok_type, dim);
    for (l = 0; l < m->n_layers; l++) {
        uint8_t* kl = (uint8_t*)kc + (size_t)l * m->seq_len * rs;
        uint8_t* vl = (uint8_t*)vc + (size_t)l * m->seq_len * rs;
        qro_rmsnorm(xb, x, m->rms_att[l], dim);
        mq(q, xb, m->wq[l], m->wtype[4 * l], qd, dim, order, m->threads);
        mq(k, xb, m->wk[l], m->wtype[4 * l + 1], kvd, dim, order, m->threads);
        mq(v, xb, m->wv[l], m->wtype[4 * l + 2], kvd, dim, order, m->threads);
        qro_rope(q, k, qd, hd, m->n_kv_heads, pos, m->rope_base);
        qro_kv_store(kl + (size_t)pos * rs, k, kvd, m->kv_type);
        qro_kv_store(vl + (size_t)pos * rs, v, kvd, m->kv_type);
        qro_attention_mt(ao, q, kl, vl, rs, m->kv_type, pos, m->n_heads, m->n_kv_heads, hd, att,
                         m->threads);
        mq(xb2, ao, m->wo[l], m->wtype[4 * l + 3], dim, qd, order, m->threads);
        for (i = 0; i < dim; i++) x[i] += xb2[i];
        qro_rmsnorm(xb, x, m->rms_ffn[l], dim);
        if (m->moe[l].n_experts == 0) qro_dense_ffn(x, xb, &m->moe[l], order, m->threads);
        else qro_moe_token(x, xb, &m->moe[l], order, order, m->threads, NULL, NULL);
    }
    qro_rmsnorm(xb, x, m->rms_final, dim);
    mq(logits, xb, m->wcls, m->wcls_type, m->vocab, dim, order, m->threads);
done:
    free(xb);
    free(xb2);
    free(q);
    free(k);
    free(v);
    free(ao);
    free(att);
}
