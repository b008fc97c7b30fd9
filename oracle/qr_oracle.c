/*
 * qr_oracle.c -- CPU restatement of quantr-in-c's quantized GEMV + MoE path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker): loaded by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg; never by the
 * product.  Built with -std=c99 -ffp-contract=off so that every float
 * operation rounds once, in the order written, exactly like the reference's
 * -std=c99 build.  Each function cites the reference lines it follows.
 */
#include "qr_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define QK8 32
#define QKK 256
#define Q8_BYTES 34
#define Q4K_BYTES 144
#define Q5K_BYTES 176
#define Q6K_BYTES 210

/* include/quant.h:53-66: fp16 bits -> fp32 by exponent rebias.  Half
 * subnormals keep exponent 0 and so decode to mant * 2^-136, like the
 * reference. */
float qro_h2f(uint16_t h) {
    uint32_t w = (uint32_t)(h & 0x7FFFu) << 13;
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    float f;
    if (e == 0x1Fu) {
        w |= 0x7F800000u;
    } else if (e != 0) {
        w += 0x38000000u;
    }
    w |= sign;
    memcpy(&f, &w, 4);
    return f;
}

/* include/quant.h:68-77: truncating fp32 -> fp16.  Exponents that land at or
 * below zero flush to signed zero; at or above 31 they saturate to infinity. */
uint16_t qro_f2h(float f) {
    uint32_t x;
    uint16_t sign;
    int e;
    memcpy(&x, &f, 4);
    sign = (uint16_t)((x >> 16) & 0x8000u);
    e = (int)((x >> 23) & 0xFFu) - 127 + 15;
    if (e <= 0) return sign;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | (uint16_t)(e << 10) | (uint16_t)((x >> 13) & 0x3FFu));
}

void qro_h2f_batch(const uint16_t* h, float* out, long n) {
    long i;
    for (i = 0; i < n; i++) out[i] = qro_h2f(h[i]);
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* src/quant.c:477-484 (and src/model.c:20-30): bytes per weight row.  Rows
 * keep only whole blocks; a tail shorter than one block is dropped. */
size_t qro_row_bytes(uint32_t type, int d) {
    switch (type & ~QRO_GGML) {
        case QRO_TYPE_Q8_0: return (size_t)(d / QK8) * Q8_BYTES;
        case QRO_TYPE_Q4_K: return (size_t)(d / QKK) * Q4K_BYTES;
        case QRO_TYPE_Q5_K: return (size_t)(d / QKK) * Q5K_BYTES;
        case QRO_TYPE_Q6_K: return (size_t)(d / QKK) * Q6K_BYTES;
        default: return (size_t)d * 4u;
    }
}

/* Number of 32-element integer units one row's dot is made of. */
int qro_units_per_row(uint32_t type, int d) {
    switch (type) {
        case QRO_TYPE_Q8_0: return d / QK8;
        case QRO_TYPE_Q4_K:
        case QRO_TYPE_Q5_K:
        case QRO_TYPE_Q6_K: return (d / QKK) * 8;
        default: return 0;
    }
}

/* src/model.c:412-414: one expert's slice of a [E][ne1][ne0] tensor. */
size_t qro_expert_slice_bytes(uint32_t type, int ne0, int ne1) {
    return qro_row_bytes(type, ne0) * (size_t)ne1;
}

/* src/quant.c:143-158.  Per 32-block: amax by strict '>', d = amax/127,
 * id = 1/d (0 when d == 0), qs = lrintf(x*id) (ties to even), d stored with
 * the truncating fp16 routine.  A tail shorter than 32 is not written. */
void qro_quantize_row_q8_0(const float* x, void* y, int k) {
    uint8_t* out = (uint8_t*)y;
    int nb = k / QK8;
    int i, j;
    for (i = 0; i < nb; i++) {
        float amax = 0.0f;
        float d, id;
        uint16_t dh;
        for (j = 0; j < QK8; j++) {
            float v = fabsf(x[i * QK8 + j]);
            if (v > amax) amax = v;
        }
        d = amax / 127.0f;
        id = d != 0.0f ? 1.0f / d : 0.0f;
        dh = qro_f2h(d);
        out[i * Q8_BYTES + 0] = (uint8_t)(dh & 0xFF);
        out[i * Q8_BYTES + 1] = (uint8_t)(dh >> 8);
        for (j = 0; j < QK8; j++) {
            out[i * Q8_BYTES + 2 + j] = (uint8_t)(int8_t)lrintf(x[i * QK8 + j] * id);
        }
    }
}

/* Element e (0..255) of a Q4_K super-block: src/quant.c:190. */
static int q4k_q(const uint8_t* blk, int e) {
    return (blk[16 + e / 2] >> ((e % 2) * 4)) & 0xF;
}
/* Element e of a Q5_K super-block: src/quant.c:207-209. */
static int q5k_q(const uint8_t* blk, int e) {
    int lo = (blk[48 + e / 2] >> ((e % 2) * 4)) & 0xF;
    int hi = (blk[16 + e / 8] >> (e % 8)) & 1;
    return lo | (hi << 4);
}
/* Element e of a Q6_K super-block (210 B: ql@0, qh@128, i8 scales@192,
 * d@208): src/quant.c:230-232. */
static int q6k_q(const uint8_t* blk, int e) {
    int ql = (blk[e / 2] >> ((e % 2) * 4)) & 0xF;
    int qh = (blk[128 + e / 4] >> ((e % 4) * 2)) & 3;
    return (ql | (qh << 4)) - 32;
}

/* src/quant.c:160-240. */
void qro_dequantize_row(float* out, const void* src, uint32_t type, int n) {
    const uint8_t* b = (const uint8_t*)src;
    int i, j, l;
    if (src == NULL) {
        memset(out, 0, (size_t)n * sizeof(float));
        return;
    }
    if (type == QRO_TYPE_F32) {
        memcpy(out, src, (size_t)n * sizeof(float));
        return;
    }
    if (type == QRO_TYPE_Q8_0) {
        for (i = 0; i < n / QK8; i++) {
            const uint8_t* blk = b + (size_t)i * Q8_BYTES;
            float d = qro_h2f(rd16(blk));
            for (j = 0; j < QK8; j++) out[i * QK8 + j] = (float)(int8_t)blk[2 + j] * d;
        }
        return;
    }
    if (type == QRO_TYPE_Q4_K || type == QRO_TYPE_Q5_K) {
        size_t bb = type == QRO_TYPE_Q4_K ? Q4K_BYTES : Q5K_BYTES;
        for (i = 0; i < n / QKK; i++) {
            const uint8_t* blk = b + (size_t)i * bb;
            float d = qro_h2f(rd16(blk));
            float dmin = qro_h2f(rd16(blk + 2));
            for (j = 0; j < 8; j++) {
                float sc = (float)(blk[4 + j] & 63) * d;
                float m = (float)(blk[4 + j] >> 6) * dmin;
                for (l = 0; l < 32; l++) {
                    int e = j * 32 + l;
                    int q = type == QRO_TYPE_Q4_K ? q4k_q(blk, e) : q5k_q(blk, e);
                    out[i * QKK + e] = (float)q * sc - m;
                }
            }
        }
        return;
    }
    if (type == QRO_TYPE_Q6_K) {
        for (i = 0; i < n / QKK; i++) {
            const uint8_t* blk = b + (size_t)i * Q6K_BYTES;
            float d = qro_h2f(rd16(blk + 208));
            for (j = 0; j < 8; j++) {
                float sc = (float)(int8_t)blk[192 + j] * d;
                for (l = 0; l < 32; l++) {
                    int e = j * 32 + l;
                    out[i * QKK + e] = (float)q6k_q(blk, e) * sc;
                }
            }
        }
        return;
    }
    memset(out, 0, (size_t)n * sizeof(float));
}

/* Integer sums of one row against a Q8_0 activation, one entry per 32-element
 * unit: isum = sum q*x_q (Q6_K uses q-32), bsum = sum x_q.  These are the
 * int32 accumulators of src/quant.c:279-283 (Q8_0), 388-397 (Q5_K; the
 * corrected Q4_K uses the same sums) and 425-431 (Q6_K). */
int qro_row_accum(uint32_t type, const void* row, const void* xq8, int d,
                  int32_t* isum, int32_t* bsum) {
    const uint8_t* w = (const uint8_t*)row;
    const uint8_t* x = (const uint8_t*)xq8;
    int u, l, units = qro_units_per_row(type, d);
    for (u = 0; u < units; u++) {
        const uint8_t* xb = x + (size_t)u * Q8_BYTES;
        int32_t is = 0, bs = 0;
        for (l = 0; l < 32; l++) {
            int xv = (int8_t)xb[2 + l];
            int q;
            if (type == QRO_TYPE_Q8_0) {
                q = (int8_t)w[(size_t)u * Q8_BYTES + 2 + l];
            } else {
                int blk = u / 8, e = (u % 8) * 32 + l;
                if (type == QRO_TYPE_Q4_K) q = q4k_q(w + (size_t)blk * Q4K_BYTES, e);
                else if (type == QRO_TYPE_Q5_K) q = q5k_q(w + (size_t)blk * Q5K_BYTES, e);
                else q = q6k_q(w + (size_t)blk * Q6K_BYTES, e);
            }
            is += q * xv;
            bs += xv;
        }
        isum[u] = is;
        if (bsum) bsum[u] = bs;
    }
    return units;
}

/* src/quant.c:279-285 (SEQ) and src/quant.c:245-277 (8 lanes): the AVX2 build
 * updates a lane with a multiply then an add (src/quant.c:271), a build with
 * AVX-512 enabled with one fused multiply-add (src/quant.c:269). */
static float dot_q8_0(const uint8_t* a, const uint8_t* b, int d, int order) {
    int nb = d / QK8, i, k;
    float sum = 0.0f;
    if (order == QRO_ORDER_SEQ) {
        for (i = 0; i < nb; i++) {
            const uint8_t* pa = a + (size_t)i * Q8_BYTES;
            const uint8_t* pb = b + (size_t)i * Q8_BYTES;
            int isum = 0, j;
            for (j = 0; j < QK8; j++) isum += (int8_t)pa[2 + j] * (int8_t)pb[2 + j];
            sum += (float)isum * qro_h2f(rd16(pa)) * qro_h2f(rd16(pb));
        }
        return sum;
    } else {
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (i = 0; i < nb; i++) {
            const uint8_t* pa = a + (size_t)i * Q8_BYTES + 2;
            const uint8_t* pb = b + (size_t)i * Q8_BYTES + 2;
            float dd = qro_h2f(rd16(pa - 2)) * qro_h2f(rd16(pb - 2));
            for (k = 0; k < 8; k++) {
                /* madd lanes: elements {2k,2k+1} of bytes 0..15 plus {16+2k,17+2k} */
                int lo = (int8_t)pa[2 * k] * (int8_t)pb[2 * k] +
                         (int8_t)pa[2 * k + 1] * (int8_t)pb[2 * k + 1];
                int hi = (int8_t)pa[16 + 2 * k] * (int8_t)pb[16 + 2 * k] +
                         (int8_t)pa[17 + 2 * k] * (int8_t)pb[17 + 2 * k];
                if (order == QRO_ORDER_AVX512) {
                    acc[k] = fmaf((float)(lo + hi), dd, acc[k]);
                } else {
                    float p = (float)(lo + hi) * dd;
                    acc[k] = p + acc[k];
                }
            }
        }
        for (k = 0; k < 8; k++) sum += acc[k];
        return sum;
    }
}

/* Q4_K (corrected; the reference's own vec_dot_q4K_q8_0, src/quant.c:291-369,
 * reads fp16 bit patterns as floats) and Q5_K (src/quant.c:372-403):
 * sumf += (sc*isum - m*bsum) * bd, sequential over super-blocks and
 * sub-blocks. */
static float dot_q45k(const uint8_t* a, const uint8_t* b, int d, uint32_t type) {
    int nb = d / QKK, i, j, l;
    size_t bb = type == QRO_TYPE_Q4_K ? Q4K_BYTES : Q5K_BYTES;
    float sumf = 0.0f;
    for (i = 0; i < nb; i++) {
        const uint8_t* blk = a + (size_t)i * bb;
        float dd = qro_h2f(rd16(blk));
        float dmin = qro_h2f(rd16(blk + 2));
        for (j = 0; j < 8; j++) {
            const uint8_t* xb = b + (size_t)(i * 8 + j) * Q8_BYTES;
            float sc = (float)(blk[4 + j] & 63) * dd;
            float m = (float)(blk[4 + j] >> 6) * dmin;
            int isum = 0, bsum = 0;
            float bd;
            for (l = 0; l < 32; l++) {
                int e = j * 32 + l;
                int q = type == QRO_TYPE_Q4_K ? q4k_q(blk, e) : q5k_q(blk, e);
                int bv = (int8_t)xb[2 + l];
                isum += q * bv;
                bsum += bv;
            }
            bd = qro_h2f(rd16(xb));
            sumf += (sc * (float)isum - m * (float)bsum) * bd;
        }
    }
    return sumf;
}

/* src/quant.c:406-437: sumf += sc * isum * bd, left to right. */
static float dot_q6k(const uint8_t* a, const uint8_t* b, int d) {
    int nb = d / QKK, i, j, l;
    float sumf = 0.0f;
    for (i = 0; i < nb; i++) {
        const uint8_t* blk = a + (size_t)i * Q6K_BYTES;
        float dd = qro_h2f(rd16(blk + 208));
        for (j = 0; j < 8; j++) {
            const uint8_t* xb = b + (size_t)(i * 8 + j) * Q8_BYTES;
            float sc = (float)(int8_t)blk[192 + j] * dd;
            int isum = 0;
            float bd;
            for (l = 0; l < 32; l++) isum += q6k_q(blk, j * 32 + l) * (int)(int8_t)xb[2 + l];
            bd = qro_h2f(rd16(xb));
            sumf += sc * (float)isum * bd;
        }
    }
    return sumf;
}

float qro_vec_dot(uint32_t type, const void* row, const void* xq8, int d, int order) {
    const uint8_t* a = (const uint8_t*)row;
    const uint8_t* b = (const uint8_t*)xq8;
    switch (type) {
        case QRO_TYPE_Q8_0: return dot_q8_0(a, b, d, order);
        case QRO_TYPE_Q4_K:
        case QRO_TYPE_Q5_K: return dot_q45k(a, b, d, type);
        case QRO_TYPE_Q6_K: return dot_q6k(a, b, d);
        default: return 0.0f;
    }
}

/* src/quant.c:441-523 for one activation: NULL weights give zeros; F32 rows
 * are a sequential multiply-add; quantized rows quantize x once to Q8_0 and
 * run the fused dot per row under an OpenMP static schedule.  Unknown types
 * dequantize to zeros (src/quant.c:239), so their rows are 0. */
void qro_matmul_q_fused(float* out, const float* x, const void* w, uint32_t type,
                        int n, int d, int threads, int order) {
    qro_matmul_q_fused_batch(out, x, w, type, n, d, 1, threads, order);
}

/* nt independent activations (x is [nt][d], out is [nt][n]); the reference
 * runs these as nt separate calls. */
void qro_matmul_q_fused_batch(float* out, const float* x, const void* w, uint32_t type,
                              int n, int d, int nt, int threads, int order) {
    int t, i;
    size_t rb;
    uint8_t* xq;
    int nbx = d / QK8 > 0 ? d / QK8 : 1;
    if (w == NULL) {
        memset(out, 0, (size_t)n * (size_t)nt * sizeof(float));
        return;
    }
    if (type == QRO_TYPE_F32) {
        for (t = 0; t < nt; t++) {
            const float* xt = x + (size_t)t * (size_t)d;
            float* ot = out + (size_t)t * (size_t)n;
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
#endif
            for (i = 0; i < n; i++) {
                const float* r = (const float*)w + (size_t)i * (size_t)d;
                float sum = 0.0f;
                int j;
                for (j = 0; j < d; j++) sum += r[j] * xt[j];
                ot[i] = sum;
            }
        }
        return;
    }
    rb = qro_row_bytes(type, d);
    xq = (uint8_t*)calloc((size_t)nbx * (size_t)nt, Q8_BYTES);
    if (!xq) {
        memset(out, 0, (size_t)n * (size_t)nt * sizeof(float));
        return;
    }
    for (t = 0; t < nt; t++)
        qro_quantize_row_q8_0(x + (size_t)t * (size_t)d, xq + (size_t)t * nbx * Q8_BYTES, d);
    for (t = 0; t < nt; t++) {
        const uint8_t* xt = xq + (size_t)t * nbx * Q8_BYTES;
        float* ot = out + (size_t)t * (size_t)n;
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
#endif
        for (i = 0; i < n; i++) {
            const uint8_t* r = (const uint8_t*)w + (size_t)i * rb;
            if (type == QRO_TYPE_Q8_0 || type == QRO_TYPE_Q4_K || type == QRO_TYPE_Q5_K ||
                type == QRO_TYPE_Q6_K)
                ot[i] = qro_vec_dot(type, r, xt, d, order);
            else
                ot[i] = 0.0f;
        }
    }
    free(xq);
}

/* src/kernels.c:18-28 (SEQ: multiply then add, j ascending),
 * src/kernels.c:50-65 (AVX2: lane k holds the FMA chain over j = 8i+k, lanes
 * summed 0..7 into a zero, then a multiply-add tail) and src/kernels.c:38-49
 * (AVX512: 16 FMA chains, _mm512_reduce_add_ps as GCC defines it: upper 8 +
 * lower 8, upper 4 + lower 4, then [0]+[2], [1]+[3], then ([0]+[2])+([1]+[3])). */
void qro_matmul_f32(float* out, const float* x, const float* w, int n, int d, int order) {
    int i, j, k;
    for (i = 0; i < n; i++) {
        const float* r = w + (size_t)i * (size_t)d;
        float sum = 0.0f;
        if (order == QRO_ORDER_SEQ) {
            for (j = 0; j < d; j++) sum += r[j] * x[j];
        } else if (order == QRO_ORDER_AVX2) {
            float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (j = 0; j + 8 <= d; j += 8)
                for (k = 0; k < 8; k++) acc[k] = fmaf(r[j + k], x[j + k], acc[k]);
            for (k = 0; k < 8; k++) sum += acc[k];
            for (; j < d; j++) sum += r[j] * x[j];
        } else {
            float acc[16], t8[8], t4[4], a02, a13;
            memset(acc, 0, sizeof(acc));
            for (j = 0; j + 16 <= d; j += 16)
                for (k = 0; k < 16; k++) acc[k] = fmaf(r[j + k], x[j + k], acc[k]);
            for (k = 0; k < 8; k++) t8[k] = acc[8 + k] + acc[k];
            for (k = 0; k < 4; k++) t4[k] = t8[4 + k] + t8[k];
            a02 = t4[0] + t4[2];
            a13 = t4[1] + t4[3];
            sum += a02 + a13;
            for (; j < d; j++) sum += r[j] * x[j];
        }
        out[i] = sum;
    }
}

/* src/kernels.c:191-207. */
void qro_softmax(float* x, int n) {
    float max_val = x[0], sum = 0.0f, inv;
    int i;
    for (i = 1; i < n; i++)
        if (x[i] > max_val) max_val = x[i];
    for (i = 0; i < n; i++) {
        x[i] = expf(x[i] - max_val);
        sum += x[i];
    }
    inv = 1.0f / sum;
    for (i = 0; i < n; i++) x[i] *= inv;
}

/* src/runtime.c:15-17. */
float qro_silu(float x) { return x / (1.0f + expf(-x)); }

void qro_expf_batch(const float* in, float* out, size_t n) {
    size_t i;
    for (i = 0; i < n; i++) out[i] = expf(in[i]);
}

/* src/runtime.c:205-230: router logits, softmax, K argmax passes (strict '>',
 * start -1e9f, lowest index wins ties, winner masked to -1e9f), then each
 * weight divided by the sequential sum of the K weights. */
int qro_route(const float* xb, const float* router_w, int dim, int E, int K, int order,
              float* logits, float* probs, int32_t* idx, float* wts) {
    float* p = (float*)malloc((size_t)E * sizeof(float));
    float wsum = 0.0f;
    int k, e;
    if (!p) return -1;
    qro_matmul_f32(p, xb, router_w, E, dim, order);
    if (logits) memcpy(logits, p, (size_t)E * sizeof(float));
    qro_softmax(p, E);
    if (probs) memcpy(probs, p, (size_t)E * sizeof(float));
    for (k = 0; k < K; k++) {
        float max_val = -1e9f;
        int max_idx = -1;
        for (e = 0; e < E; e++) {
            if (p[e] > max_val) {
                max_val = p[e];
                max_idx = e;
            }
        }
        idx[k] = max_idx;
        wts[k] = max_val;
        if (max_idx >= 0) p[max_idx] = -1e9f;
    }
    for (k = 0; k < K; k++) wsum += wts[k];
    for (k = 0; k < K; k++) wts[k] /= wsum;
    free(p);
    return 0;
}

static void matmul_any(float* out, const float* x, const void* w, uint32_t type, int n, int d,
                       int threads, int router_order, int dot_order) {
    /* src/runtime.c:58-70: NULL -> zeros, F32 -> KernelOps.matmul (the
     * backend's order), otherwise the fused quantized path. */
    if (w == NULL) {
        memset(out, 0, (size_t)n * sizeof(float));
    } else if (type == QRO_TYPE_F32) {
        qro_matmul_f32(out, x, (const float*)w, n, d, router_order);
    } else if (type & QRO_GGML) {
        qro_ggml_matmul_mt(out, x, w, (int)(type & ~QRO_GGML), n, d, 1, threads);
    } else {
        qro_matmul_q_fused(out, x, w, type, n, d, threads, dot_order);
    }
}

/* Shared expert with a sigmoid gate (no reference counterpart):
 * y = sigmoid(sum_j g[j]*xb[j]) * down(silu(up(xb)) * gate(xb)), the gate dot
 * in sequential order, the SwiGLU in the reference's slot convention. */
void qro_shared_expert(float* y, const float* xb, const qro_moe_layer* L, int threads) {
    int H = L->sh_hidden, dim = L->dim, i;
    float* hb = (float*)malloc((size_t)H * 2 * sizeof(float));
    float g = 0.0f, sg;
    if (!hb) return;
    matmul_any(hb, xb, L->sh_up, L->sh_up_type, H, dim, threads, QRO_ORDER_SEQ, QRO_ORDER_SEQ);
    matmul_any(hb + H, xb, L->sh_gate, L->sh_gate_type, H, dim, threads, QRO_ORDER_SEQ,
               QRO_ORDER_SEQ);
    for (i = 0; i < H; i++) hb[i] = qro_silu(hb[i]) * hb[H + i];
    matmul_any(y, hb, L->sh_down, L->sh_down_type, dim, H, threads, QRO_ORDER_SEQ, QRO_ORDER_SEQ);
    for (i = 0; i < dim; i++) g += L->sh_gate_inp[i] * xb[i];
    sg = 1.0f / (1.0f + expf(-g));
    for (i = 0; i < dim; i++) y[i] = sg * y[i];
    free(hb);
}

/* src/runtime.c:202-269 for one token: route, then for each slot in order run
 * up (SiLU slot), gate, silu(up)*gate, down, and accumulate xb2 += y*w in slot
 * order; finally x += xb2.  A shared expert, when present, adds its output to
 * xb2 after the routed slots. */
void qro_moe_token(float* x, const float* xb, const qro_moe_layer* L, int router_order,
                   int dot_order, int threads, int32_t* idx_out, float* w_out) {
    int dim = L->dim, H = L->hidden, K = L->n_used, k, i;
    int32_t idx[64];
    float wts[64];
    float* buf = (float*)malloc(((size_t)dim * 2 + (size_t)H * 2) * sizeof(float));
    float *xb2, *y, *hb, *hb2;
    size_t s_up, s_gate, s_down;
    if (!buf || K > 64) {
        free(buf);
        return;
    }
    xb2 = buf;
    y = buf + dim;
    hb = buf + 2 * dim;
    hb2 = hb + H;
    qro_route(xb, L->router, dim, L->n_experts, K, router_order, NULL, NULL, idx, wts);
    s_up = qro_expert_slice_bytes(L->up_type, dim, H);
    s_gate = qro_expert_slice_bytes(L->gate_type, dim, H);
    s_down = qro_expert_slice_bytes(L->down_type, H, dim);
    memset(xb2, 0, (size_t)dim * sizeof(float));
    for (k = 0; k < K; k++) {
        int e = idx[k];
        float ew = wts[k];
        const uint8_t* wu = (const uint8_t*)L->up + (size_t)e * s_up;
        const uint8_t* wg = (const uint8_t*)L->gate + (size_t)e * s_gate;
        const uint8_t* wd = (const uint8_t*)L->down + (size_t)e * s_down;
        matmul_any(hb, xb, wu, L->up_type, H, dim, threads, router_order, dot_order);
        matmul_any(hb2, xb, wg, L->gate_type, H, dim, threads, router_order, dot_order);
        for (i = 0; i < H; i++) hb[i] = qro_silu(hb[i]) * hb2[i];
        matmul_any(y, hb, wd, L->down_type, dim, H, threads, router_order, dot_order);
        for (i = 0; i < dim; i++) xb2[i] += y[i] * ew;
    }
    if (L->sh_hidden > 0) {
        qro_shared_expert(y, xb, L, threads);
        for (i = 0; i < dim; i++) xb2[i] += y[i];
    }
    for (i = 0; i < dim; i++) x[i] += xb2[i];
    if (idx_out) memcpy(idx_out, idx, (size_t)K * sizeof(int32_t));
    if (w_out) memcpy(w_out, wts, (size_t)K * sizeof(float));
    free(buf);
}

/* The dense FFN of forward_runtime (src/runtime.c:270-284), a layer with
 * n_experts == 0: hb = up . xb (w1, the SiLU slot), hb2 = gate . xb (w3),
 * hb = silu(hb) * hb2, xb = down . hb (w2), x += xb. */
void qro_dense_ffn(float* x, const float* xb, const qro_moe_layer* L, int order, int threads) {
    int dim = L->dim, H = L->hidden, i;
    float* buf = (float*)malloc(((size_t)dim + (size_t)H * 2) * sizeof(float));
    float *y, *hb, *hb2;
    if (!buf) return;
    y = buf;
    hb = buf + dim;
    hb2 = hb + H;
    matmul_any(hb, xb, L->up, L->up_type, H, dim, threads, order, order);
    matmul_any(hb2, xb, L->gate, L->gate_type, H, dim, threads, order, order);
    for (i = 0; i < H; i++) hb[i] = qro_silu(hb[i]) * hb2[i];
    matmul_any(y, hb, L->down, L->down_type, dim, H, threads, order, order);
    for (i = 0; i < dim; i++) x[i] += y[i];
    free(buf);
}

/* T independent tokens: the reference runs one forward_runtime per token
 * (src/runtime.c:294-304), so the batch is the per-token block in order. */
void qro_moe_forward(float* x, const float* xb, int T, const qro_moe_layer* L, int router_order,
                     int dot_order, int threads, int32_t* idx_out, float* w_out) {
    int t, K = L->n_used;
    for (t = 0; t < T; t++)
        qro_moe_token(x + (size_t)t * L->dim, xb + (size_t)t * L->dim, L, router_order, dot_order,
                      threads,
                      idx_out ? idx_out + (size_t)t * K : NULL, w_out ? w_out + (size_t)t * K : NULL);
}

/* Token-to-expert dispatch (no reference counterpart; the reference runs one
 * token at a time).  Pairs p = t*K + k are counted per expert, offsets is the
 * exclusive scan (E+1 entries), perm lists the pairs grouped by expert and, in
 * each group, in increasing p (a stable counting sort), inv[p] is the position
 * of pair p in perm. */
int qro_moe_dispatch(const int32_t* idx, int T, int K, int E, int32_t* counts,
                     int32_t* offsets, int32_t* perm, int32_t* inv) {
    int p, e, P = T * K;
    int32_t* cur = (int32_t*)malloc((size_t)(E > 0 ? E : 1) * sizeof(int32_t));
    if (!cur) return -1;
    for (e = 0; e < E; e++) counts[e] = 0;
    for (p = 0; p < P; p++) {
        if (idx[p] < 0 || idx[p] >= E) {
            free(cur);
            return -2;
        }
        counts[idx[p]]++;
    }
    offsets[0] = 0;
    for (e = 0; e < E; e++) offsets[e + 1] = offsets[e] + counts[e];
    for (e = 0; e < E; e++) cur[e] = offsets[e];
    for (p = 0; p < P; p++) {
        int pos = cur[idx[p]]++;
        perm[pos] = p;
        inv[p] = pos;
    }
    free(cur);
    return 0;
}
