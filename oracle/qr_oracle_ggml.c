/* qr_oracle_ggml.c -- test infrastructure only (the parity checker, never the
 * product): a C99 restatement of llama.cpp / ggml's K-quant formats and their
 * CPU reference arithmetic, which the reference (bharqav/quantr-in-c) does not
 * implement (its Q4_K / Q5_K / Q6_K bit layouts are its own, src/quant.c:180-238).
 *
 * Restated from ggml's published source (ggml-common.h block layouts,
 * ggml-quants.c: get_scale_min_k4, dequantize_row_q{4,5,6}_K,
 * quantize_row_q8_K_ref, and the generic ggml_vec_dot_q{4,5,6}_K_q8_K) --
 * ggml is not present in this container, so nothing here is checked against
 * it; the functions are pinned by closed forms (tests/test_oracle_ggml.py):
 * the IEEE half conversion against numpy on all 65,536 codes, packing and
 * unpacking written independently, the integer parts against brute force,
 * the dots against a float64 dequantize-then-dot.
 *
 *   block_q4_K: f16 d, f16 dmin, u8 scales[12], u8 qs[128]          (144 B)
 *   block_q5_K: f16 d, f16 dmin, u8 scales[12], u8 qh[32], qs[128]  (176 B)
 *   block_q6_K: u8 ql[128], u8 qh[64], i8 scales[16], f16 d          (210 B)
 *   block_q8_K: f32 d, i8 qs[256], i16 bsums[16]                     (292 B)
 *
 * Compiled -std=c99 -ffp-contract=off: every float operation rounds once, in
 * the written order (ggml's generic C path is plain scalar C).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define QK 256

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* IEEE binary16 -> binary32, exact (subnormals, infinities, NaN payloads). */
float qro_ggml_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1F;
    uint32_t man = h & 0x3FF;
    uint32_t bits;
    float f;
    if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: man * 2^-24, exact in binary32 */
            int e = -1;
            do {
                man <<= 1;
                e++;
            } while (!(man & 0x400));
            man &= 0x3FF;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    }
    memcpy(&f, &bits, 4);
    return f;
}

void qro_ggml_h2f_batch(const uint16_t* h, float* out, long n) {
    long i;
    for (i = 0; i < n; i++) out[i] = qro_ggml_h2f(h[i]);
}

size_t qro_ggml_block_bytes(int type) {
    return type == 12 ? 144 : type == 13 ? 176 : type == 14 ? 210 : 0;
}

/* get_scale_min_k4: 6-bit scale and min of sub-block j from the 12 bytes. */
static void scale_min_k4(int j, const uint8_t* q, int* d, int* m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

void qro_ggml_scale_min(const uint8_t* scales12, int* sc, int* mn) {
    int j;
    for (j = 0; j < 8; j++) scale_min_k4(j, scales12, &sc[j], &mn[j]);
}

/* dequantize_row_q{4,5,6}_K of n elements (whole 256-element blocks). */
void qro_ggml_dequantize_row(int type, const void* src, float* y, int n) {
    const uint8_t* b = (const uint8_t*)src;
    const int nb = n / QK;
    int i, j, l;
    for (i = 0; i < nb; i++) {
        if (type == 12 || type == 13) {
            const uint8_t* blk = b + (size_t)i * (type == 12 ? 144 : 176);
            const float d = qro_ggml_h2f(rd16(blk)), min = qro_ggml_h2f(rd16(blk + 2));
            const uint8_t* scales = blk + 4;
            const uint8_t* qh = blk + 16;
            const uint8_t* q = blk + (type == 12 ? 16 : 48);
            int is = 0, sc, m;
            uint8_t u1 = 1, u2 = 2;
            for (j = 0; j < QK; j += 64) {
                float d1, m1, d2, m2;
                scale_min_k4(is + 0, scales, &sc, &m);
                d1 = d * sc;
                m1 = min * m;
                scale_min_k4(is + 1, scales, &sc, &m);
                d2 = d * sc;
                m2 = min * m;
                for (l = 0; l < 32; l++) {
                    int v = q[l] & 0xF;
                    if (type == 13) v += (qh[l] & u1) ? 16 : 0;
                    *y++ = d1 * v - m1;
                }
                for (l = 0; l < 32; l++) {
                    int v = q[l] >> 4;
                    if (type == 13) v += (qh[l] & u2) ? 16 : 0;
                    *y++ = d2 * v - m2;
                }
                q += 32;
                is += 2;
                u1 <<= 2;
                u2 <<= 2;
            }
        } else if (type == 14) {
            const uint8_t* blk = b + (size_t)i * 210;
            const float d = qro_ggml_h2f(rd16(blk + 208));
            const uint8_t* ql = blk;
            const uint8_t* qh = blk + 128;
            const int8_t* sc = (const int8_t*)(blk + 192);
            int n0;
            for (n0 = 0; n0 < QK; n0 += 128) {
                for (l = 0; l < 32; l++) {
                    const int is = l / 16;
                    const int8_t q1 = (int8_t)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    const int8_t q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    const int8_t q3 = (int8_t)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    const int8_t q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    y[l + 0] = d * sc[is + 0] * q1;
                    y[l + 32] = d * sc[is + 2] * q2;
                    y[l + 64] = d * sc[is + 4] * q3;
                    y[l + 96] = d * sc[is + 6] * q4;
                }
                y += 128;
                ql += 64;
                qh += 32;
                sc += 8;
            }
        } else {
            for (j = 0; j < QK; j++) *y++ = 0.0f;
        }
    }
}

/* nearest_int: round to nearest, ties to even, by the 1.5 * 2^23 addition. */
static int nearest_int(float fval) {
    float val = fval + 12582912.f;
    int i;
    memcpy(&i, &val, sizeof(int));
    return (i & 0x007fffff) - 0x00400000;
}

/* quantize_row_q8_K_ref: per block, the value of largest magnitude (the first
 * one on ties) sets iscale = -127 / max; q = min(127, nearest_int(iscale x));
 * d = 1 / iscale; bsums over 16-element groups.  An all-zero block gets d = 0
 * and zero quants (and zero bsums here). */
void qro_quantize_row_q8_K(const float* x, void* vy, int k) {
    uint8_t* y = (uint8_t*)vy;
    const int nb = k / QK;
    int i, j, ii;
    for (i = 0; i < nb; i++) {
        uint8_t* blk = y + (size_t)i * 292;
        float* d = (float*)blk;
        int8_t* qs = (int8_t*)(blk + 4);
        int16_t bs[16];
        float max = 0, amax = 0, iscale, dv;
        for (j = 0; j < QK; j++) {
            const float ax = fabsf(x[j]);
            if (ax > amax) {
                amax = ax;
                max = x[j];
            }
        }
        if (!amax) {
            dv = 0.0f;
            memcpy(d, &dv, 4);
            memset(qs, 0, QK);
            memset(blk + 260, 0, 32);
            x += QK;
            continue;
        }
        iscale = -127.f / max;
        for (j = 0; j < QK; j++) {
            const int v = nearest_int(iscale * x[j]);
            qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (j = 0; j < QK / 16; j++) {
            int sum = 0;
            for (ii = 0; ii < 16; ii++) sum += qs[j * 16 + ii];
            bs[j] = (int16_t)sum;
        }
        memcpy(blk + 260, bs, 32);
        dv = 1 / iscale;
        memcpy(d, &dv, 4);
        x += QK;
    }
}

/* The integer parts of one block's dot: aux32[8] (lane l sums the products of
 * elements 8t + l, each 8-element group scaled by its sub-block's scale) and,
 * for Q4_K / Q5_K, sumi = sum_j bsums[j] * min[j / 2]. */
static void block_ints(int type, const uint8_t* blk, const uint8_t* yb, int32_t* aux32,
                       int32_t* sumi) {
    int8_t a[QK];
    const int8_t* q8 = (const int8_t*)(yb + 4);
    const int16_t* bsums = (const int16_t*)(yb + 260);
    int j, l, t;
    int sc[16], mn[8];
    int16_t bsv[16];
    memcpy(bsv, bsums, 32);
    for (l = 0; l < 8; l++) aux32[l] = 0;
    *sumi = 0;
    if (type == 12 || type == 13) {
        const uint8_t* q4 = blk + (type == 12 ? 16 : 48);
        const uint8_t* hm = blk + 16;
        uint8_t m = 1;
        int8_t* p = a;
        for (j = 0; j < QK / 64; j++) {
            for (l = 0; l < 32; l++) p[l] = (int8_t)(q4[l] & 0xF);
            if (type == 13)
                for (l = 0; l < 32; l++) p[l] += (hm[l] & m ? 16 : 0);
            p += 32;
            m <<= 1;
            for (l = 0; l < 32; l++) p[l] = (int8_t)(q4[l] >> 4);
            if (type == 13)
                for (l = 0; l < 32; l++) p[l] += (hm[l] & m ? 16 : 0);
            p += 32;
            m <<= 1;
            q4 += 32;
        }
        qro_ggml_scale_min(blk + 4, sc, mn);
        for (j = 0; j < QK / 16; j++) *sumi += bsv[j] * mn[j / 2];
        for (j = 0; j < QK / 32; j++)      /* 8 sub-blocks of 32 */
            for (t = 0; t < 4; t++)        /* 4 groups of 8 */
                for (l = 0; l < 8; l++) aux32[l] += sc[j] * (q8[32 * j + 8 * t + l] * a[32 * j + 8 * t + l]);
    } else {
        const uint8_t* q4 = blk;
        const uint8_t* qh = blk + 128;
        const int8_t* scales = (const int8_t*)(blk + 192);
        int8_t* p = a;
        for (j = 0; j < QK; j += 128) {
            for (l = 0; l < 32; l++) {
                p[l + 0] = (int8_t)((q4[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                p[l + 32] = (int8_t)((q4[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                p[l + 64] = (int8_t)((q4[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                p[l + 96] = (int8_t)((q4[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            }
            p += 128;
            q4 += 64;
            qh += 32;
        }
        for (j = 0; j < QK / 16; j++)      /* 16 sub-blocks of 16 */
            for (t = 0; t < 2; t++)
                for (l = 0; l < 8; l++) aux32[l] += scales[j] * (q8[16 * j + 8 * t + l] * a[16 * j + 8 * t + l]);
    }
}

/* The exposed integer parts (for the brute-force check). */
void qro_ggml_block_ints(int type, const void* blk, const void* yb, int32_t* aux32,
                         int32_t* sumi) {
    block_ints(type, (const uint8_t*)blk, (const uint8_t*)yb, aux32, sumi);
}

/* ggml_vec_dot_q{4,5,6}_K_q8_K, generic path: per block
 *   d = h2f(x.d) * y.d;  sums[l] += d * aux32[l]  (l = 0..7)
 *   dmin = h2f(x.dmin) * y.d;  sumf -= dmin * sumi   (Q4_K / Q5_K)
 * and after the blocks sumf += sums[0] ... sums[7]. */
float qro_ggml_vec_dot(int type, const void* row, const void* q8k, int n) {
    const uint8_t* x = (const uint8_t*)row;
    const uint8_t* y = (const uint8_t*)q8k;
    const size_t bb = qro_ggml_block_bytes(type);
    const int nb = n / QK;
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float sumf = 0;
    int i, l;
    for (i = 0; i < nb; i++) {
        const uint8_t* blk = x + (size_t)i * bb;
        const uint8_t* yb = y + (size_t)i * 292;
        int32_t aux32[8], sumi;
        float yd, d;
        memcpy(&yd, yb, 4);
        block_ints(type, blk, yb, aux32, &sumi);
        d = qro_ggml_h2f(rd16(type == 14 ? blk + 208 : blk)) * yd;
        for (l = 0; l < 8; l++) sums[l] += d * aux32[l];
        if (type != 14) {
            const float dmin = qro_ggml_h2f(rd16(blk + 2)) * yd;
            sumf -= dmin * sumi;
        }
    }
    for (l = 0; l < 8; l++) sumf += sums[l];
    return sumf;
}

/* out[t][r] = dot(row r, Q8_K(x[t])) for t < nt; rows split over `threads`
 * (each row's dot is independent: the same bits at any width). */
void qro_ggml_matmul_mt(float* out, const float* x, const void* w, int type, int n, int d, int nt,
                        int threads) {
    const size_t rb = qro_ggml_block_bytes(type) * (size_t)(d / QK);
    uint8_t yq[292 * 64];
    int t, r;
    for (t = 0; t < nt; t++) {
        qro_quantize_row_q8_K(x + (size_t)t * d, yq, d);
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
        for (r = 0; r < n; r++)
            out[(size_t)t * n + r] = qro_ggml_vec_dot(type, (const uint8_t*)w + (size_t)r * rb, yq, d);
    }
}

void qro_ggml_matmul(float* out, const float* x, const void* w, int type, int n, int d, int nt) {
    qro_ggml_matmul_mt(out, x, w, type, n, d, nt, 1);
}
