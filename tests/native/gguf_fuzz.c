/*
 * Mutation fuzzing of the GGUF container parser and model mapping
 * (quantr-in-c_amd/host/qr_gguf.c), built with AddressSanitizer and
 * UndefinedBehaviorSanitizer on the CPU by tests/test_gguf_fuzz.py -- the
 * counterpart of the reference's tests/fuzz_gguf.c:46-77 (tiny and corrupt
 * headers, random payloads, magic-prefixed payloads), plus structure-aware
 * mutations of valid model files: byte and bit flips, truncations, and 4- and
 * 8-byte little-endian fields overwritten with boundary values (counts,
 * lengths, dimensions, offsets, types).
 *
 *   gguf_fuzz SEED ITERATIONS FILE...
 *
 * Every input goes through qr_gguf_parse; an accepted one through the lookups,
 * qr_gguf_model_host (count, then fill) and qr_gguf_expert_host of every
 * layer and expert the mapping reports, and the first and last byte of every
 * tensor range those hand out is read (the ranges qr_gguf_load copies).  Any sanitizer report ends the run
 * with a non-zero status.  The device functions qr_gguf.c references (used
 * only by qr_gguf_load, never called here) are stubs that abort.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qr_hip.h"

/* ---- what qr_gguf.c takes from the rest of the library ------------------ */
size_t qr_row_bytes(uint32_t type, int d) {
    type &= ~(uint32_t)(QR_TILED | QR_GGML);
    if (d < 0) return 0;
    switch (type) {
        case 0: return (size_t)d * 4;
        case 8: return (size_t)(d / 32) * 34;
        case 12: return (size_t)(d / 256) * 144;
        case 13: return (size_t)(d / 256) * 176;
        case 14: return (size_t)(d / 256) * 210;
        default: return 0;
    }
}
int qrint_set_error(int code, const char* msg) {
    (void)msg;
    return code;
}
int qr_malloc(qr_ctx* c, size_t n, void** p) { (void)c; (void)n; (void)p; abort(); }
int qr_free(qr_ctx* c, void* p) { (void)c; (void)p; abort(); }
int qr_memcpy_h2d(qr_ctx* c, void* d, const void* s, size_t n) { (void)c; (void)d; (void)s; (void)n; abort(); }
int qr_sync(qr_ctx* c) { (void)c; abort(); }
int qr_weights_tile(qr_ctx* c, uint32_t t, const void* s, void* d, int n, int k) {
    (void)c; (void)t; (void)s; (void)d; (void)n; (void)k; abort();
}

/* ---- one input ----------------------------------------------------------- */
static long accepted, mapped;
static volatile uint8_t sink;

/* The first and last byte of a range the mapping hands out (what
 * qr_gguf_load would copy): a range past the buffer is a sanitizer report. */
static void touch(const void* p, size_t bytes) {
    if (!p || !bytes) return;
    sink ^= ((const uint8_t*)p)[0];
    sink ^= ((const uint8_t*)p)[bytes - 1];
}

static void touch_model(const qr_gguf* g, const qr_model* m, const qr_layer* layers) {
    const int dim = m->dim, qd = m->n_heads * m->head_dim, kvd = m->n_kv_heads * m->head_dim;
    int l, e;
    touch(m->tok_embd, qr_row_bytes(m->tok_type, dim) * (size_t)m->vocab);
    touch(m->rms_final, (size_t)dim * 4);
    touch(m->wcls, qr_row_bytes(m->wcls_type, dim) * (size_t)m->vocab);
    for (l = 0; l < m->n_layers; l++) {
        const qr_layer* y = &layers[l];
        const qr_moe_layer* M = &y->moe;
        const size_t su = qr_row_bytes(M->up_type, dim) * (size_t)M->hidden;
        const size_t sg = qr_row_bytes(M->gate_type, dim) * (size_t)M->hidden;
        const size_t sd = qr_row_bytes(M->down_type, M->hidden) * (size_t)dim;
        touch(y->rms_att, (size_t)dim * 4);
        touch(y->rms_ffn, (size_t)dim * 4);
        touch(y->wq, qr_row_bytes(y->wq_type, dim) * (size_t)qd);
        touch(y->wk, qr_row_bytes(y->wk_type, dim) * (size_t)kvd);
        touch(y->wv, qr_row_bytes(y->wv_type, dim) * (size_t)kvd);
        touch(y->wo, qr_row_bytes(y->wo_type, qd) * (size_t)dim);
        if (M->n_experts == 0) { /* dense FFN */
            touch(M->up, su);
            touch(M->gate, sg);
            touch(M->down, sd);
            continue;
        }
        touch(M->router, (size_t)M->n_experts * (size_t)dim * 4);
        for (e = 0; e < M->n_experts && e < 4096; e++) {
            const void *u = NULL, *d = NULL, *gt = NULL;
            if (qr_gguf_expert_host(g, l, e, &u, &d, &gt) != QR_OK) continue;
            touch(u, su);
            touch(gt, sg);
            touch(d, sd);
        }
    }
}

static void one(const uint8_t* data, size_t size) {
    /* a private copy of exactly `size` bytes, so the sanitizer sees any read
     * past the end */
    uint8_t* buf = (uint8_t*)malloc(size ? size : 1);
    qr_gguf* g = NULL;
    if (!buf) return;
    memcpy(buf, data, size);
    if (qr_gguf_parse(buf, size, &g) == QR_OK && g) {
        qr_model m;
        int L;
        accepted++;
        (void)qr_gguf_find(g, "token_embd.weight");
        (void)qr_gguf_get_u32(g, "general.alignment", 32);
        (void)qr_gguf_get_f32(g, "qwen3moe.rope.freq_base", 1.0f);
        (void)qr_gguf_get_str(g, "general.architecture");
        (void)qr_gguf_get_arr_len(g, "tokenizer.ggml.tokens");
        L = qr_gguf_model_host(g, 64, &m, NULL, 0);
        if (L > 0 && L <= 4096) {
            qr_layer* layers = (qr_layer*)calloc((size_t)L, sizeof(qr_layer));
            if (layers && qr_gguf_model_host(g, 64, &m, layers, L) == L) {
                mapped++;
                touch_model(g, &m, layers);
            }
            free(layers);
        }
        qr_gguf_close(g);
    }
    free(buf);
}

/* ---- mutations ------------------------------------------------------------ */
static uint64_t rng = 0x9E3779B97F4A7C15ull;
static uint64_t next(void) {
    rng ^= rng << 13;
    rng ^= rng >> 7;
    rng ^= rng << 17;
    return rng;
}

static const uint64_t kEdge[] = {0, 1, 2, 3, 4, 5, 31, 32, 63, 64, 255, 256, 4095, 65535, 65536,
                                 65537, 1u << 20, (1u << 20) + 1, 0x7FFFFFFF, 0x80000000u,
                                 0xFFFFFFFFu, 0x100000000ull, 0x7FFFFFFFFFFFFFFFull,
                                 0x8000000000000000ull, 0xFFFFFFFFFFFFFFFFull};

static void mutate(uint8_t* b, size_t* n, size_t cap) {
    const int ops = 1 + (int)(next() % 4);
    int i;
    for (i = 0; i < ops && *n > 0; i++) {
        const size_t at = (size_t)(next() % *n);
        switch (next() % 6) {
            case 0: b[at] = (uint8_t)next(); break;
            case 1: b[at] ^= (uint8_t)(1u << (next() % 8)); break;
            case 2: { /* a 4-byte field */
                const uint64_t v = kEdge[next() % (sizeof(kEdge) / sizeof(kEdge[0]))];
                if (at + 4 <= *n) memcpy(b + at, &v, 4);
                break;
            }
            case 3: { /* an 8-byte field */
                const uint64_t v = kEdge[next() % (sizeof(kEdge) / sizeof(kEdge[0]))];
                if (at + 8 <= *n) memcpy(b + at, &v, 8);
                break;
            }
            case 4: *n = at; break; /* truncate */
            default: { /* grow with random bytes */
                const size_t add = (size_t)(next() % 64);
                size_t j;
                for (j = 0; j < add && *n < cap; j++) b[(*n)++] = (uint8_t)next();
                break;
            }
        }
    }
}

static uint8_t* read_file(const char* path, size_t* n) {
    FILE* f = fopen(path, "rb");
    uint8_t* b;
    long sz;
    if (!f) return NULL;
    fseek(f, 0, SEEK_END);
    sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    b = (uint8_t*)malloc((size_t)sz + 1);
    if (b && fread(b, 1, (size_t)sz, f) != (size_t)sz) {
        free(b);
        b = NULL;
    }
    fclose(f);
    *n = (size_t)sz;
    return b;
}

int main(int argc, char** argv) {
    long iters, it;
    int nseeds = argc - 3, s;
    uint8_t** seeds;
    size_t* sizes;
    size_t cap = 0;
    uint8_t *work, tiny[8] = {'G', 'G', 'U', 'F', 3, 0, 0, 0}, hdr[64];
    if (argc < 3) {
        fprintf(stderr, "usage: gguf_fuzz SEED ITERATIONS FILE...\n");
        return 2;
    }
    rng ^= strtoull(argv[1], NULL, 0) * 0x2545F4914F6CDD1Dull;
    iters = strtol(argv[2], NULL, 0);
    seeds = (uint8_t**)calloc((size_t)(nseeds > 0 ? nseeds : 1), sizeof(uint8_t*));
    sizes = (size_t*)calloc((size_t)(nseeds > 0 ? nseeds : 1), sizeof(size_t));
    for (s = 0; s < nseeds; s++) {
        seeds[s] = read_file(argv[3 + s], &sizes[s]);
        if (!seeds[s]) {
            fprintf(stderr, "cannot read %s\n", argv[3 + s]);
            return 2;
        }
        if (sizes[s] > cap) cap = sizes[s];
    }
    cap += 4096;
    work = (uint8_t*)malloc(cap);
    if (!work) return 2;
    /* the reference harness's fixed cases */
    one(tiny, sizeof(tiny));
    memset(hdr, 0xFF, sizeof(hdr));
    memcpy(hdr, "GGUF", 4);
    hdr[4] = 3;
    one(hdr, sizeof(hdr));
    for (s = 0; s < nseeds; s++) one(seeds[s], sizes[s]);
    for (it = 0; it < iters; it++) {
        size_t n;
        const int kind = (int)(next() % 8);
        if (kind == 0 || nseeds == 0) { /* random payload, magic and version 3 on two of three */
            size_t j;
            n = 16 + (size_t)(next() % 4096);
            for (j = 0; j < n; j++) work[j] = (uint8_t)next();
            if (next() % 3 != 0) {
                memcpy(work, "GGUF", 4);
                work[4] = 3;
                work[5] = work[6] = work[7] = 0;
            }
        } else { /* a mutated valid file */
            s = (int)(next() % (uint64_t)nseeds);
            n = sizes[s];
            memcpy(work, seeds[s], n);
            mutate(work, &n, cap);
        }
        one(work, n);
    }
    printf("gguf_fuzz: %ld inputs, %ld parsed, %ld mapped\n", iters + 2 + nseeds, accepted, mapped);
    for (s = 0; s < nseeds; s++) free(seeds[s]);
    free(seeds);
    free(sizes);
    free(work);
    return 0;
}
