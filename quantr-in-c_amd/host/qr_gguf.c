/*
 * qr_gguf.c -- GGUF files into the decoder (include/qr_hip.h): the container
 * parser of gguf_init_from_buffer (src/gguf.c:50-177) and the tensor mapping of
 * load_gguf_transformer (src/model.c:253-449), then one device upload per
 * tensor through the weight registry.
 *
 * The parser accepts and refuses exactly what the reference's does: magic
 * "GGUF", at most 65536 key/values and 65536 tensors, strings of at most 1 MiB,
 * arrays of at most 1,000,000 entries, at most 4 dimensions, key/value types
 * with a known size, general.alignment (u32 or u64; 0 or absent means 32), every
 * tensor's start within the buffer.  Tensor data offsets are the aligned end
 * of the header plus the tensor's offset.
 */
#define _POSIX_C_SOURCE 200809L
#include <fcntl.h>
#include <limits.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "qr_hip.h"

enum { KV_U8 = 0, KV_I8, KV_U16, KV_I16, KV_U32, KV_I32, KV_F32, KV_BOOL, KV_STR, KV_ARR,
       KV_U64, KV_I64, KV_F64 };

typedef struct {
    const char* key; /* into the buffer is not NUL-terminated: copied */
    char* key_c;
    uint32_t type;
    const uint8_t* val;  /* scalar value bytes, or the string's bytes */
    uint64_t len;        /* string length, or array length */
    uint32_t arr_type;
} kv_t;

typedef struct {
    char* name;
    uint32_t type, n_dims;
    uint64_t ne[4];
    uint64_t offset;
    const uint8_t* data;
} tensor_t;

struct qr_gguf {
    const uint8_t* base;
    size_t size;
    void* map;  /* non-null when qr_gguf_open mapped the file */
    size_t map_size;
    uint32_t version;
    uint64_t n_tensors, n_kv, alignment, data_offset;
    kv_t* kv;
    tensor_t* t;
    char** str_cache;  /* NUL-terminated copies of string values, per kv */
};

/* qr_last_error()'s message of the calling thread (qr_runtime.hip; local to
 * the library). */
int qrint_set_error(int code, const char* msg);

static int gg_fail(int code, const char* what) {
    char buf[256];
    snprintf(buf, sizeof(buf), "qr_gguf: %s", what);
    return qrint_set_error(code, buf);
}

typedef struct { const uint8_t* p; const uint8_t* end; } rd_t;

static int rd_u32(rd_t* r, uint32_t* v) {
    if ((size_t)(r->end - r->p) < 4) return 0;
    memcpy(v, r->p, 4);
    r->p += 4;
    return 1;
}
static int rd_u64(rd_t* r, uint64_t* v) {
    if ((size_t)(r->end - r->p) < 8) return 0;
    memcpy(v, r->p, 8);
    r->p += 8;
    return 1;
}
/* a string: u64 length + bytes (src/gguf.c:20-32: the length within the
 * buffer and at most 1 MiB) */
static int rd_str(rd_t* r, const uint8_t** s, uint64_t* len) {
    if (!rd_u64(r, len)) return 0;
    if (*len > (uint64_t)(r->end - r->p)) return 0;
    if (*len > 1024 * 1024) return 0;
    *s = r->p;
    r->p += *len;
    return 1;
}
static size_t kv_size(uint32_t t) {
    switch (t) {
        case KV_U8: case KV_I8: case KV_BOOL: return 1;
        case KV_U16: case KV_I16: return 2;
        case KV_U32: case KV_I32: case KV_F32: return 4;
        case KV_U64: case KV_I64: case KV_F64: return 8;
        default: return 0;
    }
}
static char* dup_n(const uint8_t* s, uint64_t n) {
    char* c = (char*)malloc((size_t)n + 1);
    if (!c) return NULL;
    memcpy(c, s, (size_t)n);
    c[n] = '\0';
    return c;
}

int qr_gguf_close(qr_gguf* g) {
    uint64_t i;
    if (!g) return QR_OK;
    if (g->kv) {
        for (i = 0; i < g->n_kv; i++) free(g->kv[i].key_c);
        free(g->kv);
    }
    if (g->str_cache) {
        for (i = 0; i < g->n_kv; i++) free(g->str_cache[i]);
        free(g->str_cache);
    }
    if (g->t) {
        for (i = 0; i < g->n_tensors; i++) free(g->t[i].name);
        free(g->t);
    }
    if (g->map) munmap(g->map, g->map_size);
    free(g);
    return QR_OK;
}

int qr_gguf_parse(const void* data, size_t size, qr_gguf** out) {
    rd_t r;
    uint32_t magic;
    uint64_t i;
    qr_gguf* g;
    size_t hdr, rem;
    if (!out) return QR_ERR_INVALID;
    *out = NULL;
    if (!data) return gg_fail(QR_ERR_INVALID, "null buffer");
    r.p = (const uint8_t*)data;
    r.end = r.p + size;
    if (!rd_u32(&r, &magic) || magic != 0x46554747u) return gg_fail(QR_ERR_INVALID, "not a GGUF buffer");
    g = (qr_gguf*)calloc(1, sizeof(qr_gguf));
    if (!g) return QR_ERR_NOMEM;
    g->base = (const uint8_t*)data;
    g->size = size;
    if (!rd_u32(&r, &g->version) || !rd_u64(&r, &g->n_tensors) || !rd_u64(&r, &g->n_kv)) goto bad;
    if (g->n_kv > 65536 || g->n_tensors > 65536) goto bad;
    g->kv = (kv_t*)calloc(g->n_kv ? g->n_kv : 1, sizeof(kv_t));
    g->str_cache = (char**)calloc(g->n_kv ? g->n_kv : 1, sizeof(char*));
    if (!g->kv || !g->str_cache) goto nomem;
    for (i = 0; i < g->n_kv; i++) {
        kv_t* k = &g->kv[i];
        const uint8_t* s;
        uint64_t n;
        if (!rd_str(&r, &s, &n)) goto bad;
        k->key_c = dup_n(s, n);
        if (!k->key_c) goto nomem;
        if (!rd_u32(&r, &k->type)) goto bad;
        if (k->type == KV_STR) {
            if (!rd_str(&r, &k->val, &k->len)) goto bad;
        } else if (k->type == KV_ARR) {
            uint64_t j;
            if (!rd_u32(&r, &k->arr_type) || !rd_u64(&r, &k->len)) goto bad;
            if (k->len > 1000000) goto bad;
            k->val = r.p;
            if (k->arr_type == KV_STR) {
                for (j = 0; j < k->len; j++)
                    if (!rd_str(&r, &s, &n)) goto bad;
            } else {
                const size_t el = kv_size(k->arr_type);
                if (el == 0) goto bad;
                if (k->len > (uint64_t)(r.end - r.p) / el) goto bad;
                r.p += (size_t)k->len * el;
            }
        } else {
            const size_t el = kv_size(k->type);
            if (el == 0 || (size_t)(r.end - r.p) < el) goto bad;
            k->val = r.p;
            r.p += el;
        }
    }
    g->alignment = 32;
    for (i = 0; i < g->n_kv; i++) {
        if (strcmp(g->kv[i].key_c, "general.alignment") == 0) {
            if (g->kv[i].type == KV_U32) {
                uint32_t a;
                memcpy(&a, g->kv[i].val, 4);
                g->alignment = a;
            } else if (g->kv[i].type == KV_U64) {
                memcpy(&g->alignment, g->kv[i].val, 8);
            }
        }
    }
    if (g->alignment == 0) g->alignment = 32;
    g->t = (tensor_t*)calloc(g->n_tensors ? g->n_tensors : 1, sizeof(tensor_t));
    if (!g->t) goto nomem;
    for (i = 0; i < g->n_tensors; i++) {
        tensor_t* t = &g->t[i];
        const uint8_t* s;
        uint64_t n;
        uint32_t j;
        if (!rd_str(&r, &s, &n)) goto bad;
        t->name = dup_n(s, n);
        if (!t->name) goto nomem;
        if (!rd_u32(&r, &t->n_dims) || t->n_dims > 4) goto bad;
        for (j = 0; j < t->n_dims; j++)
            if (!rd_u64(&r, &t->ne[j])) goto bad;
        if (!rd_u32(&r, &t->type) || !rd_u64(&r, &t->offset)) goto bad;
    }
    hdr = (size_t)(r.p - g->base);
    rem = hdr % g->alignment;
    g->data_offset = hdr + (rem ? g->alignment - rem : 0);
    for (i = 0; i < g->n_tensors; i++) {
        const uint64_t start = g->data_offset + g->t[i].offset;
        if (start > size || start < g->data_offset) goto bad;
        g->t[i].data = g->base + start;
    }
    *out = g;
    return QR_OK;
bad:
    qr_gguf_close(g);
    return gg_fail(QR_ERR_INVALID, "malformed GGUF");
nomem:
    qr_gguf_close(g);
    return QR_ERR_NOMEM;
}

int qr_gguf_open(const char* path, qr_gguf** out) {
    int fd, rc;
    struct stat st;
    void* m;
    if (!out || !path) return QR_ERR_INVALID;
    *out = NULL;
    fd = open(path, O_RDONLY);
    if (fd < 0) return gg_fail(QR_ERR_INVALID, "cannot open the file");
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        close(fd);
        return gg_fail(QR_ERR_INVALID, "cannot stat the file");
    }
    m = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return gg_fail(QR_ERR_NOMEM, "mmap failed");
    rc = qr_gguf_parse(m, (size_t)st.st_size, out);
    if (rc != QR_OK) {
        munmap(m, (size_t)st.st_size);
        return rc;
    }
    (*out)->map = m;
    (*out)->map_size = (size_t)st.st_size;
    return QR_OK;
}

int qr_gguf_info(const qr_gguf* g, uint32_t* version, uint64_t* n_tensors, uint64_t* n_kv,
                 uint64_t* alignment, uint64_t* data_offset) {
    if (!g) return QR_ERR_INVALID;
    if (version) *version = g->version;
    if (n_tensors) *n_tensors = g->n_tensors;
    if (n_kv) *n_kv = g->n_kv;
    if (alignment) *alignment = g->alignment;
    if (data_offset) *data_offset = g->data_offset;
    return QR_OK;
}

int qr_gguf_tensor(const qr_gguf* g, uint64_t i, const char** name, uint32_t* type,
                   uint32_t* n_dims, uint64_t* ne, const void** data) {
    uint32_t j;
    if (!g || i >= g->n_tensors) return QR_ERR_INVALID;
    if (name) *name = g->t[i].name;
    if (type) *type = g->t[i].type;
    if (n_dims) *n_dims = g->t[i].n_dims;
    if (ne)
        for (j = 0; j < 4; j++) ne[j] = g->t[i].ne[j];
    if (data) *data = g->t[i].data;
    return QR_OK;
}

int64_t qr_gguf_find(const qr_gguf* g, const char* name) {
    uint64_t i;
    if (!g || !name) return -1;
    for (i = 0; i < g->n_tensors; i++)
        if (strcmp(g->t[i].name, name) == 0) return (int64_t)i;
    return -1;
}

/* gguf_get_val_* (src/gguf.c:211-269): the first key of that name holding the
 * requested type; arrays report their length. */
static const kv_t* kv_find(const qr_gguf* g, const char* key, uint32_t type) {
    uint64_t i;
    if (!g || !key) return NULL;
    for (i = 0; i < g->n_kv; i++)
        if (strcmp(g->kv[i].key_c, key) == 0 && g->kv[i].type == type) return &g->kv[i];
    return NULL;
}

uint32_t qr_gguf_get_u32(const qr_gguf* g, const char* key, uint32_t def) {
    const kv_t* k = kv_find(g, key, KV_U32);
    uint32_t v;
    if (!k) return def;
    memcpy(&v, k->val, 4);
    return v;
}

float qr_gguf_get_f32(const qr_gguf* g, const char* key, float def) {
    const kv_t* k = kv_find(g, key, KV_F32);
    float v;
    if (!k) return def;
    memcpy(&v, k->val, 4);
    return v;
}

const char* qr_gguf_get_str(const qr_gguf* g, const char* key) {
    const kv_t* k = kv_find(g, key, KV_STR);
    size_t i;
    if (!k) return NULL;
    i = (size_t)(k - g->kv);
    if (!g->str_cache[i]) g->str_cache[i] = dup_n(k->val, k->len);
    return g->str_cache[i];
}

int64_t qr_gguf_get_arr_len(const qr_gguf* g, const char* key) {
    const kv_t* k = kv_find(g, key, KV_ARR);
    return k ? (int64_t)k->len : -1;
}

/* ---- the decoder model (load_gguf_transformer, src/model.c:253-449) ------ */

#define QR_GGUF_MAX_WIDTH (1 << 20) /* dim, ffn width, q and kv widths */
#define QR_GGUF_MAX_COUNT 4096      /* layers, experts */
#define QR_GGUF_MAX_VOCAB (1 << 24)

static int known_wtype(uint32_t t) { return t == 0 || t == 8 || t == 12 || t == 13 || t == 14; }

/* tensor i's bytes when it is [ne0][ne1] (ne2 = experts, or 1) of a type */
static int check_tensor(const qr_gguf* g, int64_t i, uint64_t ne0, uint64_t ne1, uint64_t ne2,
                        int need_f32, size_t* bytes) {
    const tensor_t* t;
    size_t rb, off;
    if (i < 0) return 0;
    t = &g->t[i];
    if (!known_wtype(t->type) || (need_f32 && t->type != 0)) return 0;
    if (t->ne[0] != ne0 || (t->n_dims > 1 ? t->ne[1] : 1) != ne1 ||
        (t->n_dims > 2 ? t->ne[2] : 1) != ne2)
        return 0;
    if (ne0 > (uint64_t)INT_MAX || ne1 > (uint64_t)SIZE_MAX || ne2 > (uint64_t)SIZE_MAX) return 0;
    rb = qr_row_bytes(t->type, (int)ne0);
    if (!rb && ne0) return 0;
    /* the product and the end offset are checked before they are formed: a
     * crafted header must not wrap them past the bounds check */
    if (ne1 && rb > SIZE_MAX / (size_t)ne1) return 0;
    *bytes = rb * (size_t)ne1;
    if (ne2 && *bytes > SIZE_MAX / (size_t)ne2) return 0;
    *bytes *= (size_t)ne2;
    off = (size_t)(t->data - g->base);
    if (off > g->size || *bytes > g->size - off) return 0;
    return 1;
}

int qr_gguf_model_host(const qr_gguf* g, int seq_len, qr_model* m, qr_layer* layers,
                       int max_layers) {
    char arch[64] = "qwen2", key[160], name[160];
    const char* a;
    int l, dim, H, KVH, hd, L, E, K, hid, V, fill;
    int64_t it;
    size_t b;
    qr_layer scratch_layer;
    if (!g || !m) return QR_ERR_INVALID;
    memset(m, 0, sizeof(*m));
    a = qr_gguf_get_str(g, "general.architecture");
    if (a) {
        strncpy(arch, a, sizeof(arch) - 1);
        arch[sizeof(arch) - 1] = '\0';
    }
#define U32(suffix, def) (snprintf(key, sizeof(key), "%s.%s", arch, suffix), qr_gguf_get_u32(g, key, def))
    dim = (int)U32("embedding_length", 0);
    L = (int)U32("block_count", 0);
    H = (int)U32("attention.head_count", 0);
    KVH = (int)U32("attention.head_count_kv", (uint32_t)H);
    E = (int)U32("expert_count", 0);
    K = (int)U32("expert_used_count", 0);
    hid = (int)U32("expert_feed_forward_length", 0);
    if (!(E > 0 && hid > 0)) hid = (int)U32("feed_forward_length", 0);
    /* head_dim: the reference always takes dim / n_heads (src/runtime.c:102);
     * a file that states attention.key_length gets that */
    hd = H > 0 ? (int)U32("attention.key_length", (uint32_t)(dim / H)) : 0;
#undef U32
    snprintf(key, sizeof(key), "%s.rope.freq_base", arch);
    m->rope_base = qr_gguf_get_f32(g, key, 1000000.0f);
    /* expert_count 0 (or absent) is a dense model (src/runtime.c:270-284) */
    if (E < 0 || (E > 0 && K <= 0)) return gg_fail(QR_ERR_UNSUPPORTED, "expert counts");
    if (E == 0) K = 0;
    if (dim <= 0 || L <= 0 || H <= 0 || KVH <= 0 || hd <= 0 || hid <= 0)
        return gg_fail(QR_ERR_UNSUPPORTED, "not a model this decoder serves");
    /* sizes the later products (rows x row bytes x experts, in int and size_t)
     * stay far from overflow with; every real model is well inside them */
    if (dim > QR_GGUF_MAX_WIDTH || hid > QR_GGUF_MAX_WIDTH ||
        (int64_t)H * hd > QR_GGUF_MAX_WIDTH || (int64_t)KVH * hd > QR_GGUF_MAX_WIDTH ||
        L > QR_GGUF_MAX_COUNT || E > QR_GGUF_MAX_COUNT || K > E)
        return gg_fail(QR_ERR_UNSUPPORTED, "model sizes beyond the loader's limits");
    it = qr_gguf_find(g, "token_embd.weight");
    if (it < 0) return gg_fail(QR_ERR_INVALID, "no token_embd.weight");
    /* vocab: the tokenizer's token count (src/model.c:306-312), else the
     * embedding's rows */
    {
        int64_t nv = qr_gguf_get_arr_len(g, "tokenizer.ggml.tokens");
        if (nv <= 0) nv = (int64_t)g->t[it].ne[1];
        if (nv <= 0 || nv > QR_GGUF_MAX_VOCAB)
            return gg_fail(QR_ERR_UNSUPPORTED, "vocabulary size beyond the loader's limits");
        V = (int)nv;
    }
    if (!check_tensor(g, it, (uint64_t)dim, (uint64_t)V, 1, 0, &b))
        return gg_fail(QR_ERR_INVALID, "token_embd.weight shape or type");
    m->dim = dim;
    m->n_heads = H;
    m->n_kv_heads = KVH;
    m->head_dim = hd;
    m->n_layers = L;
    m->vocab = V;
    m->seq_len = seq_len;
    m->tok_embd = g->t[it].data;
    m->tok_type = g->t[it].type;
    it = qr_gguf_find(g, "output_norm.weight");
    if (!check_tensor(g, it, (uint64_t)dim, 1, 1, 1, &b))
        return gg_fail(QR_ERR_INVALID, "output_norm.weight");
    m->rms_final = (const float*)g->t[it].data;
    it = qr_gguf_find(g, "output.weight");
    if (it >= 0) {
        if (!check_tensor(g, it, (uint64_t)dim, (uint64_t)V, 1, 0, &b))
            return gg_fail(QR_ERR_INVALID, "output.weight shape or type");
        m->wcls = g->t[it].data;
        m->wcls_type = g->t[it].type;
    } else { /* tied embeddings (src/model.c:323-330) */
        m->wcls = m->tok_embd;
        m->wcls_type = m->tok_type;
    }
    /* every layer is checked on each call; the caller's array is filled only
     * when it holds all L layers (a shorter one gets the count) */
    fill = layers != NULL && max_layers >= L;
    for (l = 0; l < L; l++) {
        qr_layer* y = fill ? &layers[l] : &scratch_layer;
        const char* nm[4] = {"attn_q", "attn_k", "attn_v", "attn_output"};
        const void** wp[4];
        uint32_t* tp[4];
        const uint64_t rows[4] = {(uint64_t)H * hd, (uint64_t)KVH * hd, (uint64_t)KVH * hd,
                                  (uint64_t)dim};
        const uint64_t cols[4] = {(uint64_t)dim, (uint64_t)dim, (uint64_t)dim,
                                  (uint64_t)H * hd};
        int j;
        memset(y, 0, sizeof(*y));
        wp[0] = &y->wq; wp[1] = &y->wk; wp[2] = &y->wv; wp[3] = &y->wo;
        tp[0] = &y->wq_type; tp[1] = &y->wk_type; tp[2] = &y->wv_type; tp[3] = &y->wo_type;
        snprintf(name, sizeof(name), "blk.%d.attn_norm.weight", l);
        it = qr_gguf_find(g, name);
        if (!check_tensor(g, it, (uint64_t)dim, 1, 1, 1, &b)) return gg_fail(QR_ERR_INVALID, name);
        y->rms_att = (const float*)g->t[it].data;
        snprintf(name, sizeof(name), "blk.%d.ffn_norm.weight", l);
        it = qr_gguf_find(g, name);
        if (!check_tensor(g, it, (uint64_t)dim, 1, 1, 1, &b)) return gg_fail(QR_ERR_INVALID, name);
        y->rms_ffn = (const float*)g->t[it].data;
        for (j = 0; j < 4; j++) {
            snprintf(name, sizeof(name), "blk.%d.%s.weight", l, nm[j]);
            it = qr_gguf_find(g, name);
            if (!check_tensor(g, it, cols[j], rows[j], 1, 0, &b)) return gg_fail(QR_ERR_INVALID, name);
            *wp[j] = g->t[it].data;
            *tp[j] = g->t[it].type;
        }
        y->moe.dim = dim;
        y->moe.hidden = hid;
        y->moe.n_experts = E;
        y->moe.n_used = K;
        if (E == 0) {
            /* the dense FFN: w1 = ffn_up (the SiLU slot), w2 = ffn_down,
             * w3 = ffn_gate (src/model.c:434-446), in the expert fields */
            const char* kinds[3] = {"ffn_up", "ffn_down", "ffn_gate"};
            const void** fp[3];
            uint32_t* ft[3];
            fp[0] = &y->moe.up; fp[1] = &y->moe.down; fp[2] = &y->moe.gate;
            ft[0] = &y->moe.up_type; ft[1] = &y->moe.down_type; ft[2] = &y->moe.gate_type;
            for (j = 0; j < 3; j++) {
                const int down = j == 1;
                snprintf(name, sizeof(name), "blk.%d.%s.weight", l, kinds[j]);
                it = qr_gguf_find(g, name);
                if (!check_tensor(g, it, (uint64_t)(down ? hid : dim), (uint64_t)(down ? dim : hid),
                                  1, 0, &b))
                    return gg_fail(QR_ERR_INVALID, name);
                *fp[j] = g->t[it].data;
                *ft[j] = g->t[it].type;
            }
            continue;
        }
        snprintf(name, sizeof(name), "blk.%d.ffn_gate_inp.weight", l);
        it = qr_gguf_find(g, name);
        if (!check_tensor(g, it, (uint64_t)dim, (uint64_t)E, 1, 1, &b)) return gg_fail(QR_ERR_INVALID, name);
        y->moe.router = (const float*)g->t[it].data;
        {
            /* expert_w1 = ffn_up_exps (the SiLU slot), expert_w3 = ffn_gate_exps,
             * expert_w2 = ffn_down_exps (src/model.c:404-419); one 3-D tensor
             * each, or per-expert tensors (src/model.c:421-433), whose base is
             * expert 0's here (qr_gguf_load gathers them) */
            int64_t iu, idn, ig;
            snprintf(name, sizeof(name), "blk.%d.ffn_up_exps.weight", l);
            iu = qr_gguf_find(g, name);
            snprintf(name, sizeof(name), "blk.%d.ffn_down_exps.weight", l);
            idn = qr_gguf_find(g, name);
            snprintf(name, sizeof(name), "blk.%d.ffn_gate_exps.weight", l);
            ig = qr_gguf_find(g, name);
            if (iu >= 0 && idn >= 0 && ig >= 0) {
                if (!check_tensor(g, iu, (uint64_t)dim, (uint64_t)hid, (uint64_t)E, 0, &b) ||
                    !check_tensor(g, ig, (uint64_t)dim, (uint64_t)hid, (uint64_t)E, 0, &b) ||
                    !check_tensor(g, idn, (uint64_t)hid, (uint64_t)dim, (uint64_t)E, 0, &b))
                    return gg_fail(QR_ERR_INVALID, "expert tensor shape or type");
            } else {
                snprintf(name, sizeof(name), "blk.%d.ffn_up_exps.0.weight", l);
                iu = qr_gguf_find(g, name);
                snprintf(name, sizeof(name), "blk.%d.ffn_down_exps.0.weight", l);
                idn = qr_gguf_find(g, name);
                snprintf(name, sizeof(name), "blk.%d.ffn_gate_exps.0.weight", l);
                ig = qr_gguf_find(g, name);
                if (!check_tensor(g, iu, (uint64_t)dim, (uint64_t)hid, 1, 0, &b) ||
                    !check_tensor(g, ig, (uint64_t)dim, (uint64_t)hid, 1, 0, &b) ||
                    !check_tensor(g, idn, (uint64_t)hid, (uint64_t)dim, 1, 0, &b))
                    return gg_fail(QR_ERR_INVALID, "expert tensors missing");
            }
            y->moe.up = g->t[iu].data;
            y->moe.gate = g->t[ig].data;
            y->moe.down = g->t[idn].data;
            y->moe.up_type = g->t[iu].type;
            y->moe.gate_type = g->t[ig].type;
            y->moe.down_type = g->t[idn].type;
        }
    }
    m->layers = fill ? layers : NULL;
    return L;
}

int qr_gguf_expert_host(const qr_gguf* g, int layer, int e, const void** up, const void** down,
                        const void** gate) {
    char name[160];
    const char* kinds[3] = {"ffn_up_exps", "ffn_down_exps", "ffn_gate_exps"};
    const void** outs[3];
    int j;
    if (!g || layer < 0 || e < 0) return QR_ERR_INVALID;
    outs[0] = up; outs[1] = down; outs[2] = gate;
    for (j = 0; j < 3; j++) {
        int64_t i;
        snprintf(name, sizeof(name), "blk.%d.%s.weight", layer, kinds[j]);
        i = qr_gguf_find(g, name);
        if (i >= 0) {
            const tensor_t* t = &g->t[i];
            const size_t slice = qr_row_bytes(t->type, (int)t->ne[0]) * (size_t)t->ne[1];
            if ((uint64_t)e >= (t->n_dims > 2 ? t->ne[2] : 1)) return QR_ERR_INVALID;
            if (outs[j]) *outs[j] = t->data + (size_t)e * slice;
        } else {
            /* expert e's own tensor: the type and shape of expert 0's (which
             * qr_gguf_model_host checked) and inside the file, as the
             * gather reads expert 0's byte count from it */
            int64_t i0;
            const tensor_t *t, *t0;
            size_t bytes;
            snprintf(name, sizeof(name), "blk.%d.%s.0.weight", layer, kinds[j]);
            i0 = qr_gguf_find(g, name);
            snprintf(name, sizeof(name), "blk.%d.%s.%d.weight", layer, kinds[j], e);
            i = qr_gguf_find(g, name);
            if (i < 0 || i0 < 0) return QR_ERR_INVALID;
            t = &g->t[i];
            t0 = &g->t[i0];
            const uint64_t rows = t->n_dims > 1 ? t->ne[1] : 1;
            if (t->type != t0->type || t->ne[0] != t0->ne[0] ||
                rows != (t0->n_dims > 1 ? t0->ne[1] : 1) || t->n_dims > 2 ||
                t->ne[0] > (uint64_t)INT_MAX || rows > (uint64_t)SIZE_MAX)
                return QR_ERR_INVALID;
            bytes = qr_row_bytes(t->type, (int)t->ne[0]);
            if (rows && bytes > SIZE_MAX / (size_t)rows) return QR_ERR_INVALID;
            bytes *= (size_t)rows;
            if ((size_t)(t->data - g->base) > g->size ||
                bytes > g->size - (size_t)(t->data - g->base))
                return QR_ERR_INVALID;
            if (outs[j]) *outs[j] = t->data;
        }
    }
    return QR_OK;
}

/* ---- upload ------------------------------------------------------------- */

struct qr_gguf_model {
    qr_ctx* ctx;
    qr_model model;
    qr_layer* layers;
    void* slab;  /* every tensor of the model, one device allocation */
    size_t slab_bytes;
};

/* One host range to copy into the slab; `fix` (may be NULL for the second and
 * later parts of a gathered tensor) receives the device address. */
typedef struct {
    const void* src;
    size_t bytes, off;
    const void** fix;
    uint32_t* tile_type;  /* non-NULL: stored in the tiled layout, this type gets QR_TILED */
    int rows, cols;
} copy_op;

typedef struct {
    copy_op* op;
    int n, cap;
    size_t end;
} copy_plan;

#define QR_SLAB_ALIGN 256

static int plan_add(copy_plan* p, const void* src, size_t bytes, const void** fix, int new_tensor) {
    if (p->n == p->cap) {
        int cap = p->cap ? 2 * p->cap : 256;
        copy_op* o = (copy_op*)realloc(p->op, (size_t)cap * sizeof(copy_op));
        if (!o) return QR_ERR_NOMEM;
        p->op = o;
        p->cap = cap;
    }
    /* a tensor starts on a 256-byte boundary; the parts of a gathered
     * tensor follow one another with no gap */
    if (new_tensor) p->end = (p->end + QR_SLAB_ALIGN - 1) & ~(size_t)(QR_SLAB_ALIGN - 1);
    p->op[p->n].src = src;
    p->op[p->n].bytes = bytes;
    p->op[p->n].off = p->end;
    p->op[p->n].fix = fix;
    p->op[p->n].tile_type = NULL;
    p->op[p->n].rows = p->op[p->n].cols = 0;
    p->n++;
    p->end += bytes;
    return QR_OK;
}

int qr_gguf_model_free(qr_gguf_model* gm) {
    if (!gm) return QR_OK;
    if (gm->slab) (void)qr_free(gm->ctx, gm->slab);
    free(gm->layers);
    free(gm);
    return QR_OK;
}

const qr_model* qr_gguf_model_get(const qr_gguf_model* gm) { return gm ? &gm->model : NULL; }

/* Q4_K / Q5_K matrices whose rows are whole super-blocks (at most 64) are
 * stored tiled (qr_weights_tile): the decoder's GEMV streams them faster. */
static int tileable(uint32_t type, int cols) {
    return (type == QR_TYPE_Q4_K || type == QR_TYPE_Q5_K) && cols > 0 && cols % 256 == 0 &&
           cols / 256 <= 64;
}

/* The lm_head also in Q6_K, when rows x (cols / 256) is a multiple of 8 (the
 * Q6_K tiled layout's condition): the decode step reads it with the tiled
 * GEMV (the projections stay row-major in Q6_K, which the prompt's row
 * products read with int8 MFMA). */
static int tileable_out(uint32_t type, int rows, int cols) {
    return tileable(type, cols) ||
           (type == QR_TYPE_Q6_K && rows > 0 && cols > 0 && cols % 256 == 0 && cols / 256 <= 64 &&
            ((long)rows * (cols / 256)) % 8 == 0);
}

static void plan_tile_if(copy_plan* p, uint32_t* type, int rows, int cols, int ok) {
    copy_op* o = &p->op[p->n - 1];
    if (!ok) return;
    o->tile_type = type;
    o->rows = rows;
    o->cols = cols;
}

static void plan_tile(copy_plan* p, uint32_t* type, int rows, int cols) {
    plan_tile_if(p, type, rows, cols, tileable(*type, cols));
}

/* The copy plan of every tensor the decoder reads: the tied output shares
 * the embedding; per-expert tensors are gathered into one range per kind
 * (expert e at e * slice), as a 3-D tensor is laid out. */
static int plan_model(const qr_gguf* g, qr_gguf_model* gm, copy_plan* p) {
    qr_model* m = &gm->model;
    const int tied = m->wcls == m->tok_embd;
    int l, rc;
#define ADD(src, bytes, fix) \
    do { if ((rc = plan_add(p, (src), (bytes), (const void**)(fix), 1)) != QR_OK) return rc; } while (0)
    ADD(m->tok_embd, qr_row_bytes(m->tok_type, m->dim) * (size_t)m->vocab, &m->tok_embd);
    ADD(m->rms_final, (size_t)m->dim * 4, &m->rms_final);
    if (!tied) {
        ADD(m->wcls, qr_row_bytes(m->wcls_type, m->dim) * (size_t)m->vocab, &m->wcls);
        plan_tile_if(p, &m->wcls_type, m->vocab, m->dim, tileable_out(m->wcls_type, m->vocab, m->dim));
    }
    for (l = 0; l < m->n_layers; l++) {
        qr_layer* y = &gm->layers[l];
        qr_moe_layer* e = &y->moe;
        const int qd = m->n_heads * m->head_dim, kvd = m->n_kv_heads * m->head_dim;
        const size_t su = qr_row_bytes(e->up_type, m->dim) * (size_t)e->hidden;
        const size_t sd = qr_row_bytes(e->down_type, e->hidden) * (size_t)m->dim;
        const void *u1 = NULL, *d1 = NULL, *g1 = NULL;
        ADD(y->rms_att, (size_t)m->dim * 4, &y->rms_att);
        ADD(y->rms_ffn, (size_t)m->dim * 4, &y->rms_ffn);
        ADD(y->wq, qr_row_bytes(y->wq_type, m->dim) * (size_t)qd, &y->wq);
        plan_tile(p, &y->wq_type, qd, m->dim);
        ADD(y->wk, qr_row_bytes(y->wk_type, m->dim) * (size_t)kvd, &y->wk);
        plan_tile(p, &y->wk_type, kvd, m->dim);
        ADD(y->wv, qr_row_bytes(y->wv_type, m->dim) * (size_t)kvd, &y->wv);
        plan_tile(p, &y->wv_type, kvd, m->dim);
        ADD(y->wo, qr_row_bytes(y->wo_type, qd) * (size_t)m->dim, &y->wo);
        plan_tile(p, &y->wo_type, m->dim, qd);
        if (e->n_experts == 0) { /* a dense FFN: three matrices, tiled where they can be */
            ADD(e->up, su, &e->up);
            plan_tile(p, &e->up_type, e->hidden, m->dim);
            ADD(e->gate, qr_row_bytes(e->gate_type, m->dim) * (size_t)e->hidden, &e->gate);
            plan_tile(p, &e->gate_type, e->hidden, m->dim);
            ADD(e->down, sd, &e->down);
            plan_tile(p, &e->down_type, m->dim, e->hidden);
            continue;
        }
        ADD(e->router, (size_t)e->n_experts * (size_t)m->dim * 4, &e->router);
        if (e->n_experts > 1 && qr_gguf_expert_host(g, l, 1, &u1, &d1, &g1) != QR_OK)
            return QR_ERR_INVALID;
        if (e->n_experts == 1 || ((const char*)u1 == (const char*)e->up + su &&
                                  (const char*)d1 == (const char*)e->down + sd &&
                                  (const char*)g1 == (const char*)e->gate + su)) {
            ADD(e->up, su * (size_t)e->n_experts, &e->up);
            ADD(e->gate, su * (size_t)e->n_experts, &e->gate);
            ADD(e->down, sd * (size_t)e->n_experts, &e->down);
        } else {
            const void** fix[3];
            const size_t sz[3] = {su, su, sd};
            int k, x;
            fix[0] = &e->up; fix[1] = &e->gate; fix[2] = &e->down;
            for (k = 0; k < 3; k++) {
                for (x = 0; x < e->n_experts; x++) {
                    const void* part[3] = {NULL, NULL, NULL};
                    if (qr_gguf_expert_host(g, l, x, &part[0], &part[2], &part[1]) != QR_OK)
                        return QR_ERR_INVALID;
                    rc = plan_add(p, part[k], sz[k], x == 0 ? fix[k] : NULL, x == 0);
                    if (rc != QR_OK) return rc;
                }
            }
        }
    }
#undef ADD
    return QR_OK;
}

/* The file's K-quant tensors read in llama.cpp's layouts: their types carry
 * QR_GGML (which no tiling plan accepts). */
static void mark_ggml(uint32_t* type) {
    if (*type == QR_TYPE_Q4_K || *type == QR_TYPE_Q5_K || *type == QR_TYPE_Q6_K) *type |= QR_GGML;
}

static void mark_ggml_model(qr_gguf_model* gm) {
    qr_model* m = &gm->model;
    int l;
    mark_ggml(&m->tok_type);
    mark_ggml(&m->wcls_type);
    for (l = 0; l < m->n_layers; l++) {
        qr_layer* y = &gm->layers[l];
        mark_ggml(&y->wq_type);
        mark_ggml(&y->wk_type);
        mark_ggml(&y->wv_type);
        mark_ggml(&y->wo_type);
        mark_ggml(&y->moe.up_type);
        mark_ggml(&y->moe.gate_type);
        mark_ggml(&y->moe.down_type);
        mark_ggml(&y->moe.sh_up_type);
        mark_ggml(&y->moe.sh_gate_type);
        mark_ggml(&y->moe.sh_down_type);
    }
}

int qr_gguf_load(qr_ctx* ctx, const qr_gguf* g, int seq_len, qr_gguf_model** out) {
    return qr_gguf_load_ex(ctx, g, seq_len, 0, out);
}

int qr_gguf_load_ex(qr_ctx* ctx, const qr_gguf* g, int seq_len, uint32_t flags,
                    qr_gguf_model** out) {
    qr_gguf_model* gm;
    copy_plan plan = {NULL, 0, 0, 0};
    int L, i, rc, tied;
    void* stage = NULL;
    size_t stage_bytes = 0;
    if (!out) return QR_ERR_INVALID;
    *out = NULL;
    if (!ctx || !g) return QR_ERR_INVALID;
    if (flags & ~QR_GGUF_GGML_KQUANTS) return gg_fail(QR_ERR_INVALID, "qr_gguf_load: unknown flags");
    gm = (qr_gguf_model*)calloc(1, sizeof(*gm));
    if (!gm) return QR_ERR_NOMEM;
    gm->ctx = ctx;
    L = qr_gguf_model_host(g, seq_len, &gm->model, NULL, 0);
    if (L <= 0) {
        free(gm);
        return L < 0 ? L : QR_ERR_INVALID;
    }
    gm->layers = (qr_layer*)calloc((size_t)L, sizeof(qr_layer));
    if (!gm->layers) {
        free(gm);
        return QR_ERR_NOMEM;
    }
    rc = qr_gguf_model_host(g, seq_len, &gm->model, gm->layers, L);
    if (rc != L) goto fail;
    if (flags & QR_GGUF_GGML_KQUANTS) mark_ggml_model(gm);
    tied = gm->model.wcls == gm->model.tok_embd;
    rc = plan_model(g, gm, &plan);
    if (rc != QR_OK) {
        if (rc == QR_ERR_NOMEM) gg_fail(rc, "qr_gguf_load: out of host memory");
        goto fail;
    }
    gm->slab_bytes = plan.end;
    rc = qr_malloc(ctx, plan.end, &gm->slab);
    if (rc != QR_OK) goto fail;
    for (i = 0; i < plan.n; i++) /* the staging buffer of the tiled tensors */
        if (plan.op[i].tile_type && plan.op[i].bytes > stage_bytes) stage_bytes = plan.op[i].bytes;
    if (stage_bytes) {
        rc = qr_malloc(ctx, stage_bytes, &stage);
        if (rc != QR_OK) goto fail;
    }
    for (i = 0; i < plan.n; i++) {
        char* dst = (char*)gm->slab + plan.op[i].off;
        const copy_op* o = &plan.op[i];
        if (o->tile_type) {
            rc = qr_memcpy_h2d(ctx, stage, o->src, o->bytes);
            if (rc == QR_OK) rc = qr_weights_tile(ctx, *o->tile_type, stage, dst, o->rows, o->cols);
            if (rc == QR_OK) rc = qr_sync(ctx);  /* the stage is reused by the next tensor */
            if (rc != QR_OK) goto fail;
            *o->tile_type |= QR_TILED;
        } else {
            rc = qr_memcpy_h2d(ctx, dst, o->src, o->bytes);
            if (rc != QR_OK) goto fail;
        }
        if (o->fix) *o->fix = dst;
    }
    if (stage) {
        (void)qr_free(ctx, stage);
        stage = NULL;
    }
    if (tied) gm->model.wcls = gm->model.tok_embd;  /* the embedding's device copy */
    free(plan.op);
    *out = gm;
    return QR_OK;
fail:
    if (stage) (void)qr_free(ctx, stage);
    free(plan.op);
    qr_gguf_model_free(gm);
    return rc;
}
