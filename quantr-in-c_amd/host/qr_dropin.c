/*
 * qr_dropin.c -- C99 host layer with quantr-in-c's entry-point signatures
 * (declared in include/qr_dropin.h) over the device C ABI of libqr_hip.so.
 *
 * One process-wide context on the selected GPU, device staging buffers that
 * grow on demand, and the weight registry keyed by host address.  Every entry
 * is synchronous: host inputs are copied in, the kernels run, outputs are
 * copied back before returning.
 */
#define _POSIX_C_SOURCE 200809L
#include "qr_dropin.h"

#include <pthread.h>
#include <stdio.h>
#include <string.h>

#include "qr_hip.h"

static pthread_mutex_t g_mu = PTHREAD_MUTEX_INITIALIZER;
static qr_ctx* g_ctx = NULL;
static int g_order = QR_ORDER_AVX2;
static int g_init_rc = 1; /* 1: not tried yet */
static void* g_buf[4] = {NULL, NULL, NULL, NULL};
static size_t g_cap[4] = {0, 0, 0, 0};

static void report(const char* who, int rc) {
    fprintf(stderr, "[qr_dropin] %s failed (%d): %s\n", who, rc, qr_last_error());
}

static int init_locked(int device, int order) {
    int rc;
    if (g_ctx) return 0;
    rc = qr_ctx_create(device, &g_ctx);
    if (rc != QR_OK) {
        g_ctx = NULL;
        return rc;
    }
    g_order = order;
    return 0;
}

/* Lazily initialise device 0 with the default order; 0 when usable. */
static int ensure(void) {
    int rc;
    pthread_mutex_lock(&g_mu);
    if (g_init_rc == 1) g_init_rc = init_locked(0, QR_ORDER_AVX2);
    rc = g_init_rc;
    pthread_mutex_unlock(&g_mu);
    return rc;
}

/* Device staging buffer `slot` of at least `bytes`. */
static void* staging(int slot, size_t bytes) {
    if (bytes > g_cap[slot]) {
        size_t want = bytes < 4096 ? 4096 : bytes;
        if (g_buf[slot]) qr_free(g_ctx, g_buf[slot]);
        g_buf[slot] = NULL;
        g_cap[slot] = 0;
        if (qr_malloc(g_ctx, want, &g_buf[slot]) != QR_OK) return NULL;
        g_cap[slot] = want;
    }
    return g_buf[slot];
}

int qr_dropin_init(int device, int router_order) {
    int rc;
    if (router_order < QR_ORDER_SEQ || router_order > QR_ORDER_AVX512) return QR_ERR_INVALID;
    pthread_mutex_lock(&g_mu);
    if (g_ctx) {
        g_order = router_order;
        rc = 0;
    } else {
        rc = init_locked(device, router_order);
        g_init_rc = rc;
    }
    pthread_mutex_unlock(&g_mu);
    return rc;
}

void qr_dropin_shutdown(void) {
    int i;
    pthread_mutex_lock(&g_mu);
    if (g_ctx) {
        for (i = 0; i < 4; i++) {
            if (g_buf[i]) qr_free(g_ctx, g_buf[i]);
            g_buf[i] = NULL;
            g_cap[i] = 0;
        }
        qr_ctx_destroy(g_ctx);
    }
    g_ctx = NULL;
    g_init_rc = 1;
    pthread_mutex_unlock(&g_mu);
}

int qr_gpu_available(void) { return ensure() == 0 ? 3 : 0; }

static int type_known(uint32_t t) {
    return t == QR_TYPE_F32 || t == QR_TYPE_Q8_0 || t == QR_TYPE_Q4_K || t == QR_TYPE_Q5_K ||
           t == QR_TYPE_Q6_K;
}

void qr_matmul_q_fused(float* out, const float* x, const void* w, uint32_t type, int n, int d,
                       int threads) {
    const void* wd = NULL;
    float *xd, *yd;
    int rc;
    (void)threads;
    if (n <= 0) return;
    if (w == NULL || !type_known(type) || d <= 0) {
        memset(out, 0, (size_t)n * sizeof(float));
        return;
    }
    if (ensure() != 0) {
        report("qr_matmul_q_fused: no device", QR_ERR_NODEV);
        memset(out, 0, (size_t)n * sizeof(float));
        return;
    }
    pthread_mutex_lock(&g_mu);
    rc = qr_weights_upload(g_ctx, w, qr_row_bytes(type, d) * (size_t)n, &wd);
    xd = (float*)staging(0, (size_t)d * sizeof(float));
    yd = (float*)staging(1, (size_t)n * sizeof(float));
    if (rc == QR_OK && (!xd || !yd)) rc = QR_ERR_NOMEM;
    if (rc == QR_OK) rc = qr_memcpy_h2d(g_ctx, xd, x, (size_t)d * sizeof(float));
    if (rc == QR_OK) rc = qr_gemv_ord(g_ctx, g_order, type, wd, xd, d, yd, n, n, d, 1, NULL, NULL);
    if (rc == QR_OK) rc = qr_memcpy_d2h(g_ctx, out, yd, (size_t)n * sizeof(float));
    pthread_mutex_unlock(&g_mu);
    if (rc != QR_OK) {
        report("qr_matmul_q_fused", rc);
        memset(out, 0, (size_t)n * sizeof(float));
    }
}

void qr_quantize_row_q8_0(const float* x, void* y, int k) {
    float* xd;
    void* yd;
    int rc, nb = k / 32;
    if (nb <= 0) return;
    if (ensure() != 0) {
        report("qr_quantize_row_q8_0: no device", QR_ERR_NODEV);
        return;
    }
    pthread_mutex_lock(&g_mu);
    xd = (float*)staging(0, (size_t)nb * 32 * sizeof(float));
    yd = staging(1, (size_t)nb * 34);
    rc = (xd && yd) ? QR_OK : QR_ERR_NOMEM;
    if (rc == QR_OK) rc = qr_memcpy_h2d(g_ctx, xd, x, (size_t)nb * 32 * sizeof(float));
    if (rc == QR_OK) rc = qr_quantize_q8_0(g_ctx, xd, yd, (long)nb * 32);
    if (rc == QR_OK) rc = qr_memcpy_d2h(g_ctx, y, yd, (size_t)nb * 34);
    pthread_mutex_unlock(&g_mu);
    if (rc != QR_OK) report("qr_quantize_row_q8_0", rc);
}

void qr_ops_matmul(float* out, const float* x, const float* w, int n, int d, int threads) {
    const void* wd = NULL;
    float *xd, *yd;
    int rc;
    (void)threads;
    if (n <= 0) return;
    if (w == NULL || d < 0) {
        memset(out, 0, (size_t)n * sizeof(float));
        return;
    }
    if (ensure() != 0) {
        report("qr_ops_matmul: no device", QR_ERR_NODEV);
        memset(out, 0, (size_t)n * sizeof(float));
        return;
    }
    pthread_mutex_lock(&g_mu);
    rc = qr_weights_upload(g_ctx, w, (size_t)n * (size_t)d * sizeof(float), &wd);
    xd = (float*)staging(0, (size_t)(d > 0 ? d : 1) * sizeof(float));
    yd = (float*)staging(1, (size_t)n * sizeof(float));
    if (rc == QR_OK && (!xd || !yd)) rc = QR_ERR_NOMEM;
    if (rc == QR_OK) rc = qr_memcpy_h2d(g_ctx, xd, x, (size_t)d * sizeof(float));
    if (rc == QR_OK) rc = qr_matmul_f32(g_ctx, g_order, (const float*)wd, xd, yd, n, d, 1);
    if (rc == QR_OK) rc = qr_memcpy_d2h(g_ctx, out, yd, (size_t)n * sizeof(float));
    pthread_mutex_unlock(&g_mu);
    if (rc != QR_OK) {
        report("qr_ops_matmul", rc);
        memset(out, 0, (size_t)n * sizeof(float));
    }
}

void qr_ops_softmax(float* x, int size) {
    float* xd;
    int rc;
    if (size <= 0) return;
    if (ensure() != 0) {
        report("qr_ops_softmax: no device", QR_ERR_NODEV);
        return;
    }
    pthread_mutex_lock(&g_mu);
    xd = (float*)staging(0, (size_t)size * sizeof(float));
    rc = xd ? QR_OK : QR_ERR_NOMEM;
    if (rc == QR_OK) rc = qr_memcpy_h2d(g_ctx, xd, x, (size_t)size * sizeof(float));
    if (rc == QR_OK) rc = qr_softmax(g_ctx, xd, 1, size);
    if (rc == QR_OK) rc = qr_memcpy_d2h(g_ctx, x, xd, (size_t)size * sizeof(float));
    pthread_mutex_unlock(&g_mu);
    if (rc != QR_OK) report("qr_ops_softmax", rc);
}

/* Device copy of one [E] expert tensor given its E host slice pointers:
 * one upload when the slices are consecutive parts of one slab
 * (src/model.c:412-419), otherwise a gather keyed by the pointer array. */
static int expert_tensor(float* const* parts, int E, size_t slice, const void** dev) {
    int e, contiguous = 1;
    for (e = 1; e < E; e++)
        if ((const char*)parts[e] != (const char*)parts[0] + (size_t)e * slice) contiguous = 0;
    if (contiguous) return qr_weights_upload(g_ctx, parts[0], slice * (size_t)E, dev);
    return qr_weights_upload_parts(g_ctx, (const void*)parts, (const void* const*)parts, slice, E,
                                   dev);
}

int qr_moe_block(float* x, const float* xb, const float* router, float* const* up_e,
                 float* const* gate_e, float* const* down_e, uint32_t up_type,
                 uint32_t gate_type, uint32_t down_type, int dim, int hidden, int n_experts,
                 int n_used, int threads) {
    qr_moe_layer L;
    const void *rd = NULL, *ud = NULL, *gd = NULL, *dd = NULL;
    float *xd, *xbd;
    int rc;
    (void)threads;
    if (!x || !xb || !router || !up_e || !gate_e || !down_e || dim <= 0 || hidden <= 0 ||
        n_experts <= 0 || n_used <= 0)
        return QR_ERR_INVALID;
    if (ensure() != 0) {
        report("qr_moe_block: no device", QR_ERR_NODEV);
        return QR_ERR_NODEV;
    }
    pthread_mutex_lock(&g_mu);
    rc = qr_weights_upload(g_ctx, router, (size_t)n_experts * (size_t)dim * sizeof(float), &rd);
    if (rc == QR_OK)
        rc = expert_tensor(up_e, n_experts, qr_row_bytes(up_type, dim) * (size_t)hidden, &ud);
    if (rc == QR_OK)
        rc = expert_tensor(gate_e, n_experts, qr_row_bytes(gate_type, dim) * (size_t)hidden, &gd);
    if (rc == QR_OK)
        rc = expert_tensor(down_e, n_experts, qr_row_bytes(down_type, hidden) * (size_t)dim, &dd);
    xd = (float*)staging(2, (size_t)dim * sizeof(float));
    xbd = (float*)staging(3, (size_t)dim * sizeof(float));
    if (rc == QR_OK && (!xd || !xbd)) rc = QR_ERR_NOMEM;
    if (rc == QR_OK) rc = qr_memcpy_h2d(g_ctx, xd, x, (size_t)dim * sizeof(float));
    if (rc == QR_OK) rc = qr_memcpy_h2d(g_ctx, xbd, xb, (size_t)dim * sizeof(float));
    if (rc == QR_OK) {
        memset(&L, 0, sizeof(L));
        L.dim = dim;
        L.hidden = hidden;
        L.n_experts = n_experts;
        L.n_used = n_used;
        L.router = (const float*)rd;
        L.up = ud;
        L.gate = gd;
        L.down = dd;
        L.up_type = up_type;
        L.gate_type = gate_type;
        L.down_type = down_type;
        rc = qr_moe_forward(g_ctx, &L, xd, xbd, 1, g_order, NULL, NULL);
    }
    if (rc == QR_OK) rc = qr_memcpy_d2h(g_ctx, x, xd, (size_t)dim * sizeof(float));
    pthread_mutex_unlock(&g_mu);
    if (rc != QR_OK) report("qr_moe_block", rc);
    return rc;
}

int qr_dropin_register_weights(const void* host, size_t bytes) {
    const void* dev = NULL;
    int rc;
    if (ensure() != 0) return QR_ERR_NODEV;
    pthread_mutex_lock(&g_mu);
    rc = qr_weights_upload(g_ctx, host, bytes, &dev);
    pthread_mutex_unlock(&g_mu);
    if (rc != QR_OK) report("qr_dropin_register_weights", rc);
    return rc;
}

void qr_dropin_release_weights(void) {
    pthread_mutex_lock(&g_mu);
    if (g_ctx) qr_weights_release_all(g_ctx);
    pthread_mutex_unlock(&g_mu);
}
