/*
 * ref_gpu_bind.c -- TEST INFRASTRUCTURE: binds the reference's own, unmodified
 * runtime (src/runtime.c, src/quant.c, src/kernels.c, ... compiled where they
 * lie) to libqr_hip.so's drop-ins with the linker instead of source edits:
 *
 *   -Wl,--wrap=matmul_q_fused       every matmul_q_fused call made from another
 *                                   file (matmul_q, src/runtime.c:58-70, and
 *                                   ref_driver.c) runs qr_matmul_q_fused;
 *   -Wl,--wrap=resolve_backend      BACKEND_GPU stays BACKEND_GPU when the GPU is
 *                                   usable (src/kernels.c:267-291 would fall back);
 *   -Wl,--wrap=kernels_for_backend  BACKEND_GPU gets the GPU table: the router's
 *                                   matmul and softmax on the GPU, dot and
 *                                   rmsnorm from the build's own CPU table.
 *
 * This is INTEGRATION.md's binding (call sites 1-3) applied by the linker.
 * refgpu_bind(order) selects the reference build whose numbers the GPU must
 * reproduce (QR_ORDER_*) and the CPU table dot/rmsnorm come from.  Only the
 * GPU tests load the result (oracle/_ref/libqref_gpu_*.so).
 */
#include <stddef.h>
#include <stdint.h>

#include "kernels.h"
#include "qr_dropin.h"

void __real_matmul_q_fused(float* out, const float* x, const void* w, uint32_t type, int n,
                           int d, int threads);
KernelBackend __real_resolve_backend(KernelBackend requested);
const KernelOps* __real_kernels_for_backend(KernelBackend backend);

static KernelOps g_gpu_ops;
static KernelBackend g_cpu_backend = BACKEND_REF;
static int g_calls = 0;

void __wrap_matmul_q_fused(float* out, const float* x, const void* w, uint32_t type, int n,
                           int d, int threads) {
    g_calls++;
    qr_matmul_q_fused(out, x, w, type, n, d, threads);
}

KernelBackend __wrap_resolve_backend(KernelBackend requested) {
    if (requested == BACKEND_GPU && qr_gpu_available()) return BACKEND_GPU;
    return __real_resolve_backend(requested);
}

const KernelOps* __wrap_kernels_for_backend(KernelBackend backend) {
    if (backend != BACKEND_GPU) return __real_kernels_for_backend(backend);
    return &g_gpu_ops;
}

/* order: QR_ORDER_SEQ / _AVX2 / _AVX512, the build to reproduce. */
int refgpu_bind(int order) {
    const KernelOps* cpu;
    g_cpu_backend = order == QR_ORDER_SEQ ? BACKEND_REF
                  : order == QR_ORDER_AVX2 ? BACKEND_AVX2 : BACKEND_AVX512;
    cpu = __real_kernels_for_backend(g_cpu_backend);
    g_gpu_ops.matmul = qr_ops_matmul;
    g_gpu_ops.dot = cpu->dot;
    g_gpu_ops.rmsnorm = cpu->rmsnorm;
    g_gpu_ops.softmax = qr_ops_softmax;
    g_gpu_ops.name = "gpu-mi355x";
    return qr_dropin_init(0, order);
}

/* How many matmul_q_fused calls went to the GPU since the last call. */
int refgpu_take_calls(void) {
    int c = g_calls;
    g_calls = 0;
    return c;
}
