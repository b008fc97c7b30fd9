/*
 * qr_dropin.h -- quantr-in-c's hot-path entry points, same signatures, same
 * meaning, running on one MI355X through libqr_hip.so.
 *
 * Host pointers in, host results out, synchronous: each call returns with its
 * output written, like the reference's.  Weights are borrowed host pointers
 * (the reference's mmap); the first call that sees a weight pointer uploads it
 * once into a device registry keyed by that address, later calls reuse the
 * device copy (qr_dropin_release_weights drops them, the free_transformer
 * hook).  On any failure the output is zero-filled and a message goes to
 * stderr, the reference's convention (src/quant.c:443-446, 470-473).  The
 * `threads` arguments are OpenMP widths on the CPU and are ignored here.
 *
 * Each entry names the reference interface it replaces; a build of the
 * reference binds them at those call sites (kernels.c / runtime.c / model.c).
 */
#ifndef QR_DROPIN_H
#define QR_DROPIN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The reference build whose arithmetic the results match (the router's
 * KernelOps.matmul order and the Q8_0 dot order; see qr_hip.h):
 * QR_ORDER_SEQ the Makefile's -std=c99 build, QR_ORDER_AVX2 the CI's
 * -mavx2 -mfma build, QR_ORDER_AVX512 a build with -mavx512f. */
#ifndef QR_ORDER_SEQ
#define QR_ORDER_SEQ 0
#define QR_ORDER_AVX2 1
#define QR_ORDER_AVX512 2
#endif

/* Field-for-field the layout of KernelOps (include/kernels.h:6-12), so a
 * table of these functions can be used where the reference takes KernelOps. */
typedef struct {
    void (*matmul)(float* out, const float* x, const float* w, int n, int d, int threads);
    float (*dot)(const float* a, const float* b, int n);
    void (*rmsnorm)(float* o, const float* x, const float* weight, int size);
    void (*softmax)(float* x, int size);
    const char* name;
} qr_kernel_ops;

/* Select the GPU and the reference build to match (QR_ORDER_SEQ /
 * QR_ORDER_AVX2 / QR_ORDER_AVX512): it sets the router's fp32 accumulation
 * order and the Q8_0 dot order of every entry below.  Optional: the first
 * call of any entry initialises device 0 with QR_ORDER_AVX2 (the CI build).
 * Returns 0 or a qr_status. */
int qr_dropin_init(int device, int router_order);
void qr_dropin_shutdown(void);

/* Replaces gpu_available (include/kernels.h:18, src/kernels.c:248-265):
 * nonzero when an MI355X (gfx950) is usable.  Returns 3 (HIP); the
 * reference's own codes are 1 (CUDA) and 2 (Vulkan). */
int qr_gpu_available(void);

/* Replaces matmul_q_fused (include/quant.h:91-92, src/quant.c:441-523):
 * out[n] = W[n x d] . x[d] for F32, Q8_0, Q4_K, Q5_K, Q6_K weights; x is
 * quantized to Q8_0 once per call; NULL weights and unknown types give
 * zeros.  Q8_0 dots follow the build selected by qr_dropin_init.  Q4_K is the
 * corrected dot (see qr_hip.h).
 *
 * Weight registry: the first call that sees a weight pointer uploads the
 * matrix; later calls with the same pointer and size reuse the device copy
 * while the host bytes at both ends of the matrix still hash the same.
 * Weights must not change in place while registered;
 * qr_dropin_release_weights drops every copy. */
void qr_matmul_q_fused(float* out, const float* x, const void* w, uint32_t type, int n, int d,
                       int threads);

/* Replaces quantize_row_q8_0 (include/quant.h:84, src/quant.c:143-158). */
void qr_quantize_row_q8_0(const float* x, void* y, int k);

/* KernelOps.matmul (include/kernels.h:7) for the BACKEND_GPU table: the fp32
 * GEMV of the router (src/runtime.c:205) in the configured order. */
void qr_ops_matmul(float* out, const float* x, const float* w, int n, int d, int threads);

/* KernelOps.softmax (include/kernels.h:10): softmax_ref (src/kernels.c:191-207),
 * expf bit-exact with glibc's. */
void qr_ops_softmax(float* x, int size);

/* The MoE block of forward_runtime (src/runtime.c:202-269) for one token:
 * route xb, run the K selected experts, x += sum_k w_k * expert_k(xb).
 * up_e / gate_e / down_e are TransformerWeights.expert_w1[l] / expert_w3[l] /
 * expert_w2[l] (src/model.c:416-418): E pointers each; contiguous slices of one
 * GGUF tensor are uploaded as one slab, separate tensors are gathered.
 * up and gate must share a type.  Returns 0, or a qr_status after zeroing
 * nothing (x is left untouched on failure). */
int qr_moe_block(float* x, const float* xb, const float* router, float* const* up_e,
                 float* const* gate_e, float* const* down_e, uint32_t up_type,
                 uint32_t gate_type, uint32_t down_type, int dim, int hidden, int n_experts,
                 int n_used, int threads);

/* load_transformer / free_transformer hooks (include/model.h:14-15): upload a
 * mapped tensor ahead of first use; drop every device copy. */
int qr_dropin_register_weights(const void* host, size_t bytes);
void qr_dropin_release_weights(void);

#ifdef __cplusplus
}
#endif
#endif /* QR_DROPIN_H */
