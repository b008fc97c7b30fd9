/*
 * qr_oracle.h -- CPU restatement of quantr-in-c's quantized GEMV and MoE path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker: it is loaded
 * by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg, and
 * by nothing else.  The product (libqr_hip.so) never links, loads or calls it.
 *
 * Each function restates the reference's arithmetic in plain C99, in the
 * reference's evaluation order, compiled with -ffp-contract=off so that no
 * multiply-add is fused unless the reference fuses it explicitly.
 *
 * Pinning (what checks each function against something other than itself):
 *   qro_h2f / qro_f2h           golden vectors from the compiled reference (all
 *                               65536 codes / special floats), round-trip laws
 *   qro_quantize_row_q8_0       golden vectors from the compiled reference
 *   qro_dequantize_row          golden vectors (types 8, 12, 13, 14)
 *   qro_vec_dot Q8_0 SEQ/AVX2/  golden vectors from the -std=c99, the
 *              AVX512           -mavx2 -mfma and the -mavx512f builds of the
 *                               reference
 *   qro_vec_dot Q5_K, Q6_K      golden vectors
 *   qro_vec_dot Q4_K            the reference's Q4_K dot is defective; the
 *                               corrected form equals the reference's Q5_K dot
 *                               on the same block with a zero high-bit plane,
 *                               checked bit-exactly against golden Q5_K vectors,
 *                               and against an fp64 dequantize-then-dot
 *   qro_row_accum               brute-force integer sums on tiny rows
 *   qro_matmul_f32 SEQ/AVX2     golden vectors (matmul_ref, matmul_omp AVX2)
 *   qro_softmax                 golden vectors (softmax_ref)
 *   qro_moe_token               golden vectors of the reference's
 *                               forward_runtime MoE block
 *   qro_moe_dispatch            invariants (bijection, counts, stable order)
 *                               and brute force; no reference counterpart
 *   qro_shared_expert           closed form; no reference counterpart
 *                               (parity unpinned by the reference)
 */
#ifndef QR_ORACLE_H
#define QR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids used by the reference (src/quant.c:478-483, src/model.c:20-30). */
#define QRO_TYPE_F32 0
#define QRO_TYPE_Q8_0 8
#define QRO_TYPE_Q4_K 12
#define QRO_TYPE_Q5_K 13
#define QRO_TYPE_Q6_K 14
/* llama.cpp / ggml's own K-quant layouts (qr_oracle_ggml.c) when set on a
 * Q4_K / Q5_K / Q6_K type: the dot against Q8_K activations of ggml's
 * generic ggml_vec_dot_q*_K_q8_K (same block sizes as the reference's). */
#define QRO_GGML 0x200u

/* fp32 accumulation orders of the reference builds.
 * SEQ:    the portable C99 loops (Makefile CFLAGS -O3 -std=c99, no FMA):
 *         matmul_ref (src/kernels.c:18-28), the scalar vec_dot_q8_0_q8_0
 *         (src/quant.c:279-285) and every K-quant dot.
 * AVX2:   the -mavx2 -mfma build (.github/workflows/ci.yml:21): matmul_omp's
 *         8-lane FMA chains (src/kernels.c:50-65) and vec_dot_q8_0_q8_0's
 *         8-lane accumulators (src/quant.c:245-277).
 * AVX512: an -mavx512f build: matmul_omp's 16-lane FMA chains +
 *         _mm512_reduce_add_ps tree (src/kernels.c:38-49), and
 *         vec_dot_q8_0_q8_0's 8 lanes updated by fused multiply-adds
 *         (src/quant.c:268-269). */
#define QRO_ORDER_SEQ 0
#define QRO_ORDER_AVX2 1
#define QRO_ORDER_AVX512 2

float qro_h2f(uint16_t h);
uint16_t qro_f2h(float f);
void qro_h2f_batch(const uint16_t* h, float* out, long n);

size_t qro_row_bytes(uint32_t type, int d);
int qro_units_per_row(uint32_t type, int d);

void qro_quantize_row_q8_0(const float* x, void* y, int k);
void qro_dequantize_row(float* out, const void* src, uint32_t type, int n);

float qro_vec_dot(uint32_t type, const void* row, const void* xq8, int d, int order);
int qro_row_accum(uint32_t type, const void* row, const void* xq8, int d,
                  int32_t* isum, int32_t* bsum);

void qro_matmul_q_fused(float* out, const float* x, const void* w, uint32_t type,
                        int n, int d, int threads, int order);
void qro_matmul_q_fused_batch(float* out, const float* x, const void* w, uint32_t type,
                              int n, int d, int nt, int threads, int order);
void qro_matmul_f32(float* out, const float* x, const float* w, int n, int d, int order);

void qro_softmax(float* x, int n);
float qro_silu(float x);
void qro_expf_batch(const float* in, float* out, size_t n);

int qro_route(const float* xb, const float* router_w, int dim, int E, int K, int order,
              float* logits, float* probs, int32_t* idx, float* wts);

typedef struct {
    int dim;          /* model width (Config.dim) */
    int hidden;       /* expert ffn width (Config.hidden_dim) */
    int n_experts;    /* Config.expert_count */
    int n_used;       /* Config.expert_used_count */
    const float* router;      /* ffn_gate_inp [E][dim] fp32 */
    const void* up;           /* ffn_up_exps   [E][hidden][dim], the SiLU slot (expert_w1) */
    const void* gate;         /* ffn_gate_exps [E][hidden][dim], the linear slot (expert_w3) */
    const void* down;         /* ffn_down_exps [E][dim][hidden] (expert_w2) */
    uint32_t up_type, gate_type, down_type;
    /* Optional shared expert with a sigmoid gate (no reference counterpart). */
    int sh_hidden;            /* 0 = none */
    const float* sh_gate_inp; /* [dim] fp32 */
    const void* sh_up;
    const void* sh_gate;
    const void* sh_down;
    uint32_t sh_up_type, sh_gate_type, sh_down_type;
} qro_moe_layer;

size_t qro_expert_slice_bytes(uint32_t type, int ne0, int ne1);

/* router_order: the router's KernelOps.matmul order (and F32 experts');
 * dot_order: the Q8_0 fused-dot order of the build (K-quant dots have one). */
void qro_dense_ffn(float* x, const float* xb, const qro_moe_layer* L, int order, int threads);
/* qr_oracle_ggml.c: rows of a ggml-layout matrix against Q8_K(x) (rows in
 * parallel, any width: the same bits), and one row's dequantization. */
void qro_ggml_matmul_mt(float* out, const float* x, const void* w, int type, int n, int d, int nt,
                        int threads);
void qro_ggml_dequantize_row(int type, const void* src, float* y, int n);
void qro_moe_token(float* x, const float* xb, const qro_moe_layer* L, int router_order,
                   int dot_order, int threads, int32_t* idx_out, float* w_out);
void qro_moe_forward(float* x, const float* xb, int T, const qro_moe_layer* L, int router_order,
                     int dot_order, int threads, int32_t* idx_out, float* w_out);
void qro_shared_expert(float* y, const float* xb, const qro_moe_layer* L, int threads);
int qro_moe_dispatch(const int32_t* idx, int T, int K, int E, int32_t* counts,
                     int32_t* offsets, int32_t* perm, int32_t* inv);

/* ---- the single-token decode step (qr_oracle_decode.c) ------------------ */
#define QRO_KV_F32 0
#define QRO_KV_F16 1
#define QRO_KV_Q8_0 2

typedef struct {
    int dim, n_layers, n_heads, n_kv_heads, head_dim, vocab, seq_len;
    float rope_base;
    int kv_type;                 /* QRO_KV_F32, QRO_KV_F16 or QRO_KV_Q8_0 */
    const void* tok_embd;        /* [vocab] rows of tok_row_bytes */
    uint32_t tok_type;
    size_t tok_row_bytes;
    const float* const* rms_att; /* [L] -> [dim] */
    const float* const* rms_ffn;
    const void* const* wq;       /* [L] -> [n_heads*head_dim][dim] */
    const void* const* wk;       /* [L] -> [n_kv_heads*head_dim][dim] */
    const void* const* wv;
    const void* const* wo;       /* [L] -> [dim][n_heads*head_dim] */
    const uint32_t* wtype;       /* [L][4]: wq, wk, wv, wo */
    const qro_moe_layer* moe;    /* [L] */
    const float* rms_final;
    const void* wcls;            /* [vocab][dim] */
    uint32_t wcls_type;
    int threads;                 /* OpenMP width of the quantized GEMVs and of the attention's
                                    heads (rows and heads are independent: any width gives
                                    the same bits) */
} qro_model;

void qro_rmsnorm(float* o, const float* x, const float* w, int n);
void qro_rope(float* q, float* k, int qlen, int head_dim, int n_kv_heads, int pos, float base);
void qro_rope_table(float* cs, int qlen, int head_dim, int pos, float base);
size_t qro_kv_row_bytes(int kv_type, int kv_dim);
void qro_kv_store(void* row, const float* src, int kv_dim, int kv_type);
void qro_attention(float* out, const float* q, const void* kc, const void* vc, size_t row_stride,
                   int kv_type, int pos, int n_heads, int n_kv_heads, int head_dim, float* att);
void qro_attention_mt(float* out, const float* q, const void* kc, const void* vc,
                      size_t row_stride, int kv_type, int pos, int n_heads, int n_kv_heads,
                      int head_dim, float* att, int threads);
void qro_forward(const qro_model* m, void* kc, void* vc, int token, int pos, int order, float* x,
                 float* logits);

#ifdef __cplusplus
}
#endif
#endif
