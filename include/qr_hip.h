/*
 * qr_hip.h -- C ABI of libqr_hip.so: quantr-in-c's quantized GEMV and MoE hot
 * path on one MI355X (gfx950), with device-resident weights and activations.
 *
 * Plain C, plain pointers and sizes.  Every function returns a qr_status
 * (0 on success, a negative code on failure; qr_last_error() then holds a
 * message for the calling thread).  Unless a function says otherwise, pointer
 * arguments are DEVICE pointers, work is enqueued on the context's stream and
 * the call returns without waiting (qr_sync() waits).
 *
 * Block formats are the reference's own (include/quant.h:28-50 and the raw
 * 210-byte Q6_K of src/quant.c:220-226); type ids are GGML's (0 F32, 8 Q8_0,
 * 12 Q4_K, 13 Q5_K, 14 Q6_K).  Results equal the reference's C99 build bit for
 * bit: int32 unit sums, fp32 GEMV outputs (fp32 terms added in the
 * reference's sequential order), router indices and weights, and the MoE
 * layer output.  The reference's Q4_K dot is defective (it reads fp16 bit
 * patterns as floats, src/quant.c:302-309); Q4_K here is the corrected form,
 * which equals the reference's Q5_K dot on the same block with a zero fifth
 * bit plane.
 *
 * The host-pointer drop-ins with the reference's own signatures are in
 * qr_dropin.h.
 */
#ifndef QR_HIP_H
#define QR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    QR_OK = 0,
    QR_ERR_INVALID = -1,     /* bad argument (null, size, alignment, type) */
    QR_ERR_HIP = -2,         /* HIP runtime error */
    QR_ERR_NOMEM = -3,       /* device or host allocation failed */
    QR_ERR_UNSUPPORTED = -4, /* valid but not implemented (e.g. a token count) */
    QR_ERR_NODEV = -5        /* no usable GPU */
} qr_status;

#define QR_TYPE_F32 0
#define QR_TYPE_Q8_0 8
#define QR_TYPE_Q4_K 12
#define QR_TYPE_Q5_K 13
#define QR_TYPE_Q6_K 14

/* The reference build whose fp32 accumulation orders a call reproduces:
 *   SEQ    the Makefile's -std=c99 build: matmul_ref (src/kernels.c:18-28) and
 *          the scalar Q8_0 dot (src/quant.c:279-285);
 *   AVX2   the CI's -mavx2 -mfma build: matmul_omp's 8 FMA chains
 *          (src/kernels.c:50-65) and the Q8_0 dot's 8 lane accumulators,
 *          updated by a multiply then an add (src/quant.c:245-277);
 *   AVX512 a build with -mavx512f: matmul_omp's 16 FMA chains
 *          (src/kernels.c:38-49) and the Q8_0 dot's 8 lanes updated by fused
 *          multiply-adds (src/quant.c:268-269).
 * K-quant dots are scalar in every build and do not depend on the order.
 * (The same values are defined in qr_dropin.h.) */
#ifndef QR_ORDER_SEQ
#define QR_ORDER_SEQ 0
#define QR_ORDER_AVX2 1
#define QR_ORDER_AVX512 2
#endif

typedef struct qr_ctx qr_ctx;

/* ---- context, memory, timing ------------------------------------------ */
const char* qr_last_error(void);
const char* qr_version(void);
int qr_device_count(int* count);
int qr_ctx_create(int device, qr_ctx** out);
int qr_ctx_destroy(qr_ctx* ctx);
/* Use an existing hipStream_t (NULL restores the context's own stream). */
int qr_ctx_set_stream(qr_ctx* ctx, void* hip_stream);

/* The expert products of this context's MoE calls with T > 1 tokens (no
 * reference counterpart: the reference has one CPU loop).  AUTO and MFMA take
 * the int8 MFMA products where both expert types have an MFMA form (measured
 * faster than the grouped GEMV at every T >= 2 at the Qwen3-30B-A3B shape);
 * GEMV forces the grouped GEMV.  Results are identical on every path. */
#define QR_MOE_PATH_AUTO 0
#define QR_MOE_PATH_GEMV 1
#define QR_MOE_PATH_MFMA 2
int qr_ctx_set_moe_path(qr_ctx* ctx, int path);
void* qr_ctx_get_stream(qr_ctx* ctx);
int qr_sync(qr_ctx* ctx);
int qr_malloc(qr_ctx* ctx, size_t bytes, void** dptr);
int qr_free(qr_ctx* ctx, void* dptr);
/* Copies are ordered on the context stream and complete before returning. */
int qr_memcpy_h2d(qr_ctx* ctx, void* dst, const void* src, size_t bytes);
int qr_memcpy_d2h(qr_ctx* ctx, void* dst, const void* src, size_t bytes);
int qr_memcpy_d2d(qr_ctx* ctx, void* dst, const void* src, size_t bytes);
int qr_memset(qr_ctx* ctx, void* dst, int value, size_t bytes);
/* HIP events on the context stream: start, then stop -> elapsed ms. */
int qr_timer_start(qr_ctx* ctx);
int qr_timer_stop(qr_ctx* ctx, float* ms);
/* HIP graph capture of the context stream: calls between begin and end are
 * recorded, not run; the instantiated graph replays them back to back.
 * Calls that would allocate, free, synchronize or record a memset while the
 * stream is capturing return QR_ERR_INVALID instead (qr_malloc, qr_free,
 * the synchronous copies, qr_timer_stop, qr_weights_upload*, and qr_moe_route /
 * qr_moe_forward when they need more scratch than any earlier call).  The
 * scratch a call needs depends on the layer (dim, hidden, E, K, the shared
 * expert) as well as on T: run the largest captured call once outside
 * capture first.  Scratch that a larger call outgrows is kept until
 * qr_ctx_destroy, so graphs captured earlier stay valid.  qr_gemv with NULL
 * weights zero-fills with a kernel and qr_memset uses a fill kernel while
 * capturing, so neither records a memset node. */
int qr_capture_begin(qr_ctx* ctx);
int qr_capture_end(qr_ctx* ctx, void** graph);
int qr_graph_launch(qr_ctx* ctx, void* graph);
int qr_graph_destroy(void* graph);
/* A plain streaming copy kernel (dst = src, 16-byte chunks): the reference
 * point for hardware byte counters. */
int qr_copy_kernel(qr_ctx* ctx, void* dst, const void* src, size_t bytes);
/* A plain streaming read of `bytes` (16-byte chunks, each read once): the
 * achievable rate for a kernel that reads the same bytes once.  sink is a
 * 4-byte device word it may write. */
int qr_read_kernel(qr_ctx* ctx, const void* src, size_t bytes, void* sink);

/* ---- quantized GEMV ------------------------------------------------------ */

/* quantize_row_q8_0 (src/quant.c:143-158) of n floats into n/32 block_q8_0
 * (34-byte) blocks; a tail shorter than 32 is not written. */
int qr_quantize_q8_0(qr_ctx* ctx, const float* x, void* y, long n);

/* y[t*ystride + r] = W[r] . x[t*xstride ...] for r < n, t < nt, with W an
 * [n][row_bytes(type, d)] weight matrix (16-byte aligned) and x fp32,
 * quantized to Q8_0 inside the call as matmul_q_fused does
 * (src/quant.c:441-523).  type F32 runs the fp32 GEMV in SEQ order.
 * nt in {1, 2, 3, 4, 8}.  acc (optional, [nt][n][units]) receives the int32
 * sum of every 32-element unit, accb (optional, [nt][units]) the activation
 * block sums -- a parity mode for bit-exact integer checks. */
int qr_gemv_ex(qr_ctx* ctx, uint32_t type, const void* w, const float* x, int xstride,
               float* y, int ystride, int n, int d, int nt, int32_t* acc, int32_t* accb);
int qr_gemv(qr_ctx* ctx, uint32_t type, const void* w, const float* x, float* y, int n, int d,
            int nt);
/* qr_gemv_ex for the reference build `order` (QR_ORDER_*): Q8_0 weights use
 * that build's dot order; other types are the same in every build.
 * qr_gemv_ex is qr_gemv_ord with QR_ORDER_SEQ. */
int qr_gemv_ord(qr_ctx* ctx, int order, uint32_t type, const void* w, const float* x,
                int xstride, float* y, int ystride, int n, int d, int nt, int32_t* acc,
                int32_t* accb);

/* T tokens through one quantized matrix as a grouped int8 MFMA product (the
 * kernel of qr_decoder_prefill's projections): y[t * ystride + r] = W[r] .
 * x[t * xstride ...] for r < n, t < T, the same bits as qr_gemv_ord gives
 * token by token (every 32-element unit's fp32 term added in unit order).
 * Q4_K / Q5_K (row-major or QR_TILED), Q6_K and Q8_0 (QR_ORDER_SEQ only),
 * d a multiple of 256 and at most 16384; any T.  Uses the context scratch
 * (48 bytes per 32 activation values, plus 4 T + 32).  No counterpart in the
 * reference, which runs one matmul_q_fused per token (speculative
 * verification, src/speculative.c:107-140; prompts, src/runtime.c:294-304). */
int qr_gemv_rows(qr_ctx* ctx, int order, uint32_t type, const void* w, const float* x,
                 int xstride, float* y, int ystride, int n, int d, int T);

/* The tiled layout of a Q4_K / Q5_K / Q6_K / Q8_0 matrix: the same bytes as
 * the reference's row-major blocks, permuted so that the GEMV streams each
 * wave's tile in the order it is consumed (no reference counterpart; the
 * results are the same bits).  A lane holds 256 elements of a row (a K-quant
 * super-block, or 8 Q8_0 blocks) and a tile is 64 / (d / 256) rows; within
 * it, the k-th 16-byte chunk of every lane is stored together (Q4_K / Q5_K:
 * the header chunk first; Q6_K: its scales, then each unit pair's high bits
 * and low nibbles, and the fp16 d fields of all super-blocks after all the
 * tiles, in row-major order; Q8_0: the 8 scales, then the blocks' values).
 * Pass `type | QR_TILED` to qr_gemv / qr_gemv_ex / qr_gemv_ord (no integer
 * sums; Q8_0 in QR_ORDER_SEQ only) and in a decoder model's wq / wk / wv / wo
 * / wcls types.  qr_weights_tile writes the tiled copy of an n x d matrix (d
 * a multiple of 256, at most 16384; Q6_K with n * (d / 256) a multiple of 8)
 * into dst, qr_weights_untile the reverse; device pointers, 16-byte aligned,
 * not overlapping; enqueued on the context stream.  qr_row_bytes(type | QR_TILED, d) is the plain row size. */
#define QR_TILED 0x100u

/* llama.cpp / ggml's own K-quant layouts (ggml-common.h: block_q4_K with its
 * 12 packed 6-bit scales and mins, block_q5_K, block_q6_K with 16 int8
 * scales; 144 / 176 / 210 bytes), which the reference does not implement (its
 * layouts are its own, src/quant.c:180-238): pass `QR_TYPE_Q4_K | QR_GGML`
 * (Q5_K, Q6_K) to qr_gemv / qr_gemv_ex / qr_gemv_ord (no integer sums) and
 * qr_dequantize.  The activation is quantized to Q8_K (quantize_row_q8_K_ref)
 * and each row's dot follows ggml's generic ggml_vec_dot_q*_K_q8_K: eight
 * lane sums and the min sum accumulated block by block, then added.
 * qr_quantize_q8_k writes n / 256 block_q8_K (292 bytes: f32 d, i8 qs[256],
 * i16 bsums[16]). */
#define QR_GGML 0x200u
int qr_quantize_q8_k(qr_ctx* ctx, const float* x, void* y, long n);
int qr_weights_tile(qr_ctx* ctx, uint32_t type, const void* src, void* dst, int n, int d);
int qr_weights_untile(qr_ctx* ctx, uint32_t type, const void* src, void* dst, int n, int d);

/* fp32 GEMV in a reference accumulation order (router logits):
 * y[t][r] = sum_j w[r][j] * x[t][j]. */
int qr_matmul_f32(qr_ctx* ctx, int order, const float* w, const float* x, float* y, int n, int d,
                  int nt);

/* softmax_ref (src/kernels.c:191-207) of each of `rows` rows of n floats,
 * in place; expf is bit-exact with glibc's. */
int qr_softmax(qr_ctx* ctx, float* x, int rows, int n);

/* Bytes per weight row (whole blocks only, src/quant.c:477-484). */
size_t qr_row_bytes(uint32_t type, int d);

/* ---- MoE layer --------------------------------------------------------- */

/* One MoE layer's device weights.  Expert tensors are [E][rows][cols] in
 * GGUF order, expert e's matrix at base + e * rows * row_bytes(type, cols)
 * (src/model.c:412-419).  up is ffn_up_exps (the SiLU slot, expert_w1), gate
 * is ffn_gate_exps (the linear slot, expert_w3), down is ffn_down_exps
 * (expert_w2); hb = silu(up . xb) * (gate . xb) (src/runtime.c:252-256).
 * sh_* describe an optional shared expert with a sigmoid gate (no reference
 * counterpart; sh_hidden 0 disables it). */
typedef struct {
    int dim;
    int hidden;
    int n_experts;
    int n_used;
    const float* router;          /* ffn_gate_inp [E][dim] fp32 */
    const void* up;
    const void* gate;
    const void* down;
    uint32_t up_type, gate_type, down_type;
    int sh_hidden;
    const float* sh_gate_inp;     /* [dim] fp32 */
    const void* sh_up;
    const void* sh_gate;
    const void* sh_down;
    uint32_t sh_up_type, sh_gate_type, sh_down_type;
} qr_moe_layer;

/* Router for T tokens (src/runtime.c:205-230): logits in `order`, softmax,
 * K argmax passes (strict '>', lowest index on ties), weights renormalised by
 * their sequential sum.  idx/wts are [T][K]; probs (optional) [T][E]. */
int qr_moe_route(qr_ctx* ctx, const qr_moe_layer* L, const float* xb, int T, int order,
                 float* probs, int32_t* idx, float* wts);

/* Token-to-expert dispatch of T*K (token, slot) pairs p = t*K + k:
 * counts[E], offsets[E+1] (exclusive scan), perm[T*K] = pairs grouped by
 * expert and ascending p inside each group, inv[p] = position of p in perm.
 * Deterministic (no dependence on atomic ordering). */
int qr_moe_dispatch(qr_ctx* ctx, const int32_t* idx, int T, int K, int E, int32_t* counts,
                    int32_t* offsets, int32_t* perm, int32_t* inv);

/* The whole layer for T tokens: x[t] += sum_k w[t][k] * expert(xb[t]) in slot
 * order (src/runtime.c:242-269), plus the shared expert when present.
 * `order` is the reference build (QR_ORDER_*): the router's accumulation
 * order and, for Q8_0 experts, the dot order.  The shared expert has no
 * reference counterpart and always uses the sequential order.
 * idx_out / w_out (optional, [T][K]) receive the routing. */
int qr_moe_forward(qr_ctx* ctx, const qr_moe_layer* L, float* x, const float* xb, int T,
                   int order, int32_t* idx_out, float* w_out);

/* qr_moe_forward without any allocation: no reference counterpart; it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc).  Same arguments, same
 * results as qr_moe_forward.  Its scratch is one fixed device array of
 * QR_NOALLOC_SCRATCH_BYTES per GPU, held from library load until the process
 * ends; a call whose layer and T need more returns QR_ERR_INVALID (about
 * 111 KiB per token at the Qwen3-30B-A3B shape: up to T = 150).  Every call on
 * one GPU, from any context, shares that array: calls that overlap on one GPU
 * (other streams, other threads) race, so serialize them.  It calls no
 * hipMalloc / hipFree. */
#define QR_NOALLOC_SCRATCH_BYTES (16 * 1024 * 1024)
int qr_moe_forward_noalloc(qr_ctx* ctx, const qr_moe_layer* L, float* x, const float* xb, int T,
                           int order, int32_t* idx_out, float* w_out);

/* ---- single-token decode step (forward_runtime, src/runtime.c:94-288) ---- */

/* KV cache row formats.  F32 is the reference's kv_cache_type 0 and F16 its
 * kv_cache_type 1 (src/runtime.c:74-92, selected by --kv-cache-quant fp16,
 * src/main.c:140): each value stored with the truncating fp32_to_fp16 and read
 * with fp16_to_fp32 (include/quant.h:53-77), half subnormals decoding as the
 * reference decodes them.  Q8_0 rows are quantize_row_q8_0
 * (src/quant.c:143-158) of each position's kv_dim values, read back as qs * d
 * like dequantize_row: the reference's own type 2 is declared but
 * unimplemented (kv_store_row writes fp32 into a buffer sized at one byte per
 * element, src/runtime.c:74-84 against src/model.c:82-88). */
#define QR_KV_F32 0
#define QR_KV_F16 1
#define QR_KV_Q8_0 2

/* Bytes of one position's K (or V) row: kv_dim floats, kv_dim halves, or
 * kv_dim / 32 Q8_0 blocks; 0 for a bad type or size. */
size_t qr_kv_row_bytes(int kv_type, int kv_dim);

/* dequantize_row (src/quant.c:160-240) of `rows` rows of n elements each
 * (row stride qr_row_bytes(type, n)); a null src or an unknown type gives
 * zeros, as there.  out is [rows][n] fp32. */
int qr_dequantize(qr_ctx* ctx, uint32_t type, const void* src, int rows, int n, float* out);

/* rmsnorm_ref (src/kernels.c:170-180): o = w * (x * (1 / sqrtf(sum x^2 / n +
 * 1e-5))), the sum of squares formed in index order.  With add non-null, x +=
 * add first (the residual of src/runtime.c:196-198) and x is updated.
 * n <= 8192. */
int qr_rmsnorm(qr_ctx* ctx, float* o, float* x, const float* add, const float* w, int n);

/* The attention of forward_runtime (src/runtime.c:136-193) over positions
 * 0..npos-1 of a paged cache (page a power of two): position t's row is at page ptab[t / page],
 * slot t % page (rows of qr_kv_row_bytes(kv_type, n_kv_heads * head_dim)
 * bytes, kv head h's elements at h * head_dim).  Scores are dot_ref
 * (src/kernels.c:162-168) times 1 / sqrtf(head_dim), softmax_ref per head,
 * then each output element sums att * v over the positions in order.
 * q, out: [n_heads][head_dim]; att: scratch [n_heads][npos] (left holding the
 * normalised weights).  head_dim a multiple of 32 up to 512; npos <= 22528. */
int qr_attention(qr_ctx* ctx, const float* q, const void* kc, const void* vc,
                 const int32_t* ptab, int page, int kv_type, int npos, int n_heads,
                 int n_kv_heads, int head_dim, float* att, float* out);

/* One transformer layer's device weights (src/model.c:358-446): attention
 * projections [rows][cols] in GGUF row order (wq [n_heads * head_dim][dim],
 * wk / wv [n_kv_heads * head_dim][dim], wo [dim][n_heads * head_dim]) and the
 * MoE block (moe.dim == dim).  moe.n_experts == 0 makes the layer dense, as
 * expert_count == 0 does in the reference (src/runtime.c:270-284): moe.up,
 * moe.gate and moe.down are then its ffn_up (w1, the SiLU slot), ffn_gate
 * (w3) and ffn_down (w2) matrices of moe.hidden rows (columns for down), and
 * the router and n_used are not read. */
typedef struct {
    const float* rms_att;  /* [dim] */
    const float* rms_ffn;  /* [dim] */
    const void* wq;
    const void* wk;
    const void* wv;
    const void* wo;
    uint32_t wq_type, wk_type, wv_type, wo_type;
    qr_moe_layer moe;
} qr_layer;

/* A MoE decoder's device weights (Config / TransformerWeights,
 * include/types.h).  head_dim is explicit; the reference fixes it at
 * dim / n_heads (src/runtime.c:102), which this generalises.  tok_embd holds
 * vocab rows of qr_row_bytes(tok_type, dim) bytes; wcls is [vocab][dim].
 * `layers` is a host array of n_layers entries (copied at creation). */
typedef struct {
    int dim;
    int n_heads;
    int n_kv_heads;
    int head_dim;
    int n_layers;
    int vocab;
    int seq_len;     /* KV cache capacity in positions */
    float rope_base; /* rope_freq_base; <= 0 means 10000 */
    const void* tok_embd;
    uint32_t tok_type;
    const float* rms_final;
    const void* wcls;
    uint32_t wcls_type;
    const qr_layer* layers;
} qr_model;

typedef struct qr_decoder qr_decoder;

/* Replay the decode step as one HIP graph (captured on the second call and
 * again whenever logits / x_out change). */
#define QR_DEC_GRAPH 1

/* A decoder over `model` (its weights stay the caller's): the activations, a
 * paged KV cache of seq_len positions per layer (pages of `page` positions,
 * a power of two, 0 = 256; identity page table), and the RoPE cos / sin of every position,
 * computed at creation with the host C library's powf / cosf / sinf as
 * apply_rope calls them (src/runtime.c:19-41; its frequency index runs over
 * the whole q vector, as there).  `order` is the reference build
 * (QR_ORDER_*): the order of the fp32 matmuls and the router, and of the
 * Q8_0 dot.  Where a layer's wq and wk are one tiled Q4_K / Q5_K matrix
 * (wk's bytes right after wq's) and wv is Q6_K (kv_dim * dim / 256 a
 * multiple of 8) or C99-order Q8_0, the decoder keeps a tiled copy of a
 * row-major wv (about rows x row bytes per layer) so that the norm, q / k and
 * v run as one launch. */
int qr_decoder_create(qr_ctx* ctx, const qr_model* model, int kv_type, int order, int page,
                      int flags, qr_decoder** out);
int qr_decoder_destroy(qr_decoder* dec);

/* Replace the page table: table is host [n_layers][pages_per_layer], each
 * layer a permutation of 0 .. pages_per_layer - 1. */
int qr_decoder_set_pages(qr_decoder* dec, const int32_t* table);
int qr_decoder_pages(const qr_decoder* dec, int* pages_per_layer, int* page);

/* Fill positions [pos0, pos0 + n) of layer `layer`'s cache from fp32 K and V
 * values (device [n][n_kv_heads * head_dim], after RoPE): a prefill. */
int qr_decoder_kv_write(qr_decoder* dec, int layer, int pos0, int n, const float* k,
                        const float* v);
/* Device addresses of the K and V rows of one position (synchronous). */
int qr_decoder_kv_rows(const qr_decoder* dec, int layer, int pos, const void** krow,
                       const void** vrow);

/* forward_runtime (src/runtime.c:94-288) for `token` at position `pos`: the
 * cache must hold positions 0 .. pos-1; this step writes position pos.
 * logits: device [vocab]; x_out (optional): device [dim], the residual after
 * the last layer.  Enqueued on the context's stream. */
int qr_decoder_forward(qr_decoder* dec, int token, int pos, float* logits, float* x_out);

/* Prompt prefill and speculative verification (prefill_runtime,
 * src/runtime.c:294-304, which calls forward_runtime once per token; the
 * verify loop of src/speculative.c:107-140 does the same): tokens[0..n) (a
 * host array) at positions pos0 .. pos0 + n - 1, in chunks of `chunk` tokens
 * (0: QR_PREFILL_CHUNK; at most QR_PREFILL_MAX_CHUNK).  Each chunk goes
 * through every layer at once: the projections as multi-row int8 MFMA
 * products, RoPE and the cache stores for all its positions, attention with
 * one query per token (each over the positions up to its own), the MoE layer
 * at T tokens.  The cache rows of every position are written; logits
 * (optional, device) receive the last token's [vocab] logits, or with
 * QR_PREFILL_ALL_LOGITS every token's [n][vocab]; x_out (optional) the last
 * token's residual.  Every result equals n calls of qr_decoder_forward bit
 * for bit.  Allocates a workspace on first use (not under stream capture);
 * enqueued on the context stream. */
#define QR_PREFILL_ALL_LOGITS 1
/* The default chunk: a 512-token prompt of the Qwen3-30B-A3B shape takes
 * 49.0 / 36.2 / 29.3 ms in chunks of 128 / 256 / 512 (larger chunks make
 * larger MFMA products and fewer passes over the weights); the workspace
 * holds chunk x n_heads x cap attention scores. */
#define QR_PREFILL_CHUNK 512
#define QR_PREFILL_MAX_CHUNK 1024
int qr_decoder_prefill(qr_decoder* dec, const int32_t* tokens, int n, int pos0, int chunk,
                       float* logits, float* x_out, int flags);

/* ---- GGUF files (src/gguf.c, src/model.c:253-449) ----------------------- */

/* A parsed GGUF container.  qr_gguf_parse reads a buffer the caller keeps
 * alive; qr_gguf_open maps a file read-only (load_transformer's mmap,
 * src/model.c:451-470).  Both accept and refuse exactly what
 * gguf_init_from_buffer (src/gguf.c:50-177) does: magic "GGUF", at most 65536
 * key/values and tensors, strings of at most 1 MiB, arrays of at most
 * 1,000,000 entries, at most 4 dimensions, known key/value types,
 * general.alignment (u32 or u64; 0 or absent: 32), every tensor starting
 * inside the buffer.  Host-only: no device is needed. */
typedef struct qr_gguf qr_gguf;
int qr_gguf_parse(const void* data, size_t size, qr_gguf** out);
int qr_gguf_open(const char* path, qr_gguf** out);
int qr_gguf_close(qr_gguf* g);
int qr_gguf_info(const qr_gguf* g, uint32_t* version, uint64_t* n_tensors, uint64_t* n_kv,
                 uint64_t* alignment, uint64_t* data_offset);
/* Tensor i: name, GGML type, dimensions (ne[0] innermost; ne has 4 entries)
 * and its data in the buffer. */
int qr_gguf_tensor(const qr_gguf* g, uint64_t i, const char** name, uint32_t* type,
                   uint32_t* n_dims, uint64_t* ne, const void** data);
int64_t qr_gguf_find(const qr_gguf* g, const char* name); /* index, or -1 */
/* gguf_get_val_u32 / _f32 / _str (src/gguf.c:211-269): the first key of that
 * name holding that type, else the default (NULL for strings). */
uint32_t qr_gguf_get_u32(const qr_gguf* g, const char* key, uint32_t def);
float qr_gguf_get_f32(const qr_gguf* g, const char* key, float def);
const char* qr_gguf_get_str(const qr_gguf* g, const char* key);
int64_t qr_gguf_get_arr_len(const qr_gguf* g, const char* key); /* -1 if absent */

/* The decoder model of a MoE or dense GGUF as HOST pointers into the buffer, mapped as
 * load_gguf_transformer does (src/model.c:253-449): {arch}.embedding_length,
 * block_count, attention.head_count(_kv), expert_count, expert_used_count,
 * expert_feed_forward_length, rope.freq_base (default 1e6); token_embd,
 * output_norm, output (else tied to token_embd), blk.N.attn_norm / ffn_norm /
 * attn_q / attn_k / attn_v / attn_output / ffn_gate_inp, and the experts with
 * expert_w1 = ffn_up_exps (the SiLU slot), expert_w3 = ffn_gate_exps,
 * expert_w2 = ffn_down_exps as one 3-D tensor each or per-expert tensors
 * (then the pointers are expert 0's; see qr_gguf_expert_host); a file
 * without expert_count is dense: ffn_up (w1), ffn_gate (w3) and ffn_down (w2)
 * of feed_forward_length rows, in a layer with n_experts = 0.  Beyond the
 * reference: head_dim is attention.key_length when the file states it
 * (else dim / n_heads, as there); vocab is the tokenizer's token count, else
 * the embedding's rows; every tensor's shape and type is checked, all
 * layers on every call.  Returns n_layers; fills `layers` only when
 * max_layers >= n_layers. */
int qr_gguf_model_host(const qr_gguf* g, int seq_len, qr_model* model, qr_layer* layers,
                       int max_layers);
/* Expert e of layer `layer`: host pointers to its up, down and gate matrices. */
int qr_gguf_expert_host(const qr_gguf* g, int layer, int e, const void** up, const void** down,
                        const void** gate);

/* The same model copied to the device: every tensor the decoder reads in one
 * allocation (each tensor 256-byte aligned; per-expert tensors gathered
 * into one range per kind, expert e at e * slice, as a 3-D tensor is laid
 * out; a tied output shares the embedding's copy; Q4_K / Q5_K attention
 * projections, dense FFN matrices and output matrices with at most 64
 * super-blocks per row, and a Q6_K output matrix with rows a multiple of
 * 2048, are stored tiled and their types carry QR_TILED).  Returns a qr_model of
 * device pointers for qr_decoder_create.  The copy owns its memory: the
 * qr_gguf may be closed after loading, two loads are two copies, and
 * qr_gguf_model_free releases one of them (after the context stream has
 * drained; no decoder built on it may be used afterwards). */
typedef struct qr_gguf_model qr_gguf_model;
int qr_gguf_load(qr_ctx* ctx, const qr_gguf* g, int seq_len, qr_gguf_model** out);
/* qr_gguf_load with flags.  QR_GGUF_GGML_KQUANTS: the file's Q4_K / Q5_K /
 * Q6_K tensors are in llama.cpp's own block layouts (a checkpoint quantized
 * by llama.cpp; the reference reads the same bytes in its layouts,
 * src/quant.c:180-238): their types carry QR_GGML, none is tiled, and the
 * decoder computes them with ggml's Q8_K dots (a MoE layer's experts then all
 * three ggml K-quants, and no shared expert).  No counterpart in the
 * reference, which has no such option. */
#define QR_GGUF_GGML_KQUANTS 1u
int qr_gguf_load_ex(qr_ctx* ctx, const qr_gguf* g, int seq_len, uint32_t flags,
                    qr_gguf_model** out);
const qr_model* qr_gguf_model_get(const qr_gguf_model* m);
int qr_gguf_model_free(qr_gguf_model* m);

/* ---- weight registry (host pointer -> device copy) ---------------------- */

/* Upload `bytes` from host memory once and return the device copy; later
 * calls with the same host pointer return the same copy.  The registry keys
 * on the host address; an entry is reused only for the same size and while
 * the first and last 64 bytes of the host memory still hash to what was
 * uploaded (so a freed and reused address with other contents is uploaded
 * again).  Weights are expected not to change in place while registered
 * (the reference's mmap).  Copies live until released. */
int qr_weights_upload(qr_ctx* ctx, const void* host, size_t bytes, const void** dev);
/* Upload nparts host blocks of part_bytes each into one contiguous device
 * tensor (part i at offset i * part_bytes), registered under `key`: the
 * per-expert weight tensors of src/model.c:421-433 that are not one 3-D
 * slab.  The entry remembers a digest of the part pointers, the part size and
 * the two ends of every part: a later call under the same key with other
 * parts (or other contents) gathers again. */
int qr_weights_upload_parts(qr_ctx* ctx, const void* key, const void* const* parts,
                            size_t part_bytes, int nparts, const void** dev);
int qr_weights_lookup(qr_ctx* ctx, const void* host, const void** dev);
int qr_weights_release(qr_ctx* ctx, const void* host);
int qr_weights_release_all(qr_ctx* ctx);

/* ---- test hooks ---------------------------------------------------------- */
/* y[i] = expf(x[i]) with the device restatement of glibc's expf. */
int qr_test_expf(qr_ctx* ctx, const float* x, float* y, long n);

#ifdef __cplusplus
}
#endif
#endif /* QR_HIP_H */
