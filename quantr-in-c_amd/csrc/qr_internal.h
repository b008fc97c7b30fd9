// qr_internal.h -- declarations shared between the .hip translation units of
// libqr_hip.so (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include <atomic>
#include <stdint.h>

#include "../../include/qr_hip.h"

namespace qr {

// qr_runtime.hip: context internals used by other translation units.
// set_error records the calling thread's qr_last_error() message and returns
// code.  moe_check validates a MoE layer as qr_moe_forward does; gemv_check
// validates one weight matrix [n][d] of `type` for a one-token GEMV in
// `order` (w may be null: the GEMV then writes zeros).
int set_error(int code, const char* fmt, ...);
hipStream_t ctx_stream(qr_ctx* c);
int ctx_device(qr_ctx* c);
bool ctx_capturing(qr_ctx* c);
int moe_check(const qr_moe_layer* L, const char* who);
int gemv_check(uint32_t type, int order, const void* w, int n, int d, const char* who);

// qr_gemv.hip
// q8o: the Q8_0 dot order (kQ8Seq / kQ8Avx2 / kQ8Avx512 of qr_gemv.h, equal to
// QR_ORDER_*); it only changes Q8_0 weights.
size_t gemv_lds_bytes(int type, int q8o, int d, int nt, int R);
bool gemv_stream_ok(int type, int q8o, int d, int nt);
bool gemv_blk_ok(int type, int d, int nt);
int device_cus();
// Let kernel fn use up to 160 KiB of dynamic LDS on the current device (once
// per device; done[] is the caller's per-device flag array of 64 entries).
hipError_t lds_opt_in(const void* fn, std::atomic<bool>* done);
// Workgroups of `threads` threads that one CU holds at once by the kernel's
// registers and wave slots alone (the caller counts its dynamic LDS); asked of
// the runtime once per kernel and kept in `cache` (0 = not asked yet).
int resident_by_regs(const void* fn, int threads, std::atomic<int>& cache);
int gemv_rows_per_wg(int type, int q8o, int n, int d, int nt);
// R (one token only): Y = R + W X, the residual add of src/runtime.c:196-198
// and 282-284 in the GEMV's store (R may be Y).
hipError_t gemv_launch(int type, int q8o, const void* W, const float* X, float* Y, int n, int d,
                       int nt, int xstride, int ystride, int32_t* acc, int32_t* accb,
                       hipStream_t st, const float* R = nullptr);
// Tiled layout (qr_tiled.h, qr_tiled_sq.h): type is the base type (QR_T_Q4_K /
// QR_T_Q5_K / QR_T_Q6_K / QR_T_Q8_0).
// Q6_K / Q8_0 tiles (qr_tiled_sq.h) too; Q8_0 in the sequential dot order
// only (q8o, kQ8Seq = 0).
bool gemv_tiled_ok(int type, int n, int d, int nt, int q8o = 0);
hipError_t gemv_tiled_launch(int type, const void* W, const float* X, float* Y, int n, int d,
                             int nt, int xstride, int ystride, hipStream_t st, int q8o = 0,
                             const float* R = nullptr);
// One token of a tiled Q4_K / Q5_K matrix against rmsnorm_ref(x, nw) formed
// inside the launch (qr_norm.h); xb (optional) receives the normalised
// vector.  d <= kNormFuseMax.
bool gemv_tiled_norm_ok(int type, int d);
hipError_t gemv_tiled_norm_launch(int type, const void* W, const float* x, const float* nw,
                                  float* xb, float* Y, int n, int d, hipStream_t st);
// The same normalisation feeding two matrices in one launch: tiled Q4_K /
// Q5_K A (na rows into Ya; xb from its workgroup 0) and tiled Q6_K / Q8_0 B
// (nb rows into Yb; Q8_0 in the sequential dot order).
bool gemv_norm2_ok(int ta, int tb, int nb_rows, int d);
hipError_t gemv_norm2_launch(int ta, const void* Wa, float* Ya, int na, int tb, const void* Wb,
                             float* Yb, int nb, const float* x, const float* nw, float* xb, int d,
                             hipStream_t st);
hipError_t tile_pack_launch(int type, const void* src, void* dst, int n, int d, bool reverse,
                            hipStream_t st);
// llama.cpp / ggml K-quants (qr_ggml.h): type is 12 / 13 / 14 (Q4_K / Q5_K / Q6_K).
bool gemv_ggml_ok(int type, int d, int nt);
hipError_t gemv_ggml_launch(int type, const void* W, const float* X, float* Y, int n, int d, int nt,
                            int xstride, int ystride, hipStream_t st, const float* R = nullptr);
hipError_t quantize_q8k_launch(const float* x, void* y, long nblocks, hipStream_t st);
hipError_t gemv_ggml_pairs_launch(int type, const void* W, size_t eslice, const int32_t* eidx,
                                  int E, int xk, const float* X, int xstride, float* Y,
                                  int ystride, int n, int d, int P, hipStream_t st);
hipError_t ggml_dequant_launch(int type, const void* src, int rows, int n, float* out,
                               hipStream_t st);
hipError_t gemv_f32_launch(int order, const float* W, const float* X, float* Y, int n, int d,
                           int nt, int xstride, int ystride, hipStream_t st);
hipError_t quantize_q8_0_launch(const float* x, void* y, long nblocks, hipStream_t st);

// qr_moe.hip
struct MoeScratch {
  // Device buffers sized for T tokens (grown on demand by the runtime).
  float* logits;      // [T][E]
  int32_t* idx;       // [T][K]
  float* wts;         // [T][K]
  int32_t* counts;    // [E]
  int32_t* offsets;   // [E+1]
  int32_t* tiles;     // [E+1] exclusive scan of ceil(counts[e] / token tile)
  int32_t* perm;      // [T*K]
  int32_t* inv;       // [T*K]
  float* hb;          // [T*K][hidden]
  float* y;           // [T*K][dim]
  float* hbs;         // [T][sh_hidden]  shared expert
  float* ysh;         // [T][dim]        shared expert output
  float* sgl;         // [T]             shared expert gate logit
  uint8_t* xq;        // [T][dim/32] quantized activation records (MFMA path)
  uint8_t* hq;        // [T*K][hidden/32] quantized hb records (MFMA path)
  // the shared expert's own (empty without one)
  float* ush;         // [T][sh_hidden]  its up rows (GEMV path)
  uint8_t* xqs;       // [T][dim/32]     records of xb in its up type's order (MFMA path)
  uint8_t* hqs;       // [T][sh_hidden/32] records of its hb (MFMA path)
  int32_t* shoff;     // [2]   single-"expert" dispatch of the T tokens
  int32_t* shtiles;   // [2]
  int32_t* shperm;    // [T]
  float* hu;          // [T*K][hidden]  up rows of llama.cpp-layout experts (else null)
};
size_t moe_scratch_bytes(const qr_moe_layer* L, int T);
void moe_scratch_carve(void* base, const qr_moe_layer* L, int T, MoeScratch* s);
hipError_t moe_route_launch(const qr_moe_layer* L, const float* xb, int T, int order,
                            float* logits, float* probs, int32_t* idx, float* wts,
                            hipStream_t st);
hipError_t moe_dispatch_launch(const int32_t* idx, int T, int K, int E, int tile, int32_t* counts,
                               int32_t* offsets, int32_t* tiles, int32_t* perm, int32_t* inv,
                               hipStream_t st);
// path: QR_MOE_PATH_* (include/qr_hip.h); AUTO picks by the pairs per expert.
// norm_w (one token, where moe_t1_norm_ok): xb is written, not read -- the
// router's launch forms xb = rmsnorm_ref(x, norm_w) (src/kernels.c:170-180)
// before the layer uses it.
bool moe_t1_norm_ok(const qr_moe_layer* L, const float* x, const float* xb, const float* nw,
                    int order);
hipError_t moe_forward_launch(const qr_moe_layer* L, float* x, const float* xb, int T, int order,
                              const MoeScratch& s, hipStream_t st, int path = QR_MOE_PATH_AUTO,
                              const float* norm_w = nullptr);
hipError_t softmax_launch(float* x, int rows, int n, hipStream_t st);
// qr_decode.hip: a single-"expert" dispatch of T rows for the grouped MFMA
// product (offsets {0, T}, the identity permutation, tiles {0, ceil(T / tile)}).
hipError_t rows_dispatch_launch(int T, int tile, int32_t* off, int32_t* perm, int32_t* tiles,
                                hipStream_t st);

// qr_moe_t1.hip
bool router1_ok(int dim);
bool router1_norm_ok(int dim);
// Router logits of T tokens (grid E x T), and with W2 the sequential-order dot
// of the one row W2 with each token into out2[t] (E = 0: that dot alone).
// With nw (one token): xb is the residual x, normalised inside the launch
// (rmsnorm_ref with weights nw), the normalised vector stored at xb_out.
hipError_t router1_launch(int order, const float* W, const float* xb, int E, int d, float* logits,
                          hipStream_t st, int T = 1, const float* W2 = nullptr,
                          float* out2 = nullptr, const float* nw = nullptr,
                          float* xb_out = nullptr);
bool gateup1_ok(int type, int dim, int E, int K);
// With sh_up / sh_gate (the shared expert's rows, of the routed up type and
// width), its hb = silu(sh_up . xb) * (sh_gate . xb) into hbs as well.
hipError_t gateup1_launch(int type, const void* up, const void* gate, size_t slice, int dim,
                          int hidden, int E, int K, const float* xb, const float* logits,
                          int32_t* idx, float* wts, float* hb, hipStream_t st,
                          const void* sh_up = nullptr, const void* sh_gate = nullptr,
                          int sh_hidden = 0, float* hbs = nullptr);
bool down1v2_ok(int type, int K, int dim, int hidden);
hipError_t down1v2_launch(int type, const void* down, size_t slice, int dim, int hidden, int E,
                          int K, const float* hb, const int32_t* idx, const float* wts, float* x,
                          const float* ysh, const float* sgl, hipStream_t st);

// qr_moe_tn.hip
bool rlogits_ok(int d);
hipError_t rlogits_launch(int order, const float* W, const float* X, int T, int E, int d,
                          float* logits, hipStream_t st);
hipError_t route_rank_launch(const float* logits, int T, int E, int K, float* probs, int32_t* idx,
                             float* wts, const float* X, int d, bool perm, uint8_t* XQ,
                             hipStream_t st);

// qr_moe_mfma.hip
bool mfma_type_ok(int type);
hipError_t quant_rows_launch(const float* x, int xstride, int nrows, int cols, bool perm,
                             uint8_t* out, hipStream_t st);
// Pairs per work item of the grouped MFMA products for T tokens (the
// dispatch's tile size).
int mfma_tile(int T, int K, int E);
hipError_t expert_mfma_launch(int type, bool gateup, const uint8_t* W1, const uint8_t* W2,
                              size_t slice, int E, int K, int rows, int cols, const uint8_t* XQ,
                              int x_by_token, const int32_t* offsets, const int32_t* perm,
                              const int32_t* tiles, float* Y, int ystride, int items, int tile,
                              uint8_t* QO, bool qperm, hipStream_t st, bool tiled = false);

}  // namespace qr
