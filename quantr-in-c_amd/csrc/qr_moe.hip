// qr_moe.hip -- the MoE layer of quantr-in-c (src/runtime.c:202-269) for T
// tokens on gfx950, bit-exact with the reference's per-token block:
//
//   logits  = W_r . xb          (KernelOps.matmul order: SEQ / AVX2 / AVX512)
//   probs   = softmax_ref(logits)                       src/kernels.c:191-207
//   idx,w   = K argmax passes, strict '>', mask -1e9f   src/runtime.c:208-222
//   w      /= sequential sum of w                       src/runtime.c:224-230
//   per slot k:  hb = silu(up_e . xb) * (gate_e . xb)   src/runtime.c:252-256
//                y  = down_e . hb   (hb re-quantised)   src/runtime.c:259-260
//                xb2 += y * w_k     (slot order)        src/runtime.c:262-264
//   x += xb2                                            src/runtime.c:267-269
//
// Kernels:
//   k_route_topk     one wave per token: softmax (glibc-exact expf), top-K,
//                    renormalisation.
//   k_dispatch       T > 1: histogram, exclusive scan and a stable permute of
//                    the T*K (token, slot) pairs by expert; ranks come from
//                    wave ballots and per-wave counts, never from the order in
//                    which atomics land.
//   k_expert         grouped GEMV over (row tile, work item); a work item is
//                    up to NT pairs of one expert, so each weight tile is
//                    read once for NT tokens.  Gate/up mode runs both
//                    matrices and writes silu(up) * gate.
//   k_down_combine1  T == 1: all K down projections of the token plus the
//                    slot-order combine (and the shared expert) in one pass.
//   k_combine        T > 1: slot-order gather-combine.
// llama.cpp-layout experts (ggml K-quants) take ggml's Q8_K dot instead: the
// routing, then the ggml GEMV in pair mode (qr_ggml.h; one matrix-vector
// product per (token, slot) pair, the pair's expert chosen on the device) for
// up, gate and down, k_silu_mul between them, and k_combine.
#include <cstdlib>

#include "qr_gemv.h"
#include "qr_internal.h"
#include "qr_route.h"
#include "qr_tokens.h"

namespace qr {

// ---------------------------------------------------------------------------
// Scratch.
// ---------------------------------------------------------------------------
static size_t a256(size_t v) { return (v + 255) & ~(size_t)255; }

size_t moe_scratch_bytes(const qr_moe_layer* L, int T) {
  const size_t E = L->n_experts, K = L->n_used, P = (size_t)T * K;
  size_t b = 0;
  b += a256(T * E * 4);            // logits
  b += a256(P * 4) * 2;            // idx, wts
  b += a256(E * 4);                // counts
  b += a256((E + 1) * 4) * 2;      // offsets, tiles
  b += a256(P * 4) * 2;            // perm, inv
  b += a256(P * (size_t)L->hidden * 4);
  b += a256(P * (size_t)L->dim * 4);
  const size_t sh = L->sh_hidden > 0 ? (size_t)L->sh_hidden : 0;
  b += a256((size_t)T * (sh ? sh : 1) * 4);
  b += a256((size_t)T * L->dim * 4);
  b += a256((size_t)T * 4);
  b += a256((size_t)T * (L->dim / 32) * 48);
  b += a256(P * (size_t)(L->hidden / 32) * 48);
  if (sh) {
    b += a256((size_t)T * sh * 4);                  // ush
    b += a256((size_t)T * (L->dim / 32) * 48);      // xqs
    b += a256((size_t)T * (sh / 32) * 48);          // hqs
    b += a256(2 * 4) * 2 + a256((size_t)T * 4);     // shoff, shtiles, shperm
  }
  if (L->up_type & QR_GGML) b += a256(P * (size_t)L->hidden * 4);  // hu
  return b;
}

void moe_scratch_carve(void* base, const qr_moe_layer* L, int T, MoeScratch* s) {
  const size_t E = L->n_experts, K = L->n_used, P = (size_t)T * K;
  uint8_t* p = static_cast<uint8_t*>(base);
  auto take = [&](size_t bytes) {
    uint8_t* r = p;
    p += a256(bytes);
    return r;
  };
  s->logits = reinterpret_cast<float*>(take(T * E * 4));
  s->idx = reinterpret_cast<int32_t*>(take(P * 4));
  s->wts = reinterpret_cast<float*>(take(P * 4));
  s->counts = reinterpret_cast<int32_t*>(take(E * 4));
  s->offsets = reinterpret_cast<int32_t*>(take((E + 1) * 4));
  s->tiles = reinterpret_cast<int32_t*>(take((E + 1) * 4));
  s->perm = reinterpret_cast<int32_t*>(take(P * 4));
  s->inv = reinterpret_cast<int32_t*>(take(P * 4));
  s->hb = reinterpret_cast<float*>(take(P * (size_t)L->hidden * 4));
  s->y = reinterpret_cast<float*>(take(P * (size_t)L->dim * 4));
  const size_t sh = L->sh_hidden > 0 ? (size_t)L->sh_hidden : 0;
  s->hbs = reinterpret_cast<float*>(take((size_t)T * (sh ? sh : 1) * 4));
  s->ysh = reinterpret_cast<float*>(take((size_t)T * L->dim * 4));
  s->sgl = reinterpret_cast<float*>(take((size_t)T * 4));
  s->xq = take((size_t)T * (L->dim / 32) * 48);
  s->hq = take(P * (size_t)(L->hidden / 32) * 48);
  s->ush = nullptr;
  s->xqs = s->hqs = nullptr;
  s->shoff = s->shtiles = s->shperm = nullptr;
  if (sh) {
    s->ush = reinterpret_cast<float*>(take((size_t)T * sh * 4));
    s->xqs = take((size_t)T * (L->dim / 32) * 48);
    s->hqs = take((size_t)T * (sh / 32) * 48);
    s->shoff = reinterpret_cast<int32_t*>(take(2 * 4));
    s->shtiles = reinterpret_cast<int32_t*>(take(2 * 4));
    s->shperm = reinterpret_cast<int32_t*>(take((size_t)T * 4));
  }
  s->hu = nullptr;
  if (L->up_type & QR_GGML) s->hu = reinterpret_cast<float*>(take(P * (size_t)L->hidden * 4));
}

// ---------------------------------------------------------------------------
// Router: softmax + top-K + renormalisation, one wave per token, no
// workgroup barriers (each wave owns its LDS row).
// ---------------------------------------------------------------------------
constexpr int kRouteWaves = 4;

__global__ __launch_bounds__(64 * kRouteWaves) void k_route_topk(const float* __restrict__ logits,
                                                                  int T, int E, int K,
                                                                  float* __restrict__ probs,
                                                                  int32_t* __restrict__ idx,
                                                                  float* __restrict__ wts) {
  __shared__ __align__(16) float P[kRouteWaves][kRouteRow];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * kRouteWaves + wave;
  if (t >= T) return;  // whole wave; no workgroup barriers below
  route_one(logits + (size_t)t * E, E, K, P[wave], lane, probs ? probs + (size_t)t * E : nullptr,
            idx + (size_t)t * K, wts + (size_t)t * K);
}

hipError_t moe_route_launch(const qr_moe_layer* L, const float* xb, int T, int order,
                            float* logits, float* probs, int32_t* idx, float* wts,
                            hipStream_t st) {
  const int E = L->n_experts;
  hipError_t e;
  if (T <= 0) return hipSuccess;
  if (rlogits_ok(L->dim) && E <= 256 && L->n_used <= 16 &&
      (reinterpret_cast<uintptr_t>(L->router) & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(xb) & 15) == 0) {
    // tiled logits (qr_moe_tn.hip), then one workgroup per token ranks the top K
    e = rlogits_launch(order, L->router, xb, T, E, L->dim, logits, st);
    if (e != hipSuccess) return e;
    return route_rank_launch(logits, T, E, L->n_used, probs, idx, wts, xb, L->dim, false,
                             nullptr, st);
  }
  e = gemv_f32_launch(order, L->router, xb, logits, E, L->dim, T, L->dim, E, st);
  if (e != hipSuccess) return e;
  const int grid = (T + kRouteWaves - 1) / kRouteWaves;
  hipLaunchKernelGGL(k_route_topk, dim3(grid), dim3(64 * kRouteWaves), 0, st, logits, T, E,
                     L->n_used, probs, idx, wts);
  return hipGetLastError();
}

// softmax_ref rows (the KernelOps.softmax drop-in): one wave per row.
__global__ __launch_bounds__(256) void k_softmax(float* __restrict__ x, int rows, int n) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + wave;
  if (r >= rows) return;  // no barriers below
  float* p = x + (size_t)r * n;
  float mx = p[0];
  for (int e = lane; e < n; e += 64)
    if (p[e] > mx) mx = p[e];
  for (int o = 32; o > 0; o >>= 1) {
    const float v = __shfl_xor(mx, o);
    if (v > mx) mx = v;
  }
  for (int e = lane; e < n; e += 64) p[e] = qr_expf(p[e] - mx);
  // the sequential sum runs in lane 0 over values written by this wave; make
  // them visible to it first
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  __builtin_amdgcn_wave_barrier();
  float inv = 0.0f;
  if (lane == 0) {
    float sum = 0.0f;
    for (int e = 0; e < n; e++) sum += p[e];
    inv = 1.0f / sum;
  }
  inv = __shfl(inv, 0);
  for (int e = lane; e < n; e += 64) p[e] *= inv;
}

hipError_t softmax_launch(float* x, int rows, int n, hipStream_t st) {
  hipLaunchKernelGGL(k_softmax, dim3((rows + 3) / 4), dim3(256), 0, st, x, rows, n);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Dispatch: one workgroup of kDispThreads threads (qr_tokens.h).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kDispThreads) void k_dispatch(const int32_t* __restrict__ idx, int P,
                                                           int E, int tile,
                                                           int32_t* __restrict__ counts,
                                                           int32_t* __restrict__ offsets,
                                                           int32_t* __restrict__ tiles,
                                                           int32_t* __restrict__ perm,
                                                           int32_t* __restrict__ inv) {
  dispatch_wg(idx, P, E, tile, counts, offsets, tiles, perm, inv);
}

hipError_t moe_dispatch_launch(const int32_t* idx, int T, int K, int E, int tile, int32_t* counts,
                               int32_t* offsets, int32_t* tiles, int32_t* perm, int32_t* inv,
                               hipStream_t st) {
  if (E > 256) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(kDispThreads), 0, st, idx, T * K, E, tile, counts,
                     offsets, tiles, perm, inv);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Grouped expert GEMV.
// ---------------------------------------------------------------------------
enum { kModeSingle = 0, kModeDispatched = 1, kModeDense = 2 };

struct ExpertArgs {
  const uint8_t* W1;   // [E][rows][rb]  (up in gate/up mode)
  const uint8_t* W2;   // [E][rows][rb]  (gate in gate/up mode)
  size_t slice;        // bytes per expert (0: one dense expert)
  int rows, cols, rows_per_wg;
  const float* X;      // activation rows
  int xstride;
  float* Y;            // output rows, one per pair position
  int ystride;
  int mode;
  int x_by_token;      // dispatched mode: activation row = perm[p] / K (else p)
  const int32_t* idx;
  const int32_t* offsets;
  const int32_t* perm;
  const int32_t* tiles;
  int E, K, P;
};

__host__ __device__ inline size_t expert_lds_layout(int type, int q8o, int cols, int nt, int R,
                                                    int nmat, size_t* o_bd, size_t* o_bs,
                                                    size_t* o_terms, size_t* o_tile,
                                                    size_t* o_rows, size_t* tile_stride) {
  const int nxb = cols / 32;
  const int U = qr_units(type, cols);
  size_t off = align16((size_t)nt * nxb * 32);
  *o_bd = off;
  off = align16(off + (size_t)nt * nxb * 4);
  *o_bs = off;
  off = align16(off + (size_t)nt * nxb * 4);
  *o_rows = off;
  off = align16(off + (size_t)nt * 4);
  *o_terms = off;
  off = align16(off + (size_t)nmat * nt * R * q8_slots(type, q8o) * (U + 1) * 4);
  *o_tile = off;
  *tile_stride = 0;
  if (type == QR_T_Q8_0 || type == QR_T_Q6_K) {
    *tile_stride = stage_bytes((size_t)R * qr_wrow_bytes(type, cols));
    off += (size_t)nmat * *tile_stride;
  }
  return off;
}

// Resolve a work item to (expert, first pair, pair count).  Returns false if
// the item is past the end of the work.
__device__ inline bool expert_item(const ExpertArgs& a, int item, int NT, int* e, int* p0,
                                   int* np) {
  if (a.mode == kModeSingle) {
    if (item >= a.K) return false;
    *e = a.idx[item];
    *p0 = item;
    *np = 1;
  } else if (a.mode == kModeDense) {
    *p0 = item * NT;
    if (*p0 >= a.P) return false;
    *e = 0;
    *np = min(NT, a.P - *p0);
  } else {
    const int ntiles = a.tiles[a.E];
    if (item >= ntiles) return false;
    int lo = 0, hi = a.E;  // largest e with tiles[e] <= item
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (a.tiles[mid] <= item) lo = mid;
      else hi = mid;
    }
    *e = lo;
    *p0 = a.offsets[lo] + (item - a.tiles[lo]) * NT;
    *np = min(NT, a.offsets[lo + 1] - *p0);
  }
  return *e >= 0 && *e < a.E && *np > 0;
}

template <int TYPE, int NT, bool GATEUP, int Q8O>
__global__ __launch_bounds__(256) void k_expert(ExpertArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  int e, p0, np;
  if (!expert_item(a, blockIdx.y, NT, &e, &p0, &np)) return;  // uniform per workgroup
  const int R0 = a.rows_per_wg;
  const int r0 = blockIdx.x * R0;
  const int R = min(R0, a.rows - r0);
  if (R <= 0) return;
  constexpr int NMAT = GATEUP ? 2 : 1;
  const int cols = a.cols;
  const int U = qr_units(TYPE, cols);
  const size_t rb = qr_wrow_bytes(TYPE, cols);
  size_t o_bd, o_bs, o_terms, o_tile, o_rows, tstr;
  expert_lds_layout(TYPE, Q8O, cols, NT, R0, NMAT, &o_bd, &o_bs, &o_terms, &o_tile, &o_rows,
                    &tstr);
  constexpr int SL = q8_slots(TYPE, Q8O);
  UnitSrc S;
  S.act.q = reinterpret_cast<int8_t*>(smem);
  S.act.bd = reinterpret_cast<float*>(smem + o_bd);
  S.act.bs = reinterpret_cast<int32_t*>(smem + o_bs);
  S.nxb = cols >> 5;
  int* rowmap = reinterpret_cast<int*>(smem + o_rows);
  float* terms = reinterpret_cast<float*>(smem + o_terms);
  const int tstride = U + 1;

  const uint8_t* Wm[2] = {a.W1 + (size_t)e * a.slice, GATEUP ? a.W2 + (size_t)e * a.slice : nullptr};
  const size_t gstart = (size_t)r0 * rb;
  const size_t mtotal = (size_t)a.rows * rb;
  if constexpr (!Fmt<TYPE>::kDirect) {
    for (int m = 0; m < NMAT; m++)
      stage_tile(Wm[m], mtotal, gstart, gstart + (size_t)R * rb,
                 reinterpret_cast<uint32_t*>(smem + o_tile + m * tstr));
  }
  if (threadIdx.x < NT) {
    const int t = threadIdx.x;
    int row = 0;
    if (t < np) {
      const int p = p0 + t;
      row = (a.mode == kModeDispatched && a.x_by_token) ? a.perm[p] / a.K
            : (a.mode == kModeSingle ? 0 : p);
    }
    rowmap[t] = row;
  }
  __syncthreads();
  quantize_act_lds<Fmt<TYPE>::kPerm>(a.X, (size_t)a.xstride, rowmap, np, NT, cols, S.act);
  __syncthreads();

  const int lds_base = (int)(gstart & 15);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nwaves = blockDim.x >> 6;
  const int per_mat = R * U;
  for (int fu = wave * 64 + lane; fu < NMAT * per_mat; fu += nwaves * 64) {
    const int m = fu / per_mat;
    const int rem = fu - m * per_mat;
    const int row = rem / U;
    const int u = rem - row * U;
    UnitSrc Sm = S;
    Sm.tile = reinterpret_cast<const uint32_t*>(smem + o_tile + m * tstr);
    int32_t is[NT];
    unit_to_slots<TYPE, NT, Q8O>(Wm[m] + gstart + (size_t)row * rb, lds_base + row * (int)rb, u,
                                 Sm, 0, terms + (((size_t)m * NT) * R0 + row) * SL * tstride,
                                 (size_t)R0 * SL * tstride, tstride, is);
  }
  __syncthreads();

  for (int i = threadIdx.x; i < np * R; i += blockDim.x) {
    const int t = i / R, row = i - t * R;
    const float v1 = row_value<TYPE, Q8O>(terms + ((size_t)t * R0 + row) * SL * tstride, tstride, U);
    float out = v1;
    if constexpr (GATEUP) {
      const float v2 = row_value<TYPE, Q8O>(
          terms + (((size_t)NT + t) * R0 + row) * SL * tstride, tstride, U);
      out = qr_silu(v1) * v2;
    }
    a.Y[(size_t)(p0 + t) * a.ystride + r0 + row] = out;
  }
}

static int expert_rows_per_wg(int type, int q8o, int rows, int cols, int nt, int nmat) {
  const int U = qr_units(type, cols);
  int R = 64;
  size_t a, b, c, d, e, f;
  while (R > 1 && ((size_t)nmat * R * U > 16 * 256 ||
                   expert_lds_layout(type, q8o, cols, nt, R, nmat, &a, &b, &c, &d, &e, &f) >
                       48 * 1024 ||
                   (rows + R - 1) / R < 64))
    R >>= 1;
  return R;
}

template <int TYPE, int NT, bool GATEUP, int Q8O>
static hipError_t expert_launch_t(ExpertArgs a, int items, hipStream_t st) {
  constexpr int NMAT = GATEUP ? 2 : 1;
  a.rows_per_wg = expert_rows_per_wg(TYPE, Q8O, a.rows, a.cols, NT, NMAT);
  size_t o1, o2, o3, o4, o5, o6;
  const size_t lds = expert_lds_layout(TYPE, Q8O, a.cols, NT, a.rows_per_wg, NMAT, &o1, &o2, &o3,
                                       &o4, &o5, &o6);
  const int U = qr_units(TYPE, a.cols);
  int threads = ((NMAT * a.rows_per_wg * U + 63) / 64) * 64;
  threads = threads < 64 ? 64 : (threads > 256 ? 256 : threads);
  dim3 grid((a.rows + a.rows_per_wg - 1) / a.rows_per_wg, items);
  if (grid.x == 0 || grid.y == 0) return hipSuccess;
  if (lds > 64 * 1024) return hipErrorInvalidValue;  // dynamic LDS without an opt-in
  hipLaunchKernelGGL((k_expert<TYPE, NT, GATEUP, Q8O>), grid, dim3(threads), lds, st, a);
  return hipGetLastError();
}

template <int TYPE, bool GATEUP, int Q8O>
static hipError_t expert_launch_nt(const ExpertArgs& a, int nt, int items, hipStream_t st) {
  switch (nt) {
    case 1: return expert_launch_t<TYPE, 1, GATEUP, Q8O>(a, items, st);
    case 2: return expert_launch_t<TYPE, 2, GATEUP, Q8O>(a, items, st);
    case 4: return expert_launch_t<TYPE, 4, GATEUP, Q8O>(a, items, st);
    case 8: return expert_launch_t<TYPE, 8, GATEUP, Q8O>(a, items, st);
    default: return hipErrorInvalidValue;
  }
}

template <int TYPE, int Q8O>
static hipError_t expert_launch_g(bool gateup, const ExpertArgs& a, int nt, int items,
                                  hipStream_t st) {
  return gateup ? expert_launch_nt<TYPE, true, Q8O>(a, nt, items, st)
                : expert_launch_nt<TYPE, false, Q8O>(a, nt, items, st);
}

// q8o: the Q8_0 dot order (kQ8Seq / kQ8Avx2 / kQ8Avx512); other types ignore it.
static hipError_t expert_launch(int type, int q8o, bool gateup, const ExpertArgs& a, int nt,
                                int items, hipStream_t st) {
  switch (type) {
    case QR_T_Q4_K: return expert_launch_g<QR_T_Q4_K, kQ8Seq>(gateup, a, nt, items, st);
    case QR_T_Q5_K: return expert_launch_g<QR_T_Q5_K, kQ8Seq>(gateup, a, nt, items, st);
    case QR_T_Q6_K: return expert_launch_g<QR_T_Q6_K, kQ8Seq>(gateup, a, nt, items, st);
    case QR_T_Q8_0:
      switch (q8o) {
        case kQ8Seq: return expert_launch_g<QR_T_Q8_0, kQ8Seq>(gateup, a, nt, items, st);
        case kQ8Avx2: return expert_launch_g<QR_T_Q8_0, kQ8Avx2>(gateup, a, nt, items, st);
        case kQ8Avx512: return expert_launch_g<QR_T_Q8_0, kQ8Avx512>(gateup, a, nt, items, st);
        default: return hipErrorInvalidValue;
      }
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------
// T == 1: the K down projections of one token plus the slot-order combine.
// A workgroup owns R rows of every selected expert's down matrix.
// ---------------------------------------------------------------------------
struct DownArgs {
  const uint8_t* W;    // [E][dim][rb]
  size_t slice;
  int dim, hidden, rows_per_wg, K, E;
  const float* hb;     // [K][hidden]
  const int32_t* idx;  // [K]
  const float* wts;    // [K]
  float* x;            // [dim], updated in place
  const float* ysh;    // optional shared-expert output [dim]
  const float* sgl;    // its gate logit (scalar)
};

__host__ __device__ inline size_t down1_lds_layout(int type, int q8o, int hidden, int K, int R,
                                                   size_t* o_bd, size_t* o_bs, size_t* o_terms,
                                                   size_t* o_tile, size_t* tile_stride) {
  const int nxb = hidden / 32;
  const int U = qr_units(type, hidden);
  size_t off = align16((size_t)K * nxb * 32);
  *o_bd = off;
  off = align16(off + (size_t)K * nxb * 4);
  *o_bs = off;
  off = align16(off + (size_t)K * nxb * 4);
  *o_terms = off;
  off = align16(off + (size_t)K * R * q8_slots(type, q8o) * (U + 1) * 4);
  *o_tile = off;
  *tile_stride = 0;
  if (type == QR_T_Q8_0 || type == QR_T_Q6_K) {
    *tile_stride = stage_bytes((size_t)R * qr_wrow_bytes(type, hidden));
    off += (size_t)K * *tile_stride;
  }
  return off;
}

template <int TYPE, int Q8O>
__global__ __launch_bounds__(256) void k_down_combine1(DownArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int R0 = a.rows_per_wg;
  const int r0 = blockIdx.x * R0;
  const int R = min(R0, a.dim - r0);
  if (R <= 0) return;
  const int K = a.K;
  const int U = qr_units(TYPE, a.hidden);
  const size_t rb = qr_wrow_bytes(TYPE, a.hidden);
  size_t o_bd, o_bs, o_terms, o_tile, tstr;
  down1_lds_layout(TYPE, Q8O, a.hidden, K, R0, &o_bd, &o_bs, &o_terms, &o_tile, &tstr);
  constexpr int SL = q8_slots(TYPE, Q8O);
  UnitSrc S;
  S.act.q = reinterpret_cast<int8_t*>(smem);
  S.act.bd = reinterpret_cast<float*>(smem + o_bd);
  S.act.bs = reinterpret_cast<int32_t*>(smem + o_bs);
  S.nxb = a.hidden >> 5;
  float* terms = reinterpret_cast<float*>(smem + o_terms);
  const int tstride = U + 1;
  const size_t gstart = (size_t)r0 * rb;
  const size_t mtotal = (size_t)a.dim * rb;
  // A slot whose index is out of range (only NaN router inputs produce one)
  // contributes nothing and its weights are never touched.
  auto valid = [&](int k) { return a.idx[k] >= 0 && a.idx[k] < a.E; };
  if constexpr (!Fmt<TYPE>::kDirect) {
    for (int k = 0; k < K; k++) {
      if (!valid(k)) continue;
      const uint8_t* Wk = a.W + (size_t)a.idx[k] * a.slice;
      stage_tile(Wk, mtotal, gstart, gstart + (size_t)R * rb,
                 reinterpret_cast<uint32_t*>(smem + o_tile + k * tstr));
    }
  }
  quantize_act_lds<Fmt<TYPE>::kPerm>(a.hb, (size_t)a.hidden, nullptr, K, K, a.hidden, S.act);
  __syncthreads();

  const int lds_base = (int)(gstart & 15);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nwaves = blockDim.x >> 6;
  const int per_k = R * U;
  for (int fu = wave * 64 + lane; fu < K * per_k; fu += nwaves * 64) {
    const int k = fu / per_k;
    const int rem = fu - k * per_k;
    const int row = rem / U;
    const int u = rem - row * U;
    int32_t is[1];
    if (valid(k)) {  // an invalid slot's terms are never read
      UnitSrc Sk = S;
      Sk.tile = reinterpret_cast<const uint32_t*>(smem + o_tile + k * tstr);
      const uint8_t* Wk = a.W + (size_t)a.idx[k] * a.slice;
      unit_to_slots<TYPE, 1, Q8O>(Wk + gstart + (size_t)row * rb, lds_base + row * (int)rb, u, Sk,
                                  k, terms + ((size_t)k * R0 + row) * SL * tstride, 0, tstride,
                                  is);
    }
  }
  __syncthreads();

  for (int row = threadIdx.x; row < R; row += blockDim.x) {
    float acc = 0.0f;  // xb2 = 0 (src/runtime.c:242)
    for (int k = 0; k < K; k++) {
      if (!valid(k)) continue;
      const float y =
          row_value<TYPE, Q8O>(terms + ((size_t)k * R0 + row) * SL * tstride, tstride, U);
      acc += y * a.wts[k];
    }
    if (a.ysh) {
      const float sg = 1.0f / (1.0f + qr_expf(-a.sgl[0]));
      acc += sg * a.ysh[r0 + row];
    }
    a.x[r0 + row] += acc;
  }
}

static int down1_rows_per_wg(int type, int q8o, int dim, int hidden, int K) {
  const int U = qr_units(type, hidden);
  int R = 64;
  size_t a, b, c, d, e;
  while (R > 1 && ((size_t)K * R * U > 16 * 256 ||
                   down1_lds_layout(type, q8o, hidden, K, R, &a, &b, &c, &d, &e) > 48 * 1024 ||
                   (dim + R - 1) / R < 256))
    R >>= 1;
  return R;
}

template <int TYPE, int Q8O>
static hipError_t down1_launch_t(DownArgs a, hipStream_t st) {
  a.rows_per_wg = down1_rows_per_wg(TYPE, Q8O, a.dim, a.hidden, a.K);
  size_t o1, o2, o3, o4, o5;
  const size_t lds =
      down1_lds_layout(TYPE, Q8O, a.hidden, a.K, a.rows_per_wg, &o1, &o2, &o3, &o4, &o5);
  const int U = qr_units(TYPE, a.hidden);
  int threads = ((a.K * a.rows_per_wg * U + 63) / 64) * 64;
  threads = threads < 64 ? 64 : (threads > 256 ? 256 : threads);
  const int grid = (a.dim + a.rows_per_wg - 1) / a.rows_per_wg;
  if (lds > 64 * 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL((k_down_combine1<TYPE, Q8O>), dim3(grid), dim3(threads), lds, st, a);
  return hipGetLastError();
}

static hipError_t down1_launch(int type, int q8o, const DownArgs& a, hipStream_t st) {
  switch (type) {
    case QR_T_Q4_K: return down1_launch_t<QR_T_Q4_K, kQ8Seq>(a, st);
    case QR_T_Q5_K: return down1_launch_t<QR_T_Q5_K, kQ8Seq>(a, st);
    case QR_T_Q6_K: return down1_launch_t<QR_T_Q6_K, kQ8Seq>(a, st);
    case QR_T_Q8_0:
      switch (q8o) {
        case kQ8Seq: return down1_launch_t<QR_T_Q8_0, kQ8Seq>(a, st);
        case kQ8Avx2: return down1_launch_t<QR_T_Q8_0, kQ8Avx2>(a, st);
        case kQ8Avx512: return down1_launch_t<QR_T_Q8_0, kQ8Avx512>(a, st);
        default: return hipErrorInvalidValue;
      }
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------
// T > 1 combine: x[t][i] += ((0 + y_0 w_0) + y_1 w_1 + ...) (+ shared), the
// expert outputs gathered from their dispatch positions in slot order
// (src/runtime.c:262-269).  Four outputs per thread: the token's K positions
// and weights first, then all K rows' float4s, then the adds in slot order.
// ---------------------------------------------------------------------------
constexpr int kCombineMaxK = 16;

__global__ __launch_bounds__(256) void k_combine(float* __restrict__ x, const float* __restrict__ y,
                                                 const int32_t* __restrict__ inv,
                                                 const float* __restrict__ wts, int T, int K,
                                                 int dim, const float* __restrict__ ysh,
                                                 const float* __restrict__ sgl) {
  const int d4 = dim >> 2;
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (long)T * d4) return;
  const int t = (int)(gid / d4), i4 = (int)(gid - (long)t * d4);
  int pos[kCombineMaxK];
  float w[kCombineMaxK];
#pragma unroll
  for (int k = 0; k < kCombineMaxK; k++) {
    pos[k] = k < K ? inv[t * K + k] : -1;
    w[k] = k < K ? wts[t * K + k] : 0.0f;
  }
  float4 v[kCombineMaxK];
#pragma unroll
  for (int k = 0; k < kCombineMaxK; k++)
    if (pos[k] >= 0) v[k] = reinterpret_cast<const float4*>(y + (size_t)pos[k] * dim)[i4];
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int k = 0; k < kCombineMaxK; k++) {
    if (pos[k] >= 0) {
      acc.x += v[k].x * w[k];
      acc.y += v[k].y * w[k];
      acc.z += v[k].z * w[k];
      acc.w += v[k].w * w[k];
    }
  }
  if (ysh) {
    const float sg = 1.0f / (1.0f + qr_expf(-sgl[t]));
    const float4 s4 = reinterpret_cast<const float4*>(ysh + (size_t)t * dim)[i4];
    acc.x += sg * s4.x;
    acc.y += sg * s4.y;
    acc.z += sg * s4.z;
    acc.w += sg * s4.w;
  }
  float4* xp = reinterpret_cast<float4*>(x + (size_t)t * dim) + i4;
  float4 xv = *xp;
  xv.x += acc.x;
  xv.y += acc.y;
  xv.z += acc.z;
  xv.w += acc.w;
  *xp = xv;
}

static hipError_t combine_launch(float* x, const float* y, const int32_t* inv, const float* wts,
                                 int T, int K, int dim, const float* ysh, const float* sgl,
                                 hipStream_t st) {
  if (K > kCombineMaxK || (dim & 3)) return hipErrorInvalidValue;
  const long n4 = (long)T * (dim >> 2);
  hipLaunchKernelGGL(k_combine, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, x, y, inv,
                     wts, T, K, dim, ysh, sgl);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// The layer.
// ---------------------------------------------------------------------------

static int pick_tile(int P, int E) {
  const double avg = (double)P / E;
  return avg >= 6 ? 8 : avg >= 3 ? 4 : avg >= 1.5 ? 2 : 1;
}

// hb = silu(up . x) * (gate . x) of the shared expert's rows, from its up and
// gate GEMV outputs (the gate/up products' own output formula).
__global__ __launch_bounds__(256) void k_silu_mul(const float* __restrict__ u, float* __restrict__ g,
                                                  long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    g[i] = qr_silu(u[i]) * g[i];
}

static bool sh_gemv_type(int type) {
  return type == QR_T_Q4_K || type == QR_T_Q5_K || type == QR_T_Q6_K || type == QR_T_Q8_0;
}
static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// The shared expert (a dense FFN every token takes) and its gate logit.  Its
// dots are the routed experts' (C99 Q8_0 order, sequential gate logit):
//   T <= 4  three GEMVs (up, gate, down) of T tokens on the GEMV engines and
//           the silu product between them;
//   T > 4   the grouped int8 MFMA products with one "expert" (the T tokens
//           dispatched in order), gate/up leaving the down product's records;
//   else    the grouped GEMV in dense mode.
static hipError_t shared_expert(const qr_moe_layer* L, const float* xb, int T, const MoeScratch& s,
                                hipStream_t st, bool gate_done = false, bool hbs_done = false) {
  const int dim = L->dim, sh = L->sh_hidden;
  const int ut = (int)L->sh_up_type, dt = (int)L->sh_down_type;
  hipError_t e;
  const bool same_up = L->sh_gate_type == L->sh_up_type;
  const bool aligned = al16(L->sh_up) && al16(L->sh_gate) && al16(L->sh_down) && al16(xb);
  if (T <= 4 && same_up && aligned && sh_gemv_type(ut) && sh_gemv_type(dt) &&
      dim % qr_block_elems(ut) == 0 && sh % qr_block_elems(dt) == 0) {
    if (!hbs_done) {  // else the one-token gate/up launch wrote hbs
      if ((e = gemv_launch(ut, kQ8Seq, L->sh_up, xb, s.ush, sh, dim, T, dim, sh, nullptr, nullptr,
                           st)) != hipSuccess)
        return e;
      if ((e = gemv_launch(ut, kQ8Seq, L->sh_gate, xb, s.hbs, sh, dim, T, dim, sh, nullptr,
                           nullptr, st)) != hipSuccess)
        return e;
      const long n = (long)T * sh;
      hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, s.ush,
                         s.hbs, n);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if ((e = gemv_launch(dt, kQ8Seq, L->sh_down, s.hbs, s.ysh, dim, sh, T, sh, dim, nullptr,
                         nullptr, st)) != hipSuccess)
      return e;
  } else if (T > 4 && same_up && aligned && mfma_type_ok(ut) && mfma_type_ok(dt) &&
             dim % qr_block_elems(ut) == 0 && sh % 32 == 0 && sh % qr_block_elems(dt) == 0) {
    const int tile = mfma_tile(T, 1, 1);
    const int items = (T + tile - 1) / tile + 1;
    if ((e = rows_dispatch_launch(T, tile, s.shoff, s.shperm, s.shtiles, st)) != hipSuccess)
      return e;
    if ((e = quant_rows_launch(xb, dim, T, dim, ut != QR_T_Q8_0, s.xqs, st)) != hipSuccess) return e;
    const size_t su = qr_wrow_bytes(ut, dim) * (size_t)sh;
    const size_t sd = qr_wrow_bytes(dt, sh) * (size_t)dim;
    e = expert_mfma_launch(ut, true, static_cast<const uint8_t*>(L->sh_up),
                           static_cast<const uint8_t*>(L->sh_gate), su, 1, 1, sh, dim, s.xqs, 0,
                           s.shoff, s.shperm, s.shtiles, s.hbs, sh, items, tile, s.hqs,
                           dt != QR_T_Q8_0, st);
    if (e != hipSuccess) return e;
    e = expert_mfma_launch(dt, false, static_cast<const uint8_t*>(L->sh_down), nullptr, sd, 1, 1,
                           dim, sh, s.hqs, 0, s.shoff, s.shperm, s.shtiles, s.ysh, dim, items, tile,
                           nullptr, false, st);
    if (e != hipSuccess) return e;
  } else {
    const int nt = T >= 8 ? 8 : T >= 4 ? 4 : T >= 2 ? 2 : 1;
    ExpertArgs g{};
    g.W1 = static_cast<const uint8_t*>(L->sh_up);
    g.W2 = static_cast<const uint8_t*>(L->sh_gate);
    g.slice = 0;
    g.rows = sh;
    g.cols = dim;
    g.X = xb;
    g.xstride = dim;
    g.Y = s.hbs;
    g.ystride = sh;
    g.mode = kModeDense;
    g.E = 1;
    g.K = 1;
    g.P = T;
    e = expert_launch(ut, kQ8Seq, true, g, nt, (T + nt - 1) / nt, st);
    if (e != hipSuccess) return e;
    ExpertArgs dn = g;
    dn.W1 = static_cast<const uint8_t*>(L->sh_down);
    dn.W2 = nullptr;
    dn.rows = dim;
    dn.cols = sh;
    dn.X = s.hbs;
    dn.xstride = sh;
    dn.Y = s.ysh;
    dn.ystride = dim;
    e = expert_launch(dt, kQ8Seq, false, dn, nt, (T + nt - 1) / nt, st);
    if (e != hipSuccess) return e;
  }
  // gate logit: sequential dot (one row) for every token, one workgroup per
  // token (unless the router's launch computed it beside the logits)
  if (gate_done) return hipSuccess;
  if (router1_ok(dim) && al16(L->sh_gate_inp) && al16(xb))
    return router1_launch(QR_ORDER_SEQ, nullptr, xb, 0, dim, nullptr, st, T, L->sh_gate_inp, s.sgl);
  return gemv_f32_launch(QR_ORDER_SEQ, L->sh_gate_inp, xb, s.sgl, 1, dim, T, dim, 1, st);
}

// llama.cpp-layout experts (ggml K-quants, Q8_K activations): the routing,
// then one GEMV per (token, slot) pair in pair mode -- up and gate of token
// p / K through expert idx[p], the SwiGLU, down of hb row p -- and the
// weighted sum in slot order (qro_moe_token's loop: each pair's output row
// p, the identity as the combine's pair -> row map).
static hipError_t moe_forward_ggml(const qr_moe_layer* L, float* x, const float* xb, int T,
                                   int order, const MoeScratch& s, hipStream_t st) {
  const int E = L->n_experts, K = L->n_used, P = T * K;
  const int ut = (int)(L->up_type & ~(uint32_t)QR_GGML), dt = (int)(L->down_type & ~(uint32_t)QR_GGML);
  const size_t su = qr_wrow_bytes(ut, L->dim) * (size_t)L->hidden;
  const size_t sd = qr_wrow_bytes(dt, L->hidden) * (size_t)L->dim;
  hipError_t e = moe_route_launch(L, xb, T, order, s.logits, nullptr, s.idx, s.wts, st);
  if (e != hipSuccess) return e;
  e = gemv_ggml_pairs_launch(ut, L->up, su, s.idx, E, K, xb, L->dim, s.hu, L->hidden, L->hidden,
                             L->dim, P, st);
  if (e != hipSuccess) return e;
  e = gemv_ggml_pairs_launch(ut, L->gate, su, s.idx, E, K, xb, L->dim, s.hb, L->hidden, L->hidden,
                             L->dim, P, st);
  if (e != hipSuccess) return e;
  const long n = (long)P * L->hidden;
  hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, s.hu, s.hb,
                     n);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  e = gemv_ggml_pairs_launch(dt, L->down, sd, s.idx, E, 1, s.hb, L->hidden, s.y, L->dim, L->dim,
                             L->hidden, P, st);
  if (e != hipSuccess) return e;
  if ((e = rows_dispatch_launch(P, 1, s.offsets, s.inv, s.tiles, st)) != hipSuccess) return e;
  return combine_launch(x, s.y, s.inv, s.wts, T, K, L->dim, nullptr, nullptr, st);
}

// The one-token path of three launches (router, gate/up, down + combine).
static bool t1_path(const qr_moe_layer* L, const float* xb, int order) {
  const bool q8_lanes = order != QR_ORDER_SEQ &&
                        (L->up_type == QR_T_Q8_0 || L->down_type == QR_T_Q8_0);
  return !q8_lanes && !(L->up_type & QR_GGML) && router1_ok(L->dim) &&
         gateup1_ok((int)L->up_type, L->dim, L->n_experts, L->n_used) &&
         L->up_type == L->gate_type &&
         down1v2_ok((int)L->down_type, L->n_used, L->dim, L->hidden) && al16(L->router) &&
         al16(xb);
}

bool moe_t1_norm_ok(const qr_moe_layer* L, const float* x, const float* xb, const float* nw,
                    int order) {
  return t1_path(L, xb, order) && router1_norm_ok(L->dim) && al16(x) && al16(nw);
}

hipError_t moe_forward_launch(const qr_moe_layer* L, float* x, const float* xb, int T, int order,
                              const MoeScratch& s, hipStream_t st, int path, const float* norm_w) {
  if (norm_w && !(T == 1 && moe_t1_norm_ok(L, x, xb, norm_w, order))) return hipErrorInvalidValue;
  if (L->up_type & QR_GGML) return moe_forward_ggml(L, x, xb, T, order, s, st);
  const int E = L->n_experts, K = L->n_used, P = T * K;
  const bool sh = L->sh_hidden > 0;
  const size_t su = qr_wrow_bytes((int)L->up_type, L->dim) * (size_t)L->hidden;
  const size_t sd = qr_wrow_bytes((int)L->down_type, L->hidden) * (size_t)L->dim;
  hipError_t e;
  // `order` names the reference build: the router's accumulation order and
  // the Q8_0 dot order (kQ8* equal QR_ORDER_*).  Q8_0 experts in a lane order
  // run on the grouped GEMV kernels below, the only ones that form lane
  // accumulators.
  const int q8o = order;
  const bool q8_lanes = order != QR_ORDER_SEQ &&
                        (L->up_type == QR_T_Q8_0 || L->down_type == QR_T_Q8_0);

  // One token: logits, then gate/up with the routing done in every wave, then
  // down + combine (qr_moe_t1.hip): three launches, no routing kernel.  With
  // norm_w the router's workgroups also form xb = rmsnorm_ref(x, norm_w).
  if (T == 1 && t1_path(L, xb, order)) {
    // the shared expert's gate logit beside the router's (one more workgroup)
    const bool sg = sh && (reinterpret_cast<uintptr_t>(L->sh_gate_inp) & 15) == 0;
    e = router1_launch(order, L->router, norm_w ? x : xb, E, L->dim, s.logits, st, 1,
                       sg ? static_cast<const float*>(L->sh_gate_inp) : nullptr, s.sgl, norm_w,
                       norm_w ? const_cast<float*>(xb) : nullptr);
    if (e != hipSuccess) return e;
    // the shared expert's up/gate rows as more tiles of the same launch when
    // they share the routed up type (its down product then on the GEMV)
    const bool sg_up = sh && L->sh_up_type == L->up_type && L->sh_gate_type == L->up_type &&
                       sh_gemv_type((int)L->sh_down_type) &&
                       L->sh_hidden % qr_block_elems((int)L->sh_down_type) == 0 &&
                       al16(L->sh_up) && al16(L->sh_gate) && al16(L->sh_down);
    e = gateup1_launch((int)L->up_type, L->up, L->gate, su, L->dim, L->hidden, E, K, xb, s.logits,
                       s.idx, s.wts, s.hb, st, sg_up ? L->sh_up : nullptr,
                       sg_up ? L->sh_gate : nullptr, L->sh_hidden, s.hbs);
    if (e != hipSuccess) return e;
    if (sh) {
      e = shared_expert(L, xb, T, s, st, sg, sg_up);
      if (e != hipSuccess) return e;
    }
    return down1v2_launch((int)L->down_type, L->down, sd, L->dim, L->hidden, E, K, s.hb, s.idx,
                          s.wts, x, sh ? s.ysh : nullptr, s.sgl, st);
  }

  // Many tokens on int8 MFMA: tiled logits; routing + xb records; dispatch;
  // gate/up writing hb records; down; combine.  By default for every T > 1:
  // measured at the Qwen3-30B-A3B shape, the MFMA products beat the grouped
  // GEMV from T = 2 on (42.6 against 43.6 us per layer, 60 against 131 at
  // T = 16); the caller may force either product.
  const bool want_mfma = path == QR_MOE_PATH_MFMA || path == QR_MOE_PATH_AUTO;
  if (!q8_lanes && T > 1 && want_mfma && mfma_type_ok((int)L->up_type) &&
      mfma_type_ok((int)L->down_type) && rlogits_ok(L->dim) && E <= 256 && K <= 16 &&
      (reinterpret_cast<uintptr_t>(L->router) & 15) == 0) {
    const int kTile = mfma_tile(T, K, E);  // pairs per MFMA work item
    const bool perm_x = L->up_type != QR_T_Q8_0;
    // the sequential order for up to 64 tokens: one workgroup per (row,
    // token), the shared expert's gate logit beside them
    bool sg = false;
    if (order == QR_ORDER_SEQ && T <= 64 && router1_ok(L->dim) && al16(xb)) {
      sg = sh && al16(L->sh_gate_inp);
      e = router1_launch(order, L->router, xb, E, L->dim, s.logits, st, T,
                         sg ? static_cast<const float*>(L->sh_gate_inp) : nullptr, s.sgl);
    } else {
      e = rlogits_launch(order, L->router, xb, T, E, L->dim, s.logits, st);
    }
    if (e != hipSuccess) return e;
    e = route_rank_launch(s.logits, T, E, K, nullptr, s.idx, s.wts, xb, L->dim, perm_x, s.xq, st);
    if (e != hipSuccess) return e;
    e = moe_dispatch_launch(s.idx, T, K, E, kTile, s.counts, s.offsets, s.tiles, s.perm, s.inv,
                            st);
    if (e != hipSuccess) return e;
    const int items = (P + kTile - 1) / kTile + E;  // >= sum_e ceil(count_e / kTile)
    e = expert_mfma_launch((int)L->up_type, true, static_cast<const uint8_t*>(L->up),
                           static_cast<const uint8_t*>(L->gate), su, E, K, L->hidden, L->dim, s.xq,
                           1, s.offsets, s.perm, s.tiles, s.hb, L->hidden, items, kTile, s.hq,
                           L->down_type != QR_T_Q8_0, st);
    if (e != hipSuccess) return e;
    e = expert_mfma_launch((int)L->down_type, false, static_cast<const uint8_t*>(L->down), nullptr,
                           sd, E, K, L->dim, L->hidden, s.hq, 0, s.offsets, s.perm, s.tiles, s.y,
                           L->dim, items, kTile, nullptr, false, st);
    if (e != hipSuccess) return e;
    if (sh) {
      e = shared_expert(L, xb, T, s, st, sg);
      if (e != hipSuccess) return e;
    }
    return combine_launch(x, s.y, s.inv, s.wts, T, K, L->dim, sh ? s.ysh : nullptr, s.sgl, st);
  }

  e = moe_route_launch(L, xb, T, order, s.logits, nullptr, s.idx, s.wts, st);
  if (e != hipSuccess) return e;

  ExpertArgs g{};
  g.W1 = static_cast<const uint8_t*>(L->up);
  g.W2 = static_cast<const uint8_t*>(L->gate);
  g.slice = su;
  g.rows = L->hidden;
  g.cols = L->dim;
  g.X = xb;
  g.xstride = L->dim;
  g.Y = s.hb;
  g.ystride = L->hidden;
  g.idx = s.idx;
  g.offsets = s.offsets;
  g.perm = s.perm;
  g.tiles = s.tiles;
  g.E = E;
  g.K = K;
  g.P = P;

  if (T == 1) {
    g.mode = kModeSingle;
    e = expert_launch((int)L->up_type, q8o, true, g, 1, K, st);
    if (e != hipSuccess) return e;
    if (sh) {
      e = shared_expert(L, xb, T, s, st);
      if (e != hipSuccess) return e;
    }
    DownArgs dn{};
    dn.W = static_cast<const uint8_t*>(L->down);
    dn.slice = sd;
    dn.dim = L->dim;
    dn.hidden = L->hidden;
    dn.K = K;
    dn.E = E;
    dn.hb = s.hb;
    dn.idx = s.idx;
    dn.wts = s.wts;
    dn.x = x;
    dn.ysh = sh ? s.ysh : nullptr;
    dn.sgl = s.sgl;
    return down1_launch((int)L->down_type, q8o, dn, st);
  }

  // Many pairs per expert: grouped products on int8 MFMA (qr_moe_mfma.hip).
  if (!q8_lanes && want_mfma && mfma_type_ok((int)L->up_type) &&
      mfma_type_ok((int)L->down_type)) {
    const int kTile = mfma_tile(T, K, E);  // pairs per MFMA work item
    e = moe_dispatch_launch(s.idx, T, K, E, kTile, s.counts, s.offsets, s.tiles, s.perm, s.inv, st);
    if (e != hipSuccess) return e;
    const int items = (P + kTile - 1) / kTile + E;  // >= sum_e ceil(count_e / kTile)
    e = quant_rows_launch(xb, L->dim, T, L->dim, L->up_type != QR_T_Q8_0, s.xq, st);
    if (e != hipSuccess) return e;
    e = expert_mfma_launch((int)L->up_type, true, static_cast<const uint8_t*>(L->up),
                           static_cast<const uint8_t*>(L->gate), su, E, K, L->hidden, L->dim, s.xq,
                           1, s.offsets, s.perm, s.tiles, s.hb, L->hidden, items, kTile, nullptr,
                           false, st);
    if (e != hipSuccess) return e;
    e = quant_rows_launch(s.hb, L->hidden, P, L->hidden, L->down_type != QR_T_Q8_0, s.hq, st);
    if (e != hipSuccess) return e;
    e = expert_mfma_launch((int)L->down_type, false, static_cast<const uint8_t*>(L->down), nullptr,
                           sd, E, K, L->dim, L->hidden, s.hq, 0, s.offsets, s.perm, s.tiles, s.y,
                           L->dim, items, kTile, nullptr, false, st);
    if (e != hipSuccess) return e;
  } else {
  const int nt = pick_tile(P, E);
  e = moe_dispatch_launch(s.idx, T, K, E, nt, s.counts, s.offsets, s.tiles, s.perm, s.inv, st);
  if (e != hipSuccess) return e;
  const int items = (P + nt - 1) / nt + E;  // >= sum_e ceil(count_e / nt)
  g.mode = kModeDispatched;
  g.x_by_token = 1;
  e = expert_launch((int)L->up_type, q8o, true, g, nt, items, st);
  if (e != hipSuccess) return e;
  ExpertArgs dn = g;
  dn.W1 = static_cast<const uint8_t*>(L->down);
  dn.W2 = nullptr;
  dn.slice = sd;
  dn.rows = L->dim;
  dn.cols = L->hidden;
  dn.X = s.hb;
  dn.xstride = L->hidden;
  dn.Y = s.y;
  dn.ystride = L->dim;
  dn.x_by_token = 0;
  e = expert_launch((int)L->down_type, q8o, false, dn, nt, items, st);
  if (e != hipSuccess) return e;
  }
  if (sh) {
    e = shared_expert(L, xb, T, s, st);
    if (e != hipSuccess) return e;
  }
  return combine_launch(x, s.y, s.inv, s.wts, T, K, L->dim, sh ? s.ysh : nullptr, s.sgl, st);
}

}  // namespace qr
