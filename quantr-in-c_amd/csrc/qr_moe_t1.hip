// qr_moe_t1.hip -- the MoE layer for one token (decode), src/runtime.c:202-269:
// three launches, each one memory round trip deep plus its weight stream.
//
//   k_router1   logits[e] = W_r[e] . xb in the reference build's order
//               (KernelOps.matmul: SEQ / AVX2 / AVX512), one 64-thread
//               workgroup per expert row; the row and xb arrive in LDS by DMA.
//   k_gateup1   wave 0 of every workgroup routes the token from the E logits
//               (softmax_ref, K argmax passes -- the same code in every
//               workgroup, so all get the same bit-exact experts), then waves
//               stream
//               RB rows of its slot's up matrix (lanes 0-31) and the same rows
//               of gate (lanes 32-63) through LDS on the block-per-lane engine
//               (qr_blk.h):  hb[k] = silu(up_e . xb) * (gate_e . xb).  The
//               activation is staged by DMA ahead of the weights; workgroup 0
//               publishes the indices and renormalised weights.
//   k_down1     per tile of RW output rows, one wave per slot k: the expert
//               index comes in by scalar load while hb[k] is staged by DMA,
//               then the tile of down_e rows is staged by DMA;
//               y_k = down_e . hb[k] (hb re-quantised), and
//               x += ((0 + y_0 w_0) + y_1 w_1 + ...) in slot order (+ the
//               shared expert) for the tile's rows.
#include "qr_blk.h"
#include "qr_internal.h"
#include "qr_norm.h"
#include "qr_route.h"
#include "qr_stream.h"

namespace qr {

// ---------------------------------------------------------------------------
// Router logits.
// ---------------------------------------------------------------------------
// matmul_ref (src/kernels.c:18-28) of one staged row: every product w[j] * x[j]
// rounded, then added in order -- the products formed by the whole wave in
// place (w becomes the products), the chain of adds by the wave (seq_sum_wave).
__device__ inline float router_seq(float* sw, const float* sx, int d, int lane) {
  const int d4 = d >> 2;  // d % 4 == 0 (router1_ok)
#pragma unroll 4
  for (int j = lane; j < d4; j += 64) {
    float4 w = reinterpret_cast<const float4*>(sw)[j];
    const float4 x = reinterpret_cast<const float4*>(sx)[j];
    w.x = w.x * x.x;
    w.y = w.y * x.y;
    w.z = w.z * x.z;
    w.w = w.w * x.w;
    reinterpret_cast<float4*>(sw)[j] = w;
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  return seq_sum_wave<64>(sw, d, lane);
}

// Workgroup (e, t): logit e of token t (xb + t d, logits + t E).  With `W2`, the
// workgroups e = E compute, in matmul_ref's order whatever LANES is, the dot
// of the one row W2 with each token into out2[t] (the shared expert's gate
// logit, computed beside the router's).
// NORM (one token): xb is the residual stream x, and every workgroup forms
// rmsnorm_ref(x, nw) itself (qr_norm.h) while its row lands; workgroup 0
// stores the normalised vector at xb_out for the launches after it.
constexpr int kRouterNormNP = kNormFuseMax / 4 / 64;
template <int LANES, bool NORM>
__global__ __launch_bounds__(64) void k_router1(const float* __restrict__ W,
                                                const float* __restrict__ xb, int d, int E,
                                                float* __restrict__ logits,
                                                const float* __restrict__ W2,
                                                float* __restrict__ out2,
                                                const float* __restrict__ nw,
                                                float* __restrict__ xb_out) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int e = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
  const size_t rbytes = kib_round((size_t)d * 4);
  float* sw = reinterpret_cast<float*>(smem);
  float* sx = reinterpret_cast<float*>(smem + rbytes);
  const bool extra = e >= E;  // uniform
  const float* row = extra ? W2 : W + (size_t)e * d;
  dma_bytes<true>(reinterpret_cast<const uint8_t*>(row), smem, d * 4, lane);
  if constexpr (NORM) {
    NormRegs<kRouterNormNP> r;
    norm_load<kRouterNormNP>(xb, nw, d, lane, 64, r);
    norm_finish<kRouterNormNP>(r, d, sx, reinterpret_cast<float*>(smem + 2 * rbytes), lane, 64,
                               e == 0 ? xb_out : nullptr);
  } else {
    dma_bytes(reinterpret_cast<const uint8_t*>(xb + (size_t)t * d), smem + rbytes, d * 4, lane);
  }
  wait_vmcnt<0>();
  if (LANES == 1 || extra) {
    const float s = router_seq(sw, sx, d, lane);
    if (lane == 0) {
      if (extra) out2[t] = s;
      else logits[(size_t)t * E + e] = s;
    }
  } else {
    // matmul_omp, src/kernels.c:38-65: LANES FMA chains, lanes combined in the
    // build's order, then the multiply-add tail
    const int k = lane;
    const int dm = d - d % LANES;
    const float acc = k < LANES ? lds_chain<LANES>(sw, sx, k, dm) : 0.0f;
    float v[LANES];
#pragma unroll
    for (int i = 0; i < LANES; i++) v[i] = __shfl(acc, i);
    if (lane == 0) {
      float s = 0.0f;
      if constexpr (LANES == 8) {
#pragma unroll
        for (int i = 0; i < 8; i++) s += v[i];
      } else {
        float t8[8], t4[4];
#pragma unroll
        for (int i = 0; i < 8; i++) t8[i] = v[8 + i] + v[i];
#pragma unroll
        for (int i = 0; i < 4; i++) t4[i] = t8[4 + i] + t8[i];
        const float a02 = t4[0] + t4[2];
        const float a13 = t4[1] + t4[3];
        s += a02 + a13;
      }
      for (int j = dm; j < d; j++) s += sw[j] * sx[j];
      logits[(size_t)t * E + e] = s;
    }
  }
}

bool router1_ok(int dim) { return dim > 0 && (dim & 3) == 0 && 2 * kib_round((size_t)dim * 4) <= 64 * 1024; }
bool router1_norm_ok(int dim) { return router1_ok(dim) && dim <= kNormFuseMax; }

template <bool NORM>
static void router1_k(int order, dim3 grid, size_t lds, hipStream_t st, const float* W,
                      const float* xb, int d, int E, float* logits, const float* W2, float* out2,
                      const float* nw, float* xb_out) {
  switch (order) {
    case QR_ORDER_SEQ:
      hipLaunchKernelGGL((k_router1<1, NORM>), grid, dim3(64), lds, st, W, xb, d, E, logits, W2,
                         out2, nw, xb_out);
      break;
    case QR_ORDER_AVX2:
      hipLaunchKernelGGL((k_router1<8, NORM>), grid, dim3(64), lds, st, W, xb, d, E, logits, W2,
                         out2, nw, xb_out);
      break;
    default:
      hipLaunchKernelGGL((k_router1<16, NORM>), grid, dim3(64), lds, st, W, xb, d, E, logits, W2,
                         out2, nw, xb_out);
      break;
  }
}

hipError_t router1_launch(int order, const float* W, const float* xb, int E, int d, float* logits,
                          hipStream_t st, int T, const float* W2, float* out2, const float* nw,
                          float* xb_out) {
  if ((E > 0 && (reinterpret_cast<uintptr_t>(W) & 15)) || (reinterpret_cast<uintptr_t>(xb) & 15) ||
      (W2 && (reinterpret_cast<uintptr_t>(W2) & 15)) || T < 1)
    return hipErrorInvalidValue;
  const dim3 grid(E + (W2 ? 1 : 0), T);
  if (nw) {
    if (T != 1 || !router1_norm_ok(d) || (reinterpret_cast<uintptr_t>(nw) & 15) ||
        (xb_out && (reinterpret_cast<uintptr_t>(xb_out) & 15)))
      return hipErrorInvalidValue;
    router1_k<true>(order, grid, 2 * kib_round((size_t)d * 4) + 16, st, W, xb, d, E, logits, W2,
                    out2, nw, xb_out);
  } else {
    router1_k<false>(order, grid, 2 * kib_round((size_t)d * 4), st, W, xb, d, E, logits, W2,
                     out2, nullptr, nullptr);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Gate/up.
// ---------------------------------------------------------------------------
struct GateUp1Args {
  const uint8_t* up;    // [E][hidden][rb]
  const uint8_t* gate;  // [E][hidden][rb]
  size_t slice;         // bytes per expert
  int dim, hidden, E, K;
  const float* xb;      // [dim]
  const float* logits;  // [E]
  int32_t* idx;         // [K] out (workgroup 0)
  float* wts;           // [K] out (workgroup 0)
  float* hb;            // [K][hidden]
  // optional: the shared expert's up / gate rows (same type and width),
  // computed as tiles after the routed ones into hbs
  const uint8_t* sh_up;
  const uint8_t* sh_gate;
  int sh_hidden;        // 0: none
  float* hbs;           // [sh_hidden]
};

// LDS: activation staging | activation (NIB/NAT) | routing row | slots
__host__ __device__ inline size_t gateup1_lds(int type, int dim, size_t* o_act, size_t* o_pw,
                                              size_t* o_slots) {
  const size_t xs = blk_xs_bytes(dim, 1);
  *o_act = xs;
  *o_pw = *o_act + align16(act_tok_bytes(dim));
  *o_slots = *o_pw + (size_t)kRouteRow * 4;
  const size_t sb = (size_t)64 * (type == QR_T_Q4_K ? QR_Q4K_BYTES : QR_Q5K_BYTES);
  return *o_slots + (size_t)kBlkWaves * sb;
}

template <int TYPE>
__global__ __launch_bounds__(64 * kBlkWaves) void k_gateup1(GateUp1Args a) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int BB = BlkFmt<TYPE>::kBytes;
  constexpr int NCH = BlkFmt<TYPE>::kChunks;
  constexpr int SB = 64 * BB;
  const int nb = a.dim >> 8;
  const int RB = 32 / nb;  // rows per wave tile, per matrix
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int half = lane >> 5, l = lane & 31;
  const int rl = l / nb, b = l - rl * nb;
  const size_t rb = (size_t)nb * BB;
  const int tiles_per_slot = (a.hidden + RB - 1) / RB;
  const int routed = a.K * tiles_per_slot;  // then the shared expert's tiles
  const int tile = blockIdx.x * kBlkWaves + wave;
  const bool shared = tile >= routed;  // uniform per wave
  const bool wave_on = tile < routed + (a.sh_hidden + RB - 1) / RB;
  const int k = wave_on && !shared ? tile / tiles_per_slot : 0;
  const int r0 = shared ? (tile - routed) * RB : (tile - k * tiles_per_slot) * RB;
  const int nrows = shared ? a.sh_hidden : a.hidden;
  size_t o_act, o_pw, o_slots;
  gateup1_lds(TYPE, a.dim, &o_act, &o_pw, &o_slots);
  uint8_t* act = smem + o_act;
  float* pw = reinterpret_cast<float*>(smem + o_pw);
  uint8_t* slot = smem + o_slots + (size_t)wave * SB;

  // 1. routing: wave 0 computes the softmax and the rank keys while waves
  //    1 .. kBlkWaves - 1 stage the activation by DMA and quantize it (each
  //    its own groups: its own DMA's completion is all it waits for); after
  //    the barrier every thread ranks the E candidates (route_rank_wg);
  //    workgroup 0 publishes the routing
  const ExpTab tab = qr_expf_tab();
  const int* sidx = route_idx(pw);
  if (wave == 0) {
    float pv[4];
    route_softmax(a.logits, a.E, pw, lane, nullptr, tab, pv);
    route_rank_keys(pv, a.E, a.K, pw, lane);
  } else {
    stage_act_dma(a.xb, (size_t)a.dim, 1, a.dim, smem, wave - 1, lane, kBlkWaves - 1);
    wait_vmcnt<0>();
    ActPre pre;
    quantize_act_blk<BlkFmt<TYPE>::kNib, kActLds>(a.xb, (size_t)a.dim, 1, a.dim, act, pre,
                                         reinterpret_cast<const float*>(smem),
                                         (int)threadIdx.x - 64, 64 * (kBlkWaves - 1));
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  route_rank_wg(a.E, a.K, pw, (int)threadIdx.x, (int)blockDim.x);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  if (blockIdx.x == 0 && wave == 0) route_write(pw, a.K, lane, a.idx, a.wts);
  const int e = wave_on && !shared ? __builtin_amdgcn_readfirstlane(sidx[k]) : -1;
  const bool ok = wave_on && (shared || (e >= 0 && e < a.E));  // uniform per wave
  if (!ok) return;  // no barriers below
  // 2. the weight tile: up rows r0.. at slot bytes [0, RB rb), the same gate
  //    rows at [32 BB, 32 BB + RB rb): lane l reads its block at l * BB
  {
    const int rows = min(RB, nrows - r0);
    const int valid = rows * (int)rb;
    const uint8_t* ub = shared ? a.sh_up + (size_t)r0 * rb : a.up + (size_t)e * a.slice + (size_t)r0 * rb;
    const uint8_t* gb =
        shared ? a.sh_gate + (size_t)r0 * rb : a.gate + (size_t)e * a.slice + (size_t)r0 * rb;
    const uint32_t sbase = lds_u32addr(slot);
#pragma unroll
    for (int c = 0; c < NCH; c++) {
      const int o = c * 1024 + lane * 16;
      const uint8_t* src = o < 32 * BB ? (o < valid ? ub + o : ub)
                                       : (o - 32 * BB < valid ? gb + (o - 32 * BB) : ub);
      lds_dma16_nt(src, sbase + (uint32_t)(c * 1024));
    }
  }

  wait_vmcnt<0>();
  uint4 c[NCH];
  {
    const uint4* q = reinterpret_cast<const uint4*>(slot + (size_t)lane * BB);
#pragma unroll
    for (int j = 0; j < NCH; j++) c[j] = q[j];
  }
  float terms[1][8];
  int32_t isums[1][8];
  blk_terms<TYPE, 1>(c, b, act, act_tok_bytes(a.dim), terms, isums);
  float y[1];
  blk_chain<1>(terms, b, nb, y);
  const float g = __shfl(y[0], lane + 32);  // gate row chain of the same row
  const float sv = qr_silu_w(y[0], tab);  // every lane
  const int row = r0 + rl;
  if (half == 0 && rl < RB && row < nrows && b == nb - 1) {
    if (shared) a.hbs[row] = sv * g;
    else a.hb[(size_t)k * a.hidden + row] = sv * g;
  }
}

bool gateup1_ok(int type, int dim, int E, int K) {
  if (type != QR_T_Q4_K && type != QR_T_Q5_K) return false;
  const int nb = dim >> 8;
  if (nb < 1 || nb > 32 || (dim & 3) || E > 256 || K > 16) return false;
  size_t a, b, c;
  return blk_xs_bytes(dim, 1) <= 16 * 1024 && gateup1_lds(type, dim, &a, &b, &c) <= 64 * 1024;
}

hipError_t gateup1_launch(int type, const void* up, const void* gate, size_t slice, int dim,
                          int hidden, int E, int K, const float* xb, const float* logits,
                          int32_t* idx, float* wts, float* hb, hipStream_t st, const void* sh_up,
                          const void* sh_gate, int sh_hidden, float* hbs) {
  GateUp1Args a;
  a.up = static_cast<const uint8_t*>(up);
  a.gate = static_cast<const uint8_t*>(gate);
  a.slice = slice;
  a.dim = dim;
  a.hidden = hidden;
  a.E = E;
  a.K = K;
  a.xb = xb;
  a.logits = logits;
  a.idx = idx;
  a.wts = wts;
  a.hb = hb;
  a.sh_up = static_cast<const uint8_t*>(sh_up);
  a.sh_gate = static_cast<const uint8_t*>(sh_gate);
  a.sh_hidden = sh_up && sh_gate && hbs ? sh_hidden : 0;
  a.hbs = hbs;
  if (a.sh_hidden && ((reinterpret_cast<uintptr_t>(sh_up) & 15) ||
                      (reinterpret_cast<uintptr_t>(sh_gate) & 15)))
    return hipErrorInvalidValue;
  const int RB = 32 / (dim >> 8);
  const int tiles = K * ((hidden + RB - 1) / RB) + (a.sh_hidden + RB - 1) / RB;
  const int grid = (tiles + kBlkWaves - 1) / kBlkWaves;
  size_t o1, o2, o3;
  const size_t lds = gateup1_lds(type, dim, &o1, &o2, &o3);
  if (type == QR_T_Q4_K)
    hipLaunchKernelGGL(k_gateup1<QR_T_Q4_K>, dim3(grid), dim3(64 * kBlkWaves), lds, st, a);
  else
    hipLaunchKernelGGL(k_gateup1<QR_T_Q5_K>, dim3(grid), dim3(64 * kBlkWaves), lds, st, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Down + combine.
// ---------------------------------------------------------------------------
struct Down1Args {
  const uint8_t* down;  // [E][dim][rb]
  size_t slice;
  int dim, hidden, E, K;
  const float* hb;      // [K][hidden]
  const int32_t* idx;   // [K]
  const float* wts;     // [K]
  float* x;             // [dim], updated in place
  const float* ysh;     // optional shared-expert output [dim]
  const float* sgl;     // its gate logit
  int RW;               // rows per tile
  int o_wave;           // LDS offset of wave 0's slice
  int slice_bytes;      // LDS per wave: terms | hb staging | weight tile staging
  int o_hs, o_stage;    // offsets inside a slice
  int o_ab;             // the wave's quantized hb blocks (48 bytes each)
};

template <int TYPE>
__global__ __launch_bounds__(1024) void k_down1(Down1Args a) {
  extern __shared__ __align__(16) uint8_t smem[];
  TileShape sh = tile_shape(TYPE, a.hidden);
  sh.RW = a.RW;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int k = wave;  // slot
  const int r0 = blockIdx.x * a.RW;
  const int RWt = min(a.RW, a.dim - r0);
  float* ys = reinterpret_cast<float*>(smem);  // [K][RW]
  uint8_t* slice = smem + a.o_wave + (size_t)wave * a.slice_bytes;
  float* terms = reinterpret_cast<float*>(slice);
  float* hs = reinterpret_cast<float*>(slice + a.o_hs);
  uint8_t* stage = slice + a.o_stage;

  // the expert indices and weights by scalar loads (their own counter), hb[k]
  // by DMA meanwhile
  // (16 entries each, 64 bytes: the scratch regions of idx and wts are 256
  // bytes, and entries past K are never used)
  int eks[16];
  float wks[16];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int4 iv = reinterpret_cast<const int4*>(a.idx)[j];
    const float4 wv = reinterpret_cast<const float4*>(a.wts)[j];
    eks[4 * j] = iv.x; eks[4 * j + 1] = iv.y; eks[4 * j + 2] = iv.z; eks[4 * j + 3] = iv.w;
    wks[4 * j] = wv.x; wks[4 * j + 1] = wv.y; wks[4 * j + 2] = wv.z; wks[4 * j + 3] = wv.w;
  }
  dma_bytes(reinterpret_cast<const uint8_t*>(a.hb + (size_t)k * a.hidden),
            reinterpret_cast<uint8_t*>(hs), a.hidden * 4, lane);
  int e = -1;
#pragma unroll
  for (int kk = 0; kk < 16; kk++)
    if (kk == k) e = eks[kk];
  e = __builtin_amdgcn_readfirstlane(e);
  const bool ok = e >= 0 && e < a.E;  // uniform per wave
  if (ok) {
    // the tile's byte range [r0 rb, (r0 + RWt) rb) from its 16-byte aligned start
    const size_t gs = (size_t)r0 * sh.rb;
    const size_t a0 = gs & ~(size_t)15;
    const uint8_t* W = a.down + (size_t)e * a.slice;
    const int nbytes = (int)(gs + (size_t)RWt * sh.rb - a0);
    const int nt = dma_bytes<true>(W + a0, stage, nbytes, lane);
    // hb staged (loads complete in order: only the tile's DMA may be in flight)
    switch (nt) {
      case 1: wait_vmcnt<1>(); break;
      case 2: wait_vmcnt<2>(); break;
      case 3: wait_vmcnt<3>(); break;
      case 4: wait_vmcnt<4>(); break;
      case 5: wait_vmcnt<5>(); break;
      case 6: wait_vmcnt<6>(); break;
      case 7: wait_vmcnt<7>(); break;
      case 8: wait_vmcnt<8>(); break;
      default: wait_vmcnt<0>(); break;
    }
    const Slots sl = make_slots(sh.U, lane);
    LaneAct<1, kUPL> A;
    quantize_lane_act_wave<TYPE, kUPL>(hs, sl, sh.RW, sh.U, slice + a.o_ab, lane, A);
    wait_vmcnt<0>();
    TileRegs<TYPE> R;
    if constexpr (IsDirect<TYPE>::value) load_tile_lds<TYPE>(stage, r0, RWt, sh, sl, R);
    tile_terms<TYPE, 1, kUPL>(R, sl, RWt, r0, sh, A, reinterpret_cast<const uint32_t*>(stage),
                              terms, nullptr, a.dim);
    wave_lds_sync();
    for (int i = lane; i < RWt; i += 64) ys[k * a.RW + i] = row_sum_seq(terms + i * sh.TS, sh.U);
  } else {
    wait_vmcnt<0>();  // no DMA in flight when the wave moves on
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  for (int i = threadIdx.x; i < RWt; i += blockDim.x) {
    float acc = 0.0f;  // xb2 = 0 (src/runtime.c:242)
#pragma unroll
    for (int kk = 0; kk < 16; kk++) {
      if (kk >= a.K) break;
      const int ek = eks[kk];
      if (ek < 0 || ek >= a.E) continue;
      acc += ys[kk * a.RW + i] * wks[kk];
    }
    if (a.ysh) {
      const float sg = 1.0f / (1.0f + qr_expf(-a.sgl[0]));
      acc += sg * a.ysh[r0 + i];
    }
    a.x[r0 + i] += acc;
  }
}

// LDS of a k_down1 workgroup with RW rows per tile: ys, then K wave slices of
// [terms | hb staging | weight staging | quantized hb], the staging areas
// whole KiB (DMA).
static size_t down1_lds(int type, int K, int RW, int hidden, const TileShape& sh, Down1Args* a) {
  const size_t terms = align16((size_t)RW * sh.TS * 4);
  const size_t hsb = kib_round((size_t)hidden * 4);
  const size_t stb = kib_round((size_t)RW * sh.rb + 15);
  const size_t abb = (size_t)(hidden / 32) * 48;
  a->o_wave = (int)align16((size_t)K * RW * 4);
  a->o_hs = (int)terms;
  a->o_stage = (int)(terms + hsb);
  a->o_ab = (int)(terms + hsb + stb);
  a->slice_bytes = (int)align16(terms + hsb + stb + abb);
  (void)type;
  return (size_t)a->o_wave + (size_t)K * a->slice_bytes;
}

// Rows per tile: enough tiles to cover the CUs, within the engine's shape, a
// DMA of at most 8 KiB and K slices within 160 KiB of LDS.
static int down1_rows(int type, int K, int dim, int hidden) {
  const TileShape sh = tile_shape(type, hidden);
  const int cus = device_cus();
  int RW = (dim + cus - 1) / cus;
  if (RW > sh.RW) RW = sh.RW;
  Down1Args t;
  while (RW > 1 && ((size_t)RW * sh.rb + 15 > 8 * 1024 ||
                    down1_lds(type, K, RW, hidden, sh, &t) > 160 * 1024))
    RW--;
  return RW;
}

bool down1v2_ok(int type, int K, int dim, int hidden) {
  if (type == QR_T_F32 || K > 16 || K < 1 || (hidden & 3)) return false;
  const TileShape sh = tile_shape(type, hidden);
  if (sh.RW < 1 || kib_round((size_t)hidden * 4) > 16 * 1024) return false;
  const int RW = down1_rows(type, K, dim, hidden);
  Down1Args t;
  return RW >= 1 && (size_t)RW * sh.rb + 15 <= 8 * 1024 &&
         down1_lds(type, K, RW, hidden, sh, &t) <= 160 * 1024;
}

template <int TYPE>
static hipError_t down1_launch_t(const Down1Args& a, int grid, size_t lds, hipStream_t st) {
  static std::atomic<bool> opted[64];
  if (lds > 64 * 1024) {
    const hipError_t e = lds_opt_in((const void*)k_down1<TYPE>, opted);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(k_down1<TYPE>, dim3(grid), dim3(64 * a.K), lds, st, a);
  return hipGetLastError();
}

hipError_t down1v2_launch(int type, const void* down, size_t slice, int dim, int hidden, int E,
                          int K, const float* hb, const int32_t* idx, const float* wts, float* x,
                          const float* ysh, const float* sgl, hipStream_t st) {
  Down1Args a;
  a.down = static_cast<const uint8_t*>(down);
  a.slice = slice;
  a.dim = dim;
  a.hidden = hidden;
  a.E = E;
  a.K = K;
  a.hb = hb;
  a.idx = idx;
  a.wts = wts;
  a.x = x;
  a.ysh = ysh;
  a.sgl = sgl;
  const TileShape sh = tile_shape(type, hidden);
  a.RW = down1_rows(type, K, dim, hidden);
  const size_t lds = down1_lds(type, K, a.RW, hidden, sh, &a);
  const int grid = (dim + a.RW - 1) / a.RW;
  switch (type) {
    case QR_T_Q4_K: return down1_launch_t<QR_T_Q4_K>(a, grid, lds, st);
    case QR_T_Q5_K: return down1_launch_t<QR_T_Q5_K>(a, grid, lds, st);
    case QR_T_Q6_K: return down1_launch_t<QR_T_Q6_K>(a, grid, lds, st);
    case QR_T_Q8_0: return down1_launch_t<QR_T_Q8_0>(a, grid, lds, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qr
