// qr_moe_t1.hip -- the MoE layer's expert products for one token (decode),
// src/runtime.c:242-269 with K selected experts:
//
//   k_gateup1  hb[k] = silu(up_e . xb) * (gate_e . xb) for every slot k, on
//              the block-per-lane engine (qr_blk.h): a wave holds RB rows of
//              up in lanes 0-31 and the same rows of gate in lanes 32-63, so
//              SwiGLU pairs the two row chains with one lane shuffle.
//   k_down1    y_k = down_e . hb[k] for the K slots of a tile of rows, one wave
//              per slot on the wave-tile engine (qr_stream.h), then
//              x += ((0 + y_0 w_0) + y_1 w_1 + ...) in slot order (+ the shared
//              expert) for the tile's rows.
#include "qr_blk.h"
#include "qr_internal.h"
#include "qr_stream.h"

namespace qr {

// ---------------------------------------------------------------------------
// Gate/up.
// ---------------------------------------------------------------------------
struct GateUp1Args {
  const uint8_t* up;    // [E][hidden][rb]
  const uint8_t* gate;  // [E][hidden][rb]
  size_t slice;         // bytes per expert
  int dim, hidden, E, K;
  const float* xb;      // [dim]
  const int32_t* idx;   // [K]
  float* hb;            // [K][hidden]
};

template <int TYPE>
__global__ __launch_bounds__(64 * kBlkWaves) void k_gateup1(GateUp1Args a) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int BB = BlkFmt<TYPE>::kBytes;
  constexpr int NCH = BlkFmt<TYPE>::kChunks;
  const int nb = a.dim >> 8;
  const int RB = 32 / nb;  // rows per wave tile, per matrix
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int half = lane >> 5, l = lane & 31;
  const int rl = l / nb, b = l - rl * nb;
  const size_t rb = (size_t)nb * BB;
  const int tiles_per_slot = (a.hidden + RB - 1) / RB;
  const int tile = blockIdx.x * kBlkWaves + wave;
  const bool wave_on = tile < a.K * tiles_per_slot;
  const int k = wave_on ? tile / tiles_per_slot : 0;
  const int r0 = (tile - k * tiles_per_slot) * RB;
  const int e = wave_on ? a.idx[k] : -1;
  const bool ok = wave_on && e >= 0 && e < a.E;  // uniform per wave

  // activation first (see k_gemv_blk), then the weight stream
  ActPre pre;
  act_prefetch(a.xb, (size_t)a.dim, 1, a.dim, pre);
  quantize_act_blk<BlkFmt<TYPE>::kNib>(a.xb, (size_t)a.dim, 1, a.dim, smem, pre);
  asm volatile("" ::: "memory");
  uint4 c[NCH];
  const int row = r0 + rl;
  const bool lane_on = ok && rl < RB && row < a.hidden;
  if (lane_on) {
    const uint8_t* W = half ? a.gate : a.up;
    const uint4* p = reinterpret_cast<const uint4*>(W + (size_t)e * a.slice + (size_t)row * rb +
                                                    (size_t)b * BB);
#pragma unroll
    for (int q = 0; q < NCH; q++) c[q] = p[q];
  } else {
#pragma unroll
    for (int q = 0; q < NCH; q++) c[q] = make_uint4(0, 0, 0, 0);
  }
  __syncthreads();
  if (!ok) return;  // no barriers below

  float terms[1][8];
  int32_t isums[1][8];
  blk_terms<TYPE, 1>(c, b, smem, act_tok_bytes(a.dim), terms, isums);
  float y[1];
  blk_chain<1>(terms, b, nb, y);
  const float g = __shfl(y[0], lane + 32);  // gate row chain of the same row
  if (half == 0 && rl < RB && row < a.hidden && b == nb - 1)
    a.hb[(size_t)k * a.hidden + row] = qr_silu(y[0]) * g;
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
  size_t slice_bytes;   // LDS per wave: terms, then the staged tile
  size_t terms_bytes;
};

template <int TYPE>
__global__ __launch_bounds__(1024) void k_down1(Down1Args a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const TileShape sh0 = tile_shape(TYPE, a.hidden);
  TileShape sh = sh0;
  sh.RW = a.RW;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int k = wave;  // slot
  const int r0 = blockIdx.x * a.RW;
  const int RWt = min(a.RW, a.dim - r0);
  float* ys = reinterpret_cast<float*>(smem);  // [K][RW]
  uint8_t* slice = smem + align16((size_t)a.K * a.RW * 4) + (size_t)wave * a.slice_bytes;
  float* terms = reinterpret_cast<float*>(slice);
  uint32_t* stage = reinterpret_cast<uint32_t*>(slice + a.terms_bytes);
  const int e = a.idx[k];
  const bool ok = e >= 0 && e < a.E;  // uniform per wave

  if (ok) {
    const Slots sl = make_slots(sh.U, lane);
    LaneAct<1, kUPL> A;
    quantize_lane_act<TYPE, 1, kUPL>(a.hb + (size_t)k * a.hidden, (size_t)a.hidden, sl, sh.RW, A);
    asm volatile("" ::: "memory");
    TileRegs<TYPE> R;
    const uint8_t* W = a.down + (size_t)e * a.slice;
    load_tile<TYPE>(W, a.slice, r0, RWt, sh, sl, lane, R);
    if constexpr (!IsDirect<TYPE>::value) {
      // the wave's stage area holds the tile's chunks only (not the engine's
      // full kCPL chunks): copy those that fit
      const int nch = (int)((a.slice_bytes - a.terms_bytes) / 16);
#pragma unroll
      for (int j = 0; j < kCPL; j++) {
        const int ci = j * 64 + lane;
        if (ci < nch) reinterpret_cast<uint4*>(stage)[ci] = R.c[j];
      }
      wave_lds_sync();
    }
    tile_terms<TYPE, 1, kUPL>(R, sl, RWt, r0, sh, A, stage, terms, nullptr, a.dim);
    wave_lds_sync();
    for (int i = lane; i < RWt; i += 64) ys[k * a.RW + i] = row_sum_seq(terms + i * sh.TS, sh.U);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < RWt; i += blockDim.x) {
    float acc = 0.0f;  // xb2 = 0 (src/runtime.c:242)
    for (int kk = 0; kk < a.K; kk++) {
      const int ek = a.idx[kk];
      if (ek < 0 || ek >= a.E) continue;
      acc += ys[kk * a.RW + i] * a.wts[kk];
    }
    if (a.ysh) {
      const float sg = 1.0f / (1.0f + qr_expf(-a.sgl[0]));
      acc += sg * a.ysh[r0 + i];
    }
    a.x[r0 + i] += acc;
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
bool gateup1_ok(int type, int dim) {
  if (type != QR_T_Q4_K && type != QR_T_Q5_K) return false;
  const int nb = dim >> 8;
  return nb >= 1 && nb <= 32 && (dim & 3) == 0 && act_tok_bytes(dim) <= 64 * 1024;
}

hipError_t gateup1_launch(int type, const void* up, const void* gate, size_t slice, int dim,
                          int hidden, int E, int K, const float* xb, const int32_t* idx, float* hb,
                          hipStream_t st) {
  GateUp1Args a;
  a.up = static_cast<const uint8_t*>(up);
  a.gate = static_cast<const uint8_t*>(gate);
  a.slice = slice;
  a.dim = dim;
  a.hidden = hidden;
  a.E = E;
  a.K = K;
  a.xb = xb;
  a.idx = idx;
  a.hb = hb;
  const int RB = 32 / (dim >> 8);
  const int tiles = K * ((hidden + RB - 1) / RB);
  const int grid = (tiles + kBlkWaves - 1) / kBlkWaves;
  const size_t lds = act_tok_bytes(dim);
  if (type == QR_T_Q4_K)
    hipLaunchKernelGGL(k_gateup1<QR_T_Q4_K>, dim3(grid), dim3(64 * kBlkWaves), lds, st, a);
  else
    hipLaunchKernelGGL(k_gateup1<QR_T_Q5_K>, dim3(grid), dim3(64 * kBlkWaves), lds, st, a);
  return hipGetLastError();
}

// LDS of a k_down1 workgroup with RW rows per tile.
static size_t down1_lds(int type, int K, int RW, const TileShape& sh, size_t* slice,
                        size_t* terms) {
  *terms = align16((size_t)RW * sh.TS * 4);
  const bool direct = type == QR_T_Q4_K || type == QR_T_Q5_K;
  *slice = *terms + (direct ? 0 : align16((size_t)RW * sh.rb + 15 + 4 + 15));
  return align16((size_t)K * RW * 4) + (size_t)K * *slice;
}

// Rows per tile: the engine's shape, reduced until K wave slices fit 64 KB.
static int down1_rows(int type, int K, int hidden) {
  const TileShape sh = tile_shape(type, hidden);
  int RW = sh.RW;
  size_t s, t;
  while (RW > 1 && down1_lds(type, K, RW, sh, &s, &t) > 64 * 1024) RW--;
  return RW;
}

bool down1v2_ok(int type, int K, int hidden) {
  if (type == QR_T_F32 || K > 16 || (hidden & 3)) return false;
  const TileShape sh = tile_shape(type, hidden);
  if (sh.RW < 1) return false;
  const int RW = down1_rows(type, K, hidden);
  size_t s, t;
  return RW >= 1 && down1_lds(type, K, RW, sh, &s, &t) <= 64 * 1024;
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
  a.RW = down1_rows(type, K, hidden);
  const size_t lds = down1_lds(type, K, a.RW, sh, &a.slice_bytes, &a.terms_bytes);
  const int grid = (dim + a.RW - 1) / a.RW;
  switch (type) {
    case QR_T_Q4_K:
      hipLaunchKernelGGL(k_down1<QR_T_Q4_K>, dim3(grid), dim3(64 * K), lds, st, a);
      break;
    case QR_T_Q5_K:
      hipLaunchKernelGGL(k_down1<QR_T_Q5_K>, dim3(grid), dim3(64 * K), lds, st, a);
      break;
    case QR_T_Q6_K:
      hipLaunchKernelGGL(k_down1<QR_T_Q6_K>, dim3(grid), dim3(64 * K), lds, st, a);
      break;
    case QR_T_Q8_0:
      hipLaunchKernelGGL(k_down1<QR_T_Q8_0>, dim3(grid), dim3(64 * K), lds, st, a);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace qr
