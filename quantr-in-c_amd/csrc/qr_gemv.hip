// qr_gemv.hip -- quantized decode GEMV for gfx950:  y[t][r] = W[r] . x[t]
// for W in Q8_0 / Q4_K / Q5_K / Q6_K (the reference's block layouts, streamed
// straight from HBM), x fp32 quantized to Q8_0 inside the kernel, t < NT.
//
// Semantics: matmul_q_fused (src/quant.c:441-523): one Q8_0 quantization of x
// per call, then per row the fused dot in the reference's order: int32 sums per
// 32-element unit, one fp32 term per unit, the terms added sequentially from
// 0.0f.  Results are bit-identical to the reference's -std=c99 build (Q8_0,
// Q5_K, Q6_K) and to the corrected Q4_K dot.
//
// Work split: a workgroup owns R consecutive rows (one contiguous byte range
// of W).  Its waves sweep the rows' units 64 at a time (lane = unit), compute
// each unit's int32 sum with v_dot4_i32_i8 and its fp32 term, and park the
// term in LDS; then R*NT threads add their row's terms in unit order.
#include <algorithm>
#include <cstdlib>

#include "qr_gemv.h"
#include "qr_internal.h"
#include "qr_stream.h"
#include "qr_blk.h"
#include "qr_tiled.h"
#include "qr_tiled_sq.h"
#include "qr_ggml.h"

namespace qr {

constexpr int kWg = 256;


// LDS layout: act q | act bd | act bs | terms | staged tile.  Terms are
// [nt][R][slots][U + 1] floats (slots: q8_slots).
__host__ __device__ inline size_t gemv_lds_layout(int type, int q8o, int d, int nt, int R,
                                                  size_t* o_bd, size_t* o_bs, size_t* o_terms,
                                                  size_t* o_tile) {
  const int nxb = d / 32;
  const int U = qr_units(type, d);
  size_t off = align16((size_t)nt * nxb * 32);
  *o_bd = off;
  off = align16(off + (size_t)nt * nxb * 4);
  *o_bs = off;
  off = align16(off + (size_t)nt * nxb * 4);
  *o_terms = off;
  off = align16(off + (size_t)nt * R * q8_slots(type, q8o) * (U + 1) * 4);
  *o_tile = off;
  if (type == QR_T_Q8_0 || type == QR_T_Q6_K) off += stage_bytes((size_t)R * qr_wrow_bytes(type, d));
  return off;
}

template <int TYPE, int NT, int Q8O>
__global__ __launch_bounds__(kWg) void k_gemv(GemvArgs g) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int d = g.d;
  const int U = qr_units(TYPE, d);
  const int nxb = d >> 5;
  const size_t rb = qr_wrow_bytes(TYPE, d);
  const int r0 = blockIdx.x * g.rows_per_wg;
  const int R = min(g.rows_per_wg, g.n - r0);
  if (R <= 0) return;

  size_t o_bd, o_bs, o_terms, o_tile;
  gemv_lds_layout(TYPE, Q8O, d, NT, g.rows_per_wg, &o_bd, &o_bs, &o_terms, &o_tile);
  constexpr int SL = q8_slots(TYPE, Q8O);
  UnitSrc S;
  S.act.q = reinterpret_cast<int8_t*>(smem);
  S.act.bd = reinterpret_cast<float*>(smem + o_bd);
  S.act.bs = reinterpret_cast<int32_t*>(smem + o_bs);
  S.tile = reinterpret_cast<const uint32_t*>(smem + o_tile);
  S.nxb = nxb;
  float* terms = reinterpret_cast<float*>(smem + o_terms);
  const int tstride = U + 1;

  const size_t gstart = (size_t)r0 * rb;
  int lds_base = 0;
  if constexpr (!Fmt<TYPE>::kDirect) {
    stage_tile(g.W, (size_t)g.n * rb, gstart, gstart + (size_t)R * rb,
               reinterpret_cast<uint32_t*>(smem + o_tile));
    lds_base = (int)(gstart & 15);
  }
  quantize_act_lds<Fmt<TYPE>::kPerm>(g.X, (size_t)g.xstride, nullptr, NT, NT, d, S.act);
  __syncthreads();

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nwaves = blockDim.x >> 6;
  const int total_units = R * U;
  for (int fu = wave * 64 + lane; fu < total_units; fu += nwaves * 64) {
    const int row = fu / U;
    const int u = fu - row * U;
    int32_t is[NT];
    unit_to_slots<TYPE, NT, Q8O>(g.W + gstart + (size_t)row * rb, lds_base + row * (int)rb, u, S,
                                 0, terms + (size_t)row * SL * tstride,
                                 (size_t)g.rows_per_wg * SL * tstride, tstride, is);
#pragma unroll
    for (int t = 0; t < NT; t++)
      if (g.acc) g.acc[((size_t)t * g.n + r0 + row) * U + u] = is[t];
    if (g.accb && blockIdx.x == 0 && row == 0) {
#pragma unroll
      for (int t = 0; t < NT; t++) g.accb[(size_t)t * U + u] = S.act.bs[t * nxb + u];
    }
  }
  __syncthreads();

  for (int i = threadIdx.x; i < R * NT; i += blockDim.x) {
    const int t = i / R, row = i - t * R;
    const float v = row_value<TYPE, Q8O>(terms + ((size_t)t * g.rows_per_wg + row) * SL * tstride,
                                         tstride, U);
    g.Y[(size_t)t * g.ystride + r0 + row] = g.R ? g.R[r0 + row] + v : v;
  }
}

// ---------------------------------------------------------------------------
// Streaming GEMV (the wave-tile engine of qr_stream.h): persistent
// workgroups of independent waves, each walking tiles of RW rows with its
// activation blocks in registers and the next tile's loads in flight while it
// sums.  NS = 1 when every slot of a lane has the same unit (U divides 64).
// ---------------------------------------------------------------------------
template <int TYPE, int NT, int NS, int Q8O>
__global__ __launch_bounds__(64 * kStreamWaves) void k_gemv_stream(GemvArgs g) {
  extern __shared__ __align__(16) uint8_t smem[];
  const TileShape sh = tile_shape(TYPE, g.d, Q8O);
  const StreamLds L = stream_lds(TYPE, NT, sh);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  uint8_t* slice = smem + (size_t)wave * L.slice;
  float* terms = reinterpret_cast<float*>(slice);
  uint32_t* stage = reinterpret_cast<uint32_t*>(slice + wave_terms_bytes(NT, sh));

  const int ntiles = (g.n + sh.RW - 1) / sh.RW;
  const int tstep = gridDim.x * kStreamWaves;
  int tile = blockIdx.x * kStreamWaves + wave;
  if (tile >= ntiles) return;  // no workgroup barriers below
  const size_t total = (size_t)g.n * sh.rb;
  const Slots sl = make_slots(sh.U, lane);
  TileRegs<TYPE> R;
  load_tile<TYPE>(g.W, total, tile * sh.RW, min(sh.RW, g.n - tile * sh.RW), sh, sl, lane, R);
  LaneAct<NT, NS> A;
  quantize_lane_act<TYPE, NT, NS>(g.X, (size_t)g.xstride, sl, sh.RW, A);
  if (g.accb && tile == 0) {
#pragma unroll
    for (int i = 0; i < NS; i++)
      if (sl.row[i] == 0)
#pragma unroll
        for (int t = 0; t < NT; t++) g.accb[t * sh.U + sl.u[i]] = A.a[t][i].bs;
  }

  for (;;) {
    const int r0 = tile * sh.RW;
    const int RWt = min(sh.RW, g.n - r0);
    if constexpr (!IsDirect<TYPE>::value) {
      stage_regs<TYPE>(R, stage, lane);
      wave_lds_sync();
    }
    tile_terms<TYPE, NT, NS, Q8O>(R, sl, RWt, r0, sh, A, stage, terms, g.acc, g.n);
    wave_lds_sync();
    const int next = tile + tstep;
    if (next < ntiles)
      load_tile<TYPE>(g.W, total, next * sh.RW, min(sh.RW, g.n - next * sh.RW), sh, sl, lane, R);
    if constexpr (q8_slots(TYPE, Q8O) == 9) {
      // eight lanes per (token, row): lane k runs accumulator k, then the
      // row's first lane adds the eight into 0.0f in lane order (groups of
      // eight lanes stay whole: RWt * NT * 8 and 64 are multiples of 8)
      for (int i = lane; i < RWt * NT * 8; i += 64) {
        const int rt = i >> 3, k = i & 7;
        const int t = rt / RWt, row = rt - t * RWt;
        const float acc = q8_chain<Q8O>(terms + (t * sh.RW + row) * 9 * sh.TS, sh.TS, sh.U, k);
        const int base = lane & ~7;
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = __shfl(acc, base + j);
        if (k == 0) {
          float sum = 0.0f;
#pragma unroll
          for (int j = 0; j < 8; j++) sum += v[j];
          g.Y[(size_t)t * g.ystride + r0 + row] = g.R ? g.R[r0 + row] + sum : sum;
        }
      }
    } else {
      for (int i = lane; i < RWt * NT; i += 64) {
        const int t = i / RWt, row = i - t * RWt;
        const float v = row_sum_seq(terms + (t * sh.RW + row) * sh.TS, sh.U);
        g.Y[(size_t)t * g.ystride + r0 + row] = g.R ? g.R[r0 + row] + v : v;
      }
    }
    if (next >= ntiles) break;
    wave_lds_sync();
    tile = next;
  }
}

// ---------------------------------------------------------------------------
// Block-per-lane GEMV for Q4_K / Q5_K (qr_blk.h): each wave walks tiles of
// RB = 64/nb rows with lane = super-block.  A tile's bytes come into the
// wave's LDS slot by DMA (coalesced 1 KiB instructions), one tile in flight
// per wave; the lane copies its block out of the slot, the slot is refilled
// with the wave's next tile, and only then are the lane's terms formed, so the
// next tile streams while this one is reduced.
//
// Start-up: the activation's DMA into an LDS staging area goes first (XS),
// then the first tile's DMA; each wave waits only for its own part of the
// activation (loads complete in issue order: at most NCH operations -- the
// tile's -- still in flight) and the workgroup quantizes it from LDS, while
// the weight stream is already on its way.  The quantizer reads only LDS, so
// the compiler has no vector load of its own to wait for and the tile DMA
// stays in flight across it.  Without staging (large activations) the
// activation is loaded into registers before the tile DMA.  ACC: the parity
// mode (int32 unit sums written out).
// ---------------------------------------------------------------------------
template <int TYPE>
__host__ __device__ constexpr size_t blk_slot_bytes() {
  return (size_t)64 * BlkFmt<TYPE>::kBytes;
}

template <int TYPE, int NT, bool XS, bool ACC>
__global__ __launch_bounds__(64 * kBlkWaves) void k_gemv_blk(GemvArgs g) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int BB = BlkFmt<TYPE>::kBytes;
  constexpr int NCH = BlkFmt<TYPE>::kChunks;
  constexpr size_t SB = blk_slot_bytes<TYPE>();
  const int nb = g.d >> 8;
  const int U = nb * 8;
  const int RB = 64 / nb;
  // wave-uniform (scalar) tile indices
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int rl = lane / nb, b = lane - rl * nb;
  const bool lane_on = rl < RB;
  const size_t rb = (size_t)nb * BB;
  const size_t tokb = act_tok_bytes(g.d);
  const int ntiles = (g.n + RB - 1) / RB;
  const int tstep = gridDim.x * kBlkWaves;
  const size_t total = (size_t)g.n * rb;
  int tile = blockIdx.x * kBlkWaves + wave;
  const size_t tile_bytes = (size_t)RB * rb;
  const size_t xsb = XS ? blk_xs_bytes(g.d, NT) : 0;
  float* xs = reinterpret_cast<float*>(smem);
  uint8_t* act = smem + xsb;
  uint8_t* slot = act + align16((size_t)NT * tokb) + (size_t)wave * SB;
  const uint32_t sbase = lds_u32addr(slot);

  // DMA of tile t into the slot: NCH KiB (64 blocks) from the tile's start
  // when they all lie inside the matrix (bytes past the tile's rows land in
  // slot bytes that only lanes without a row read); otherwise lanes past the
  // tile's end are clamped (tile_dma)
  auto dma = [&](int t) {
    if (t >= ntiles) return;
    const uint8_t* src = g.W + (size_t)t * tile_bytes;
    if ((size_t)t * tile_bytes + (size_t)NCH * 1024 <= total) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slot's earlier reads are done
#pragma unroll
      for (int k = 0; k < NCH; k++)
        lds_dma16_nt(src + k * 1024 + lane * 16, sbase + (uint32_t)(k * 1024));
    } else {
      tile_dma<NCH>(src, slot, (g.n - t * RB) * (int)rb, lane);
    }
  };
  ActPre pre;
  if constexpr (XS) {
    stage_act_dma(g.X, (size_t)g.xstride, NT, g.d, smem, wave, lane);
    const bool has = tile < ntiles;
    dma(tile);
    if (has) wait_vmcnt<NCH>();
    else wait_vmcnt<0>();
    quantize_act_blk<BlkFmt<TYPE>::kNib, kActLds>(g.X, (size_t)g.xstride, NT, g.d, act, pre, xs);
  } else {
    // the compiler's wait for these loads also covers the first tile's DMA
    act_prefetch(g.X, (size_t)g.xstride, NT, g.d, pre);
    dma(tile);
    quantize_act_blk<BlkFmt<TYPE>::kNib>(g.X, (size_t)g.xstride, NT, g.d, act, pre);
  }
  // LDS-only barrier: the tile DMA stays in flight across it
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  if constexpr (ACC) {
    if (g.accb && blockIdx.x == 0) {
      for (int i = threadIdx.x; i < NT * U; i += blockDim.x) {
        const int t = i / U, u = i - t * U;
        g.accb[i] = reinterpret_cast<const int*>(act + (size_t)t * tokb + act_off(u) + 44)[0];
      }
    }
  }
  if (tile >= ntiles) return;  // no barriers below

  for (;;) {
    wait_vmcnt<0>();
    uint4 c[NCH];
    {
      const uint4* q = reinterpret_cast<const uint4*>(slot + (size_t)lane * BB);
#pragma unroll
      for (int k = 0; k < NCH; k++) c[k] = q[k];
    }
    const int cur = tile;
    tile += tstep;
    dma(tile);
    const int row = cur * RB + rl;
    const bool live = lane_on && row < g.n;
    float terms[NT][8];
    int32_t isums[NT][8];
    blk_terms<TYPE, NT>(c, b, act, tokb, terms, isums);
    if constexpr (ACC) {
      if (g.acc && live) {
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
          for (int q = 0; q < 8; q++) g.acc[((size_t)t * g.n + row) * U + 8 * b + q] = isums[t][q];
      }
    }
    float y[NT];
    blk_chain<NT>(terms, b, nb, y);
    if (live && b == nb - 1) {
#pragma unroll
      for (int t = 0; t < NT; t++) g.Y[(size_t)t * g.ystride + row] = g.R ? g.R[row] + y[t] : y[t];
    }
    if (tile >= ntiles) break;
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
size_t gemv_lds_bytes(int type, int q8o, int d, int nt, int R) {
  size_t a, b, c, e;
  return gemv_lds_layout(type, q8o, d, nt, R, &a, &b, &c, &e);
}

// Compute units of the current device (cached per device).
int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int cu = 0;
    if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cu <= 0)
      cu = 256;
    cached[dev] = cu;
  }
  return cached[dev];
}

bool gemv_stream_ok(int type, int q8o, int d, int nt) {
  if (type == QR_T_F32) return false;
  const TileShape sh = tile_shape(type, d, q8o);
  if (sh.RW < 1 || (d & 3)) return false;
  // activation registers: nt blocks per distinct slot unit (1 when U divides
  // 64, else kUPL); more than 4 blocks per lane spill
  const int ns = (64 % sh.U == 0) ? 1 : kUPL;
  if (nt * ns > 4) return false;
  return stream_lds(type, nt, sh).total <= 64 * 1024;
}

// Workgroups per CU of the streaming kernel: 3 for one or two tokens, 2 for
// more, fewer where LDS does not hold that many.  Measured on 32000 x 2048
// Q6_K / Q8_0 and the 151936 x 2048 Q6_K lm_head: 3 per CU streams 4.3 TB/s
// for one token where 2 and 4 give 3.6-4.0 and 1 gives 2.6; with 4 tokens 2
// per CU takes 28.9 us where 3 takes 33.8 (Q6_K) and 40.8 (Q8_0).
template <int TYPE, int NT, int Q8O>
static hipError_t launch_stream_t(const GemvArgs& a, hipStream_t st) {
  const TileShape sh = tile_shape(TYPE, a.d, Q8O);
  const size_t lds = stream_lds(TYPE, NT, sh).total;
  const int ntiles = (a.n + sh.RW - 1) / sh.RW;
  const int want = (ntiles + kStreamWaves - 1) / kStreamWaves;
  constexpr int kDefault = NT > 2 ? 2 : 3;
  int per_cu = lds > 0 ? (int)((160 * 1024) / lds) : kDefault;
  per_cu = per_cu < 1 ? 1 : (per_cu > kDefault ? kDefault : per_cu);
  // no more than stay resident by registers (Q8_0 at two tokens in the AVX2 /
  // AVX-512 orders holds 190: two per CU)
  static std::atomic<int> by_regs[2];  // the two kernel forms below
  const bool one = 64 % sh.U == 0;
  const void* fn = one ? (const void*)k_gemv_stream<TYPE, NT, 1, Q8O>
                       : (const void*)k_gemv_stream<TYPE, 1, kUPL, Q8O>;
  per_cu = std::min(per_cu, resident_by_regs(fn, 64 * kStreamWaves, by_regs[one ? 0 : 1]));
  const int cap = device_cus() * per_cu;
  const int grid = want < cap ? want : cap;
  if (grid <= 0) return hipSuccess;
  if (64 % sh.U == 0) {
    hipLaunchKernelGGL((k_gemv_stream<TYPE, NT, 1, Q8O>), dim3(grid), dim3(64 * kStreamWaves), lds,
                       st, a);
  } else {
    if constexpr (NT == 1)
      hipLaunchKernelGGL((k_gemv_stream<TYPE, 1, kUPL, Q8O>), dim3(grid), dim3(64 * kStreamWaves),
                         lds, st, a);
    else
      return hipErrorInvalidValue;  // excluded by gemv_stream_ok
  }
  return hipGetLastError();
}

// Rows per workgroup: enough workgroups to cover the 256 CUs several times,
// at most 16 units per thread, and an LDS footprint that leaves room for
// several workgroups per CU.
int gemv_rows_per_wg(int type, int q8o, int n, int d, int nt) {
  const int U = qr_units(type, d);
  int R = 64;
  while (R > 1 && ((n + R - 1) / R < 1024 || (size_t)R * U > 16 * kWg)) R >>= 1;
  while (R > 1 && gemv_lds_bytes(type, q8o, d, nt, R) > 48 * 1024) R >>= 1;
  return R;
}

template <int TYPE, int NT, int Q8O>
static hipError_t launch_t(const GemvArgs& a, hipStream_t st) {
  const size_t lds = gemv_lds_bytes(TYPE, Q8O, a.d, NT, a.rows_per_wg);
  const int U = qr_units(TYPE, a.d);
  int threads = ((a.rows_per_wg * U + 63) / 64) * 64;
  threads = threads < 64 ? 64 : (threads > kWg ? kWg : threads);
  const int grid = (a.n + a.rows_per_wg - 1) / a.rows_per_wg;
  if (lds > 64 * 1024) return hipErrorInvalidValue;  // dynamic LDS without an opt-in
  hipLaunchKernelGGL((k_gemv<TYPE, NT, Q8O>), dim3(grid), dim3(threads), lds, st, a);
  return hipGetLastError();
}

template <int TYPE>
static size_t blk_lds_bytes(int d, int nt, int D, bool xs) {
  return (xs ? blk_xs_bytes(d, nt) : 0) + align16((size_t)nt * act_tok_bytes(d)) +
         (size_t)kBlkWaves * D * blk_slot_bytes<TYPE>();
}
static size_t blk_lds_bytes_t(int type, int d, int nt, int D, bool xs) {
  return type == QR_T_Q4_K ? blk_lds_bytes<QR_T_Q4_K>(d, nt, D, xs)
                           : blk_lds_bytes<QR_T_Q5_K>(d, nt, D, xs);
}
constexpr size_t kLdsMax = 160 * 1024;  // LDS per workgroup on gfx950

bool gemv_blk_ok(int type, int d, int nt) {
  if (type != QR_T_Q4_K && type != QR_T_Q5_K) return false;
  const int nb = d >> 8;
  if (nb < 1 || nb > 64 || (d & 3) || nt > 4) return false;
  return blk_lds_bytes_t(type, d, nt, 1, false) <= kLdsMax;
}

// Opt a kernel into LDS beyond 64 KiB, once per device.
// done[dev] records the opt-in per device (several host threads may race to
// make it; the attribute call is idempotent).
hipError_t lds_opt_in(const void* fn, std::atomic<bool>* done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  if (!done[dev].load(std::memory_order_acquire)) {
    // the dynamic allowance is what the kernel's static LDS leaves of the CU's
    hipFuncAttributes fa;
    e = hipFuncGetAttributes(&fa, fn);
    if (e != hipSuccess) return e;
    const size_t stat = fa.sharedSizeBytes;
    if (stat >= kLdsMax) return hipErrorInvalidValue;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(kLdsMax - stat));
    if (e != hipSuccess) return e;
    done[dev].store(true, std::memory_order_release);
  }
  return hipSuccess;
}

int resident_by_regs(const void* fn, int threads, std::atomic<int>& cache) {
  int v = cache.load(std::memory_order_relaxed);
  if (v > 0) return v;
  int nb = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, threads, 0) != hipSuccess) {
    (void)hipGetLastError();  // not this launch's error; leave the grid unbounded by it
    nb = 64;
  }
  v = nb < 1 ? 1 : nb;
  cache.store(v, std::memory_order_relaxed);
  return v;
}

template <int TYPE, int NT, bool XS, bool ACC>
static hipError_t launch_blk_k(const GemvArgs& a, int grid, size_t lds, hipStream_t st) {
  static std::atomic<bool> opted[64];
  if (lds > 64 * 1024) {
    hipError_t e = lds_opt_in((const void*)k_gemv_blk<TYPE, NT, XS, ACC>, opted);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((k_gemv_blk<TYPE, NT, XS, ACC>), dim3(grid), dim3(64 * kBlkWaves), lds, st, a);
  return hipGetLastError();
}

// One tile in flight per wave and as many workgroups per CU as LDS holds, up
// to three.  Measured on the 32000 x 2048 Q4_K GEMV: three per CU (48 KiB
// each) take 8.39 us per launch against 8.65 us at two; two tiles in flight
// per wave measured slower (9.2 us and more: the memory system then serves
// every wave's tiles late, and the arithmetic bunches at the end).  The
// activation is staged through LDS by DMA when it fits kXsMax, else loaded
// into registers (d = 5632 at 3 or 4 tokens).
template <int TYPE, int NT>
static hipError_t launch_blk_t(const GemvArgs& a, hipStream_t st) {
  const int nb = a.d >> 8;
  const int RB = 64 / nb;
  const bool xs = blk_xs_bytes(a.d, NT) <= kXsMax;
  const size_t lds = blk_lds_bytes<TYPE>(a.d, NT, 1, xs);
  if (lds > kLdsMax) return hipErrorInvalidValue;  // excluded by gemv_blk_ok
  const int ntiles = (a.n + RB - 1) / RB;
  const int want = (ntiles + kBlkWaves - 1) / kBlkWaves;
  int per_cu = (int)(kLdsMax / lds);
  per_cu = per_cu < 1 ? 1 : (per_cu > 3 ? 3 : per_cu);
  const int cap = device_cus() * per_cu;
  const int grid = want < cap ? want : cap;
  if (grid <= 0) return hipSuccess;
  const bool acc = a.acc || a.accb;
  if (xs) return acc ? launch_blk_k<TYPE, NT, true, true>(a, grid, lds, st)
                     : launch_blk_k<TYPE, NT, true, false>(a, grid, lds, st);
  return acc ? launch_blk_k<TYPE, NT, false, true>(a, grid, lds, st)
             : launch_blk_k<TYPE, NT, false, false>(a, grid, lds, st);
}

template <int TYPE, int NT, int Q8O>
static hipError_t launch_any_t(const GemvArgs& a, hipStream_t st) {
  if constexpr ((TYPE == QR_T_Q4_K || TYPE == QR_T_Q5_K) && NT <= 4) {
    if (gemv_blk_ok(TYPE, a.d, NT)) return launch_blk_t<TYPE, NT>(a, st);
  }
  if constexpr (NT <= 4) {
    if (gemv_stream_ok(TYPE, Q8O, a.d, NT)) return launch_stream_t<TYPE, NT, Q8O>(a, st);
  }
  return launch_t<TYPE, NT, Q8O>(a, st);
}

template <int TYPE, int Q8O>
static hipError_t launch_nt(const GemvArgs& a, int nt, hipStream_t st) {
  switch (nt) {
    case 1: return launch_any_t<TYPE, 1, Q8O>(a, st);
    case 2: return launch_any_t<TYPE, 2, Q8O>(a, st);
    case 3: return launch_any_t<TYPE, 3, Q8O>(a, st);
    case 4: return launch_any_t<TYPE, 4, Q8O>(a, st);
    case 8: return launch_any_t<TYPE, 8, Q8O>(a, st);
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------
// Tiled-layout GEMV (qr_tiled.h).
// ---------------------------------------------------------------------------
size_t tiled_lds_bytes(int type, int d, int nt, int nw) {
  const int nch = type == QR_T_Q4_K ? TiledFmt<QR_T_Q4_K>::kChunks : TiledFmt<QR_T_Q5_K>::kChunks;
  return align16((size_t)nt * act_tok_bytes(d)) + (size_t)nw * nch * 1024;
}

static size_t sq_lds_bytes(int type, int d, int nt, int nw) {
  return align16((size_t)nt * act_tok_bytes(d)) + (size_t)nw * sq_slot_kib(type) * 1024;
}

bool gemv_tiled_ok(int type, int n, int d, int nt, int q8o) {
  if (!(nt >= 1 && nt <= 4) && nt != 8) return false;
  if (type == QR_T_Q6_K || type == QR_T_Q8_0) {
    // the Q8_0 lane orders keep eight accumulators per row: streaming engine only
    if (!sq_shape_ok(type, n, d) || (type == QR_T_Q8_0 && q8o != kQ8Seq)) return false;
    return sq_lds_bytes(type, d, nt == 8 ? 4 : nt, 2) <= kLdsMax;
  }
  if (type != QR_T_Q4_K && type != QR_T_Q5_K) return false;
  if (d <= 0 || (d & 255) || (d >> 8) > 64) return false;
  return tiled_lds_bytes(type, d, nt == 8 ? 4 : nt, 4) <= kLdsMax;
}

// Q6_K / Q8_0 (qr_tiled_sq.h): four waves per workgroup (a 14 / 17 KiB slot
// each; two where four do not fit beside a long activation), as many
// workgroups per CU as the LDS holds (up to 4), the waves then walking their
// tiles.
template <int TYPE, int NT, int NW>
static hipError_t launch_sq_nw(const GemvArgs& a, hipStream_t st) {
  static std::atomic<bool> opted[64];
  const SqGeom g = sq_geom(TYPE, a.n, a.d);
  if (g.ntiles <= 0) return hipSuccess;
  const size_t lds = sq_lds_bytes(TYPE, a.d, NT, NW);
  if (lds > 64 * 1024) {
    hipError_t e = lds_opt_in((const void*)k_gemv_tiled_sq<TYPE, NT, NW>, opted);
    if (e != hipSuccess) return e;
  }
  int per_cu = (int)(kLdsMax / lds);
  per_cu = per_cu < 1 ? 1 : (per_cu > 4 ? 4 : per_cu);
  const int want = (g.ntiles + NW - 1) / NW;
  const int cap = device_cus() * per_cu;
  const int grid = want < cap ? want : cap;
  hipLaunchKernelGGL((k_gemv_tiled_sq<TYPE, NT, NW>), dim3(grid), dim3(64 * NW), lds, st, a);
  return hipGetLastError();
}
template <int TYPE, int NT>
static hipError_t launch_sq_t(const GemvArgs& a, hipStream_t st) {
  if (sq_lds_bytes(TYPE, a.d, NT, 4) <= kLdsMax) return launch_sq_nw<TYPE, NT, 4>(a, st);
  return launch_sq_nw<TYPE, NT, 2>(a, st);
}

template <int TYPE>
static hipError_t launch_sq_type(GemvArgs a, int nt, hipStream_t st) {
  switch (nt) {
    case 1: return launch_sq_t<TYPE, 1>(a, st);
    case 2: return launch_sq_t<TYPE, 2>(a, st);
    case 3: return launch_sq_t<TYPE, 3>(a, st);
    case 4: return launch_sq_t<TYPE, 4>(a, st);
    case 8: {  // two launches of four tokens
      hipError_t e = launch_sq_t<TYPE, 4>(a, st);
      if (e != hipSuccess) return e;
      a.X += (size_t)4 * a.xstride;
      a.Y += (size_t)4 * a.ystride;
      return launch_sq_t<TYPE, 4>(a, st);
    }
    default: return hipErrorInvalidValue;
  }
}

template <int TYPE, int NT, int NW, int PRO>
static hipError_t launch_tiled_k(const GemvArgs& a, int grid, size_t lds, hipStream_t st) {
  static std::atomic<bool> opted[64];
  if (lds > 64 * 1024) {
    hipError_t e = lds_opt_in((const void*)k_gemv_tiled<TYPE, NT, NW, PRO>, opted);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((k_gemv_tiled<TYPE, NT, NW, PRO>), dim3(grid), dim3(64 * NW), lds, st, a);
  return hipGetLastError();
}

template <int TYPE, int NT, int NW>
static hipError_t launch_tiled_nw(const GemvArgs& a, int grid, size_t lds, hipStream_t st) {
  constexpr int QW = NW < 4 ? NW : 4;
  const int groups = NT * (a.d >> 3);
  if (groups <= 64 * QW) return launch_tiled_k<TYPE, NT, NW, kProAsm1>(a, grid, lds, st);
  if (groups <= 128 * QW) return launch_tiled_k<TYPE, NT, NW, kProAsm2>(a, grid, lds, st);
  return launch_tiled_k<TYPE, NT, NW, kProLate>(a, grid, lds, st);
}

// Waves per workgroup: 8 where two such workgroups fit a CU's LDS and the
// tiles give every CU one, else 4 (four quantizing waves either way).  The
// grid is at most what stays resident (as many workgroups per CU as LDS
// holds, up to 4); the waves then walk their tiles.  Measured on the
// 32000 x 2048 Q4_K GEMV (4000 tiles): 8 waves, two workgroups per CU (every
// wave one tile), 7.65 us; 4 waves, four per CU, 7.9 us; 16 waves, one per
// CU, 8.3 us.
template <int TYPE, int NT>
static hipError_t launch_tiled_t(const GemvArgs& a, hipStream_t st) {
  const TiledGeom g = tiled_geom(TYPE, a.n, a.d);
  if (g.ntiles <= 0) return hipSuccess;
  const int cus = device_cus();
  const int nw =
      (2 * tiled_lds_bytes(TYPE, a.d, NT, 8) <= kLdsMax && (g.ntiles + 7) / 8 >= cus) ? 8 : 4;
  const size_t lds = tiled_lds_bytes(TYPE, a.d, NT, nw);
  int per_cu = (int)(kLdsMax / lds);
  per_cu = per_cu < 1 ? 1 : (per_cu > 4 ? 4 : per_cu);
  const int want = (g.ntiles + nw - 1) / nw;
  const int grid = want < cus * per_cu ? want : cus * per_cu;
  if (nw == 8) return launch_tiled_nw<TYPE, NT, 8>(a, grid, lds, st);
  return launch_tiled_nw<TYPE, NT, 4>(a, grid, lds, st);
}

template <int TYPE>
static hipError_t launch_tiled_type(GemvArgs a, int nt, hipStream_t st) {
  switch (nt) {
    case 1: return launch_tiled_t<TYPE, 1>(a, st);
    case 2: return launch_tiled_t<TYPE, 2>(a, st);
    case 3: return launch_tiled_t<TYPE, 3>(a, st);
    case 4: return launch_tiled_t<TYPE, 4>(a, st);
    case 8: {  // two launches of four tokens
      hipError_t e = launch_tiled_t<TYPE, 4>(a, st);
      if (e != hipSuccess) return e;
      a.X += (size_t)4 * a.xstride;
      a.Y += (size_t)4 * a.ystride;
      return launch_tiled_t<TYPE, 4>(a, st);
    }
    default: return hipErrorInvalidValue;
  }
}

hipError_t gemv_tiled_launch(int type, const void* W, const float* X, float* Y, int n, int d,
                             int nt, int xstride, int ystride, hipStream_t st, int q8o,
                             const float* R) {
  if (R && nt != 1) return hipErrorInvalidValue;
  GemvArgs a{};
  a.R = R;
  a.W = static_cast<const uint8_t*>(W);
  a.X = X;
  a.Y = Y;
  a.n = n;
  a.d = d;
  a.xstride = xstride;
  a.ystride = ystride;
  a.rows_per_wg = 0;
  a.acc = nullptr;
  a.accb = nullptr;
  if (type == QR_T_Q6_K || type == QR_T_Q8_0) {
    if (!gemv_tiled_ok(type, n, d, nt, q8o)) return hipErrorInvalidValue;
    const SqGeom g = sq_geom(type, n, d);
    a.t_nb = g.nb;
    a.t_rb = g.RB;
    a.t_ntiles = g.ntiles;
    a.t_tile_bytes = g.tile_bytes;
    if (type == QR_T_Q6_K) return launch_sq_type<QR_T_Q6_K>(a, nt, st);
    return launch_sq_type<QR_T_Q8_0>(a, nt, st);
  }
  const TiledGeom g = tiled_geom(type, n, d);
  a.t_nb = g.nb;
  a.t_rb = g.RB;
  a.t_ntiles = g.ntiles;
  a.t_tile_bytes = g.tile_bytes;
  if (type == QR_T_Q4_K) return launch_tiled_type<QR_T_Q4_K>(a, nt, st);
  if (type == QR_T_Q5_K) return launch_tiled_type<QR_T_Q5_K>(a, nt, st);
  return hipErrorInvalidValue;
}

// The normalising start-up (kProNorm): LDS of the one-token kernel plus the
// normalised vector and its scale.
static size_t tiled_norm_lds(int type, int d, int nw) {
  return tiled_lds_bytes(type, d, 1, nw) + (size_t)d * 4 + 16;
}

bool gemv_tiled_norm_ok(int type, int d) {
  return (type == QR_T_Q4_K || type == QR_T_Q5_K) && d % 256 == 0 && (d >> 8) <= 64 &&
         d <= kNormFuseMax && tiled_norm_lds(type, d, 4) <= kLdsMax;
}

template <int TYPE>
static hipError_t launch_tiled_norm(const GemvArgs& a, hipStream_t st) {
  const TiledGeom g = tiled_geom(TYPE, a.n, a.d);
  if (g.ntiles <= 0) return hipSuccess;
  const int cus = device_cus();
  const size_t lds8 = tiled_norm_lds(TYPE, a.d, 8);
  const int nw = (2 * lds8 <= kLdsMax && (g.ntiles + 7) / 8 >= cus) ? 8 : 4;
  const size_t lds = tiled_norm_lds(TYPE, a.d, nw);
  int per_cu = (int)(kLdsMax / lds);
  per_cu = per_cu < 1 ? 1 : (per_cu > 4 ? 4 : per_cu);
  // every workgroup is resident at once (each forms the same chain; a second
  // wave of workgroups would form it again after the first)
  const int want = (g.ntiles + nw - 1) / nw;
  const int grid = want < cus * per_cu ? want : cus * per_cu;
  if (nw == 8) return launch_tiled_k<TYPE, 1, 8, kProNorm>(a, grid, lds, st);
  return launch_tiled_k<TYPE, 1, 4, kProNorm>(a, grid, lds, st);
}

// Two matrices after one normalisation (k_gemv_norm2): a tiled Q4_K / Q5_K
// matrix A and a tiled Q6_K / Q8_0 matrix B, four waves per workgroup.
static size_t norm2_lds(int ta, int tb, int d) {
  const size_t la = tiled_norm_lds(ta, d, 4);
  const size_t lb = sq_lds_bytes(tb, d, 1, 4) + (size_t)d * 4 + 16;
  return la > lb ? la : lb;
}

bool gemv_norm2_ok(int ta, int tb, int nb_rows, int d) {
  return gemv_tiled_norm_ok(ta, d) && (tb == QR_T_Q6_K || tb == QR_T_Q8_0) &&
         sq_shape_ok(tb, nb_rows, d) &&
         norm2_lds(ta, tb, d) <= kLdsMax;
}

template <int TA, int TB>
static hipError_t launch_norm2(const GemvArgs& a, const GemvArgs& b, hipStream_t st) {
  static std::atomic<bool> opted[64];
  const size_t lds = norm2_lds(TA, TB, a.d);
  if (lds > 64 * 1024) {
    hipError_t e = lds_opt_in((const void*)k_gemv_norm2<TA, TB, 4>, opted);
    if (e != hipSuccess) return e;
  }
  // every workgroup resident at once (each forms the chain): the two roles
  // share the CUs in proportion to their tiles
  int per_cu = (int)(kLdsMax / lds);
  per_cu = per_cu < 1 ? 1 : (per_cu > 4 ? 4 : per_cu);
  const int cap = device_cus() * per_cu;
  int ga = (a.t_ntiles + 3) / 4, gb = (b.t_ntiles + 3) / 4;
  if (ga + gb > cap) {
    const int ga2 = (int)((long)cap * ga / (ga + gb));
    gb = cap - (ga2 < 1 ? 1 : ga2);
    ga = ga2 < 1 ? 1 : ga2;
    if (gb < 1) return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL((k_gemv_norm2<TA, TB, 4>), dim3(ga + gb), dim3(256), lds, st, a, b, ga);
  return hipGetLastError();
}

hipError_t gemv_norm2_launch(int ta, const void* Wa, float* Ya, int na, int tb, const void* Wb,
                             float* Yb, int nb_rows, const float* x, const float* nw, float* xb,
                             int d, hipStream_t st) {
  if (!gemv_norm2_ok(ta, tb, nb_rows, d) || na <= 0 || nb_rows <= 0) return hipErrorInvalidValue;
  GemvArgs a{}, b{};
  a.W = static_cast<const uint8_t*>(Wa);
  b.W = static_cast<const uint8_t*>(Wb);
  a.X = b.X = x;
  a.nw = b.nw = nw;
  a.nxb = xb;  // the q / k role's workgroup 0 stores the normalised vector
  a.Y = Ya;
  b.Y = Yb;
  a.n = na;
  b.n = nb_rows;
  a.d = b.d = d;
  a.xstride = b.xstride = d;
  a.ystride = na;
  b.ystride = nb_rows;
  const TiledGeom g = tiled_geom(ta, na, d);
  a.t_nb = g.nb;
  a.t_rb = g.RB;
  a.t_ntiles = g.ntiles;
  a.t_tile_bytes = g.tile_bytes;
  const SqGeom h = sq_geom(tb, nb_rows, d);
  b.t_nb = h.nb;
  b.t_rb = h.RB;
  b.t_ntiles = h.ntiles;
  b.t_tile_bytes = h.tile_bytes;
  if (ta == QR_T_Q4_K)
    return tb == QR_T_Q6_K ? launch_norm2<QR_T_Q4_K, QR_T_Q6_K>(a, b, st)
                           : launch_norm2<QR_T_Q4_K, QR_T_Q8_0>(a, b, st);
  return tb == QR_T_Q6_K ? launch_norm2<QR_T_Q5_K, QR_T_Q6_K>(a, b, st)
                         : launch_norm2<QR_T_Q5_K, QR_T_Q8_0>(a, b, st);
}

hipError_t gemv_tiled_norm_launch(int type, const void* W, const float* x, const float* nw,
                                  float* xb, float* Y, int n, int d, hipStream_t st) {
  if (!gemv_tiled_norm_ok(type, d)) return hipErrorInvalidValue;
  GemvArgs a{};
  a.W = static_cast<const uint8_t*>(W);
  a.X = x;
  a.Y = Y;
  a.n = n;
  a.d = d;
  a.xstride = d;
  a.ystride = n;
  a.nw = nw;
  a.nxb = xb;
  const TiledGeom g = tiled_geom(type, n, d);
  a.t_nb = g.nb;
  a.t_rb = g.RB;
  a.t_ntiles = g.ntiles;
  a.t_tile_bytes = g.tile_bytes;
  if (type == QR_T_Q4_K) return launch_tiled_norm<QR_T_Q4_K>(a, st);
  return launch_tiled_norm<QR_T_Q5_K>(a, st);
}

// ---------------------------------------------------------------------------
// llama.cpp / ggml K-quants against Q8_K (qr_ggml.h).
// ---------------------------------------------------------------------------
static bool ggml_xs(int d, int nt) { return blk_xs_bytes(d, nt) <= kXsMax; }
// The register start-up: one token, Q4_K / Q5_K, G = d / 2048 groups of 8
// per thread (G <= 2)
static int ggml_regs_g(int type, int d, int nt) {
  if (nt != 1 || (type != kGgmlQ4 && type != kGgmlQ5)) return 0;
  return d <= 2048 ? 1 : d <= 4096 ? 2 : 0;
}
static size_t ggml_lds_bytes(int type, int d, int nt, int xm) {
  const int ndma = type == kGgmlQ4 ? GgmlFmt<kGgmlQ4>::kDma
                   : type == kGgmlQ5 ? GgmlFmt<kGgmlQ5>::kDma : GgmlFmt<kGgmlQ6>::kDma;
  return (xm == kXmLds ? blk_xs_bytes(d, nt) : 0) + align16((size_t)nt * q8k_tok_bytes(d)) +
         (size_t)4 * ndma * 1024;
}
static int ggml_xm(int type, int d, int nt) {
  return ggml_regs_g(type, d, nt) ? kXmRegs : ggml_xs(d, nt) ? kXmLds : kXmLate;
}

bool gemv_ggml_ok(int type, int d, int nt) {
  if (type != kGgmlQ4 && type != kGgmlQ5 && type != kGgmlQ6) return false;
  if (d <= 0 || (d & 255) || (d >> 8) > 64) return false;
  if (!(nt >= 1 && nt <= 4) && nt != 8) return false;
  const int n4 = nt == 8 ? 4 : nt;
  return ggml_lds_bytes(type, d, n4, ggml_xm(type, d, n4)) <= kLdsMax;
}

template <int T, int NT, int XM, int G = 1>
static hipError_t launch_ggml_x(const GemvArgs& a, hipStream_t st, int pairs = 0) {
  static std::atomic<bool> opted[64];
  const int nb = a.d >> 8, RB = 64 / nb;
  const int ntiles = (a.n + RB - 1) / RB;
  const size_t lds = ggml_lds_bytes(T, a.d, NT, XM);
  if (lds > 64 * 1024) {
    hipError_t e = lds_opt_in((const void*)k_gemv_ggml<T, NT, XM, G>, opted);
    if (e != hipSuccess) return e;
  }
  static std::atomic<int> by_regs{0};
  int per_cu = (int)(kLdsMax / lds);
  per_cu = per_cu < 1 ? 1 : (per_cu > 4 ? 4 : per_cu);
  // a grid beyond what stays resident would leave its last workgroups a round
  // of their own after the others (Q4_K at 4 tokens holds 209 registers: two
  // workgroups per CU, not the four its LDS allows)
  per_cu = std::min(per_cu, resident_by_regs((const void*)k_gemv_ggml<T, NT, XM, G>, 256, by_regs));
  const int want = (ntiles + 3) / 4;
  // pair mode: the pairs' matrices share the resident workgroups
  const int cap = pairs > 0 ? (device_cus() * per_cu + pairs - 1) / pairs : device_cus() * per_cu;
  // as few rounds of the resident grid as the tiles need, the tiles spread
  // evenly over them (every wave the same number of tiles, give or take one)
  const int rounds = (want + cap - 1) / cap;
  int grid = (want + rounds - 1) / rounds;
  if (grid < 1) grid = 1;
  if (ntiles <= 0) return hipSuccess;
  hipLaunchKernelGGL((k_gemv_ggml<T, NT, XM, G>), dim3(grid, pairs > 0 ? pairs : 1), dim3(256),
                     lds, st, a);
  return hipGetLastError();
}

template <int T, int NT>
static hipError_t launch_ggml_t(const GemvArgs& a, hipStream_t st, int pairs = 0) {
  if constexpr (NT == 1 && (T == kGgmlQ4 || T == kGgmlQ5)) {
    const int G = ggml_regs_g(T, a.d, NT);
    if (G == 1) return launch_ggml_x<T, 1, kXmRegs, 1>(a, st, pairs);
    if (G == 2) return launch_ggml_x<T, 1, kXmRegs, 2>(a, st, pairs);
  }
  return ggml_xs(a.d, NT) ? launch_ggml_x<T, NT, kXmLds>(a, st, pairs)
                          : launch_ggml_x<T, NT, kXmLate>(a, st, pairs);
}

template <int T>
static hipError_t launch_ggml_type(GemvArgs a, int nt, hipStream_t st) {
  switch (nt) {
    case 1: return launch_ggml_t<T, 1>(a, st);
    case 2: return launch_ggml_t<T, 2>(a, st);
    case 3: return launch_ggml_t<T, 3>(a, st);
    case 4: return launch_ggml_t<T, 4>(a, st);
    case 8: {
      hipError_t e = launch_ggml_t<T, 4>(a, st);
      if (e != hipSuccess) return e;
      a.X += (size_t)4 * a.xstride;
      a.Y += (size_t)4 * a.ystride;
      return launch_ggml_t<T, 4>(a, st);
    }
    default: return hipErrorInvalidValue;
  }
}

hipError_t gemv_ggml_launch(int type, const void* W, const float* X, float* Y, int n, int d, int nt,
                            int xstride, int ystride, hipStream_t st, const float* R) {
  if (R && nt != 1) return hipErrorInvalidValue;
  GemvArgs a{};
  a.R = R;
  a.W = static_cast<const uint8_t*>(W);
  a.X = X;
  a.Y = Y;
  a.n = n;
  a.d = d;
  a.xstride = xstride;
  a.ystride = ystride;
  if (type == kGgmlQ4) return launch_ggml_type<kGgmlQ4>(a, nt, st);
  if (type == kGgmlQ5) return launch_ggml_type<kGgmlQ5>(a, nt, st);
  if (type == kGgmlQ6) return launch_ggml_type<kGgmlQ6>(a, nt, st);
  return hipErrorInvalidValue;
}

// Expert products of llama.cpp-layout experts, one GEMV per (token, slot)
// pair p: Y[p] = W_{eidx[p]} . X[p / xk] (n rows of d, one token each).
hipError_t gemv_ggml_pairs_launch(int type, const void* W, size_t eslice, const int32_t* eidx,
                                  int E, int xk, const float* X, int xstride, float* Y,
                                  int ystride, int n, int d, int P, hipStream_t st) {
  if (P <= 0) return hipSuccess;
  if (!gemv_ggml_ok(type, d, 1) || xk < 1 || P > 65535) return hipErrorInvalidValue;
  GemvArgs a{};
  a.W = static_cast<const uint8_t*>(W);
  a.X = X;
  a.Y = Y;
  a.n = n;
  a.d = d;
  a.xstride = xstride;
  a.ystride = ystride;
  a.eidx = eidx;
  a.eslice = eslice;
  a.xk = xk;
  a.E = E;
  if (type == kGgmlQ4) return launch_ggml_t<kGgmlQ4, 1>(a, st, P);
  if (type == kGgmlQ5) return launch_ggml_t<kGgmlQ5, 1>(a, st, P);
  if (type == kGgmlQ6) return launch_ggml_t<kGgmlQ6, 1>(a, st, P);
  return hipErrorInvalidValue;
}

hipError_t quantize_q8k_launch(const float* x, void* y, long nblocks, hipStream_t st) {
  if (nblocks <= 0) return hipSuccess;
  const long grid = (nblocks + 3) / 4;
  hipLaunchKernelGGL(k_quantize_q8k, dim3((unsigned)grid), dim3(256), 0, st, x,
                     static_cast<uint8_t*>(y), nblocks);
  return hipGetLastError();
}

hipError_t ggml_dequant_launch(int type, const void* src, int rows, int n, float* out,
                               hipStream_t st) {
  const size_t rb = (size_t)(n >> 8) * (type == kGgmlQ4 ? 144 : type == kGgmlQ5 ? 176 : 210);
  long grid = ((long)rows * n + 255) / 256;
  if (grid > 4096) grid = 4096;
  if (grid <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_ggml_dequant_rows, dim3((unsigned)grid), dim3(256), 0, st,
                     static_cast<const uint8_t*>(src), type, rb, rows, n, out);
  return hipGetLastError();
}

hipError_t tile_pack_launch(int type, const void* src, void* dst, int n, int d, bool reverse,
                            hipStream_t st) {
  if (type == QR_T_Q6_K || type == QR_T_Q8_0) {
    const long per = type == QR_T_Q6_K ? SqFmt<QR_T_Q6_K>::kChunks + 1 : SqFmt<QR_T_Q8_0>::kChunks;
    const long total = (long)n * (d >> 8) * per;
    if (total <= 0) return hipSuccess;
    long grid = (total + 255) / 256;
    if (grid > 65536) grid = 65536;
    const uint8_t* s = static_cast<const uint8_t*>(src);
    uint8_t* o = static_cast<uint8_t*>(dst);
    if (type == QR_T_Q6_K)
      hipLaunchKernelGGL(k_tile_pack_sq<QR_T_Q6_K>, dim3((unsigned)grid), dim3(256), 0, st, s, o,
                         n, d, reverse ? 1 : 0);
    else
      hipLaunchKernelGGL(k_tile_pack_sq<QR_T_Q8_0>, dim3((unsigned)grid), dim3(256), 0, st, s, o,
                         n, d, reverse ? 1 : 0);
    return hipGetLastError();
  }
  const long nch = type == QR_T_Q4_K ? TiledFmt<QR_T_Q4_K>::kChunks : TiledFmt<QR_T_Q5_K>::kChunks;
  const long total = (long)n * (d >> 8) * nch;
  if (total <= 0) return hipSuccess;
  long grid = (total + 255) / 256;
  if (grid > 65536) grid = 65536;
  const uint8_t* s = static_cast<const uint8_t*>(src);
  uint8_t* o = static_cast<uint8_t*>(dst);
  if (type == QR_T_Q4_K)
    hipLaunchKernelGGL(k_tile_pack<QR_T_Q4_K>, dim3((unsigned)grid), dim3(256), 0, st, s, o, n, d,
                       reverse ? 1 : 0);
  else if (type == QR_T_Q5_K)
    hipLaunchKernelGGL(k_tile_pack<QR_T_Q5_K>, dim3((unsigned)grid), dim3(256), 0, st, s, o, n, d,
                       reverse ? 1 : 0);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t gemv_launch(int type, int q8o, const void* W, const float* X, float* Y, int n, int d,
                       int nt, int xstride, int ystride, int32_t* acc, int32_t* accb,
                       hipStream_t st, const float* R) {
  if (R && nt != 1) return hipErrorInvalidValue;
  GemvArgs a{};
  a.R = R;
  a.W = static_cast<const uint8_t*>(W);
  a.X = X;
  a.Y = Y;
  a.n = n;
  a.d = d;
  a.xstride = xstride;
  a.ystride = ystride;
  a.rows_per_wg = gemv_rows_per_wg(type, q8o, n, d, nt);
  a.acc = acc;
  a.accb = accb;
  switch (type) {
    case QR_T_Q4_K: return launch_nt<QR_T_Q4_K, kQ8Seq>(a, nt, st);
    case QR_T_Q5_K: return launch_nt<QR_T_Q5_K, kQ8Seq>(a, nt, st);
    case QR_T_Q6_K: return launch_nt<QR_T_Q6_K, kQ8Seq>(a, nt, st);
    case QR_T_Q8_0:
      switch (q8o) {
        case kQ8Seq: return launch_nt<QR_T_Q8_0, kQ8Seq>(a, nt, st);
        case kQ8Avx2: return launch_nt<QR_T_Q8_0, kQ8Avx2>(a, nt, st);
        case kQ8Avx512: return launch_nt<QR_T_Q8_0, kQ8Avx512>(a, nt, st);
        default: return hipErrorInvalidValue;
      }
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------
// fp32 GEMV in the reference's accumulation orders (router logits and F32
// weights):  out[t][r] = sum_j W[r][j] * x[t][j].
//   SEQ    matmul_ref (src/kernels.c:18-28) and matmul_q_fused's F32 rows
//          (src/quant.c:455-462): j ascending, multiply then add.
//   AVX2   matmul_omp built -mavx2 -mfma (src/kernels.c:50-65): lane k keeps
//          the FMA chain over j = 8i + k; lanes added 0..7 into 0.0f; then a
//          multiply-add tail for d % 8.
//   AVX512 matmul_omp built -mavx512f (src/kernels.c:38-49): 16 FMA chains,
//          GCC's _mm512_reduce_add_ps tree (upper 8 + lower 8, upper 4 +
//          lower 4, [0]+[2] and [1]+[3], then their sum), then the tail.
// One thread per chain; the LANES chains of one row sit in adjacent lanes.
// ---------------------------------------------------------------------------
template <int LANES>
__global__ __launch_bounds__(256) void k_gemv_f32(const float* __restrict__ W,
                                                  const float* __restrict__ X,
                                                  float* __restrict__ Y, int n, int d, int nt,
                                                  int xstride, int ystride) {
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int k = (int)(gid % LANES);
  const long rt = gid / LANES;  // (token, row) pair
  const bool live = rt < (long)n * nt;
  const int t = live ? (int)(rt / n) : 0;
  const int r = live ? (int)(rt - (long)t * n) : 0;
  const float* w = W + (size_t)r * d;
  const float* x = X + (size_t)t * xstride;
  if constexpr (LANES == 1) {
    if (!live) return;
    float s = 0.0f;
    for (int j = 0; j < d; j++) s += w[j] * x[j];
    Y[(size_t)t * ystride + r] = s;
  } else {
    const int dm = d - d % LANES;
    float acc = 0.0f;
    if (live)
      for (int j = k; j < dm; j += LANES) acc = __builtin_fmaf(w[j], x[j], acc);
    float v[LANES];
    const int base = (int)(threadIdx.x & 63) - k;
#pragma unroll
    for (int i = 0; i < LANES; i++) v[i] = __shfl(acc, base + i);
    if (!live || k != 0) return;
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
    for (int j = dm; j < d; j++) s += w[j] * x[j];
    Y[(size_t)t * ystride + r] = s;
  }
}

// LDS-staged variant: a workgroup copies RPW weight rows into LDS with one
// round trip of 128-bit loads, then LANES x RPW x TPW threads run the chains
// out of LDS (row stride RS floats, RS = 8 mod 32, so the RPW rows' chains
// read distinct banks), the activation read through the cache with the next
// 8 loads in flight.
template <int LANES>
__global__ __launch_bounds__(256) void k_gemv_f32_lds(const float* __restrict__ W,
                                                      const float* __restrict__ X,
                                                      float* __restrict__ Y, int n, int d, int nt,
                                                      int xstride, int ystride, int RPW, int RS) {
  extern __shared__ __align__(16) float sw[];
  const int TPW = 256 / (LANES * RPW);
  const int r0 = blockIdx.x * RPW;
  const int t0 = blockIdx.y * TPW;
  const int nr = min(RPW, n - r0);
  // stage rows r0 .. r0+nr-1
  if ((d & 3) == 0 && ((reinterpret_cast<uintptr_t>(W) & 15) == 0)) {
    // each thread's 8 loads of a batch are in flight before its LDS stores
    const int d4 = d >> 2;
    const int total = nr * d4;
    for (int base = 0; base < total; base += 8 * (int)blockDim.x) {
      float4 v0, v1, v2, v3, v4, v5, v6, v7;
      float4* v[8] = {&v0, &v1, &v2, &v3, &v4, &v5, &v6, &v7};
#pragma unroll
      for (int b = 0; b < 8; b++) {
        const int i = base + b * (int)blockDim.x + (int)threadIdx.x;
        const int ic = i < total ? i : 0;
        const int rr = ic / d4, j4 = ic - rr * d4;
        *v[b] = reinterpret_cast<const float4*>(W + (size_t)(r0 + rr) * d)[j4];
      }
#pragma unroll
      for (int b = 0; b < 8; b++) {
        const int i = base + b * (int)blockDim.x + (int)threadIdx.x;
        if (i < total) {
          const int rr = i / d4, j4 = i - rr * d4;
          *reinterpret_cast<float4*>(sw + rr * RS + 4 * j4) = *v[b];
        }
      }
    }
  } else {
    for (int i = threadIdx.x; i < nr * d; i += blockDim.x) {
      const int rr = i / d, j = i - rr * d;
      sw[rr * RS + j] = W[(size_t)(r0 + rr) * d + j];
    }
  }
  __syncthreads();
  const int k = threadIdx.x % LANES;
  const int rr = (threadIdx.x / LANES) % RPW;
  const int tt = threadIdx.x / (LANES * RPW);
  const bool live = rr < nr && t0 + tt < nt;
  const float* w = sw + rr * RS;
  const float* x = X + (size_t)(live ? t0 + tt : 0) * xstride;
  if constexpr (LANES == 1) {
    if (!live) return;  // no barriers below
    float s = 0.0f;
    int j = 0;
    for (; j + 8 <= d; j += 8) {
      float xv[8];
#pragma unroll
      for (int q = 0; q < 8; q++) xv[q] = x[j + q];
#pragma unroll
      for (int q = 0; q < 8; q++) s += w[j + q] * xv[q];
    }
    for (; j < d; j++) s += w[j] * x[j];
    Y[(size_t)(t0 + tt) * ystride + r0 + rr] = s;
  } else {
    const int dm = d - d % LANES;
    float acc = 0.0f;
    if (live) {
      int j = k;
      for (; j + 7 * LANES < dm; j += 8 * LANES) {
        float xv[8];
#pragma unroll
        for (int q = 0; q < 8; q++) xv[q] = x[j + q * LANES];
#pragma unroll
        for (int q = 0; q < 8; q++) acc = __builtin_fmaf(w[j + q * LANES], xv[q], acc);
      }
      for (; j < dm; j += LANES) acc = __builtin_fmaf(w[j], x[j], acc);
    }
    float v[LANES];
    const int base = (int)(threadIdx.x & 63) - k;
#pragma unroll
    for (int i = 0; i < LANES; i++) v[i] = __shfl(acc, base + i);
    if (!live || k != 0) return;
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
    for (int j = dm; j < d; j++) s += w[j] * x[j];
    Y[(size_t)(t0 + tt) * ystride + r0 + rr] = s;
  }
}

template <int LANES>
static hipError_t launch_f32_lds(const float* W, const float* X, float* Y, int n, int d, int nt,
                                 int xstride, int ystride, hipStream_t st) {
  const int RS = ((d + 31) & ~31) + 8;
  int RPW = 4;
  while (RPW > 1 && (size_t)RPW * RS * 4 > 64 * 1024) RPW >>= 1;
  if ((size_t)RPW * RS * 4 > 64 * 1024) return hipErrorInvalidValue;
  const int TPW = 256 / (LANES * RPW);
  dim3 grid((n + RPW - 1) / RPW, (nt + TPW - 1) / TPW);
  hipLaunchKernelGGL(k_gemv_f32_lds<LANES>, grid, dim3(256), (size_t)RPW * RS * 4, st, W, X, Y, n,
                     d, nt, xstride, ystride, RPW, RS);
  return hipGetLastError();
}

hipError_t gemv_f32_launch(int order, const float* W, const float* X, float* Y, int n, int d,
                           int nt, int xstride, int ystride, hipStream_t st) {
  const int lanes = order == QR_ORDER_SEQ ? 1 : order == QR_ORDER_AVX2 ? 8 : 16;
  if (n <= 0 || nt <= 0) return hipSuccess;
  // rows that fit LDS go through the staged kernel
  if ((size_t)(((d + 31) & ~31) + 8) * 4 <= 64 * 1024) {
    switch (lanes) {
      case 1: return launch_f32_lds<1>(W, X, Y, n, d, nt, xstride, ystride, st);
      case 8: return launch_f32_lds<8>(W, X, Y, n, d, nt, xstride, ystride, st);
      default: return launch_f32_lds<16>(W, X, Y, n, d, nt, xstride, ystride, st);
    }
  }
  const long total = (long)n * nt * lanes;
  const int threads = 256;
  const long grid = (total + threads - 1) / threads;
  if (grid == 0) return hipSuccess;
  switch (lanes) {
    case 1:
      hipLaunchKernelGGL(k_gemv_f32<1>, dim3((unsigned)grid), dim3(threads), 0, st, W, X, Y, n, d,
                         nt, xstride, ystride);
      break;
    case 8:
      hipLaunchKernelGGL(k_gemv_f32<8>, dim3((unsigned)grid), dim3(threads), 0, st, W, X, Y, n, d,
                         nt, xstride, ystride);
      break;
    default:
      hipLaunchKernelGGL(k_gemv_f32<16>, dim3((unsigned)grid), dim3(threads), 0, st, W, X, Y, n,
                         d, nt, xstride, ystride);
      break;
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// quantize_row_q8_0 (src/quant.c:143-158) to block_q8_0 bytes in HBM, one
// thread per 32-element block: the activation quantizer's drop-in and the
// Q8_0 weight quantizer.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_quantize_q8_0(const float* __restrict__ x,
                                                       uint8_t* __restrict__ y, long nblocks) {
  const long b = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const float* p = x + b * 32;
  float v[32];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; j++) {
    v[j] = p[j];
    const float av = __builtin_fabsf(v[j]);
    amax = av > amax ? av : amax;
  }
  const float dd = amax / 127.0f;
  const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
  const uint32_t dh = qr_f2h(dd);
  uint8_t* o = y + b * QR_Q8_BYTES;
  o[0] = (uint8_t)(dh & 0xFFu);
  o[1] = (uint8_t)(dh >> 8);
#pragma unroll
  for (int j = 0; j < 32; j++) o[2 + j] = (uint8_t)(int8_t)(int)__builtin_rintf(v[j] * id);
}

hipError_t quantize_q8_0_launch(const float* x, void* y, long nblocks, hipStream_t st) {
  if (nblocks <= 0) return hipSuccess;
  const int threads = 256;
  const long grid = (nblocks + threads - 1) / threads;
  hipLaunchKernelGGL(k_quantize_q8_0, dim3((unsigned)grid), dim3(threads), 0, st, x,
                     static_cast<uint8_t*>(y), nblocks);
  return hipGetLastError();
}

}  // namespace qr
