// qr_moe_tn.hip -- the router side of the MoE layer for T > 1 tokens
// (src/runtime.c:202-230 applied to every token):
//
//   k_rlogits        logits[t][e] = W_r[e] . xb[t] in the reference build's
//                    accumulation order (KernelOps.matmul: SEQ / AVX2 / AVX512),
//                    a tile of tokens x router rows per workgroup from K-chunks
//                    of both double-buffered into LDS by DMA.
//   k_route_rank     one workgroup per token: softmax_ref, top-K as an exact
//                    rank over the workgroup, renormalisation; the other waves
//                    quantize the token's xb into the activation records of
//                    the grouped products meanwhile.
#include <cstdlib>

#include "qr_blk.h"
#include "qr_internal.h"
#include "qr_route.h"
#include "qr_tokens.h"

namespace qr {

// ---------------------------------------------------------------------------
// Router logits for many tokens.  Thread (k, tb, rb) of the 256 runs chain k
// of the TT x RT outputs (token tb TT + i, row rb RT + q) of the workgroup's
// tile: LANES = 1 is matmul_ref's sequential mul-then-add (src/kernels.c:18-28),
// LANES = 8 / 16 matmul_omp's FMA chains over j = k mod LANES, combined in the
// build's lane order, then the multiply-add tail (src/kernels.c:38-65).  A
// chain walks the K-chunks in order, so chunking keeps every chain's order.
// ---------------------------------------------------------------------------
constexpr int kRlCk = 256;          // elements per chunk: one 1 KiB DMA per row
constexpr int kRlRs = kRlCk + 8;    // LDS row stride (floats): 8-bank skew per row

template <int TW, int RW, int NBUF>
__host__ __device__ constexpr size_t rlogits_lds() {
  return (size_t)NBUF * (TW + RW) * kRlRs * 4;
}

// NBUF chunk buffers: NBUF - 1 chunks in flight while one is consumed.
template <int LANES, int NTB, int TT, int NRB, int RT, int NBUF>
__global__ __launch_bounds__(256) void k_rlogits(const float* __restrict__ W,
                                                 const float* __restrict__ X, int T, int E, int d,
                                                 float* __restrict__ logits) {
  static_assert(LANES * NTB * NRB == 256, "thread layout");
  constexpr int TW = NTB * TT, RW = NRB * RT;
  static_assert((TW + RW) % 4 == 0, "rows per wave");
  constexpr int NIW = (TW + RW) / 4;  // DMA instructions per wave and chunk
  static_assert(NIW * (NBUF - 1) <= 63, "vmcnt range");
  constexpr int BUF = (TW + RW) * kRlRs;
  extern __shared__ __align__(16) float sm[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int k = tid % LANES, tb = (tid / LANES) % NTB, rb = tid / (LANES * NTB);
  const int r0 = blockIdx.x * RW, t0 = blockIdx.y * TW;
  const int nch = (d + kRlCk - 1) / kRlCk;
  const int dm = d - d % LANES;

  // chunk c of LDS row i (rows 0..RW-1: router rows r0 + i, then tokens
  // t0 + i - RW; past-the-end rows and tokens reload the last one) into
  // buffer b; wave w moves rows w, w + 4, ...
  auto issue = [&](int c, int b) {
    const int nb = min(kRlCk, d - c * kRlCk) * 4;
    const int o = lane * 16;
#pragma unroll
    for (int n = 0; n < NIW; n++) {
      const int i = wave + 4 * n;
      const float* src = i < RW ? W + (size_t)min(r0 + i, E - 1) * d
                                : X + (size_t)min(t0 + i - RW, T - 1) * d;
      lds_dma16(reinterpret_cast<const uint8_t*>(src + c * kRlCk) + (o < nb ? o : 0),
                lds_u32addr(sm + b * BUF + i * kRlRs));
    }
  };

  float acc[TT][RT];
#pragma unroll
  for (int i = 0; i < TT; i++)
#pragma unroll
    for (int q = 0; q < RT; q++) acc[i][q] = 0.0f;

#pragma unroll
  for (int c = 0; c < NBUF - 1; c++)
    if (c < nch) issue(c, c);
  for (int c = 0; c < nch; c++) {
    if (c + NBUF - 1 < nch) issue(c + NBUF - 1, (c + NBUF - 1) % NBUF);
    // chunk c has landed once only the later chunks' DMA is in flight
    const int later = min(NBUF - 1, nch - 1 - c);
    switch (later) {
      case 0: wait_vmcnt<0>(); break;
      case 1: wait_vmcnt<NIW>(); break;
      case 2: wait_vmcnt<(NBUF > 2 ? 2 : 0) * NIW>(); break;
      case 3: wait_vmcnt<(NBUF > 3 ? 3 : 0) * NIW>(); break;
      case 4: wait_vmcnt<(NBUF > 4 ? 4 : 0) * NIW>(); break;
      default: wait_vmcnt<(NBUF > 5 ? 5 : 0) * NIW>(); break;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    const float* sw = sm + (c % NBUF) * BUF + (rb * RT) * kRlRs;
    const float* sx = sm + (c % NBUF) * BUF + (RW + tb * TT) * kRlRs;
    const int jend = min(dm, (c + 1) * kRlCk) - c * kRlCk;
    if (jend == kRlCk) {
      // a whole chunk, fully unrolled, each step's reads P steps ahead of
      // its adds in a register ring held there by scheduling barriers (as in
      // k_rlogits4); every chain keeps its element order
      constexpr int NS = kRlCk / LANES, P = 8;
      float wr[P][RT], xr[P][TT];
#pragma unroll
      for (int s = 0; s < P; s++) {
#pragma unroll
        for (int q = 0; q < RT; q++) wr[s][q] = sw[q * kRlRs + k + LANES * s];
#pragma unroll
        for (int i = 0; i < TT; i++) xr[s][i] = sx[i * kRlRs + k + LANES * s];
      }
#pragma unroll
      for (int s = 0; s < NS; s++) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < TT; i++)
#pragma unroll
          for (int q = 0; q < RT; q++) {
            if constexpr (LANES == 1) acc[i][q] += wr[s % P][q] * xr[s % P][i];
            else acc[i][q] = __builtin_fmaf(wr[s % P][q], xr[s % P][i], acc[i][q]);
          }
        __builtin_amdgcn_sched_barrier(0);
        if (s + P < NS) {
#pragma unroll
          for (int q = 0; q < RT; q++) wr[s % P][q] = sw[q * kRlRs + k + LANES * (s + P)];
#pragma unroll
          for (int i = 0; i < TT; i++) xr[s % P][i] = sx[i * kRlRs + k + LANES * (s + P)];
        }
      }
    } else {
#pragma unroll 4
      for (int j = k; j < jend; j += LANES) {
        float wv[RT], xv[TT];
#pragma unroll
        for (int q = 0; q < RT; q++) wv[q] = sw[q * kRlRs + j];
#pragma unroll
        for (int i = 0; i < TT; i++) xv[i] = sx[i * kRlRs + j];
#pragma unroll
        for (int i = 0; i < TT; i++)
#pragma unroll
          for (int q = 0; q < RT; q++) {
            if constexpr (LANES == 1) acc[i][q] += wv[q] * xv[i];
            else acc[i][q] = __builtin_fmaf(wv[q], xv[i], acc[i][q]);
          }
      }
    }
    if (c + NBUF < nch) {
      // every thread is done with this buffer before chunk c + NBUF lands in it
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
    }
  }

  // combine the LANES chains of each output (adjacent lanes) and add the tail
  const int base = lane - k;
  const int last0 = (nch - 1) * kRlCk;  // the tail lies in the last chunk
  const float* lw = sm + ((nch - 1) % NBUF) * BUF + (rb * RT) * kRlRs;
  const float* lx = sm + ((nch - 1) % NBUF) * BUF + (RW + tb * TT) * kRlRs;
#pragma unroll
  for (int i = 0; i < TT; i++)
#pragma unroll
    for (int q = 0; q < RT; q++) {
      const int t = t0 + tb * TT + i, e = r0 + rb * RT + q;
      float s;
      if constexpr (LANES == 1) {
        s = acc[i][q];
      } else {
        float v[LANES];
#pragma unroll
        for (int l = 0; l < LANES; l++) v[l] = __shfl(acc[i][q], base + l);
        s = 0.0f;
        if constexpr (LANES == 8) {
#pragma unroll
          for (int l = 0; l < 8; l++) s += v[l];
        } else {
          float t8[8], t4[4];
#pragma unroll
          for (int l = 0; l < 8; l++) t8[l] = v[8 + l] + v[l];
#pragma unroll
          for (int l = 0; l < 4; l++) t4[l] = t8[4 + l] + t8[l];
          const float a02 = t4[0] + t4[2];
          const float a13 = t4[1] + t4[3];
          s += a02 + a13;
        }
        for (int j = dm; j < d; j++) s += lw[q * kRlRs + j - last0] * lx[i * kRlRs + j - last0];
      }
      if (k == 0 && t < T && e < E) logits[(size_t)t * E + e] = s;
    }
}

// The FMA-chain orders with four adjacent chains per thread: thread (cg, tb,
// rb) runs chains 4 cg .. 4 cg + 3 of its TT x RT outputs, so each step reads
// one float4 per token and per row (chain k's element j = s LANES + k sits
// next to chain k + 1's); the LANES chains of an output live in LANES / 4
// adjacent lanes and are combined as above.
template <int LANES, int NTB, int TT, int NRB, int RT, int NBUF>
__global__ __launch_bounds__(256) void k_rlogits4(const float* __restrict__ W,
                                                  const float* __restrict__ X, int T, int E, int d,
                                                  float* __restrict__ logits) {
  constexpr int G = LANES / 4;  // threads per output
  static_assert(LANES == 8 || LANES == 16, "FMA-chain orders");
  static_assert(G * NTB * NRB == 256, "thread layout");
  constexpr int TW = NTB * TT, RW = NRB * RT;
  static_assert((TW + RW) % 4 == 0, "rows per wave");
  constexpr int NIW = (TW + RW) / 4;
  static_assert(NIW * (NBUF - 1) <= 63, "vmcnt range");
  constexpr int BUF = (TW + RW) * kRlRs;
  extern __shared__ __align__(16) float sm[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cg = tid % G, tb = (tid / G) % NTB, rb = tid / (G * NTB);
  const int r0 = blockIdx.x * RW, t0 = blockIdx.y * TW;
  const int nch = (d + kRlCk - 1) / kRlCk;
  const int dm = d - d % LANES;

  auto issue = [&](int c, int b) {
    const int nb = min(kRlCk, d - c * kRlCk) * 4;
    const int o = lane * 16;
#pragma unroll
    for (int n = 0; n < NIW; n++) {
      const int i = wave + 4 * n;
      const float* src = i < RW ? W + (size_t)min(r0 + i, E - 1) * d
                                : X + (size_t)min(t0 + i - RW, T - 1) * d;
      lds_dma16(reinterpret_cast<const uint8_t*>(src + c * kRlCk) + (o < nb ? o : 0),
                lds_u32addr(sm + b * BUF + i * kRlRs));
    }
  };

  float acc[TT][RT][4];
#pragma unroll
  for (int i = 0; i < TT; i++)
#pragma unroll
    for (int q = 0; q < RT; q++)
#pragma unroll
      for (int c = 0; c < 4; c++) acc[i][q][c] = 0.0f;

#pragma unroll
  for (int c = 0; c < NBUF - 1; c++)
    if (c < nch) issue(c, c);
  for (int c = 0; c < nch; c++) {
    if (c + NBUF - 1 < nch) issue(c + NBUF - 1, (c + NBUF - 1) % NBUF);
    const int later = min(NBUF - 1, nch - 1 - c);
    switch (later) {
      case 0: wait_vmcnt<0>(); break;
      case 1: wait_vmcnt<NIW>(); break;
      case 2: wait_vmcnt<(NBUF > 2 ? 2 : 0) * NIW>(); break;
      default: wait_vmcnt<(NBUF > 3 ? 3 : 0) * NIW>(); break;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    const float* sw = sm + (c % NBUF) * BUF + (rb * RT) * kRlRs;
    const float* sx = sm + (c % NBUF) * BUF + (RW + tb * TT) * kRlRs;
    const int jend = min(dm, (c + 1) * kRlCk) - c * kRlCk;
    if (jend == kRlCk) {
      // a whole chunk, fully unrolled: step s (elements 4 cg + LANES s ..)
      // reads its float4s P steps ahead into a register ring, the
      // scheduling barriers keeping them there (left alone, the scheduler
      // sinks each read to just before its FMAs and the wave waits on LDS
      // every few FMAs); each accumulator's FMAs stay in element order
      constexpr int NS = kRlCk / LANES, P = 4;
      float4 wr[P][RT], xr[P][TT];
#pragma unroll
      for (int s = 0; s < P; s++) {
#pragma unroll
        for (int q = 0; q < RT; q++)
          wr[s][q] = *reinterpret_cast<const float4*>(sw + q * kRlRs + 4 * cg + LANES * s);
#pragma unroll
        for (int i = 0; i < TT; i++)
          xr[s][i] = *reinterpret_cast<const float4*>(sx + i * kRlRs + 4 * cg + LANES * s);
      }
#pragma unroll
      for (int s = 0; s < NS; s++) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < TT; i++)
#pragma unroll
          for (int q = 0; q < RT; q++) {
            acc[i][q][0] = __builtin_fmaf(wr[s % P][q].x, xr[s % P][i].x, acc[i][q][0]);
            acc[i][q][1] = __builtin_fmaf(wr[s % P][q].y, xr[s % P][i].y, acc[i][q][1]);
            acc[i][q][2] = __builtin_fmaf(wr[s % P][q].z, xr[s % P][i].z, acc[i][q][2]);
            acc[i][q][3] = __builtin_fmaf(wr[s % P][q].w, xr[s % P][i].w, acc[i][q][3]);
          }
        __builtin_amdgcn_sched_barrier(0);
        if (s + P < NS) {
#pragma unroll
          for (int q = 0; q < RT; q++)
            wr[s % P][q] =
                *reinterpret_cast<const float4*>(sw + q * kRlRs + 4 * cg + LANES * (s + P));
#pragma unroll
          for (int i = 0; i < TT; i++)
            xr[s % P][i] =
                *reinterpret_cast<const float4*>(sx + i * kRlRs + 4 * cg + LANES * (s + P));
        }
      }
    } else {
#pragma unroll 4
      for (int j = 4 * cg; j < jend; j += LANES) {
        float4 wv[RT], xv[TT];
#pragma unroll
        for (int q = 0; q < RT; q++) wv[q] = *reinterpret_cast<const float4*>(sw + q * kRlRs + j);
#pragma unroll
        for (int i = 0; i < TT; i++) xv[i] = *reinterpret_cast<const float4*>(sx + i * kRlRs + j);
#pragma unroll
        for (int i = 0; i < TT; i++)
#pragma unroll
          for (int q = 0; q < RT; q++) {
            acc[i][q][0] = __builtin_fmaf(wv[q].x, xv[i].x, acc[i][q][0]);
            acc[i][q][1] = __builtin_fmaf(wv[q].y, xv[i].y, acc[i][q][1]);
            acc[i][q][2] = __builtin_fmaf(wv[q].z, xv[i].z, acc[i][q][2]);
            acc[i][q][3] = __builtin_fmaf(wv[q].w, xv[i].w, acc[i][q][3]);
          }
      }
    }
    if (c + NBUF < nch) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
    }
  }

  const int base = lane - cg;
  const int last0 = (nch - 1) * kRlCk;
  const float* lw = sm + ((nch - 1) % NBUF) * BUF + (rb * RT) * kRlRs;
  const float* lx = sm + ((nch - 1) % NBUF) * BUF + (RW + tb * TT) * kRlRs;
#pragma unroll
  for (int i = 0; i < TT; i++)
#pragma unroll
    for (int q = 0; q < RT; q++) {
      const int t = t0 + tb * TT + i, e = r0 + rb * RT + q;
      float v[LANES];
#pragma unroll
      for (int g = 0; g < G; g++)
#pragma unroll
        for (int c = 0; c < 4; c++) v[4 * g + c] = __shfl(acc[i][q][c], base + g);
      float s = 0.0f;
      if constexpr (LANES == 8) {
#pragma unroll
        for (int l = 0; l < 8; l++) s += v[l];
      } else {
        float t8[8], t4[4];
#pragma unroll
        for (int l = 0; l < 8; l++) t8[l] = v[8 + l] + v[l];
#pragma unroll
        for (int l = 0; l < 4; l++) t4[l] = t8[4 + l] + t8[l];
        const float a02 = t4[0] + t4[2];
        const float a13 = t4[1] + t4[3];
        s += a02 + a13;
      }
      for (int j = dm; j < d; j++) s += lw[q * kRlRs + j - last0] * lx[i * kRlRs + j - last0];
      if (cg == 0 && t < T && e < E) logits[(size_t)t * E + e] = s;
    }
}

// Few tokens, the FMA-chain orders: one workgroup per router row e.  The row
// and the T token rows arrive whole in LDS by DMA (row i at i RS floats, RS
// = the row's whole KiB plus a LANES-float skew, so the chains of LANES
// adjacent lanes and of different tokens read different banks); thread
// t LANES + k then runs chain k of token t over the whole row with no
// barrier, and the LANES chains are combined as in k_rlogits.
template <int LANES>
__global__ __launch_bounds__(256) void k_rlogits_row(const float* __restrict__ W,
                                                     const float* __restrict__ X, int T, int E,
                                                     int d, float* __restrict__ logits) {
  extern __shared__ __align__(16) float sm[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int e = blockIdx.x;
  const int rbytes = (int)kib_round((size_t)d * 4);
  const int RS = rbytes / 4 + LANES;
  // row i (0: W[e], 1 + t: X[t]) by wave i % 4
  for (int i = wave; i <= T; i += 4) {
    const float* src = i == 0 ? W + (size_t)e * d : X + (size_t)(i - 1) * d;
    if (i == 0)  // the router row: read once
      dma_bytes<true>(reinterpret_cast<const uint8_t*>(src), reinterpret_cast<uint8_t*>(sm), d * 4,
                      lane);
    else
      dma_bytes(reinterpret_cast<const uint8_t*>(src), reinterpret_cast<uint8_t*>(sm + i * RS),
                d * 4, lane);
  }
  wait_vmcnt<0>();
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  const int t = tid / LANES, k = tid % LANES;
  if (tid >= ((T * LANES + 63) & ~63)) return;  // whole waves past the last token
  const int tc = t < T ? t : T - 1;
  const float* sw = sm;
  const float* sx = sm + (1 + tc) * RS;
  const int dm = d - d % LANES;
  const float acc = lds_chain<LANES>(sw, sx, k, dm);
  float v[LANES];
  const int base = lane - k;
#pragma unroll
  for (int l = 0; l < LANES; l++) v[l] = __shfl(acc, base + l);
  float sum = 0.0f;
  if constexpr (LANES == 8) {
#pragma unroll
    for (int l = 0; l < 8; l++) sum += v[l];
  } else {
    float t8[8], t4[4];
#pragma unroll
    for (int l = 0; l < 8; l++) t8[l] = v[8 + l] + v[l];
#pragma unroll
    for (int l = 0; l < 4; l++) t4[l] = t8[4 + l] + t8[l];
    const float a02 = t4[0] + t4[2];
    const float a13 = t4[1] + t4[3];
    sum += a02 + a13;
  }
  for (int j = dm; j < d; j++) sum += sw[j] * sx[j];
  if (k == 0 && t < T) logits[(size_t)t * E + e] = sum;
}

template <int LANES>
static size_t rlogits_row_lds(int T, int d) {
  return (size_t)(T + 1) * (kib_round((size_t)d * 4) + 4 * LANES);
}

// Whether k_rlogits_row takes T tokens: LANES threads per token, the T + 1
// rows within 160 KiB, and a wave's DMA within the vmcnt range.
template <int LANES>
static bool rlogits_row_ok(int T, int d) {
  const int nkb = (int)(kib_round((size_t)d * 4) >> 10);
  return T >= 1 && T * LANES <= 256 && rlogits_row_lds<LANES>(T, d) <= 160 * 1024 &&
         ((T + 4) / 4) * nkb <= 63;
}

template <int LANES>
static hipError_t rlogits_row_launch_t(const float* W, const float* X, int T, int E, int d,
                                       float* logits, hipStream_t st) {
  const size_t lds = rlogits_row_lds<LANES>(T, d);
  static std::atomic<bool> opted[64];
  if (lds > 64 * 1024) {
    const hipError_t e = lds_opt_in((const void*)k_rlogits_row<LANES>, opted);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(k_rlogits_row<LANES>, dim3(E), dim3(256), lds, st, W, X, T, E, d, logits);
  return hipGetLastError();
}

bool rlogits_ok(int d) { return d > 0 && (d & 3) == 0; }

template <int LANES, int NTB, int TT, int NRB, int RT, int NBUF>
static hipError_t rlogits4_launch_t(const float* W, const float* X, int T, int E, int d,
                                    float* logits, hipStream_t st) {
  constexpr int TW = NTB * TT, RW = NRB * RT;
  constexpr size_t lds = rlogits_lds<TW, RW, NBUF>();
  static_assert(lds <= 160 * 1024, "LDS");
  static std::atomic<bool> opted[64];
  if (lds > 64 * 1024) {
    const hipError_t e =
        lds_opt_in((const void*)k_rlogits4<LANES, NTB, TT, NRB, RT, NBUF>, opted);
    if (e != hipSuccess) return e;
  }
  const dim3 grid((E + RW - 1) / RW, (T + TW - 1) / TW);
  hipLaunchKernelGGL((k_rlogits4<LANES, NTB, TT, NRB, RT, NBUF>), grid, dim3(256), lds, st, W, X,
                     T, E, d, logits);
  return hipGetLastError();
}

template <int LANES, int NTB, int TT, int NRB, int RT, int NBUF>
static hipError_t rlogits_launch_t(const float* W, const float* X, int T, int E, int d,
                                   float* logits, hipStream_t st) {
  constexpr int TW = NTB * TT, RW = NRB * RT;
  constexpr size_t lds = rlogits_lds<TW, RW, NBUF>();
  static_assert(lds <= 160 * 1024, "LDS");
  static std::atomic<bool> opted[64];
  if (lds > 64 * 1024) {
    const hipError_t e =
        lds_opt_in((const void*)k_rlogits<LANES, NTB, TT, NRB, RT, NBUF>, opted);
    if (e != hipSuccess) return e;
  }
  const dim3 grid((E + RW - 1) / RW, (T + TW - 1) / TW);
  hipLaunchKernelGGL((k_rlogits<LANES, NTB, TT, NRB, RT, NBUF>), grid, dim3(256), lds, st, W, X,
                     T, E, d, logits);
  return hipGetLastError();
}

// Tiles of 16 tokens x 4 router rows up to 128 tokens (more workgroups for
// the same work -- 256 at 128 tokens and 128 experts, against 64 of 16 x 16;
// one chain per thread); 16 x 16 tiles with four chains per thread beyond (a
// quarter of the LDS read instructions); two chunk buffers (deeper rings
// measured no faster).
hipError_t rlogits_launch(int order, const float* W, const float* X, int T, int E, int d,
                          float* logits, hipStream_t st) {
  if (!rlogits_ok(d) || (reinterpret_cast<uintptr_t>(W) & 15) ||
      (reinterpret_cast<uintptr_t>(X) & 15))
    return hipErrorInvalidValue;
  if (T <= 0 || E <= 0) return hipSuccess;
  const bool small = T <= 128;
  switch (order) {
    case QR_ORDER_SEQ: return rlogits_launch_t<1, 16, 1, 16, 1, 2>(W, X, T, E, d, logits, st);
    case QR_ORDER_AVX2:
      if (rlogits_row_ok<8>(T, d)) return rlogits_row_launch_t<8>(W, X, T, E, d, logits, st);
      if (small) return rlogits_launch_t<8, 8, 2, 4, 1, 2>(W, X, T, E, d, logits, st);
      // 8-row by 16-token workgroup tiles: at 128 experts and 512 tokens, 512
      // workgroups (two per CU) against 256 for 16 x 16 (239.1 -> 236.4 us
      // per layer measured)
      return rlogits4_launch_t<8, 16, 1, 8, 1, 2>(W, X, T, E, d, logits, st);
    default:
      if (rlogits_row_ok<16>(T, d)) return rlogits_row_launch_t<16>(W, X, T, E, d, logits, st);
      if (small) return rlogits_launch_t<16, 4, 4, 4, 1, 2>(W, X, T, E, d, logits, st);
      return rlogits4_launch_t<16, 4, 4, 16, 1, 2>(W, X, T, E, d, logits, st);
  }
}

// One workgroup of 4 waves per token: wave 0 computes the softmax and the
// rank keys while the others quantize the token's xb into its activation
// records; every thread then ranks the E candidates (route_rank_wg) and wave
// 0 writes the renormalised routing.
__global__ __launch_bounds__(256) void k_route_rank(
    const float* __restrict__ logits, int T, int E, int K, float* __restrict__ probs,
    int32_t* __restrict__ idx, float* __restrict__ wts, const float* __restrict__ X, int d,
    int perm, uint8_t* __restrict__ XQ) {
  __shared__ __align__(16) float pw[kRouteRow];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x;
  if (wave == 0) {
    const ExpTab tab = qr_expf_tab();
    float pv[4];
    route_softmax(logits + (size_t)t * E, E, pw, lane, probs ? probs + (size_t)t * E : nullptr,
                  tab, pv);
    route_rank_keys(pv, E, K, pw, lane);
  } else if (XQ) {
    // waves 1..3: the token's activation records, 48 blocks per pass
    const int groups = (d >> 5) * 4;
    uint8_t* out = XQ + (size_t)t * (d >> 5) * kXQ;
    const float* x = X + (size_t)t * d;
    for (int g0 = 0; g0 < groups; g0 += 192) {
      if (perm) quant_rows_group<true>(x, d, 1, d, out, g0 + (int)threadIdx.x - 64);
      else quant_rows_group<false>(x, d, 1, d, out, g0 + (int)threadIdx.x - 64);
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  route_rank_wg(E, K, pw, (int)threadIdx.x, (int)blockDim.x);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  if (wave == 0) route_write(pw, K, lane, idx + (size_t)t * K, wts + (size_t)t * K);
}

hipError_t route_rank_launch(const float* logits, int T, int E, int K, float* probs, int32_t* idx,
                             float* wts, const float* X, int d, bool perm, uint8_t* XQ,
                             hipStream_t st) {
  if (E > 256 || K > 16 || T <= 0) return T <= 0 ? hipSuccess : hipErrorInvalidValue;
  hipLaunchKernelGGL(k_route_rank, dim3(T), dim3(256), 0, st, logits, T, E, K, probs, idx, wts, X,
                     d, perm ? 1 : 0, XQ);
  return hipGetLastError();
}

}  // namespace qr
