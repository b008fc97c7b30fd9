// qr_tiled_sq.h -- the tiled layout of Q6_K and Q8_0 matrices and its GEMV:
// the formats whose blocks are not 16-byte aligned (210 and 34 bytes), which
// the row-major engines must stage through LDS as byte ranges.
//
// As for Q4_K / Q5_K (qr_tiled.h), a lane holds 256 elements of a row and a
// wave's tile is RB = 64 / nb rows of nb such "super-units" (nb = d / 256),
// lane l = (row l / nb, super-unit l % nb); the tile stores chunk k of all its
// L lanes together (chunk k of lane l at byte 16 (k L + l) of the tile), so
// one 1 KiB DMA instruction moves one chunk of a whole tile and the wave works
// on each chunk as it lands.  The bytes are the reference's, permuted once
// (qr_weights_tile); the matrix keeps its size.
//
//   Q6_K (a 210-byte super-block per lane, src/quant.c:220-226: ql[128],
//   qh[64], int8 scales[16], fp16 d): 13 chunks in consumption order --
//   the scales, then for each pair of 32-element units the 16 qh bytes of the
//   pair and the 16 ql bytes of each unit -- so a tile is 208 L bytes; the d
//   fields of all super-units follow all the tiles, 2 bytes each in row-major
//   order (super-unit u's at byte 208 n nb + 2 u).  A tile's L fields are one
//   2 L-byte run, which the wave moves with one more DMA instruction from the
//   16-byte unit that holds its start; the matrix needs n nb a multiple of 8
//   so that no such unit passes the end of the fields.
//   Source chunk of tiled chunk k: 12, 8, 0, 1, 9, 2, 3, 10, 4, 5, 11, 6, 7.
//
//   Q8_0 (8 consecutive 34-byte blocks per lane, 272 bytes): 17 chunks --
//   the 8 fp16 scales d_0 .. d_7, then block j's 32 int8 values as chunks
//   1 + 2 j and 2 + 2 j.
//
// The unit terms and their order are the reference's (Q6_K: sc * isum * bd,
// src/quant.c:406-437; Q8_0: isum * da * db added in block order, the
// -std=c99 build's vec_dot_q8_0_q8_0, src/quant.c:279-285); the row sum is
// the lane chain of qr_blk.h.  The Q8_0 lane orders of the AVX2 / AVX-512
// builds keep eight accumulators per row and stay on the streaming engine.
#pragma once

#include "qr_blk.h"
#include "qr_norm.h"
#include "qr_tiled.h"

namespace qr {

template <int TYPE>
struct SqFmt;
template <>
struct SqFmt<QR_T_Q6_K> {
  static constexpr int kBytes = QR_Q6K_BYTES;  // 210
  static constexpr int kChunks = 13;
  static constexpr bool kTailD = true;  // the d fields after all the tiles
  static constexpr int kOps = 14;       // DMA instructions per tile: d fields, then chunks
};
template <>
struct SqFmt<QR_T_Q8_0> {
  static constexpr int kBytes = 8 * QR_Q8_BYTES;  // 272
  static constexpr int kChunks = 17;
  static constexpr bool kTailD = false;
  static constexpr int kOps = 17;
};

__host__ __device__ inline int sq_bytes(int type) {
  return type == QR_T_Q6_K ? SqFmt<QR_T_Q6_K>::kBytes : SqFmt<QR_T_Q8_0>::kBytes;
}
// Tile bytes per lane: the chunks (Q6_K's d fields sit after all the tiles).
__host__ __device__ inline int sq_lane_bytes(int type) {
  return type == QR_T_Q6_K ? 16 * SqFmt<QR_T_Q6_K>::kChunks : SqFmt<QR_T_Q8_0>::kBytes;
}
// LDS slot KiB per wave (one per DMA instruction of a tile)
__host__ __device__ inline int sq_slot_kib(int type) {
  return type == QR_T_Q6_K ? SqFmt<QR_T_Q6_K>::kOps : SqFmt<QR_T_Q8_0>::kOps;
}
// n rows of d elements the layout takes: whole super-units (and, for Q6_K,
// n (d / 256) a multiple of 8: the d fields end on a 16-byte unit).
__host__ __device__ inline bool sq_shape_ok(int type, int n, int d) {
  if (n < 0 || d <= 0 || (d & 255) || (d >> 8) > 64) return false;
  return type == QR_T_Q8_0 || (type == QR_T_Q6_K && ((long)n * (d >> 8)) % 8 == 0);
}

struct SqGeom {
  int nb;             // super-units per row
  int RB;             // rows per full tile
  int ntiles;
  size_t tile_bytes;  // bytes of a full tile
};
__host__ __device__ inline SqGeom sq_geom(int type, int n, int d) {
  SqGeom g;
  g.nb = d >> 8;
  g.RB = g.nb > 0 ? 64 / g.nb : 0;
  g.ntiles = g.RB > 0 ? (n + g.RB - 1) / g.RB : 0;
  g.tile_bytes = (size_t)g.RB * g.nb * sq_lane_bytes(type);
  return g;
}

// Byte offset inside a lane's super-unit (reference layout) of byte i of
// tiled chunk k.
template <int TYPE>
__host__ __device__ inline int sq_src_byte(int k, int i) {
  if constexpr (TYPE == QR_T_Q6_K) {
    constexpr int kMap[13] = {12, 8, 0, 1, 9, 2, 3, 10, 4, 5, 11, 6, 7};
    return 16 * kMap[k] + i;
  } else {
    if (k == 0) return QR_Q8_BYTES * (i >> 1) + (i & 1);  // d_j
    const int j = (k - 1) >> 1, h = (k - 1) & 1;
    return QR_Q8_BYTES * j + 2 + 16 * h + i;
  }
}

// Row-major -> tiled (or back, `reverse`): thread i moves 16 bytes of chunk
// (i % NCH1) of super-unit i / NCH1 (NCH1 = NCH, plus one for Q6_K's d), byte
// by byte (a one-time repack).
template <int TYPE>
__global__ __launch_bounds__(256) void k_tile_pack_sq(const uint8_t* __restrict__ src,
                                                      uint8_t* __restrict__ dst, int n, int d,
                                                      int reverse) {
  constexpr int BB = SqFmt<TYPE>::kBytes, NCH = SqFmt<TYPE>::kChunks;
  constexpr int NCH1 = NCH + (SqFmt<TYPE>::kTailD ? 1 : 0);
  const SqGeom g = sq_geom(TYPE, n, d);
  const long total = (long)n * g.nb * NCH1;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (long)gridDim.x * blockDim.x) {
    const long su = i / NCH1;  // row-major super-unit index
    const int k = (int)(i - su * NCH1);
    const int per = g.RB * g.nb;
    const int t = (int)(su / per), l = (int)(su - (long)t * per);
    const int L = min(g.RB, n - t * g.RB) * g.nb;
    const size_t tbase = (size_t)t * g.tile_bytes;
    const size_t pbase = (size_t)su * BB;
    if (k == NCH) {  // Q6_K's d, after all the tiles in row-major order
#pragma unroll
      for (int b = 0; b < 2; b++) {
        const size_t tp = (size_t)208 * n * g.nb + 2 * (size_t)su + b;
        const size_t pp = pbase + 208 + b;
        dst[reverse ? pp : tp] = src[reverse ? tp : pp];
      }
    } else {
#pragma unroll
      for (int b = 0; b < 16; b++) {
        const size_t tp = tbase + (size_t)16 * ((size_t)k * L + l) + b;
        const size_t pp = pbase + sq_src_byte<TYPE>(k, b);
        dst[reverse ? pp : tp] = src[reverse ? tp : pp];
      }
    }
  }
}

// This lane's DMA sources in tile t: chunk k at src[k] (lanes past the tile
// reload its first 16 bytes into slot bytes nobody reads) and, Q6_K, 16
// bytes of the d fields at dsrc: the tile's run of 2 L bytes starts sq_doff
// bytes into a 16-byte unit, lane j takes unit j of the run (the lanes past
// it the first unit again).
__device__ inline int sq_doff(const GemvArgs& g, int t) {
  return (int)(((size_t)2 * t * g.t_rb * g.t_nb) & 15);  // the fields start on a 16-byte unit
}
template <int TYPE>
__device__ inline void sq_src(const GemvArgs& g, int t, int lane,
                              const uint8_t* (&src)[SqFmt<TYPE>::kChunks], const uint8_t*& dsrc) {
  constexpr int NCH = SqFmt<TYPE>::kChunks;
  const int L = min(g.t_rb, g.n - t * g.t_rb) * g.t_nb;
  const uint8_t* base = g.W + (size_t)t * g.t_tile_bytes;
  const bool on = lane < L;
#pragma unroll
  for (int k = 0; k < NCH; k++) src[k] = on ? base + (size_t)k * 16 * L + 16 * lane : base;
  if constexpr (SqFmt<TYPE>::kTailD) {
    const size_t run = (size_t)208 * g.n * g.t_nb + (size_t)2 * t * g.t_rb * g.t_nb;
    const uint8_t* unit0 = g.W + (run & ~(size_t)15);
    const int units = (sq_doff(g, t) + 2 * L + 15) >> 4;
    dsrc = lane < units ? unit0 + 16 * lane : unit0;
  } else {
    dsrc = base;
  }
}

// The slot's KiB of the d fields (Q6_K): after the chunks.
constexpr int kSqDSlot = 13;

// One tile's DMA: (Q6_K) the d fields, then the NCH chunks.
template <int TYPE>
__device__ inline void sq_dma(const uint8_t* const (&src)[SqFmt<TYPE>::kChunks],
                              const uint8_t* dsrc, uint32_t sbase) {
  constexpr int NCH = SqFmt<TYPE>::kChunks;
  if constexpr (SqFmt<TYPE>::kTailD) lds_dma16_nt(dsrc, sbase + (uint32_t)(kSqDSlot * 1024));
#pragma unroll
  for (int k = 0; k < NCH; k++) lds_dma16_nt(src[k], sbase + (uint32_t)(k * 1024));
}

// Chunk K of the current tile, once landed (the wave's vector memory
// operations complete in issue order, kOps per tile).  With RING, chunk K of
// the next tile goes into its place right after the read; before chunk 0's
// refill, the next tile's d fields replace this tile's (read together with
// chunk 0).  Operations issued after this tile's chunk K when it is waited
// for: its chunks K+1 .. NCH-1, and with RING the refills of chunks 0 .. K-1
// plus (K >= 1) the next d fields.
template <int TYPE, int K, bool RING>
__device__ inline uint4 sq_chunk(const uint8_t* slot, uint32_t sbase, int lane,
                                 const uint8_t* const (&nsrc)[SqFmt<TYPE>::kChunks],
                                 const uint8_t* ndsrc, float* dval, int doff = 0) {
  constexpr int NCH = SqFmt<TYPE>::kChunks;
  constexpr bool TD = SqFmt<TYPE>::kTailD;
  constexpr int AFTER_RING = NCH - 1 + ((TD && K >= 1) ? 1 : 0);
  constexpr int AFTER_LAST = NCH - 1 - K;
  if constexpr (RING) wait_vmcnt<AFTER_RING>();
  else wait_vmcnt<AFTER_LAST>();
  const uint4 v = *reinterpret_cast<const uint4*>(slot + K * 1024 + 16 * lane);
  if constexpr (TD && K == 0)  // the d fields landed before chunk 0 (issued first)
    *dval = qr_h2f(*reinterpret_cast<const uint16_t*>(slot + kSqDSlot * 1024 + doff + 2 * lane));
  if constexpr (RING) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the reads are done before the refill
    if constexpr (TD && K == 0) lds_dma16_nt(ndsrc, sbase + (uint32_t)(kSqDSlot * 1024));
    lds_dma16_nt(nsrc[K], sbase + (uint32_t)(K * 1024));
  }
  return v;
}

// The activation block of unit u (NAT layout) as 8 dwords.
__device__ inline void sq_act(const uint8_t* act, int u, uint32_t (&xv)[8], float& bd, int& bs) {
  const ActView a = act_read(act + act_off(u));
#pragma unroll
  for (int i = 0; i < 8; i++) xv[i] = a.q[i];
  bd = a.bd;
  bs = a.bs;
}

// Q6_K: the 8 unit terms of the lane's super-block (units 8 b .. 8 b + 7 of
// its row) for NT tokens.
template <int NT, bool RING>
__device__ inline void sq_tile_q6(const uint8_t* slot, uint32_t sbase, int lane,
                                  const uint8_t* const (&nsrc)[13], const uint8_t* ndsrc,
                                  const uint8_t* act, size_t tokb, int b, float (&terms)[NT][8],
                                  int doff) {
  float d;
  const uint4 sv = sq_chunk<QR_T_Q6_K, 0, RING>(slot, sbase, lane, nsrc, ndsrc, &d, doff);
  const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
  for (int p = 0; p < 4; p++) {
    uint4 qh, ql0, ql1;
    switch (p) {  // compile-time chunk indices
      case 0:
        qh = sq_chunk<QR_T_Q6_K, 1, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        ql0 = sq_chunk<QR_T_Q6_K, 2, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        ql1 = sq_chunk<QR_T_Q6_K, 3, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        break;
      case 1:
        qh = sq_chunk<QR_T_Q6_K, 4, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        ql0 = sq_chunk<QR_T_Q6_K, 5, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        ql1 = sq_chunk<QR_T_Q6_K, 6, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        break;
      case 2:
        qh = sq_chunk<QR_T_Q6_K, 7, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        ql0 = sq_chunk<QR_T_Q6_K, 8, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        ql1 = sq_chunk<QR_T_Q6_K, 9, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        break;
      default:
        qh = sq_chunk<QR_T_Q6_K, 10, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        ql0 = sq_chunk<QR_T_Q6_K, 11, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        ql1 = sq_chunk<QR_T_Q6_K, 12, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        break;
    }
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int s = 2 * p + h;
      const int sc8 = (int)(int8_t)((sw[s >> 2] >> (8 * (s & 3))) & 0xFFu);
      const float sc = (float)sc8 * d;
      const uint2 qh2 = h == 0 ? make_uint2(qh.x, qh.y) : make_uint2(qh.z, qh.w);
      const uint4 ql = h == 0 ? ql0 : ql1;
#pragma unroll
      for (int t = 0; t < NT; t++) {
        uint32_t xv[8];
        float bd;
        int bs;
        sq_act(act + (size_t)t * tokb, 8 * b + s, xv, bd, bs);
        const int isum = dot_q6_regs_raw(ql, qh2, xv) - 32 * bs;
        terms[t][s] = sc * (float)isum * bd;
      }
    }
  }
}

// Q8_0: the 8 block terms of the lane's super-unit for NT tokens.
template <int NT, bool RING>
__device__ inline void sq_tile_q8(const uint8_t* slot, uint32_t sbase, int lane,
                                  const uint8_t* const (&nsrc)[17], const uint8_t* ndsrc,
                                  const uint8_t* act, size_t tokb, int b, float (&terms)[NT][8]) {
  const uint4 dh = sq_chunk<QR_T_Q8_0, 0, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
  const uint32_t dw[4] = {dh.x, dh.y, dh.z, dh.w};
#pragma unroll
  for (int j = 0; j < 8; j++) {
    uint4 w0, w1;
    switch (j) {
      case 0:
        w0 = sq_chunk<QR_T_Q8_0, 1, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        w1 = sq_chunk<QR_T_Q8_0, 2, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        break;
      case 1:
        w0 = sq_chunk<QR_T_Q8_0, 3, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        w1 = sq_chunk<QR_T_Q8_0, 4, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        break;
      case 2:
        w0 = sq_chunk<QR_T_Q8_0, 5, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        w1 = sq_chunk<QR_T_Q8_0, 6, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        break;
      case 3:
        w0 = sq_chunk<QR_T_Q8_0, 7, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        w1 = sq_chunk<QR_T_Q8_0, 8, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        break;
      case 4:
        w0 = sq_chunk<QR_T_Q8_0, 9, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        w1 = sq_chunk<QR_T_Q8_0, 10, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        break;
      case 5:
        w0 = sq_chunk<QR_T_Q8_0, 11, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        w1 = sq_chunk<QR_T_Q8_0, 12, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        break;
      case 6:
        w0 = sq_chunk<QR_T_Q8_0, 13, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        w1 = sq_chunk<QR_T_Q8_0, 14, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        break;
      default:
        w0 = sq_chunk<QR_T_Q8_0, 15, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        w1 = sq_chunk<QR_T_Q8_0, 16, RING>(slot, sbase, lane, nsrc, ndsrc, nullptr);
        break;
    }
    const uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    const float da = qr_h2f((dw[j >> 1] >> (16 * (j & 1))) & 0xFFFFu);
#pragma unroll
    for (int t = 0; t < NT; t++) {
      uint32_t xv[8];
      float bd;
      int bs;
      sq_act(act + (size_t)t * tokb, 8 * b + j, xv, bd, bs);
      terms[t][j] = (float)dot_q8_regs(w, xv) * da * bd;
    }
  }
}

// The GEMV: NW waves per workgroup, wave w of workgroup g takes tiles
// g NW + w, then + (workgroups) NW, ...; its LDS slot holds one tile (kOps
// KiB).  Every wave issues its first tile's DMA at once; the first QW =
// min(NW, 4) waves then quantize the activation (NAT layout) into LDS.
// NORM (one token): the activation is rmsnorm_ref(X, nw) formed in the
// workgroup (qr_norm.h; the normalised vector after the slots), as the tiled
// Q4_K / Q5_K GEMV's kProNorm start-up does.  Workgroup `bid` of `nbid`.
template <int TYPE, int NT, int NW, bool NORM>
__device__ inline void sq_body(const GemvArgs& g, uint8_t* smem, int bid, int nbid) {
  constexpr int NSLOT = SqFmt<TYPE>::kOps;
  constexpr int NCH = SqFmt<TYPE>::kChunks;
  constexpr int QW = NW < 4 ? NW : 4;
  const int nb = g.t_nb, ntiles = g.t_ntiles;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int tstep = nbid * NW;
  int tile = bid * NW + wave;
  const bool has = tile < ntiles;
  const size_t tokb = act_tok_bytes(g.d);
  uint8_t* act = smem;
  uint8_t* slot = smem + align16((size_t)NT * tokb) + (size_t)wave * NSLOT * 1024;
  const uint32_t sbase = lds_u32addr(slot);
  const uint8_t* src[NCH];
  const uint8_t* dsrc;
  sq_src<TYPE>(g, has ? tile : 0, lane, src, dsrc);
  // every wave's first tile DMA first; the quantizing waves then load the
  // activation with ordinary loads (the compiler's wait for those, being
  // later in the same in-order stream, also covers the DMA: their quantizer
  // starts when both have landed, which is when the tile is needed anyway)
  if (has) sq_dma<TYPE>(src, dsrc, sbase);
  if constexpr (NORM) {
    static_assert(NT == 1, "the normalising start-up takes one token");
    constexpr int NP = (kNormFuseMax / 4 + 64 * NW - 1) / (64 * NW);
    float* xs = reinterpret_cast<float*>(smem + align16(tokb) + (size_t)NW * NSLOT * 1024);
    NormRegs<NP> r;
    norm_load<NP>(g.X, g.nw, g.d, (int)threadIdx.x, 64 * NW, r);
    norm_finish<NP>(r, g.d, xs, xs + g.d, (int)threadIdx.x, 64 * NW, bid == 0 ? g.nxb : nullptr);
    if (wave < QW) {
      ActPre pre;
      quantize_act_blk<false, kActLds>(g.X, (size_t)g.d, 1, g.d, act, pre, xs, (int)threadIdx.x,
                                       64 * QW);
    }
  } else if (wave < QW) {
    ActPre pre;
    act_load8(g.X, (size_t)g.xstride, NT, g.d, (int)threadIdx.x, pre.v);
    quantize_act_blk<false, kActGlobal>(g.X, (size_t)g.xstride, NT, g.d, act, pre, nullptr,
                                        (int)threadIdx.x, 64 * QW);
  }
  // LDS-only barrier: the tile DMA stays in flight across it
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  if (!has) return;  // no barriers below
  // after a normalisation: the first tile has landed, and the wait covers the
  // workgroup's stores, which would otherwise count in the ring's figures
  if constexpr (NORM) wait_vmcnt<0>();
  const int rl = lane / nb, b = lane - rl * nb;
  for (;;) {
    const int next = tile + tstep;
    float terms[NT][8];
    const int doff = TYPE == QR_T_Q6_K ? sq_doff(g, tile) : 0;
    if (next < ntiles) {
      sq_src<TYPE>(g, next, lane, src, dsrc);
      if constexpr (TYPE == QR_T_Q6_K)
        sq_tile_q6<NT, true>(slot, sbase, lane, src, dsrc, act, tokb, b, terms, doff);
      else
        sq_tile_q8<NT, true>(slot, sbase, lane, src, dsrc, act, tokb, b, terms);
    } else {
      if constexpr (TYPE == QR_T_Q6_K)
        sq_tile_q6<NT, false>(slot, sbase, lane, src, dsrc, act, tokb, b, terms, doff);
      else
        sq_tile_q8<NT, false>(slot, sbase, lane, src, dsrc, act, tokb, b, terms);
    }
    float y[NT];
    blk_chain<NT>(terms, b, nb, y);
    const int L = min(g.t_rb, g.n - tile * g.t_rb) * nb;
    if (lane < L && b == nb - 1) {
      const int row = tile * g.t_rb + rl;
#pragma unroll
      for (int t = 0; t < NT; t++) g.Y[(size_t)t * g.ystride + row] = g.R ? g.R[row] + y[t] : y[t];
    }
    if (next >= ntiles) break;
    tile = next;
  }
}

template <int TYPE, int NT, int NW>
__global__ __launch_bounds__(64 * NW) void k_gemv_tiled_sq(GemvArgs g) {
  extern __shared__ __align__(16) uint8_t smem[];
  sq_body<TYPE, NT, NW, false>(g, smem, (int)blockIdx.x, (int)gridDim.x);
}

// One token through two matrices after one normalisation: workgroups
// [0, ga) run a tiled Q4_K / Q5_K matrix (a, kProNorm), the rest a tiled
// Q6_K / Q8_0 matrix (b), every workgroup forming the same rmsnorm_ref of the
// residual (the decode step's q / k and v projections in one launch).
template <int TA, int TB, int NW>
__global__ __launch_bounds__(64 * NW) void k_gemv_norm2(GemvArgs a, GemvArgs b, int ga) {
  extern __shared__ __align__(16) uint8_t smem[];
  if ((int)blockIdx.x < ga)  // uniform per workgroup
    tiled_body<TA, 1, NW, kProNorm>(a, smem, (int)blockIdx.x, ga);
  else
    sq_body<TB, 1, NW, true>(b, smem, (int)blockIdx.x - ga, (int)gridDim.x - ga);
}

}  // namespace qr
