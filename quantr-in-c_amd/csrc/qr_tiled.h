// qr_tiled.h -- the tiled weight layout of Q4_K / Q5_K matrices and its GEMV.
//
// The same bytes as the reference's row-major super-blocks, permuted once
// (qr_weights_tile) so that a wave's tile streams in the order its lanes
// consume it.  A tile is RB = 64 / nb rows of nb super-blocks (nb = d / 256),
// lane l holding block l of the tile (row l / nb, block l % nb), as in the
// block-per-lane engine (qr_blk.h).  Each super-block is cut into its 16-byte
// chunks (header, then the sub-block data: 9 chunks for Q4_K, 11 for Q5_K);
// the tile stores chunk k of all its L lanes together:
//
//   tile t at byte t * RB * nb * BB; chunk k of lane l at + k * 16 L + 16 l,
//
// with L = (rows of tile t) * nb (only the last tile can be short).  The
// matrix keeps its size, n * nb * BB bytes.
//
// Why: a wave moves a tile into LDS with one 1 KiB DMA instruction per chunk;
// the instructions complete in issue order, so the wave can start on the
// header and the first sub-blocks while the later chunks are still in
// flight, instead of waiting for the whole tile (each lane's 144 contiguous
// bytes would span every instruction).  Measured on the 32000 x 2048 Q4_K
// GEMV: 7.65 us against 8.1 us for the same kernel over the row-major layout.
#pragma once

#include "qr_blk.h"
#include "qr_norm.h"

namespace qr {

struct TiledGeom {
  int nb;        // super-blocks per row
  int RB;        // rows per full tile
  int ntiles;
  size_t tile_bytes;  // bytes of a full tile
};

template <int TYPE>
struct TiledFmt {
  static constexpr int kBytes = BlkFmt<TYPE>::kBytes;
  static constexpr int kChunks = BlkFmt<TYPE>::kChunks;  // 9 or 11
};

__host__ __device__ inline TiledGeom tiled_geom(int type, int n, int d) {
  TiledGeom g;
  g.nb = d >> 8;
  g.RB = g.nb > 0 ? 64 / g.nb : 0;
  g.ntiles = g.RB > 0 ? (n + g.RB - 1) / g.RB : 0;
  g.tile_bytes = (size_t)g.RB * g.nb * (type == QR_T_Q4_K ? QR_Q4K_BYTES : QR_Q5K_BYTES);
  return g;
}

// Row-major blocks -> tiled layout, one thread per 16-byte chunk.
template <int TYPE>
__global__ __launch_bounds__(256) void k_tile_pack(const uint8_t* __restrict__ src,
                                                   uint8_t* __restrict__ dst, int n, int d,
                                                   int reverse) {
  constexpr int BB = TiledFmt<TYPE>::kBytes, NCH = TiledFmt<TYPE>::kChunks;
  const TiledGeom g = tiled_geom(TYPE, n, d);
  const long total = (long)n * g.nb * NCH;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (long)gridDim.x * blockDim.x) {
    const long blk = i / NCH;  // row-major block index
    const int k = (int)(i - blk * NCH);
    const int per = g.RB * g.nb;
    const int t = (int)(blk / per), l = (int)(blk - (long)t * per);
    const int rows = min(g.RB, n - t * g.RB);
    const size_t tiled = (size_t)t * g.tile_bytes + (size_t)k * 16 * rows * g.nb + 16 * (size_t)l;
    const size_t plain = (size_t)blk * BB + 16 * (size_t)k;
    const uint4* s = reinterpret_cast<const uint4*>(src + (reverse ? tiled : plain));
    *reinterpret_cast<uint4*>(dst + (reverse ? plain : tiled)) = *s;
  }
}

// ---------------------------------------------------------------------------
// The GEMV.  NW waves per workgroup; wave w of workgroup g takes tiles
// g * NW + w, then + gridDim.x * NW, ...; its LDS slot holds one tile (NCH
// KiB).  The first QW = min(NW, 4) waves also quantize the activation into
// LDS.
//
// Start-up, two forms (PRO):
//   kProAsm1 / kProAsm2 (every quantizing thread owns one / two groups of 8
//            activation values): one asm block loads the thread's values and
//            issues the first tile's DMA behind them, then waits until only
//            the DMA is in flight.  The compiler sees neither the DMA nor the
//            loads' completion, so the quantizer starts as soon as the
//            activation is in, whatever the tile is doing.
//   kProLate (larger activations): the quantizing waves load the activation
//            with ordinary loads and quantize it first, and issue their first
//            tile's DMA after the barrier; the other waves issue theirs at once.
//   kProNorm (one token): X is the residual stream and the activation is its
//            rmsnorm_ref with weights nw (qr_norm.h).  Every wave issues its
//            first tile's DMA, the workgroup loads x and nw, thread 0 forms
//            the sum of squares while the tiles land, and the normalised
//            vector goes to LDS (after the slots, d floats and the scale)
//            for the quantizer; workgroup 0 also stores it at nxb.
// Then, tile after tile, the wave takes chunk k once it has landed (the
// wave's DMA operations complete in issue order), and right after reading it
// refills chunk k of its slot with chunk k of its next tile: a ring of NCH
// operations, so with a next tile every wait is "at most NCH - 1 in flight";
// on the last tile the count runs down.  The Y stores between tiles only make
// those waits stricter.  The row sums are the sequential chain of qr_blk.h.
// ---------------------------------------------------------------------------
enum { kProAsm1 = 0, kProAsm2 = 1, kProLate = 2, kProNorm = 3 };

// How a tile's chunks are issued (tiled_chunk below): all in flight (the
// last tile), all in flight with the next tile's refills (a ring), or a
// window of kWin chunks (a wave's only tile).
enum { kChLast = 0, kChRing = 1, kChWindow = 2 };
constexpr int kWin = 5;

// One global_load_lds_dwordx4 per chunk: chunk k's 16 bytes for this lane at
// src[k], into LDS sbase + 1024 k (+ 16 lane by the hardware).
template <int NCH>
__device__ inline void tiled_dma(const uint8_t* const (&src)[NCH], uint32_t sbase) {
#pragma unroll
  for (int k = 0; k < NCH; k++) lds_dma16_nt(src[k], sbase + (uint32_t)(k * 1024));
}

#define QR_DMA1(K)                                   \
  "s_mov_b32 m0, %[m" #K "]\n\t"                     \
  "global_load_lds_dwordx4 %[v" #K "], off nt\n\t"
#define QR_DMA9 QR_DMA1(0) QR_DMA1(1) QR_DMA1(2) QR_DMA1(3) QR_DMA1(4) QR_DMA1(5) QR_DMA1(6) \
  QR_DMA1(7) QR_DMA1(8)
#define QR_DMA11 QR_DMA9 QR_DMA1(9) QR_DMA1(10)
#define QR_SRC9 [v0] "v"(src[0]), [v1] "v"(src[1]), [v2] "v"(src[2]), [v3] "v"(src[3]), \
  [v4] "v"(src[4]), [v5] "v"(src[5]), [v6] "v"(src[6]), [v7] "v"(src[7]), [v8] "v"(src[8]), \
  [m0] "s"(sb), [m1] "s"(sb + 1024), [m2] "s"(sb + 2048), [m3] "s"(sb + 3072), \
  [m4] "s"(sb + 4096), [m5] "s"(sb + 5120), [m6] "s"(sb + 6144), [m7] "s"(sb + 7168), \
  [m8] "s"(sb + 8192)
#define QR_SRC11 QR_SRC9, [v9] "v"(src[9]), [v10] "v"(src[10]), [m9] "s"(sb + 9216), \
  [m10] "s"(sb + 10240)

// G groups of activation values (two 16-byte loads each, at xp[g]), then
// NCH chunk DMAs, then a wait for the G groups.  Outputs are complete when
// the statement ends.
template <int NCH, int G>
__device__ inline void tiled_pro_asm(const float* const (&xp)[G], const uint8_t* const (&src)[NCH],
                                     uint32_t sb, float4 (&v)[2 * G]);

template <>
__device__ inline void tiled_pro_asm<9, 1>(const float* const (&xp)[1],
                                           const uint8_t* const (&src)[9], uint32_t sb,
                                           float4 (&v)[2]) {
  int save;
  asm volatile(
      "global_load_dwordx4 %[a], %[x], off\n\t"
      "global_load_dwordx4 %[b], %[x], off offset:16\n\t"
      "s_mov_b32 %[save], m0\n\t" QR_DMA9
      "s_mov_b32 m0, %[save]\n\t"
      "s_waitcnt vmcnt(9)"
      : [a] "=&v"(v[0]), [b] "=&v"(v[1]), [save] "=&s"(save)
      : [x] "v"(xp[0]), QR_SRC9
      : "memory");
}
template <>
__device__ inline void tiled_pro_asm<11, 1>(const float* const (&xp)[1],
                                            const uint8_t* const (&src)[11], uint32_t sb,
                                            float4 (&v)[2]) {
  int save;
  asm volatile(
      "global_load_dwordx4 %[a], %[x], off\n\t"
      "global_load_dwordx4 %[b], %[x], off offset:16\n\t"
      "s_mov_b32 %[save], m0\n\t" QR_DMA11
      "s_mov_b32 m0, %[save]\n\t"
      "s_waitcnt vmcnt(11)"
      : [a] "=&v"(v[0]), [b] "=&v"(v[1]), [save] "=&s"(save)
      : [x] "v"(xp[0]), QR_SRC11
      : "memory");
}
template <>
__device__ inline void tiled_pro_asm<9, 2>(const float* const (&xp)[2],
                                           const uint8_t* const (&src)[9], uint32_t sb,
                                           float4 (&v)[4]) {
  int save;
  asm volatile(
      "global_load_dwordx4 %[a], %[x], off\n\t"
      "global_load_dwordx4 %[b], %[x], off offset:16\n\t"
      "global_load_dwordx4 %[c], %[y], off\n\t"
      "global_load_dwordx4 %[d], %[y], off offset:16\n\t"
      "s_mov_b32 %[save], m0\n\t" QR_DMA9
      "s_mov_b32 m0, %[save]\n\t"
      "s_waitcnt vmcnt(9)"
      : [a] "=&v"(v[0]), [b] "=&v"(v[1]), [c] "=&v"(v[2]), [d] "=&v"(v[3]), [save] "=&s"(save)
      : [x] "v"(xp[0]), [y] "v"(xp[1]), QR_SRC9
      : "memory");
}
template <>
__device__ inline void tiled_pro_asm<11, 2>(const float* const (&xp)[2],
                                            const uint8_t* const (&src)[11], uint32_t sb,
                                            float4 (&v)[4]) {
  int save;
  asm volatile(
      "global_load_dwordx4 %[a], %[x], off\n\t"
      "global_load_dwordx4 %[b], %[x], off offset:16\n\t"
      "global_load_dwordx4 %[c], %[y], off\n\t"
      "global_load_dwordx4 %[d], %[y], off offset:16\n\t"
      "s_mov_b32 %[save], m0\n\t" QR_DMA11
      "s_mov_b32 m0, %[save]\n\t"
      "s_waitcnt vmcnt(11)"
      : [a] "=&v"(v[0]), [b] "=&v"(v[1]), [c] "=&v"(v[2]), [d] "=&v"(v[3]), [save] "=&s"(save)
      : [x] "v"(xp[0]), [y] "v"(xp[1]), QR_SRC11
      : "memory");
}
// One group of activation values, then the first kWin (5) of a Q4_K tile's 9
// chunk DMAs, then a wait for the group (the windowed single tile).
#define QR_DMA5 QR_DMA1(0) QR_DMA1(1) QR_DMA1(2) QR_DMA1(3) QR_DMA1(4)
__device__ inline void tiled_pro_asm_win(const float* const (&xp)[1],
                                         const uint8_t* const (&src)[9], uint32_t sb,
                                         float4 (&v)[2]) {
  static_assert(kWin == 5, "the asm issues five chunks");
  int save;
  asm volatile(
      "global_load_dwordx4 %[a], %[x], off\n\t"
      "global_load_dwordx4 %[b], %[x], off offset:16\n\t"
      "s_mov_b32 %[save], m0\n\t" QR_DMA5
      "s_mov_b32 m0, %[save]\n\t"
      "s_waitcnt vmcnt(5)"
      : [a] "=&v"(v[0]), [b] "=&v"(v[1]), [save] "=&s"(save)
      : [x] "v"(xp[0]), [v0] "v"(src[0]), [v1] "v"(src[1]), [v2] "v"(src[2]), [v3] "v"(src[3]),
        [v4] "v"(src[4]), [m0] "s"(sb), [m1] "s"(sb + 1024), [m2] "s"(sb + 2048),
        [m3] "s"(sb + 3072), [m4] "s"(sb + 4096)
      : "memory");
}
#undef QR_DMA5
#undef QR_DMA1
#undef QR_DMA9
#undef QR_DMA11
#undef QR_SRC9
#undef QR_SRC11

// The activation loads alone, completed.
template <int G>
__device__ inline void tiled_x_asm(const float* const (&xp)[G], float4 (&v)[2 * G]) {
#pragma unroll
  for (int g = 0; g < G; g++) {
    asm volatile(
        "global_load_dwordx4 %[a], %[x], off\n\t"
        "global_load_dwordx4 %[b], %[x], off offset:16\n\t"
        "s_waitcnt vmcnt(0)"
        : [a] "=&v"(v[2 * g]), [b] "=&v"(v[2 * g + 1])
        : [x] "v"(xp[g])
        : "memory");
  }
}

// This lane's chunk addresses in tile t (lanes past the tile reload its first
// 16 bytes into slot bytes nobody reads).
template <int TYPE>
__device__ inline void tiled_src(const GemvArgs& g, int t, int lane,
                                 const uint8_t* (&src)[TiledFmt<TYPE>::kChunks]) {
  constexpr int NCH = TiledFmt<TYPE>::kChunks;
  const int L = min(g.t_rb, g.n - t * g.t_rb) * g.t_nb;
  const uint8_t* base = g.W + (size_t)t * g.t_tile_bytes;
  const bool on = lane < L;
#pragma unroll
  for (int k = 0; k < NCH; k++) src[k] = on ? base + (size_t)k * 16 * L + 16 * lane : base;
}

// How a tile's chunks were issued, and what reading chunk K issues next:
//   kChLast:   all NCH chunks in flight; nothing.
//   kChRing:   all NCH chunks in flight; chunk K of the next tile (nsrc) into
//              chunk K's place right after the read.
//   kChWindow: chunks 0 .. kWin - 1 issued at the start; chunk K + kWin of this
//              tile (nsrc) into its own place.  A wave with a single tile
//              keeps a few chunks in flight instead of all, so its chunks land
//              spread over the whole stream and only its last unit is left
//              when the stream ends (the 32000 x 2048 Q4_K GEMV: 7.80 -> 7.67 us,
//              medians of four alternating runs).

template <int NCH, int K, int MODE>
__device__ inline uint4 tiled_chunk(const uint8_t* slot, uint32_t sbase, int lane,
                                    const uint8_t* const (&nsrc)[NCH]) {
  if constexpr (MODE == kChRing) {
    wait_vmcnt<NCH - 1>();
  } else if constexpr (MODE == kChWindow) {
    constexpr int ISSUED = kWin + K < NCH ? kWin + K : NCH;  // chunks issued before this read
    wait_vmcnt<ISSUED - 1 - K>();
  } else {
    wait_vmcnt<NCH - 1 - K>();
  }
  const uint4 v = *reinterpret_cast<const uint4*>(slot + K * 1024 + 16 * lane);
  if constexpr (MODE == kChRing) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the read is done before the refill
    lds_dma16_nt(nsrc[K], sbase + (uint32_t)(K * 1024));
  } else if constexpr (MODE == kChWindow && K + kWin < NCH) {
    lds_dma16_nt(nsrc[K + kWin], sbase + (uint32_t)((K + kWin) * 1024));
  }
  return v;
}

// Unit S's terms for NT tokens, as blk_terms (src/quant.c:384-400 for Q4_K,
// 402-437 for Q5_K): (sc * (float)isum - m * bsf) * bd.
template <int TYPE, int NT, int S, int MODE>
__device__ inline void tiled_unit(const uint8_t* slot, uint32_t sbase, int lane,
                                  const uint8_t* const (&nsrc)[TiledFmt<TYPE>::kChunks],
                                  uint4 hdr, float dd, float dm, const uint4 (&qh)[2],
                                  const uint8_t* act, size_t tokb, int b, float (&terms)[NT][8]) {
  constexpr int NCH = TiledFmt<TYPE>::kChunks;
  const uint32_t sw = S < 4 ? hdr.y : hdr.z;
  const float sc = (float)((sw >> (8 * (S & 3))) & 0x3Fu) * dd;
  const float m = (float)((sw >> (8 * (S & 3) + 6)) & 0x3u) * dm;
  const uint4 qs = tiled_chunk<NCH, BlkFmt<TYPE>::kQs + S, MODE>(slot, sbase, lane, nsrc);
  uint32_t h = 0;
  if constexpr (TYPE == QR_T_Q5_K) {
    const uint4 hv = qh[S >> 2];
    h = (S & 3) == 0 ? hv.x : (S & 3) == 1 ? hv.y : (S & 3) == 2 ? hv.z : hv.w;
  }
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const ActView a = act_read(act + (size_t)t * tokb + act_off(8 * b + S));
    int isum;
    if constexpr (TYPE == QR_T_Q4_K) isum = dot_q4_nib(qs, a);
    else isum = dot_q5_regs(qs, h, a.q);
    terms[t][S] = (sc * (float)isum - m * a.bsf) * a.bd;
  }
}

// One tile's terms (all 8 units of the lane's super-block, NT tokens).
template <int TYPE, int NT, int MODE>
__device__ inline void tiled_tile(const uint8_t* slot, uint32_t sbase, int lane,
                                  const uint8_t* const (&nsrc)[TiledFmt<TYPE>::kChunks],
                                  const uint8_t* act, size_t tokb, int b, float (&terms)[NT][8]) {
  constexpr int NCH = TiledFmt<TYPE>::kChunks;
  const uint4 hdr = tiled_chunk<NCH, 0, MODE>(slot, sbase, lane, nsrc);
  const float dd = qr_h2f(hdr.x & 0xFFFFu);
  const float dm = qr_h2f(hdr.x >> 16);
  uint4 qh[2];
  if constexpr (TYPE == QR_T_Q5_K) {
    qh[0] = tiled_chunk<NCH, 1, MODE>(slot, sbase, lane, nsrc);
    qh[1] = tiled_chunk<NCH, 2, MODE>(slot, sbase, lane, nsrc);
  }
  tiled_unit<TYPE, NT, 0, MODE>(slot, sbase, lane, nsrc, hdr, dd, dm, qh, act, tokb, b, terms);
  tiled_unit<TYPE, NT, 1, MODE>(slot, sbase, lane, nsrc, hdr, dd, dm, qh, act, tokb, b, terms);
  tiled_unit<TYPE, NT, 2, MODE>(slot, sbase, lane, nsrc, hdr, dd, dm, qh, act, tokb, b, terms);
  tiled_unit<TYPE, NT, 3, MODE>(slot, sbase, lane, nsrc, hdr, dd, dm, qh, act, tokb, b, terms);
  tiled_unit<TYPE, NT, 4, MODE>(slot, sbase, lane, nsrc, hdr, dd, dm, qh, act, tokb, b, terms);
  tiled_unit<TYPE, NT, 5, MODE>(slot, sbase, lane, nsrc, hdr, dd, dm, qh, act, tokb, b, terms);
  tiled_unit<TYPE, NT, 6, MODE>(slot, sbase, lane, nsrc, hdr, dd, dm, qh, act, tokb, b, terms);
  tiled_unit<TYPE, NT, 7, MODE>(slot, sbase, lane, nsrc, hdr, dd, dm, qh, act, tokb, b, terms);
}

// The GEMV's work as workgroup `bid` of `nbid` (a kernel of its own, or one
// role of a kernel that runs two matrices).
template <int TYPE, int NT, int NW, int PRO>
__device__ inline void tiled_body(const GemvArgs& g, uint8_t* smem, int bid, int nbid) {
  constexpr int NCH = TiledFmt<TYPE>::kChunks;
  constexpr int QW = NW < 4 ? NW : 4;  // quantizing waves
  constexpr bool NIB = BlkFmt<TYPE>::kNib;
  const int nb = g.t_nb, ntiles = g.t_ntiles;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int tstep = nbid * NW;
  int tile = bid * NW + wave;
  const bool has = tile < ntiles;
  // a wave whose first tile is its only one keeps a window of its chunks in
  // flight (Q4_K with the one-group start-up: the 32000 x 2048 GEMV gives
  // every wave one tile)
  constexpr bool WINOK = NCH == 9 && PRO == kProAsm1;
  const bool win = WINOK && has && tile + tstep >= ntiles;  // wave-uniform
  const size_t tokb = act_tok_bytes(g.d);
  uint8_t* act = smem;
  uint8_t* slot = smem + align16((size_t)NT * tokb) + (size_t)wave * NCH * 1024;
  const uint32_t sbase = lds_u32addr(slot);
  const uint8_t* src[NCH];
  tiled_src<TYPE>(g, has ? tile : 0, lane, src);
  const int qtid = (int)threadIdx.x;  // quantizing threads: 0 .. 64 QW - 1
  if constexpr (PRO == kProAsm1 || PRO == kProAsm2) {
    constexpr int G = PRO == kProAsm1 ? 1 : 2;
    if (wave < QW) {
      // groups qtid and qtid + 64 QW (of token gi / (d / 8))
      const int per_tok = g.d >> 3;
      const float* xp[G];
#pragma unroll
      for (int k = 0; k < G; k++) {
        const int q = qtid + k * 64 * QW;
        const int gi = q < NT * per_tok ? q : 0;
        int t = 0;  // gi / per_tok without a division (NT <= 4)
#pragma unroll
        for (int j = 1; j < NT; j++) t += gi >= j * per_tok;
        xp[k] = g.X + (size_t)t * g.xstride + (size_t)(gi - t * per_tok) * 8;
      }
      float4 u[2 * G];
      if constexpr (WINOK) {
        if (win) tiled_pro_asm_win(xp, src, sbase, u);
        else if (has) tiled_pro_asm<NCH, G>(xp, src, sbase, u);
        else tiled_x_asm<G>(xp, u);
      } else {
        if (has) tiled_pro_asm<NCH, G>(xp, src, sbase, u);
        else tiled_x_asm<G>(xp, u);
      }
#pragma unroll
      for (int k = 0; k < G; k++) {
        ActPre pre;
        pre.v[0] = u[2 * k].x; pre.v[1] = u[2 * k].y; pre.v[2] = u[2 * k].z;
        pre.v[3] = u[2 * k].w; pre.v[4] = u[2 * k + 1].x; pre.v[5] = u[2 * k + 1].y;
        pre.v[6] = u[2 * k + 1].z; pre.v[7] = u[2 * k + 1].w;
        quantize_act_blk<NIB, kActRegs>(g.X, (size_t)g.xstride, NT, g.d, act, pre, nullptr,
                                        qtid + k * 64 * QW, 64 * QW);
      }
    } else if (win) {
#pragma unroll
      for (int k = 0; k < kWin; k++) lds_dma16_nt(src[k], sbase + (uint32_t)(k * 1024));
    } else if (has) {
      tiled_dma<NCH>(src, sbase);
    }
  } else if constexpr (PRO == kProNorm) {
    static_assert(NT == 1, "the normalising start-up takes one token");
    constexpr int NP = (kNormFuseMax / 4 + 64 * NW - 1) / (64 * NW);
    float* xs = reinterpret_cast<float*>(smem + align16(tokb) + (size_t)NW * NCH * 1024);
    if (has) tiled_dma<NCH>(src, sbase);
    NormRegs<NP> r;
    norm_load<NP>(g.X, g.nw, g.d, (int)threadIdx.x, 64 * NW, r);
    norm_finish<NP>(r, g.d, xs, xs + g.d, (int)threadIdx.x, 64 * NW, bid == 0 ? g.nxb : nullptr);
    if (wave < QW) {
      ActPre pre;
      quantize_act_blk<NIB, kActLds>(g.X, (size_t)g.d, 1, g.d, act, pre, xs, qtid, 64 * QW);
    }
  } else {
    if (wave < QW) {
      ActPre pre;
      act_load8(g.X, (size_t)g.xstride, NT, g.d, qtid, pre.v);
      quantize_act_blk<NIB, kActGlobal>(g.X, (size_t)g.xstride, NT, g.d, act, pre, nullptr, qtid,
                                        64 * QW);
    } else if (has) {
      tiled_dma<NCH>(src, sbase);
    }
  }
  // LDS-only barrier: the tile DMA stays in flight across it
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  if (!has) return;  // no barriers below
  if constexpr (PRO == kProLate) {
    if (wave < QW) tiled_dma<NCH>(src, sbase);
  }
  // after the normalisation the first tile has long landed; the wait also
  // covers workgroup 0's stores, which would otherwise count in the ring's
  // "in flight" figures
  if constexpr (PRO == kProNorm) wait_vmcnt<0>();
  const int rl = lane / nb, b = lane - rl * nb;
  for (;;) {
    const int next = tile + tstep;
    float terms[NT][8];
    if (next < ntiles) {
      tiled_src<TYPE>(g, next, lane, src);
      tiled_tile<TYPE, NT, kChRing>(slot, sbase, lane, src, act, tokb, b, terms);
    } else if (WINOK && win) {  // the wave's only tile: src holds its own chunks
      tiled_tile<TYPE, NT, kChWindow>(slot, sbase, lane, src, act, tokb, b, terms);
    } else {
      tiled_tile<TYPE, NT, kChLast>(slot, sbase, lane, src, act, tokb, b, terms);
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

template <int TYPE, int NT, int NW, int PRO>
__global__ __launch_bounds__(64 * NW) void k_gemv_tiled(GemvArgs g) {
  extern __shared__ __align__(16) uint8_t smem[];
  tiled_body<TYPE, NT, NW, PRO>(g, smem, (int)blockIdx.x, (int)gridDim.x);
}

}  // namespace qr
