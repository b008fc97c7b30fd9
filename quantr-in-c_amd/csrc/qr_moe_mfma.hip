// qr_moe_mfma.hip -- grouped expert products on int8 MFMA (the MoE layer for
// T > 1 tokens).
//
// A work item is (64 weight rows of one expert) x (up to 16 or 32 dispatched
// (token, slot) pairs of that expert).  The K loop walks the rows one "stage"
// at a time -- one K-quant super-block, or 8 Q8_0 blocks -- with the rows'
// bytes (both matrices in gate/up mode) and the pairs' quantized activation
// records moved into LDS rings by DMA, and each (row, unit)'s fp32 scale and
// min decoded into LDS.  Each 32-element unit is one v_mfma_i32_16x16x32_i8
// per 16 x 16 tile of exact int32 unit sums.  The epilogue forms the
// reference's fp32 term of every (row, pair, unit) --
// (sc*isum - m*bsum)*bd for Q4_K/Q5_K (src/quant.c:384-400),
// sc*isum*bd for Q6_K (src/quant.c:422-434), isum*d*bd for Q8_0
// (src/quant.c:279-285) -- and adds it to the (row, pair) accumulator in
// unit order, so every output equals the reference's sequential fused dot.
//
// MFMA lane layout (v_mfma_i32_16x16x32_i8, checked on the device): A is
// lane -> row lane%16, elements 8*(lane/16)..+7 of the unit; B is lane -> pair
// lane%16, the same elements; D is lane -> pair lane%16, rows 4*(lane/16)+i.
// The 8 elements of a lane's A and B may be in any order as long as both use
// it: K-quant nibbles pair with activations stored [x0 x2 x4 x6 | x1 x3 x5 x7]
// (the order a nibble dword unpacks to), Q8_0 with natural order.
#include <stdio.h>

#include <type_traits>

#include "qr_blk.h"
#include "qr_tiled.h"
#include "qr_tokens.h"
#include "qr_internal.h"

namespace qr {

typedef int v4i __attribute__((ext_vector_type(4)));


// ---------------------------------------------------------------------------
// Activation rows -> quantized records in HBM (quantize_row_q8_0,
// src/quant.c:143-158, four lanes per 32-element block).
// ---------------------------------------------------------------------------
template <bool PERM>
__global__ __launch_bounds__(256) void k_quant_rows(const float* __restrict__ x, int xstride,
                                                   int nrows, int cols, uint8_t* __restrict__ out) {
  quant_rows_group<PERM>(x, xstride, nrows, cols, out, (long)blockIdx.x * 256 + threadIdx.x);
}

// ---------------------------------------------------------------------------
// Per-format stage geometry and unit decoding.
// ---------------------------------------------------------------------------
template <int TYPE>
struct MF {
  // bytes of one stage of a row: one super-block, or 8 Q8_0 blocks
  static constexpr int kStage = TYPE == QR_T_Q4_K ? 144 : TYPE == QR_T_Q5_K ? 176
                              : TYPE == QR_T_Q6_K ? 210 : 8 * QR_Q8_BYTES;
  // LDS slot of one row's stage: room for the up-to-15 misaligned head bytes
  // and the slack dword of unaligned reads
  static constexpr int kSlot = ((kStage + 15 + 4) + 15) / 16 * 16;
  static constexpr int kChunks = (kStage + 15 + 15) / 16;  // 16-byte loads that cover a stage
  static constexpr bool kPerm = TYPE != QR_T_Q8_0;
  static constexpr bool kMin = TYPE == QR_T_Q4_K || TYPE == QR_T_Q5_K;
};

// The bits of the float 1.5 * 2^23: adding an integer |S| < 2^22 to them
// gives the bits of the float 1.5 * 2^23 + S.
constexpr int kQ6Magic = 0x4B400000;

// Four bits (bits 0..3 of x) to bit 4 of 4 bytes.
__device__ inline uint32_t bits4_to_b4(uint32_t x) { return spread4(x) << 4; }

// A operand of unit s of a staged row (`o` = byte offset of the row's stage
// in the LDS slot area `wl`): the lane's 8 elements (k-group kg) as 8 int8.
template <int TYPE>
__device__ inline long unit_a(const uint32_t* wl, int o, int s, int kg) {
  uint32_t lo, hi;
  if constexpr (TYPE == QR_T_Q4_K) {
    const uint32_t w = wl[(o + 16 + 16 * s + 4 * kg) >> 2];  // aligned
    lo = w & 0x0F0F0F0Fu;
    hi = (w >> 4) & 0x0F0F0F0Fu;
  } else if constexpr (TYPE == QR_T_Q5_K) {
    const uint32_t w = wl[(o + 48 + 16 * s + 4 * kg) >> 2];
    const uint32_t t = (wl[(o + 16 + 4 * s) >> 2] >> (8 * kg)) & 0xFFu;
    const uint32_t ev = (t & 1u) | ((t >> 1) & 2u) | ((t >> 2) & 4u) | ((t >> 3) & 8u);
    const uint32_t od = ((t >> 1) & 1u) | ((t >> 2) & 2u) | ((t >> 3) & 4u) | ((t >> 4) & 8u);
    lo = (w & 0x0F0F0F0Fu) | bits4_to_b4(ev);
    hi = ((w >> 4) & 0x0F0F0F0Fu) | bits4_to_b4(od);
  } else {  // Q8_0 (Q6_K: unit_a_q6): block s, bytes 2 + 8 kg .. +7
    lo = lds_u32(wl, o + QR_Q8_BYTES * s + 2 + 8 * kg);
    hi = lds_u32(wl, o + QR_Q8_BYTES * s + 6 + 8 * kg);
  }
  return (long)((uint64_t)lo | ((uint64_t)hi << 32));
}

// Q6_K: a staged row starts at any even byte (210-byte stages), so the lane's
// ql and qh words of every unit are read as aligned dword pairs at indices
// fixed for the stage -- ql at dword w + 4 s shifted by wsh bytes, qh's 16
// bits at dword h + 2 s picked by the byte selector hsel -- and the 2-bit
// fields are moved to bits 4-5 of their bytes by shifts and masks.
struct Q6Ref {
  int w, h;
  uint32_t wsh, hsel;
};
__device__ inline Q6Ref q6_ref(int o, int kg) {
  Q6Ref q;
  const int ow = o + 4 * kg, oh = o + 128 + 2 * kg;
  q.w = ow >> 2;
  q.wsh = (uint32_t)(ow & 3);
  q.h = oh >> 2;
  const uint32_t k = (uint32_t)(oh & 3);
  q.hsel = k * 0x0101u + (k + 1) * 0x01010000u;  // bytes [k+1, k+1, k, k]
  return q;
}
__device__ inline long unit_a_q6(const uint32_t* wl, const Q6Ref& q, int s) {
  const uint32_t w = __builtin_amdgcn_alignbyte(wl[q.w + 4 * s + 1], wl[q.w + 4 * s], q.wsh);
  // x: qh bytes b1 b1 b0 b0; element i's low pair sits in bits 4i..4i+1 of
  // b1:b0, its high pair two bits up
  const uint32_t x = __builtin_amdgcn_perm(wl[q.h + 2 * s + 1], wl[q.h + 2 * s], q.hsel);
  const uint32_t lo = (w & 0x0F0F0F0Fu) | (((x << 4) & 0x00300030u) | (x & 0x30003000u));
  const uint32_t hi = ((w >> 4) & 0x0F0F0F0Fu) | (((x << 2) & 0x00300030u) | ((x >> 2) & 0x30003000u));
  return (long)((uint64_t)lo | ((uint64_t)hi << 32));
}

// fp32 scales (and mins) of the four units s0 .. s0 + 3 of a staged row (0
// past unit su), the row's header decoded once.
template <int TYPE>
__device__ inline void unit_scales4(const uint32_t* wl, int o, int s0, int su, float (&sc)[4],
                                    float (&mn)[4]) {
  if constexpr (TYPE == QR_T_Q4_K || TYPE == QR_T_Q5_K) {
    const uint32_t h0 = wl[o >> 2];
    const float d = qr_h2f(h0 & 0xFFFFu), dm = qr_h2f(h0 >> 16);
    const uint32_t w = wl[(o + 4 + s0) >> 2];  // 16-byte aligned stage: o % 4 == 0
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t b = (w >> (8 * i)) & 0xFFu;
      sc[i] = (float)(b & 63u) * d;
      mn[i] = (float)(b >> 6) * dm;
    }
  } else if constexpr (TYPE == QR_T_Q6_K) {
    const float d = qr_h2f(lds_u32(wl, o + 208) & 0xFFFFu);
    const uint32_t w = lds_u32(wl, o + 192 + s0);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      sc[i] = (float)(int)(int8_t)((w >> (8 * i)) & 0xFFu) * d;
      mn[i] = 0.0f;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      sc[i] = s0 + i < su ? qr_h2f(lds_u32(wl, o + QR_Q8_BYTES * (s0 + i)) & 0xFFFFu) : 0.0f;
      mn[i] = 0.0f;
    }
  }
}

// ---------------------------------------------------------------------------
// The grouped MFMA kernel.
//
// A workgroup of NW waves takes one work item: 16 NW weight rows of expert e
// (16 per wave; in gate/up mode the same 16 rows of both matrices) against
// one tile of up to NTOK = 16 NJ dispatched pairs of e.  The K loop walks the
// rows one stage at a time (one super-block, or 8 Q8_0 blocks: 8 units)
// through rings of D LDS slots filled by global_load_lds_dwordx4: the stage's
// activation records, shared by the waves (each moves its share), and each
// wave's own 16 x NMAT row stages.  With D >= 2, one barrier per stage: past
// it every wave's share of stage st has landed and every wave is done with
// stage st - 1, whose slots then take stage st + D - 1.  With one slot, a
// second barrier before each stage's DMA.  DMA waits are counted by hand
// (loads complete in issue order), so the compiler never holds a register or
// a wait for the stream.
// ---------------------------------------------------------------------------
struct MfmaArgs {
  const uint8_t* W1;      // [E][rows][rb] (up in gate/up mode)
  const uint8_t* W2;      // [E][rows][rb] (gate in gate/up mode)
  size_t slice;           // bytes per expert
  int rows, cols, E, K;
  const uint8_t* XQ;      // activation records [xrows][cols/32][kXQ]
  int x_by_token;         // activation row of dispatch position p: perm[p] / K, else p
  const int32_t* offsets; // dispatch (tile = NTOK)
  const int32_t* perm;
  const int32_t* tiles;
  float* Y;               // [P][ystride], row = dispatch position
  int ystride;
  // gate/up mode, optional: instead of Y, the activation records of the down
  // product ([P][rows/32], PERM order if qperm), quantized from the tile
  uint8_t* QO;
  int qperm;
  int skinny;             // work items of at most 4 pairs take the skinny form
  int wnt;                // weight DMA with the non-temporal hint (weights read about once)
  // Q4_K / Q5_K weights in the tiled layout (qr_tiled.h): rows per tile and
  // bytes per full tile; 0 for the row-major layout
  int t_rb;
  size_t t_tile_bytes;
};

template <int TYPE, bool GATEUP, int NJ, int RA, int D, int NW>
struct MfmaGeo {
  static constexpr int NMAT = GATEUP ? 2 : 1;
  static constexpr int NTOK = 16 * NJ;
  static constexpr int WR = 16 * RA;                       // rows per wave
  static constexpr int MR = NW * WR;                       // rows per workgroup
  // 16-byte chunks per row stage: Q4_K / Q5_K stages start 16-byte aligned,
  // the others anywhere (up to 15 bytes of head)
  static constexpr int NCH = (TYPE == QR_T_Q4_K || TYPE == QR_T_Q5_K) ? MF<TYPE>::kStage / 16
                                                                      : MF<TYPE>::kChunks;
  static constexpr int SLOT = NCH * 16;                    // LDS bytes per row stage
  static constexpr int WCH = NMAT * WR * NCH;              // a wave's chunks per stage
  static constexpr int WI = (WCH + 63) / 64;               // its DMA instructions
  static constexpr int WST = WI * 1024;                    // its LDS slot (whole instructions)
  // a pair's 8 records take 24 chunks plus one pad chunk: a 400-byte LDS
  // stride puts the 16 pairs of an MFMA B tile on different banks
  static constexpr int APC = 8 * kXQ / 16 + 1;             // chunks per pair (with pad)
  static constexpr int ACH = NTOK * APC;                   // activation chunks per stage
  static constexpr int AI = (ACH + 64 * NW - 1) / (64 * NW);  // per wave
  static constexpr int AST = NW * AI * 1024;               // LDS of one activation stage
  static constexpr int NI = WI + AI;                       // DMA instructions per wave and stage
  static constexpr int NSC = NMAT * 8 * WR;                // a wave's (matrix, unit, row)s
  static constexpr int SCL = NSC * 4;                      // their scales (or mins), bytes
  static constexpr int O_W = D * AST;                      // weight rings, wave-major
  static constexpr int O_S = O_W + NW * D * WST;           // scales, per wave
  static constexpr int O_M = O_S + NW * SCL;               // mins, per wave
  static constexpr int LDS = O_M + NW * SCL;
  // activation row of each pair, read once before the first stage: it shares
  // the scale area, first written after the first stage's barrier
  static constexpr int O_X = O_S;
  static_assert(NTOK * 4 <= NW * SCL, "xrow");
  static_assert(D >= 1 && D <= 3, "ring depth");
  static_assert(NI <= 63, "vmcnt range");
};

template <int TYPE, bool GATEUP, int NJ, int RA, int D, int NW>
__global__ __launch_bounds__(64 * NW) void k_expert_mfma(MfmaArgs a) {
  using G = MfmaGeo<TYPE, GATEUP, NJ, RA, D, NW>;
  constexpr int NMAT = G::NMAT;
  constexpr int NCH = G::NCH;
  constexpr int WR = G::WR;
  constexpr int KST = MF<TYPE>::kStage;
  extern __shared__ __align__(16) uint8_t smem[];

  // work item -> (expert e, first dispatch position p0, pair count np)
  const int item = blockIdx.y;
  const int ntiles = a.tiles[a.E];
  if (item >= ntiles) return;  // uniform
  int lo = 0, hi = a.E;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (a.tiles[mid] <= item) lo = mid;
    else hi = mid;
  }
  const int e = lo;
  const int p0 = a.offsets[e] + (item - a.tiles[e]) * G::NTOK;
  const int np = min(G::NTOK, a.offsets[e + 1] - p0);
  if (np <= 0) return;  // uniform
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int kg = lane >> 4, ln = lane & 15;
  const int rw0 = blockIdx.x * G::MR + wave * WR;  // the wave's first row
  const int U = TYPE == QR_T_Q8_0 ? a.cols / 32 : (a.cols / 256) * 8;
  const size_t rb = qr_wrow_bytes(TYPE, a.cols);
  const int nstage = (U + 7) / 8;
  int* xrow = reinterpret_cast<int*>(smem + G::O_X);
  if (threadIdx.x < G::NTOK) {
    int xr = 0;
    const int tt = threadIdx.x;
    if (tt < np) xr = a.x_by_token ? a.perm[p0 + tt] / a.K : p0 + tt;
    xrow[tt] = xr;
  }
  __syncthreads();  // xrow

  // Per-lane DMA sources, stage-invariant parts.  Weight chunk c = k*64+lane
  // of this wave: matrix c / (WR NCH), row rw0 + (c / NCH) % WR, chunk c % NCH
  // of the row's stage; chunks past the row's stage bytes, rows past the
  // matrix and lanes past the wave's chunks reload the workgroup's first row's
  // stage start.
  const size_t ebase = (size_t)e * a.slice;
  const uint32_t row0 = (uint32_t)(blockIdx.x * G::MR) * (uint32_t)rb;  // within the slice
  const uint8_t* wbase[G::WI];  // the chunk's matrix, at the expert's slice
  uint32_t wroff[G::WI];        // its row's offset in the slice, or ~0 (no row)
  int wch[G::WI];
  int wrow[G::WI];              // its row, or -1
#pragma unroll
  for (int k = 0; k < G::WI; k++) {
    const int c = k * 64 + lane;
    const int m = c / (WR * NCH);
    const int rem = c - m * WR * NCH;
    const int rr = rem / NCH;
    wch[k] = rem - rr * NCH;
    const int row = rw0 + rr;
    wroff[k] = (c < G::WCH && row < a.rows) ? (uint32_t)row * (uint32_t)rb : ~0u;
    wrow[k] = (c < G::WCH && row < a.rows) ? row : -1;
    wbase[k] = ((GATEUP && m == 1) ? a.W2 : a.W1) + ebase;
  }
  // Activation chunk c = (wave AI + k) 64 + lane: pair c / APC, chunk c % APC
  // of its 8 records (unit (c % APC) / 3; chunk 24 is the pad).  asrc: the
  // chunk's offset in XQ at stage 0, or ~0 (reload pair 0's first chunk).
  const size_t xq_row = (size_t)U * kXQ;
  size_t asrc[G::AI];
  int aunit[G::AI];
#pragma unroll
  for (int k = 0; k < G::AI; k++) {
    const int c = (wave * G::AI + k) * 64 + lane;
    const int tt = c / G::APC;
    const int ch = c - tt * G::APC;
    const bool ok = c < G::ACH && tt < np && ch < G::APC - 1;
    asrc[k] = ok ? (size_t)xrow[tt] * xq_row + 16 * (size_t)ch : ~(size_t)0;
    aunit[k] = ch / 3;
  }
  const size_t asrc0 = (size_t)xrow[0] * xq_row;
  // Q4_K / Q5_K: a row's stage is whole 16-byte chunks (rows and stages are
  // multiples of 16 bytes) and every stage's 8 units exist, so each source is
  // a stage-invariant address plus the stage's offset
  constexpr bool ALN = TYPE == QR_T_Q4_K || TYPE == QR_T_Q5_K;
  const uint8_t* wp[G::WI];
  const uint8_t* ap[G::AI];
  // In the tiled layout the stage's chunk ch of row r is chunk ch of lane
  // (r % RB) nb + stage of tile r / RB: tile start + 16 (ch L + lane), L the
  // tile's lanes, so a stage advances the address by 16 bytes instead of a
  // super-block.
  if constexpr (ALN) {
    const int nbk = a.cols >> 8;
#pragma unroll
    for (int k = 0; k < G::WI; k++) {
      if (wroff[k] == ~0u) {
        wp[k] = a.t_rb ? a.W1 + ebase : a.W1 + ebase + row0;
      } else if (a.t_rb) {
        const int r = wrow[k], t = r / a.t_rb;
        const int L = min(a.t_rb, a.rows - t * a.t_rb) * nbk;
        wp[k] = wbase[k] + (size_t)t * a.t_tile_bytes + (size_t)16 * wch[k] * L +
                (size_t)16 * (r - t * a.t_rb) * nbk;
      } else {
        wp[k] = wbase[k] + wroff[k] + 16 * wch[k];
      }
    }
#pragma unroll
    for (int k = 0; k < G::AI; k++) ap[k] = a.XQ + (asrc[k] != ~(size_t)0 ? asrc[k] : asrc0);
  }

  auto issue = [&](int st) {
    const int slot = st % D;
    const uint32_t abase = lds_u32addr(smem + slot * G::AST) + (uint32_t)(wave * G::AI * 1024);
    if constexpr (ALN) {
      const size_t ao = (size_t)(8 * st) * kXQ;
#pragma unroll
      for (int k = 0; k < G::AI; k++) lds_dma16(ap[k] + ao, abase + (uint32_t)(k * 1024));
      const uint32_t wlds = lds_u32addr(smem + G::O_W + (wave * D + slot) * G::WST);
      const uint32_t s0 = (uint32_t)st * (a.t_rb ? 16u : (uint32_t)KST);
      if (a.wnt) {
#pragma unroll
        for (int k = 0; k < G::WI; k++) lds_dma16_nt(wp[k] + s0, wlds + (uint32_t)(k * 1024));
      } else {
#pragma unroll
        for (int k = 0; k < G::WI; k++) lds_dma16(wp[k] + s0, wlds + (uint32_t)(k * 1024));
      }
      return;
    }
#pragma unroll
    for (int k = 0; k < G::AI; k++) {
      const bool ok = asrc[k] != ~(size_t)0 && 8 * st + aunit[k] < U;
      const size_t src = (ok ? asrc[k] : asrc0) + (size_t)(8 * st) * kXQ;
      lds_dma16(a.XQ + src, abase + (uint32_t)(k * 1024));
    }
    const uint32_t wlds = lds_u32addr(smem + G::O_W + (wave * D + slot) * G::WST);
    // offsets within the expert's slice: its base is 16-byte aligned, so
    // alignment within the slice is alignment in memory
    const uint32_t s0 = (uint32_t)st * KST;
    const uint32_t se = s0 + KST < (uint32_t)rb ? s0 + KST : (uint32_t)rb;
    const uint32_t clampoff = (row0 + s0) & ~15u;
#pragma unroll
    for (int k = 0; k < G::WI; k++) {
      uint32_t off = clampoff;
      const uint8_t* W = a.W1 + ebase;
      if (wroff[k] != ~0u) {
        const uint32_t o = ((wroff[k] + s0) & ~15u) + 16u * (uint32_t)wch[k];
        if (o < wroff[k] + se) {
          off = o;
          W = wbase[k];
        }
      }
      if (a.wnt) lds_dma16_nt(W + off, wlds + (uint32_t)(k * 1024));
      else lds_dma16(W + off, wlds + (uint32_t)(k * 1024));
    }
  };

  float* scl = reinterpret_cast<float*>(smem + G::O_S + wave * G::SCL);
  float* mnl = reinterpret_cast<float*>(smem + G::O_M + wave * G::SCL);

  // The stage loop and the outputs, in two forms.  Full: an MFMA per (unit,
  // matrix, 16-row tile, 16-pair column tile), A = weights, B = pairs; lane
  // (ln, kg) accumulates rows 4 kg + i of pair 16 j + ln.  Skinny (a work
  // item of at most 4 pairs): A = the pairs with each pair's 32 elements split
  // into 4 k-quarters on 4 A rows (row 4 t + q holds pair t's quarter q, zeros
  // elsewhere), B = weights; lane (ln, kg) receives the 4 quarter sums of pair
  // kg and row ln, adds them (exact integers) and forms one term -- a quarter
  // of the full form's epilogue work for the same 16 rows.
  auto run = [&](auto form_tag) {
    // form: 0 skinny, else the number of 16-pair column tiles computed (the
    // work item's pairs need no more)
    constexpr int FORM = decltype(form_tag)::value;
    constexpr bool SK = FORM == 0;
    constexpr int NJA = SK ? 1 : FORM;
    float acc[NMAT][RA][NJ][4];
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
      for (int r = 0; r < RA; r++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
          for (int i = 0; i < 4; i++) acc[m][r][j][i] = 0.0f;

#pragma unroll
    for (int s = 0; s < D - 1; s++)
      if (s < nstage) issue(s);
    for (int st = 0; st < nstage; st++) {
      if constexpr (D == 1) {
        // one slot: every wave is done with stage st - 1 before stage st
        // lands in it
        if (st > 0) {
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          __builtin_amdgcn_s_barrier();
        }
        issue(st);
      }
      // stage st has landed once no more than the later stages' DMA is in flight
      if (D == 3 && st + 1 < nstage) wait_vmcnt<G::NI>();
      else wait_vmcnt<0>();
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      if (D > 1 && st + D - 1 < nstage) issue(st + D - 1);
      const int slot = st % D;
      const uint32_t* wl =
          reinterpret_cast<const uint32_t*>(smem + G::O_W + (wave * D + slot) * G::WST);
      const uint8_t* as = smem + slot * G::AST;
      const int su = min(8, U - st * 8);
      const uint32_t s0 = (uint32_t)st * KST;
      // scales and mins of the wave's (matrix, unit, row)s, entry
      // (m * 8 + s) * WR + rr: lane (m, rr, half) decodes row rr's header once
      // for units 4 half .. 4 half + 3
      for (int i = lane; i < NMAT * WR * 2; i += 64) {
        const int m = i / (2 * WR), rem = i - m * 2 * WR;
        const int rr = rem >> 1, half = rem & 1;
        float sc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, mn[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        const int row = rw0 + rr;
        if (4 * half < su && row < a.rows) {
          const int hd = (int)(((uint32_t)row * (uint32_t)rb + s0) & 15u);
          unit_scales4<TYPE>(wl, (m * WR + rr) * G::SLOT + hd, 4 * half, su, sc, mn);
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
          scl[(m * 8 + 4 * half + q) * WR + rr] = sc[q];
          mnl[(m * 8 + 4 * half + q) * WR + rr] = mn[q];
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      // head bytes of this lane's weight rows (both matrices share them: same
      // slice and row sizes, 16-byte aligned bases)
      int hA[RA];
#pragma unroll
      for (int r = 0; r < RA; r++)
        hA[r] = (int)(((uint32_t)(rw0 + 16 * r + ln) * (uint32_t)rb + s0) & 15u);
      Q6Ref q6[NMAT][RA];
      if constexpr (TYPE == QR_T_Q6_K) {
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
          for (int r = 0; r < RA; r++) q6[m][r] = q6_ref((m * WR + 16 * r + ln) * G::SLOT + hA[r], kg);
      }
      auto term_of = [&](float sc, float mn, int isum, float bd, float bsf, int bs) {
        if constexpr (MF<TYPE>::kMin) return (sc * (float)isum - mn * bsf) * bd;
        else if constexpr (TYPE == QR_T_Q6_K) return sc * (float)(isum - 32 * bs) * bd;
        else return (float)isum * sc * bd;
      };
      auto unit_step = [&](int s) {
        long Wq[NMAT][RA];
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
          for (int r = 0; r < RA; r++)
            if constexpr (TYPE == QR_T_Q6_K) Wq[m][r] = unit_a_q6(wl, q6[m][r], s);
            else Wq[m][r] = unit_a<TYPE>(wl, (m * WR + 16 * r + ln) * G::SLOT + hA[r], s, kg);
        if constexpr (SK) {
          // A: pair ln / 4's quarter ln % 4 on A row ln (zeros in the other
          // k-groups); the term's pair is kg
          const uint8_t* ra = as + (ln >> 2) * (16 * G::APC) + s * kXQ;
          const uint2 xq = *reinterpret_cast<const uint2*>(ra + 8 * kg);
          const bool mine = kg == (ln & 3);
          const long Aq = mine ? (long)((uint64_t)xq.x | ((uint64_t)xq.y << 32)) : 0l;
          const uint8_t* rt = as + kg * (16 * G::APC) + s * kXQ;
          const float bd = *reinterpret_cast<const float*>(rt + 32);
          const float bsf = *reinterpret_cast<const float*>(rt + 36);
          const int bs = *reinterpret_cast<const int*>(rt + 40);
#pragma unroll
          for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int r = 0; r < RA; r++) {
              const v4i zero = {0, 0, 0, 0};
              const v4i Dv = __builtin_amdgcn_mfma_i32_16x16x32_i8(Aq, Wq[m][r], zero, 0, 0, 0);
              const int isum = (Dv[0] + Dv[1]) + (Dv[2] + Dv[3]);
              const int si = (m * 8 + s) * WR + 16 * r + ln;
              acc[m][r][0][0] += term_of(scl[si], mnl[si], isum, bd, bsf, bs);
            }
        } else {
#pragma unroll
          for (int j = 0; j < NJA; j++) {
            const uint8_t* rec = as + (16 * j + ln) * (16 * G::APC) + s * kXQ;
            const uint2 bq = *reinterpret_cast<const uint2*>(rec + 8 * kg);
            const long B = (long)((uint64_t)bq.x | ((uint64_t)bq.y << 32));
            const float bd = *reinterpret_cast<const float*>(rec + 32);
            const float bsf = *reinterpret_cast<const float*>(rec + 36);
            const int bs = *reinterpret_cast<const int*>(rec + 40);
            // Q6_K: the accumulator starts at the bits of 1.5 * 2^23, so each
            // exact sum S (|S| <= 32 * 63 * 127 < 2^22) comes out as the bits
            // of the float 1.5 * 2^23 + S; less 1.5 * 2^23 + 32 bs (exact
            // too) that is (float)(S - 32 bs) in one exact subtraction, the
            // value the reference's (float)isum holds
            const float q6m = __builtin_bit_cast(float, kQ6Magic + 32 * bs);
#pragma unroll
            for (int m = 0; m < NMAT; m++)
#pragma unroll
              for (int r = 0; r < RA; r++) {
                const v4i c0 = TYPE == QR_T_Q6_K ? v4i{kQ6Magic, kQ6Magic, kQ6Magic, kQ6Magic}
                                                 : v4i{0, 0, 0, 0};
                const v4i Dv = __builtin_amdgcn_mfma_i32_16x16x32_i8(Wq[m][r], B, c0, 0, 0, 0);
                const int si = (m * 8 + s) * WR + 16 * r + 4 * kg;
                const float4 sc4 = *reinterpret_cast<const float4*>(scl + si);
                const float4 mn4 = *reinterpret_cast<const float4*>(mnl + si);
                const float scv[4] = {sc4.x, sc4.y, sc4.z, sc4.w};
                const float mnv[4] = {mn4.x, mn4.y, mn4.z, mn4.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                  if constexpr (TYPE == QR_T_Q6_K) {
                    // each element passes through an empty asm before its
                    // float view: without it this compiler (ROCm 7.2 clang)
                    // folds the four subtractions of the float views of an
                    // MFMA result's elements into one, on element 0
                    int di = Dv[i];
                    asm("" : "+v"(di));
                    acc[m][r][j][i] += scv[i] * (__builtin_bit_cast(float, di) - q6m) * bd;
                  } else {
                    acc[m][r][j][i] += term_of(scv[i], mnv[i], Dv[i], bd, bsf, bs);
                  }
                }
              }
          }
        }
      };
      if (su == 8) {
        // every stage of a K-quant, and whole Q8_0 stages: unrolled, so the
        // units' LDS reads and MFMAs interleave
#pragma unroll
        for (int s = 0; s < 8; s++) unit_step(s);
      } else {
        for (int s = 0; s < su; s++) unit_step(s);
      }
    }

    // output element (j, i) of row tile r: pair tt, row
    auto out_pos = [&](int r, int j, int i, int* tt, int* row) {
      if constexpr (SK) {
        *tt = kg;
        *row = rw0 + 16 * r + ln;
      } else {
        *tt = 16 * j + ln;
        *row = rw0 + 16 * r + 4 * kg + i;
      }
    };
    constexpr int OJ = NJA, OI = SK ? 1 : 4;

    if constexpr (GATEUP) {
      if (a.QO) {
        // hb = silu(up) * gate of the tile's rows and pairs -> LDS [NTOK][MR]
        // (the activation ring is free now) -> whole 32-row blocks per pair
        // quantized (quantize_row_q8_0, as the down product's matmul_q_fused
        // does) into the down product's activation records
        float* ob = reinterpret_cast<float*>(smem);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();  // every wave is done with the last stage
#pragma unroll
        for (int j = 0; j < OJ; j++)
#pragma unroll
          for (int r = 0; r < RA; r++)
#pragma unroll
            for (int i = 0; i < OI; i++) {
              int tt, row;
              out_pos(r, j, i, &tt, &row);
              ob[tt * G::MR + (row - blockIdx.x * G::MR)] =
                  qr_silu(acc[0][r][j][i]) * acc[NMAT - 1][r][j][i];
            }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        constexpr int NB = G::MR / 32;  // blocks per pair in the tile
        constexpr int NT = SK ? 4 : 16 * NJA;
        const int nrec = a.rows >> 5;
        for (int g = threadIdx.x; g < NT * NB * 4; g += 64 * NW) {  // whole quads
          const int tt = g / (NB * 4), rem = g - tt * (NB * 4);
          const int blk = rem >> 2, part = rem & 3;
          const float* src = ob + tt * G::MR + blk * 32 + part * 8;
          float v[8];
#pragma unroll
          for (int i = 0; i < 8; i++) v[i] = src[i];
          uint2 q8;
          float bd;
          int bs;
          if (a.qperm) quant8_core<true>(v, &q8, &bd, &bs);
          else quant8_core<false>(v, &q8, &bd, &bs);
          const int row0 = blockIdx.x * G::MR + blk * 32;
          if (tt < np && row0 < a.rows)
            record_store(a.QO + ((size_t)(p0 + tt) * nrec + (row0 >> 5)) * kXQ, part, q8, bd, bs);
        }
        return;
      }
    }

#pragma unroll
    for (int j = 0; j < OJ; j++)
#pragma unroll
      for (int r = 0; r < RA; r++)
#pragma unroll
        for (int i = 0; i < OI; i++) {
          int tt, row;
          out_pos(r, j, i, &tt, &row);
          if (tt >= np || row >= a.rows) continue;
          float out = acc[0][r][j][i];
          if constexpr (GATEUP) out = qr_silu(acc[0][r][j][i]) * acc[NMAT - 1][r][j][i];
          a.Y[(size_t)(p0 + tt) * a.ystride + row] = out;
        }
  };
  if (np <= 4 && a.skinny) run(std::integral_constant<int, 0>{});
  else if (NJ == 1 || np <= 16) run(std::integral_constant<int, 1>{});
  else run(std::integral_constant<int, NJ>{});
}


// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
bool mfma_type_ok(int type) {
  return type == QR_T_Q4_K || type == QR_T_Q5_K || type == QR_T_Q6_K || type == QR_T_Q8_0;
}

hipError_t quant_rows_launch(const float* x, int xstride, int nrows, int cols, bool perm,
                             uint8_t* out, hipStream_t st) {
  const long total = (long)nrows * (cols / 32) * 4;
  if (total <= 0) return hipSuccess;
  const unsigned grid = (unsigned)((total + 255) / 256);
  if (perm) hipLaunchKernelGGL(k_quant_rows<true>, dim3(grid), dim3(256), 0, st, x, xstride, nrows, cols, out);
  else hipLaunchKernelGGL(k_quant_rows<false>, dim3(grid), dim3(256), 0, st, x, xstride, nrows, cols, out);
  return hipGetLastError();
}

// Pairs per work item: 16 while experts see few pairs each (less padding of
// the 16-pair MFMA tile), 32 beyond (half the weight re-reads).
int mfma_tile(int T, int K, int E) { return (long)T * K >= 16L * E ? 32 : 16; }

template <int TYPE, bool GATEUP, int NJ, int D, int NW>
static hipError_t mfma_launch_t(const MfmaArgs& a, int items, hipStream_t st) {
  using G = MfmaGeo<TYPE, GATEUP, NJ, 1, D, NW>;
  if constexpr (G::LDS > 160 * 1024) {
    return mfma_launch_t<TYPE, GATEUP, NJ, 2, 4>(a, items, st);  // the shape that always fits
  } else {
    static std::atomic<bool> opted[64];
    dim3 grid((a.rows + G::MR - 1) / G::MR, items);
    if (grid.x == 0 || grid.y == 0) return hipSuccess;
    if (G::LDS > 64 * 1024) {
      const hipError_t e = lds_opt_in((const void*)k_expert_mfma<TYPE, GATEUP, NJ, 1, D, NW>, opted);
      if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((k_expert_mfma<TYPE, GATEUP, NJ, 1, D, NW>), grid, dim3(64 * NW), G::LDS,
                       st, a);
    return hipGetLastError();
  }
}

// Kernel shape per product: NW waves per workgroup (4, or 2 where a single
// expert's product would otherwise leave CUs idle), each on 16 rows, and a
// ring of D stages.  Measured on the Qwen3-30B-A3B layer: one slot (the least
// LDS, the most workgroups per CU) wins where the epilogue's VALU work
// dominates -- both products with 32-pair items, the 24-unit down product
// always -- and two slots for gate/up with 16-pair items, whose eight stages
// are latency bound.
template <int TYPE, bool GATEUP, int NJ>
static hipError_t mfma_launch_shape(const MfmaArgs& a, int items, int nw, bool ring,
                                    hipStream_t st) {
  constexpr int D = (GATEUP && NJ == 1) ? 2 : 1;
  if (nw == 2) {
    if (ring) return mfma_launch_t<TYPE, GATEUP, NJ, 2, 2>(a, items, st);
    return mfma_launch_t<TYPE, GATEUP, NJ, D, 2>(a, items, st);
  }
  if (ring) return mfma_launch_t<TYPE, GATEUP, NJ, 2, 4>(a, items, st);
  return mfma_launch_t<TYPE, GATEUP, NJ, D, 4>(a, items, st);
}

template <int TYPE, bool GATEUP>
static hipError_t mfma_launch_nj(const MfmaArgs& a, int items, int tile, int nw, bool ring,
                                 hipStream_t st) {
  if (tile == 32) return mfma_launch_shape<TYPE, GATEUP, 2>(a, items, nw, ring, st);
  return mfma_launch_shape<TYPE, GATEUP, 1>(a, items, nw, ring, st);
}

hipError_t expert_mfma_launch(int type, bool gateup, const uint8_t* W1, const uint8_t* W2,
                              size_t slice, int E, int K, int rows, int cols, const uint8_t* XQ,
                              int x_by_token, const int32_t* offsets, const int32_t* perm,
                              const int32_t* tiles, float* Y, int ystride, int items, int tile,
                              uint8_t* QO, bool qperm, hipStream_t st, bool tiled) {
  if (tile != 16 && tile != 32) return hipErrorInvalidValue;
  if (slice >= ((size_t)1 << 32)) return hipErrorInvalidValue;  // 32-bit offsets in a slice
  if (QO && (!gateup || (rows & 31) || (reinterpret_cast<uintptr_t>(QO) & 15)))
    return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(W1) & 15) || (gateup && (reinterpret_cast<uintptr_t>(W2) & 15)) ||
      (reinterpret_cast<uintptr_t>(XQ) & 15))
    return hipErrorInvalidValue;
  MfmaArgs a;
  a.W1 = W1;
  a.W2 = W2;
  a.slice = slice;
  a.rows = rows;
  a.cols = cols;
  a.E = E;
  a.K = K;
  a.XQ = XQ;
  a.x_by_token = x_by_token;
  a.offsets = offsets;
  a.perm = perm;
  a.tiles = tiles;
  a.Y = Y;
  a.ystride = ystride;
  a.QO = QO;
  a.qperm = qperm ? 1 : 0;
  a.skinny = 1;
  a.t_rb = 0;
  a.t_tile_bytes = 0;
  if (tiled) {  // Q4_K / Q5_K rows of whole super-blocks, at most 64 per row
    if ((type != QR_T_Q4_K && type != QR_T_Q5_K) || (cols & 255) || (cols >> 8) > 64)
      return hipErrorInvalidValue;
    const TiledGeom tg = tiled_geom(type, rows, cols);
    a.t_rb = tg.RB;
    a.t_tile_bytes = tg.tile_bytes;
  }
  // items of up to 16 pairs: an expert rarely has more than one, so its rows
  // are read about once and the hint keeps the activation records cached;
  // with 32-pair items hot experts are re-read by several items
  a.wnt = tile <= 16;
  // one expert (a dense product): items - 1 = ceil(P / tile) exactly; with
  // fewer than two workgroups of 64 rows per CU, workgroups of 32 rows
  // and a two-slot ring for its long rows (each workgroup walks them alone)
  int nw = 4;
  if (E == 1 && (long)((rows + 63) / 64) * (items - 1) < 2L * device_cus()) nw = 2;
  const int stages = type == QR_T_Q8_0 ? (cols / 32 + 7) / 8 : cols / 256;
  const bool ring = E == 1 && stages >= 8;
  switch (type) {
    case QR_T_Q4_K: return gateup ? mfma_launch_nj<QR_T_Q4_K, true>(a, items, tile, nw, ring, st)
                                  : mfma_launch_nj<QR_T_Q4_K, false>(a, items, tile, nw, ring, st);
    case QR_T_Q5_K: return gateup ? mfma_launch_nj<QR_T_Q5_K, true>(a, items, tile, nw, ring, st)
                                  : mfma_launch_nj<QR_T_Q5_K, false>(a, items, tile, nw, ring, st);
    case QR_T_Q6_K: return gateup ? mfma_launch_nj<QR_T_Q6_K, true>(a, items, tile, nw, ring, st)
                                  : mfma_launch_nj<QR_T_Q6_K, false>(a, items, tile, nw, ring, st);
    case QR_T_Q8_0: return gateup ? mfma_launch_nj<QR_T_Q8_0, true>(a, items, tile, nw, ring, st)
                                  : mfma_launch_nj<QR_T_Q8_0, false>(a, items, tile, nw, ring, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qr
