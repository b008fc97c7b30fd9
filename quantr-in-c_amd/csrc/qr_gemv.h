// qr_gemv.h -- device building blocks of the quantized GEMV: the in-LDS Q8_0
// activation quantizer, per-format 32-element unit dots, and the sequential
// per-row fp32 reduction.  Shared by the plain GEMV kernels (qr_gemv.hip) and
// the grouped MoE expert kernels (qr_moe.hip).
#pragma once

#include "qr_common.h"

namespace qr {

// ---------------------------------------------------------------------------
// Activation in LDS.  One token's Q8_0 activation is d int8 values plus, per
// 32-element block, the decoded fp16 scale (float) and the integer sum of the
// block's values.  K-quant nibble layouts pair element 2i with 2i+1 in one
// byte; for Q4_K the int8 values are stored per 8-element group as
// [x0 x2 x4 x6 | x1 x3 x5 x7] so that the low and high nibbles of one weight
// dword multiply one activation dword each.  Other formats use natural order.
// ---------------------------------------------------------------------------
struct ActLds {
  int8_t* q;     // [nt][(d/32)*32]
  float* bd;     // [nt][d/32]  h2f(f2h(d)) of each block
  int32_t* bs;   // [nt][d/32]  sum of the block's int8 values
};

__device__ inline uint32_t pack4(int a, int b, int c, int e) {
  return (uint32_t)(uint8_t)a | ((uint32_t)(uint8_t)b << 8) | ((uint32_t)(uint8_t)c << 16) |
         ((uint32_t)(uint8_t)e << 24);
}

// quantize_row_q8_0 (src/quant.c:143-158) of nt rows x[t*xstride .. +d) into
// LDS, by the whole workgroup.  Each thread owns 8-element groups; the four
// threads of one 32-block are adjacent lanes, so amax and the block sum reduce
// with two xor-shuffles.  amax is a max (order-free); d = amax/127 and 1/d
// are correctly rounded IEEE divisions; rintf rounds ties to even like
// lrintf; the stored scale goes through the truncating fp16 routine.
//
// Rows t < nlive come from x + rows[t] * xstride (rows may be null: row t);
// rows nlive <= t < nt are filled with zeros so that every LDS slot a kernel
// may read is defined.
template <bool PERM>
__device__ inline void quantize_act_lds(const float* __restrict__ x, size_t xstride,
                                        const int* rows, int nlive, int nt, int d, ActLds a) {
  const int nxb = d >> 5;                 // whole 32-blocks; a shorter tail is ignored
  const int ngroups = nxb * 4;            // 8-element groups per row
  const int qstride = nxb * 32;           // LDS row stride of the int8 values
  const int total = nt * ngroups;
  const int nthr = blockDim.x;            // a multiple of 64
  for (int base = 0; base < ((total + nthr - 1) / nthr) * nthr; base += nthr) {
    const int gi = base + (int)threadIdx.x;
    const bool live = gi < total;
    const int t = live ? gi / ngroups : 0;
    const int g = live ? gi - t * ngroups : 0;
    float v[8];
    if (live && t < nlive) {
      const size_t row = rows ? (size_t)rows[t] : (size_t)t;
      const float4* p = reinterpret_cast<const float4*>(x + row * xstride + (size_t)g * 8);
      const float4 u0 = p[0], u1 = p[1];
      v[0] = u0.x; v[1] = u0.y; v[2] = u0.z; v[3] = u0.w;
      v[4] = u1.x; v[5] = u1.y; v[6] = u1.z; v[7] = u1.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = 0.0f;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float av = __builtin_fabsf(v[i]);
      amax = av > amax ? av : amax;
    }
    // groups g..g+3 of one block sit in lanes 4k..4k+3 when nthr % 4 == 0
    float o1 = __shfl_xor(amax, 1);
    amax = o1 > amax ? o1 : amax;
    o1 = __shfl_xor(amax, 2);
    amax = o1 > amax ? o1 : amax;
    const float dd = amax / 127.0f;
    const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
    int q[8];
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      q[i] = (int)(int8_t)(int)__builtin_rintf(v[i] * id);
      s += q[i];
    }
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    if (live) {
      uint32_t w0, w1;
      if (PERM) {
        w0 = pack4(q[0], q[2], q[4], q[6]);
        w1 = pack4(q[1], q[3], q[5], q[7]);
      } else {
        w0 = pack4(q[0], q[1], q[2], q[3]);
        w1 = pack4(q[4], q[5], q[6], q[7]);
      }
      uint2* dst = reinterpret_cast<uint2*>(a.q + (size_t)t * qstride + (size_t)g * 8);
      *dst = make_uint2(w0, w1);
      if ((g & 3) == 0) {
        const int b = t * nxb + (g >> 2);
        a.bd[b] = qr_h2f(qr_f2h(dd));
        a.bs[b] = s;
      }
    }
  }
}

__device__ inline int sdot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Spread 4 bits to bit 0 of 4 bytes (no carries: the shifted copies of the 4
// bits land on distinct positions).
__device__ inline uint32_t spread4(uint32_t x) { return ((x & 0xFu) * 0x00204081u) & 0x01010101u; }
// Spread the four 2-bit fields of a byte to bits 0-1 of 4 bytes.
__device__ inline uint32_t spread2x4(uint32_t b) {
  uint32_t t = (b | (b << 12)) & 0x000F000Fu;
  return (t | (t << 6)) & 0x03030303u;
}
// Interleave the low / high nibble bytes of a packed dword back into element
// order: lo holds elements 0,2,4,6 and hi 1,3,5,7 (one per byte).
__device__ inline uint32_t nib_lo_pair(uint32_t lo, uint32_t hi) {
  return __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // [lo0 hi0 lo1 hi1]
}
__device__ inline uint32_t nib_hi_pair(uint32_t lo, uint32_t hi) {
  return __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // [lo2 hi2 lo3 hi3]
}

// Unaligned dword from LDS (byte offset o), from two aligned dwords.
__device__ inline uint32_t lds_u32(const uint32_t* lds, int o) {
  const uint32_t lo = lds[o >> 2];
  const uint32_t hi = lds[(o >> 2) + 1];
  return __builtin_amdgcn_alignbyte(hi, lo, (uint32_t)(o & 3));
}

// ---------------------------------------------------------------------------
// Per-unit integer dots.  A unit is 32 weights against one Q8_0 activation
// block: xv holds its 32 int8 values as 8 dwords (PERM order for Q4_K,
// natural order otherwise).  The *_unit forms read them from LDS (`xa`,
// 16-byte aligned).
// ---------------------------------------------------------------------------
__device__ inline void act8_from_lds(const int8_t* xa, uint32_t xv[8]) {
  const uint4 x0 = *reinterpret_cast<const uint4*>(xa);
  const uint4 x1 = *reinterpret_cast<const uint4*>(xa + 16);
  xv[0] = x0.x; xv[1] = x0.y; xv[2] = x0.z; xv[3] = x0.w;
  xv[4] = x1.x; xv[5] = x1.y; xv[6] = x1.z; xv[7] = x1.w;
}

// Q4_K sub-block: 16 bytes of nibbles against a PERM-layout activation.
__device__ inline int dot_q4_regs(uint4 qs, const uint32_t xv[8]) {
  const uint32_t wq[4] = {qs.x, qs.y, qs.z, qs.w};
  int acc = 0;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    acc = sdot4(wq[k] & 0x0F0F0F0Fu, xv[2 * k], acc);
    acc = sdot4((wq[k] >> 4) & 0x0F0F0F0Fu, xv[2 * k + 1], acc);
  }
  return acc;
}
__device__ inline int dot_q4_unit(uint4 qs, const int8_t* xa) {
  uint32_t xv[8];
  act8_from_lds(xa, xv);
  return dot_q4_regs(qs, xv);
}

// 4-bit nibbles (+ high bits already spread per natural dword) against a
// natural-order activation.  qs holds 4 packed dwords (32 nibbles).
__device__ inline int dot_nib_regs(uint4 qs, const uint32_t hb[8], const uint32_t xv[8]) {
  const uint32_t wq[4] = {qs.x, qs.y, qs.z, qs.w};
  int acc = 0;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const uint32_t lo = wq[k] & 0x0F0F0F0Fu;
    const uint32_t hi = (wq[k] >> 4) & 0x0F0F0F0Fu;
    acc = sdot4(nib_lo_pair(lo, hi) | hb[2 * k], xv[2 * k], acc);
    acc = sdot4(nib_hi_pair(lo, hi) | hb[2 * k + 1], xv[2 * k + 1], acc);
  }
  return acc;
}

// Q5_K sub-block: nibbles plus the fifth-bit dword (bit l = element l).
__device__ inline int dot_q5_regs(uint4 qs, uint32_t qh, const uint32_t xv[8]) {
  uint32_t hb[8];
#pragma unroll
  for (int i = 0; i < 8; i++) hb[i] = spread4(qh >> (4 * i)) << 4;
  return dot_nib_regs(qs, hb, xv);
}
__device__ inline int dot_q5_unit(uint4 qs, uint32_t qh, const int8_t* xa) {
  uint32_t xv[8];
  act8_from_lds(xa, xv);
  return dot_q5_regs(qs, qh, xv);
}

// Q6_K sub-block: 16 bytes of low nibbles plus 8 bytes of 2-bit high pairs
// (byte i holds elements 4i..4i+3).  Returns sum(q * x) with q in 0..63; the
// caller subtracts 32 * bsum to get the reference's sum((q - 32) * x).
__device__ inline int dot_q6_regs_raw(uint4 ql, uint2 qh, const uint32_t xv[8]) {
  uint32_t hb[8];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    hb[i] = spread2x4((qh.x >> (8 * i)) & 0xFFu) << 4;
    hb[4 + i] = spread2x4((qh.y >> (8 * i)) & 0xFFu) << 4;
  }
  return dot_nib_regs(ql, hb, xv);
}
__device__ inline int dot_q6_unit_raw(uint4 ql, uint2 qh, const int8_t* xa) {
  uint32_t xv[8];
  act8_from_lds(xa, xv);
  return dot_q6_regs_raw(ql, qh, xv);
}

// Q8_0 block: 8 dwords of int8 weights against a natural-order activation.
__device__ inline int dot_q8_regs(const uint32_t w[8], const uint32_t xv[8]) {
  int acc = 0;
#pragma unroll
  for (int k = 0; k < 8; k++) acc = sdot4(w[k], xv[k], acc);
  return acc;
}
__device__ inline int dot_q8_unit(const uint32_t w[8], const int8_t* xa) {
  uint32_t xv[8];
  act8_from_lds(xa, xv);
  return dot_q8_regs(w, xv);
}

// ---------------------------------------------------------------------------
// Q8_0 dot orders of the reference builds (vec_dot_q8_0_q8_0,
// src/quant.c:242-288).  The integer products are the same; the fp32
// accumulation differs:
//   kQ8Seq     -std=c99 build: per block isum, sum += (isum * da) * db,
//              blocks in order (src/quant.c:279-285);
//   kQ8Avx2    -mavx2 -mfma build: 8 int32 lanes per block, lane k holding the
//              products of bytes 2k, 2k+1, 16+2k, 17+2k (madd of the low and
//              high 16 bytes, src/quant.c:249-264); lane accumulators
//              acc_k = (lane_k * (da * db)) + acc_k, a multiply then an add
//              (src/quant.c:271); finally 0 + acc_0 + ... + acc_7
//              (src/quant.c:274-276);
//   kQ8Avx512  a build with AVX-512 enabled: the same lanes, each updated by
//              one fused multiply-add (src/quant.c:268-269).
// The values equal QR_ORDER_SEQ / _AVX2 / _AVX512: one order names one build.
// ---------------------------------------------------------------------------
constexpr int kQ8Seq = 0;
constexpr int kQ8Avx2 = 1;
constexpr int kQ8Avx512 = 2;
// Term slots per unit: one fp32 term, or (lane orders) the 8 lane sums as
// floats plus the block's da * db.
__host__ __device__ constexpr int q8_slots(int type, int q8o) {
  return (type == QR_T_Q8_0 && q8o != kQ8Seq) ? 9 : 1;
}

// The 8 lane sums of one Q8_0 block (natural byte order in w and x): lane k
// gathers bytes {2k, 2k+1} of dword k/2 and of dword 4 + k/2 into one dword
// (v_perm) and takes one 4-wide dot.
__device__ inline void q8_lanes(const uint32_t w[8], const uint32_t xv[8], int l[8]) {
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const uint32_t sel = (k & 1) ? 0x07060302u : 0x05040100u;
    const uint32_t pw = __builtin_amdgcn_perm(w[4 + (k >> 1)], w[k >> 1], sel);
    const uint32_t px = __builtin_amdgcn_perm(xv[4 + (k >> 1)], xv[k >> 1], sel);
    l[k] = sdot4(pw, px, 0);
  }
}

// One lane accumulator of a row in a lane order: acc over the units' lane-k
// sums f[u] and scales dd[u], unit 0 first.
template <int Q8O>
__device__ inline float q8_lane_update(float f, float dd, float acc) {
  if constexpr (Q8O == kQ8Avx512) return __builtin_fmaf(f, dd, acc);
  else return f * dd + acc;  // contraction is off: a multiply, then an add
}

// A row's value in a lane order from its term slots: tp[k * ts + u] holds
// lane k's sum of unit u (k < 8) and tp[8 * ts + u] the unit's da * db.  The
// 8 accumulators advance together, then are added 0..7 into 0.0f.
template <int Q8O>
__device__ inline float q8_row_sum(const float* tp, int ts, int U) {
  float acc[8];
#pragma unroll
  for (int k = 0; k < 8; k++) acc[k] = 0.0f;
  for (int u = 0; u < U; u++) {
    const float dd = tp[8 * ts + u];
#pragma unroll
    for (int k = 0; k < 8; k++) acc[k] = q8_lane_update<Q8O>(tp[k * ts + u], dd, acc[k]);
  }
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; k++) s += acc[k];
  return s;
}

// fp32 terms, in the reference's operation order (contraction is off).
// Q4_K/Q5_K: (sc*isum - m*bsum) * bd   (src/quant.c:399)
__device__ inline float term_q45(uint32_t hdr0, uint32_t sbyte, int isum, int bsum, float bd) {
  const float d = qr_h2f(hdr0 & 0xFFFFu);
  const float dmin = qr_h2f(hdr0 >> 16);
  const float sc = (float)(sbyte & 63u) * d;
  const float m = (float)(sbyte >> 6) * dmin;
  return (sc * (float)isum - m * (float)bsum) * bd;
}
// Q6_K: sc * isum * bd, left to right (src/quant.c:433)
__device__ inline float term_q6(int scale_i8, uint32_t dh, int isum, float bd) {
  const float sc = (float)scale_i8 * qr_h2f(dh);
  return sc * (float)isum * bd;
}
// Q8_0: isum * da * db, left to right (src/quant.c:284)
__device__ inline float term_q8(uint32_t dh, int isum, float bd) {
  return (float)isum * qr_h2f(dh) * bd;
}


// ---------------------------------------------------------------------------
// Weight tiles.  A tile is R consecutive rows of one [rows][row_bytes]
// matrix: one contiguous byte range.
// ---------------------------------------------------------------------------
template <int TYPE>
struct Fmt {
  // 144- and 176-byte blocks keep every sub-block 16-byte aligned: lanes load
  // their own bytes with 128-bit global loads.  34- and 210-byte blocks do
  // not: the tile is first copied to LDS with 128-bit loads.
  static constexpr bool kDirect = (TYPE == QR_T_Q4_K || TYPE == QR_T_Q5_K);
  static constexpr bool kPerm = (TYPE == QR_T_Q4_K);
};

__host__ __device__ inline size_t align16(size_t v) { return (v + 15) & ~(size_t)15; }

// LDS bytes of a staged tile of `bytes` bytes starting anywhere: up to 15
// bytes of head, the tail rounded to 16, and one slack dword for lds_u32.
__host__ __device__ inline size_t stage_bytes(size_t bytes) { return align16(bytes + 15 + 4 + 15); }

// Copy matrix bytes [gstart, gend) into LDS; LDS byte 0 is matrix byte
// (gstart & ~15).  `total` is the matrix size: whole 16-byte chunks use
// 128-bit loads, a chunk reaching past `total` is read a dword or half-word
// at a time, so no load leaves the matrix (row sizes are even).
__device__ inline void stage_tile(const uint8_t* __restrict__ W, size_t total, size_t gstart,
                                  size_t gend, uint32_t* lds) {
  const size_t a0 = gstart & ~(size_t)15;
  const int nch = (int)((gend - a0 + 15) >> 4);
  for (int c = threadIdx.x; c < nch; c += blockDim.x) {
    const size_t off = a0 + (size_t)c * 16;
    uint4 v;
    if (off + 16 <= total) {
      v = *reinterpret_cast<const uint4*>(W + off);
    } else {
      uint32_t w[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const size_t o = off + 4 * k;
        if (o + 4 <= total) w[k] = *reinterpret_cast<const uint32_t*>(W + o);
        else if (o + 2 <= total) w[k] = *reinterpret_cast<const uint16_t*>(W + o);
        else w[k] = 0;
      }
      v = make_uint4(w[0], w[1], w[2], w[3]);
    }
    reinterpret_cast<uint4*>(lds)[c] = v;
  }
}

struct UnitSrc {
  const uint32_t* tile;  // staged tile (Q8_0 / Q6_K)
  ActLds act;            // quantized activation rows
  int nxb;               // activation blocks per row (d / 32)
};

// Terms (and int32 sums) of unit u of one row for NT activation rows
// tok0 .. tok0+NT-1.  `wrow` is the row in global memory (direct formats),
// `row_lds` its byte offset in the staged tile (staged formats).
// Q4_K / Q5_K unit u (super-block u/8, sub-block u%8) from registers: the
// block's 16-byte header, the sub-block's 16 bytes of nibbles and, for Q5_K,
// its fifth-bit dword.  Terms and int32 sums for activation rows
// tok0 .. tok0+NT-1.
template <int TYPE, int NT>
__device__ inline void direct_unit_terms(uint4 hdr, uint4 qs, uint32_t qh, int u, const ActLds& act,
                                         int nxb, int tok0, float* terms_out, int32_t* isum_out) {
  const int s = u & 7;
  const uint32_t sbyte = ((s < 4 ? hdr.y : hdr.z) >> (8 * (s & 3))) & 0xFFu;
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int a = (tok0 + t) * nxb + u;
    const int8_t* xa = act.q + (size_t)a * 32;
    int isum;
    if constexpr (TYPE == QR_T_Q4_K) isum = dot_q4_unit(qs, xa);
    else isum = dot_q5_unit(qs, qh, xa);
    terms_out[t] = term_q45(hdr.x, sbyte, isum, act.bs[a], act.bd[a]);
    isum_out[t] = isum;
  }
}

// Q8_0 unit u of a row staged in LDS, in a lane order: for each activation row
// tok0 + t, slot[t][k * ts] = lane k's sum (k < 8), slot[t][8 * ts] = da * db,
// where slot[t] = dst + t * tstep.  isum_out receives the unit's int32 sum.
template <int NT>
__device__ inline void q8_unit_lanes(int row_lds, int u, const UnitSrc& S, int tok0, float* dst,
                                     size_t tstep, int ts, int32_t* isum_out) {
  const int o = row_lds + u * QR_Q8_BYTES;
  const uint32_t* T = S.tile;
  const float da = qr_h2f(lds_u32(T, o) & 0xFFFFu);
  uint32_t w[8];
#pragma unroll
  for (int k = 0; k < 8; k++) w[k] = lds_u32(T, o + 2 + 4 * k);
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int a = (tok0 + t) * S.nxb + u;
    uint32_t xv[8];
    act8_from_lds(S.act.q + (size_t)a * 32, xv);
    int l[8];
    q8_lanes(w, xv, l);
    float* sp = dst + (size_t)t * tstep;
    int is = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      sp[(size_t)k * ts] = (float)l[k];
      is += l[k];
    }
    sp[(size_t)8 * ts] = da * S.act.bd[a];  // fp16_to_fp32(a.d) * fp16_to_fp32(b.d)
    isum_out[t] = is;
  }
}

template <int TYPE, int NT>
__device__ inline void unit_terms(const uint8_t* __restrict__ wrow, int row_lds, int u,
                                  const UnitSrc& S, int tok0, float* terms_out,
                                  int32_t* isum_out) {
  const int nxb = S.nxb;
  if constexpr (TYPE == QR_T_Q4_K || TYPE == QR_T_Q5_K) {
    const int b = u >> 3, s = u & 7;
    const uint8_t* blk = wrow + (size_t)b * (TYPE == QR_T_Q4_K ? QR_Q4K_BYTES : QR_Q5K_BYTES);
    const uint4 hdr = *reinterpret_cast<const uint4*>(blk);
    uint4 qs;
    uint32_t qh = 0;
    if constexpr (TYPE == QR_T_Q4_K) {
      qs = *reinterpret_cast<const uint4*>(blk + 16 + 16 * s);
    } else {
      qs = *reinterpret_cast<const uint4*>(blk + 48 + 16 * s);
      qh = *reinterpret_cast<const uint32_t*>(blk + 16 + 4 * s);
    }
    direct_unit_terms<TYPE, NT>(hdr, qs, qh, u, S.act, nxb, tok0, terms_out, isum_out);
  } else if constexpr (TYPE == QR_T_Q6_K) {
    const int b = u >> 3, s = u & 7;
    const int o = row_lds + b * QR_Q6K_BYTES;
    const uint32_t* T = S.tile;
    const uint4 ql = make_uint4(lds_u32(T, o + 16 * s), lds_u32(T, o + 16 * s + 4),
                                lds_u32(T, o + 16 * s + 8), lds_u32(T, o + 16 * s + 12));
    const uint2 qh = make_uint2(lds_u32(T, o + 128 + 8 * s), lds_u32(T, o + 128 + 8 * s + 4));
    const int scale = (int)(int8_t)(lds_u32(T, o + 192 + s) & 0xFFu);
    const uint32_t dh = lds_u32(T, o + 208) & 0xFFFFu;
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const int a = (tok0 + t) * nxb + u;
      const int8_t* xa = S.act.q + (size_t)a * 32;
      const int isum = dot_q6_unit_raw(ql, qh, xa) - 32 * S.act.bs[a];
      terms_out[t] = term_q6(scale, dh, isum, S.act.bd[a]);
      isum_out[t] = isum;
    }
  } else {  // Q8_0
    const int o = row_lds + u * QR_Q8_BYTES;
    const uint32_t* T = S.tile;
    const uint32_t dh = lds_u32(T, o) & 0xFFFFu;
    uint32_t w[8];
#pragma unroll
    for (int k = 0; k < 8; k++) w[k] = lds_u32(T, o + 2 + 4 * k);
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const int a = (tok0 + t) * nxb + u;
      const int isum = dot_q8_unit(w, S.act.q + (size_t)a * 32);
      terms_out[t] = term_q8(dh, isum, S.act.bd[a]);
      isum_out[t] = isum;
    }
  }
}

// Sequential sum of one row's terms from 0.0f, unit 0 first (the fp32
// accumulation of every reference dot, src/quant.c:279-285, 384-400, 422-434).
__device__ inline float row_sum(const float* tp, int U) {
  float s = 0.0f;
  for (int u = 0; u < U; u++) s += tp[u];
  return s;
}

// A row's value from its term slots: the sequential sum, or (Q8_0 lane
// orders) the lane accumulators of slots [9][ts].
template <int TYPE, int Q8O>
__device__ inline float row_value(const float* tp, int ts, int U) {
  if constexpr (q8_slots(TYPE, Q8O) == 9) return q8_row_sum<Q8O>(tp, ts, U);
  else return row_sum(tp, U);
}

// Terms of unit u of one row for NT activation rows into term slots: row
// block t at dst + t * tstep, unit u at [u] (one slot per unit) or at
// [k * ts + u] (lane orders).  isum_out receives the int32 sums.
template <int TYPE, int NT, int Q8O>
__device__ inline void unit_to_slots(const uint8_t* __restrict__ wrow, int row_lds, int u,
                                     const UnitSrc& S, int tok0, float* dst, size_t tstep, int ts,
                                     int32_t* isum_out) {
  if constexpr (q8_slots(TYPE, Q8O) == 9) {
    q8_unit_lanes<NT>(row_lds, u, S, tok0, dst + u, tstep, ts, isum_out);
  } else {
    float tv[NT];
    unit_terms<TYPE, NT>(wrow, row_lds, u, S, tok0, tv, isum_out);
#pragma unroll
    for (int t = 0; t < NT; t++) dst[(size_t)t * tstep + u] = tv[t];
  }
}

// Arguments of the GEMV kernels (qr_gemv.hip, qr_tiled.h).
struct GemvArgs {
  const uint8_t* W;      // [n][row_bytes], 16-byte aligned
  const float* X;        // [nt][xstride]
  float* Y;              // [nt][ystride]
  int n, d;
  int xstride, ystride;
  int rows_per_wg;
  int32_t* acc;          // optional [nt][n][units] int32 unit sums
  int32_t* accb;         // optional [nt][units] activation block sums
  // tiled layout (qr_tiled.h): super-blocks per row, rows per full tile,
  // tiles, bytes of a full tile -- set on the host
  int t_nb, t_rb, t_ntiles;
  size_t t_tile_bytes;
  // pair mode of the ggml GEMV (expert products of llama.cpp-layout
  // experts): workgroup row blockIdx.y = pair p multiplies expert eidx[p]'s
  // matrix (W + eidx[p] * eslice) by activation row p / xk, into Y row p;
  // eidx null: one matrix
  const int32_t* eidx;
  size_t eslice;
  int xk, E;
  // residual: Y = R + W X (one token; R may be Y itself); null: Y = W X
  const float* R;
  // normalising start-up of the tiled GEMV (qr_norm.h, one token): X is
  // the residual stream, nw the norm's weights, and workgroup 0 also stores
  // the normalised vector at nxb when given
  const float* nw;
  float* nxb;
};

}  // namespace qr
