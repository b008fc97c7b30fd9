// qr_blk.h -- the block-per-lane GEMV engine for the 16-byte aligned K-quant
// formats (Q4_K 144-byte and Q5_K 176-byte super-blocks).
//
// A wave tile is RB = 64 / nb whole rows of nb super-blocks each; lane
// l = r * nb + b holds super-block b of tile row r: its header and sub-blocks
// arrive as 16-byte loads of one contiguous 144 / 176-byte range (neighbouring
// lanes read neighbouring blocks, so a wave streams RB * row_bytes contiguous
// bytes).  The lane decodes the block header once for its 8 units, takes the
// int32 sum of each unit against the Q8_0 activation block in LDS with
// v_dot4_i32_i8, and forms the unit's fp32 term in the reference's operation
// order.  The row's terms must be added one after another from 0.0f, block 0
// first: the lanes of a row do that as a chain of nb stages, stage k adding
// block k's 8 terms onto the partial sum that lane k-1 handed over with a DPP
// wave shift -- no LDS round trip.
#pragma once

#include "qr_gemv.h"

namespace qr {

constexpr int kBlkWaves = 4;  // waves per workgroup

// Activation in LDS, per token: activation block u at byte
// (u / 8) * kActRow + (u % 8) * kActBlk, 48 bytes:
//   NIB layout (Q4_K):  [xh 16 B | xl 16 B | bd f32 | bsf f32 | c i32 | bs i32]
//   NAT layout (Q5_K):  [32 int8 in element order | bd f32 | bsf f32 | - | bs i32]
// bd = h2f(f2h(d)) of the block, bs its integer sum, bsf = (float)bs.  In the
// NIB layout each int8 value x is split as x + 128 = 16 * xh + xl with xh, xl
// in 0..15: xl is kept as an unsigned nibble, xh - 8 as a signed nibble (8 per
// dword, element order, nibble k = bits 4k..4k+3), and c = 128 * sum(xh - 8).
// Then for 4-bit weights q:  sum(q * x) = 16 * sum((q - 8) * (xh - 8))
// + sum(q * xl) + c, two 8-nibble dot products per weight dword and no
// unpacking of the weight nibbles (q - 8 is q ^ 8 as a signed nibble).
// kActRow = 8 blocks + 16 bytes, so the 8 blocks that the lanes of one row
// read at the same time fall on different LDS banks.
constexpr int kActBlk = 48;
constexpr int kActRow = 8 * kActBlk + 16;

__host__ __device__ inline size_t act_tok_bytes(int d) {
  return (size_t)((d / 32 + 7) / 8) * kActRow;
}
__device__ inline int act_off(int u) { return (u >> 3) * kActRow + (u & 7) * kActBlk; }

// DPP quad permutations (lane ^ 1, lane ^ 2) and the whole-wave shift by one
// lane (lane l receives lane l-1; lane 0 receives `fill`).
__device__ inline int dpp_xor1(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false); }
__device__ inline int dpp_xor2(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false); }
__device__ inline float dpp_xor1f(float v) {
  return __builtin_bit_cast(float, dpp_xor1(__builtin_bit_cast(int, v)));
}
__device__ inline float dpp_xor2f(float v) {
  return __builtin_bit_cast(float, dpp_xor2(__builtin_bit_cast(int, v)));
}
__device__ inline float wave_shr1f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x138, 0xF, 0xF, false));
}

// quantize_row_q8_0 (src/quant.c:143-158) of nt rows x[t * xstride ..+ d)
// into the LDS layout above, by the whole workgroup: four adjacent lanes per
// 32-element block, 8 elements each; amax and the integer sum reduce across
// the quad with DPP.  amax is a max (order-free); d = amax / 127 and 1 / d are
// correctly rounded divisions; rintf rounds ties to even like lrintf; the
// stored scale goes through the truncating fp16 routine.  PERM stores each
// 8-element group as [x0 x2 x4 x6 | x1 x3 x5 x7] (the Q4_K nibble order).
//
// act_prefetch loads a thread's first 8 elements: issued before a kernel's
// weight loads, the (small) activation read is not queued behind them.
struct ActPre {
  float v[8];
};
__device__ inline void act_load8(const float* __restrict__ x, size_t xstride, int nt, int d, int gi,
                                 float (&v)[8]) {
  const int per_tok = (d >> 5) * 4;
  if (gi < nt * per_tok) {
    const int t = gi / per_tok, g = gi - t * per_tok;
    const float4* p = reinterpret_cast<const float4*>(x + (size_t)t * xstride + (size_t)g * 8);
    const float4 u0 = p[0], u1 = p[1];
    v[0] = u0.x; v[1] = u0.y; v[2] = u0.z; v[3] = u0.w;
    v[4] = u1.x; v[5] = u1.y; v[6] = u1.z; v[7] = u1.w;
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = 0.0f;
  }
}
__device__ inline void act_prefetch(const float* __restrict__ x, size_t xstride, int nt, int d,
                                    ActPre& pre) {
  act_load8(x, xstride, nt, d, (int)threadIdx.x, pre.v);
}

// Where the fp32 values come from (a compile-time choice on purpose: a
// function that may also issue global loads makes the compiler wait for all
// vector memory operations before the values it reads -- vmcnt(0) -- which
// would include the weight DMA a caller has in flight):
//   kActGlobal  the first pass uses `pre`, later passes load from x;
//   kActLds     the activation is staged in LDS at xs, group gi's 8 floats at
//               xs + 8 gi (see stage_act_dma), and every pass reads there;
//   kActRegs    one pass, from `pre` only (the caller guarantees that one
//               pass covers the activation: nt * d / 8 <= nthr).
// tid / nthr (optional): the caller's index among the nthr threads that
// quantize (a multiple of 64, so quads never straddle waves); default the
// whole workgroup.
enum { kActGlobal = 0, kActLds = 1, kActRegs = 2 };
template <bool NIB, int SRC = kActGlobal>
__device__ inline void quantize_act_blk(const float* __restrict__ x, size_t xstride, int nt,
                                        int d, uint8_t* lds, const ActPre& pre,
                                        const float* xs = nullptr, int tid = -1, int nthr = 0) {
  const int nxb = d >> 5;
  const int per_tok = nxb * 4;
  const int total = nt * per_tok;
  const size_t tokb = act_tok_bytes(d);
  if (tid < 0) {
    tid = (int)threadIdx.x;
    nthr = (int)blockDim.x;
  }
  for (int base = 0; base < total; base += nthr) {
    const int gi = base + tid;
    const bool live = gi < total;
    const int t = live ? gi / per_tok : 0;
    const int g = live ? gi - t * per_tok : 0;
    float v[8];
    if constexpr (SRC == kActRegs) {
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = pre.v[i];
    } else if constexpr (SRC == kActLds) {
      const float4* p = reinterpret_cast<const float4*>(xs + (size_t)(live ? gi : 0) * 8);
      const float4 u0 = p[0], u1 = p[1];
      v[0] = u0.x; v[1] = u0.y; v[2] = u0.z; v[3] = u0.w;
      v[4] = u1.x; v[5] = u1.y; v[6] = u1.z; v[7] = u1.w;
    } else if (base == 0) {
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = pre.v[i];
    } else {
      act_load8(x, xstride, nt, d, gi, v);
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float av = __builtin_fabsf(v[i]);
      amax = av > amax ? av : amax;
    }
    float o = dpp_xor1f(amax);
    amax = o > amax ? o : amax;
    o = dpp_xor2f(amax);
    amax = o > amax ? o : amax;
    const float dd = amax / 127.0f;
    const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
    int q[8];
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      q[i] = (int)(int8_t)(int)__builtin_rintf(v[i] * id);
      s += q[i];
    }
    s += dpp_xor1(s);
    s += dpp_xor2(s);
    const int blk = g >> 2, part = g & 3;
    uint8_t* ab = lds + (size_t)t * tokb + act_off(blk);
    if constexpr (NIB) {
      uint32_t wh = 0, wl = 0;
      int hs = 0;  // sum of (xh - 8) over the 8 elements
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const uint32_t xb = (uint32_t)(q[i] + 128);  // 1..255
        wh |= ((xb >> 4) ^ 8u) << (4 * i);
        wl |= (xb & 15u) << (4 * i);
        hs += (int)(xb >> 4) - 8;
      }
      hs += dpp_xor1(hs);
      hs += dpp_xor2(hs);
      if (live) {
        reinterpret_cast<uint32_t*>(ab)[part] = wh;
        reinterpret_cast<uint32_t*>(ab + 16)[part] = wl;
        if (part == 0) {
          float* f = reinterpret_cast<float*>(ab + 32);
          f[0] = qr_h2f(qr_f2h(dd));
          f[1] = (float)s;
          reinterpret_cast<int*>(ab + 40)[0] = 128 * hs;
          reinterpret_cast<int*>(ab + 44)[0] = s;
        }
      }
    } else if (live) {
      *reinterpret_cast<uint2*>(ab + part * 8) =
          make_uint2(pack4(q[0], q[1], q[2], q[3]), pack4(q[4], q[5], q[6], q[7]));
      if (part == 0) {
        float* f = reinterpret_cast<float*>(ab + 32);
        f[0] = qr_h2f(qr_f2h(dd));
        f[1] = (float)s;
        reinterpret_cast<int*>(ab + 44)[0] = s;
      }
    }
    if constexpr (SRC == kActRegs) break;
  }
}

// ---------------------------------------------------------------------------
// Weight tiles through LDS.  A wave moves a tile's bytes from HBM into its LDS
// slot with global_load_lds_dwordx4 (one instruction = 64 lanes x 16 bytes =
// 1 KiB contiguous: fully coalesced, and no VGPRs held while in flight); each
// lane then reads its own super-block back from the slot (a 144 / 176-byte
// lane stride touches distinct banks within every 16 lanes).
//
// The DMA is issued from inline asm and waited for explicitly with the wave's
// vmcnt: the compiler, which cannot tell the slots from the activation in
// LDS, would otherwise wait for every DMA in flight before any LDS access.
// Vector-memory loads complete in issue order, so "at most N operations in
// flight" after a tile's DMA plus N later DMA operations means the tile has
// landed; later stores only make such a wait stricter.  Every DMA instruction
// is issued with all lanes active (lanes past the valid bytes reload the
// tile's first 16 bytes into slot bytes nobody reads), so the count of DMA
// operations per tile is exactly NCH.
// ---------------------------------------------------------------------------

// One global_load_lds_dwordx4: each lane's 16 bytes at src land at LDS byte
// lds + 16 * lane (lds wave-uniform).  M0 carries the LDS address; the
// compiler does not track M0 across inline asm, so the asm saves and restores
// it around the instruction.
__device__ inline void lds_dma16(const void* src, uint32_t lds) {
  int save;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "v"(src), "s"(lds)
      : "memory");
}
// The same with the non-temporal hint, for bytes read once (weight streams):
// they are the first lines L2 gives up, so data that every workgroup re-reads
// (the activation) stays cached across launches.
__device__ inline void lds_dma16_nt(const void* src, uint32_t lds) {
  int save;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dwordx4 %1, off nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "v"(src), "s"(lds)
      : "memory");
}
// The LDS byte address of a pointer into LDS, wave-uniform.
__device__ inline uint32_t lds_u32addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)p);
}

template <int NCH>
__device__ inline void tile_dma(const uint8_t* g, uint8_t* s, int valid, int lane) {
  const uint32_t sbase = lds_u32addr(s);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slot's earlier reads are done
#pragma unroll
  for (int k = 0; k < NCH; k++) {
    const int off = k * 1024 + lane * 16;
    lds_dma16_nt(g + (off < valid ? off : 0), sbase + (uint32_t)(k * 1024));
  }
}

// DMA `nbytes` from g into LDS s in whole 1 KiB instructions; lanes past the
// end reload g's first 16 bytes into bytes nobody reads (s must hold the
// rounded-up size).  Returns the number of instructions issued.
// NT: with the non-temporal hint (bytes read once).
template <bool NT = false>
__device__ inline int dma_bytes(const uint8_t* g, uint8_t* s, int nbytes, int lane) {
  const uint32_t sbase = lds_u32addr(s);
  const int n = (nbytes + 1023) >> 10;
  for (int k = 0; k < n; k++) {
    const int off = k * 1024 + lane * 16;
    if constexpr (NT) lds_dma16_nt(g + (off < nbytes ? off : 0), sbase + (uint32_t)(k * 1024));
    else lds_dma16(g + (off < nbytes ? off : 0), sbase + (uint32_t)(k * 1024));
  }
  return n;
}

__host__ __device__ inline size_t kib_round(size_t b) { return (b + 1023) & ~(size_t)1023; }

// LDS staging of the activation: whole passes of 256 groups of 8 floats.
__host__ __device__ inline size_t blk_xs_bytes(int d, int nt) {
  return (size_t)((nt * (d >> 3) + 255) >> 8) * 8192;
}
constexpr size_t kXsMax = 16 * 1024;

// Stage the fp32 activation of nt tokens into LDS xs by DMA, laid out for
// quantize_act_blk: 8-element group gi = t * (d / 8) + g at xs + 32 gi bytes.
// The nw waves that quantize (64 nw threads, group gi = pass * 64 nw +
// thread) each stage the 2 KiB of groups their own threads read in each pass,
// `wave` being the caller's index among them: 2 DMA instructions per pass,
// none that starts past the last group (d a multiple of 256 keeps every
// instruction within the groups); lanes past the last group reload group 0.
// Returns the number of DMA instructions issued.  Call with all 64 lanes.
__device__ inline int stage_act_dma(const float* __restrict__ x, size_t xstride, int nt, int d,
                                    uint8_t* xs, int wave, int lane, int nw = 4) {
  const int per_tok = d >> 3;
  const int total = nt * per_tok;
  const int pt = 64 * nw;
  const int passes = (total + pt - 1) / pt;
  const uint32_t xbase = lds_u32addr(xs);
  int issued = 0;
  for (int p = 0; p < passes; p++) {
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const int first = p * pt + wave * 64 + k * 32;  // first group of this instruction
      if (first >= total) continue;  // wave-uniform
      int gi = first + (lane >> 1);
      gi = gi < total ? gi : 0;
      const int t = gi / per_tok, g = gi - t * per_tok;
      lds_dma16(x + (size_t)t * xstride + (size_t)g * 8 + 4 * (lane & 1),
                xbase + (uint32_t)(first * 32));
      issued++;
    }
  }
  return issued;
}

// Wait until at most N of the wave's vector memory operations are in flight.
template <int N>
__device__ inline void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One activation block read back from LDS.
struct ActView {
  uint32_t q[8];  // NAT: 32 int8;  NIB: xh[0..3] = q[0..3], xl[0..3] = q[4..7]
  float bd, bsf;
  int c, bs;
};
__device__ inline ActView act_read(const uint8_t* ab) {
  const uint4 a = *reinterpret_cast<const uint4*>(ab);
  const uint4 b = *reinterpret_cast<const uint4*>(ab + 16);
  const uint4 c = *reinterpret_cast<const uint4*>(ab + 32);
  ActView v;
  v.q[0] = a.x; v.q[1] = a.y; v.q[2] = a.z; v.q[3] = a.w;
  v.q[4] = b.x; v.q[5] = b.y; v.q[6] = b.z; v.q[7] = b.w;
  v.bd = __builtin_bit_cast(float, c.x);
  v.bsf = __builtin_bit_cast(float, c.y);
  v.c = (int)c.z;
  v.bs = (int)c.w;
  return v;
}

// sum(q * x) of one 32-element unit of 4-bit weights (4 dwords of 8 nibbles,
// element order) against a NIB-layout activation block.
__device__ inline int dot_q4_nib(uint4 qs, const ActView& a) {
  int hi = __builtin_amdgcn_sdot8((int)(qs.x ^ 0x88888888u), (int)a.q[0], 0, false);
  hi = __builtin_amdgcn_sdot8((int)(qs.y ^ 0x88888888u), (int)a.q[1], hi, false);
  hi = __builtin_amdgcn_sdot8((int)(qs.z ^ 0x88888888u), (int)a.q[2], hi, false);
  hi = __builtin_amdgcn_sdot8((int)(qs.w ^ 0x88888888u), (int)a.q[3], hi, false);
  uint32_t lo = __builtin_amdgcn_udot8(qs.x, a.q[4], (uint32_t)a.c, false);
  lo = __builtin_amdgcn_udot8(qs.y, a.q[5], lo, false);
  lo = __builtin_amdgcn_udot8(qs.z, a.q[6], lo, false);
  lo = __builtin_amdgcn_udot8(qs.w, a.q[7], lo, false);
  return (int)((uint32_t)hi << 4) + (int)lo;
}

template <int TYPE>
struct BlkFmt {
  static constexpr int kBytes = TYPE == QR_T_Q4_K ? QR_Q4K_BYTES : QR_Q5K_BYTES;
  static constexpr int kChunks = kBytes / 16;           // 9 or 11
  static constexpr int kQs = TYPE == QR_T_Q4_K ? 1 : 3;  // first chunk of the nibbles
  static constexpr bool kNib = TYPE == QR_T_Q4_K;        // activation layout
};

// The 8 unit terms (and int32 sums) of one super-block held in chunks c[]
// against NT activation rows; `act` is the LDS activation, `b` the block's
// index in its row (units 8b .. 8b+7).  Term of unit s, as src/quant.c:384-400:
// (sc * (float)isum - m * (float)bsum) * bd with sc = (scale & 63) * d and
// m = (scale >> 6) * dmin, every operation rounded once.
template <int TYPE, int NT>
__device__ inline void blk_terms(const uint4* c, int b, const uint8_t* act, size_t tokb,
                                 float (&terms)[NT][8], int32_t (&isums)[NT][8]) {
  const uint4 hdr = c[0];
  const float dd = qr_h2f(hdr.x & 0xFFFFu);
  const float dm = qr_h2f(hdr.x >> 16);
  const uint32_t s6[2] = {hdr.y & 0x3F3F3F3Fu, hdr.z & 0x3F3F3F3Fu};
  const uint32_t m2[2] = {(hdr.y >> 6) & 0x03030303u, (hdr.z >> 6) & 0x03030303u};
#pragma unroll
  for (int s = 0; s < 8; s++) {
    const float sc = (float)((s6[s >> 2] >> (8 * (s & 3))) & 0xFFu) * dd;
    const float m = (float)((m2[s >> 2] >> (8 * (s & 3))) & 0xFFu) * dm;
    const uint4 qs = c[BlkFmt<TYPE>::kQs + s];
    uint32_t qh = 0;
    if constexpr (TYPE == QR_T_Q5_K) {
      const uint4 h = c[1 + (s >> 2)];
      qh = (s & 3) == 0 ? h.x : (s & 3) == 1 ? h.y : (s & 3) == 2 ? h.z : h.w;
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const ActView a = act_read(act + (size_t)t * tokb + act_off(8 * b + s));
      int isum;
      if constexpr (TYPE == QR_T_Q4_K) isum = dot_q4_nib(qs, a);
      else isum = dot_q5_regs(qs, qh, a.q);
      terms[t][s] = (sc * (float)isum - m * a.bsf) * a.bd;
      isums[t][s] = isum;
    }
  }
}

// Sequential row sums: lanes b = 0 .. nb-1 of each row hold the row's terms
// block by block; returns, in the lane holding block nb-1, the sum from 0.0f
// over block 0's 8 terms, then block 1's, ... (other lanes: unspecified).
// Stage k adds every lane's 8 terms onto the stage k-1 value of the lane
// before it (a DPP wave shift); by induction lane k holds the exact prefix at
// stage k, so no lane needs a select and the critical path is the nb*8 adds.
// Every lane of the wave must be active.
template <int NT>
__device__ inline void blk_chain(const float (&terms)[NT][8], int b, int nb, float (&out)[NT]) {
  (void)b;
#pragma unroll
  for (int t = 0; t < NT; t++) {
    float v = 0.0f;
#pragma unroll
    for (int s = 0; s < 8; s++) v += terms[t][s];
    out[t] = v;
  }
  for (int k = 1; k < nb; k++) {
#pragma unroll
    for (int t = 0; t < NT; t++) {
      float v = wave_shr1f(out[t]);
#pragma unroll
      for (int s = 0; s < 8; s++) v += terms[t][s];
      out[t] = v;
    }
  }
}

}  // namespace qr
