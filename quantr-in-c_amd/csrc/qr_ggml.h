// qr_ggml.h -- llama.cpp / ggml K-quant matrices (block_q4_K 144 B, block_q5_K
// 176 B, block_q6_K 210 B; ggml-common.h) against Q8_K activations, in ggml's
// CPU reference arithmetic (ggml-quants.c: quantize_row_q8_K_ref and the
// generic ggml_vec_dot_q{4,5,6}_K_q8_K).  The reference (bharqav/quantr-in-c)
// has its own K-quant layouts; these serve real llama.cpp checkpoints.
//
// The dot of a row with an activation, per 256-element super-block:
//   aux32[l] (l = 0..7) = sum over the block's elements e with e % 8 == l of
//                         scale(e) * q8[e] * a[e]      (exact int32)
//   sumi = sum_j bsums[j] * min[j / 2]                 (Q4_K / Q5_K)
//   d = h2f(x.d) * y.d;      sums[l] += d * (float)aux32[l]
//   dmin = h2f(x.dmin) * y.d; sumf -= dmin * (float)sumi
// and after the last block sumf += sums[0], ..., sums[7].
//
// Layout of the work: a wave tile is RB = 64 / nb rows of nb super-blocks,
// lane = super-block (as qr_blk.h), the tile moved into the wave's LDS slot
// by DMA.  The activation is quantized to Q8_K inside the kernel into LDS,
// its int8 values transposed so that one dword holds, for lane position l of
// a 32-element group, the elements l, l + 8, l + 16, l + 24: one v_dot4 of it
// with the weights transposed the same way is that group's part of aux32[l].
// The nine running sums of a row (sums[0..7], sumf) pass from block to block
// along the row's lanes with DPP shifts, one stage per block, in block order.
#pragma once

#include "qr_blk.h"
#include "qr_ggml_elem.h"
#include "qr_tiled.h"

namespace qr {

template <int T>
struct GgmlFmt {
  static constexpr int kBytes = T == kGgmlQ4 ? 144 : T == kGgmlQ5 ? 176 : 210;
  static constexpr int kDma = (64 * kBytes + 1023) / 1024;  // DMA instructions per 64-block tile
};

// Q8_K activation of one super-block in LDS: 64 transposed dwords (group m,
// lane position l at dword 8 m + l: bytes = elements 32 m + l, + 8, + 16,
// + 24), then d (fp32), then the 16 bsums as int32.
constexpr int kQ8kBlk = 336;
__host__ __device__ inline size_t q8k_tok_bytes(int d) { return (size_t)(d >> 8) * kQ8kBlk; }

// quantize_row_q8_K_ref (ggml-quants.c) of nt rows of d values into the LDS
// layout above.  One wave per (token, block): lane l takes elements l + 64 k.
// The scale comes from the element of largest magnitude, the first one on
// ties (the reference scans with a strict '>'); iscale = -127 / max; each
// q = min(127, round-half-even(iscale * x)); d = 1 / iscale.
__device__ inline void quantize_q8k_lds(const float* __restrict__ x, size_t xstride, int nt, int d,
                                        uint8_t* act, int wave, int nwaves, int lane) {
  const int nb = d >> 8;
  const size_t tokb = q8k_tok_bytes(d);
  for (int p = wave; p < nt * nb; p += nwaves) {
    const int t = p / nb, b = p - t * nb;
    const float* xb = x + (size_t)t * xstride + (size_t)b * 256;
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) v[k] = xb[lane + 64 * k];
    float best = 0.0f, vmax = 0.0f;
    int bi = 1 << 30;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const float ax = __builtin_fabsf(v[k]);
      if (ax > best) {
        best = ax;
        vmax = v[k];
        bi = lane + 64 * k;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ob = __shfl_xor(best, o);
      const float ov = __shfl_xor(vmax, o);
      const int oi = __shfl_xor(bi, o);
      if (ob > best || (ob == best && oi < bi)) {
        best = ob;
        vmax = ov;
        bi = oi;
      }
    }
    uint8_t* blk = act + (size_t)t * tokb + (size_t)b * kQ8kBlk;
    int q[4];
    float dd;
    if (best == 0.0f) {  // an all-zero block (or only NaNs): d = 0, zero quants
#pragma unroll
      for (int k = 0; k < 4; k++) q[k] = 0;
      dd = 0.0f;
    } else {
      const float iscale = -127.f / vmax;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int r = (int)__builtin_rintf(iscale * v[k]);
        q[k] = r < 127 ? r : 127;
      }
      dd = 1.0f / iscale;
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int e = lane + 64 * k;
      const int m = e >> 5, l = e & 7, tb = (e & 31) >> 3;
      blk[(m * 8 + l) * 4 + tb] = (uint8_t)(int8_t)q[k];
      // bsum of group 4 k + lane / 16: the 16 lanes of the segment
      int s = q[k];
      s += __shfl_xor(s, 8);
      s += __shfl_xor(s, 4);
      s += __shfl_xor(s, 2);
      s += __shfl_xor(s, 1);
      if ((lane & 15) == 0) reinterpret_cast<int*>(blk + 260)[4 * k + (lane >> 4)] = s;
    }
    if (lane == 0) *reinterpret_cast<float*>(blk + 256) = dd;
  }
}

// The same quantization from registers: thread tid of the workgroup holds the
// 8 values of group tid + 256 k in v[2 k], v[2 k + 1] (elements 8 (tid + 256 k)
// onward), so a 256-element block is the 32 groups of one half-wave.  d is a
// multiple of 256, so a half-wave's groups are all inside the activation or
// all past it.  Every thread of the workgroup calls it.
template <int G>
__device__ inline void quantize_q8k_regs(const float4 (&v)[2 * G], int d, uint8_t* act, int tid) {
  const int ngr = d >> 3;
#pragma unroll
  for (int k = 0; k < G; k++) {
    const int gi = tid + 256 * k;
    const bool live = gi < ngr;
    float x[8] = {v[2 * k].x, v[2 * k].y, v[2 * k].z, v[2 * k].w,
                  v[2 * k + 1].x, v[2 * k + 1].y, v[2 * k + 1].z, v[2 * k + 1].w};
    const int tq = gi & 31;  // the group's place in its block
    float best = 0.0f, vmax = 0.0f;
    int bi = 1 << 30;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float ax = __builtin_fabsf(x[i]);
      if (ax > best) {
        best = ax;
        vmax = x[i];
        bi = 8 * tq + i;
      }
    }
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) {
      const float ob = __shfl_xor(best, o);
      const float ov = __shfl_xor(vmax, o);
      const int oi = __shfl_xor(bi, o);
      if (ob > best || (ob == best && oi < bi)) {
        best = ob;
        vmax = ov;
        bi = oi;
      }
    }
    int q[8];
    float dd;
    if (best == 0.0f) {  // an all-zero block (or only NaNs): d = 0, zero quants
#pragma unroll
      for (int i = 0; i < 8; i++) q[i] = 0;
      dd = 0.0f;
    } else {
      const float iscale = -127.f / vmax;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const int r = (int)__builtin_rintf(iscale * x[i]);
        q[i] = r < 127 ? r : 127;
      }
      dd = 1.0f / iscale;
    }
    // bsum of the 16 elements of groups tq and tq ^ 1
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) s += q[i];
    s += __shfl_xor(s, 1);
    if (live) {
      uint8_t* blk = act + (size_t)(gi >> 5) * kQ8kBlk;
      const int m = tq >> 2, tb = tq & 3;  // element 8 tq + i: dword 8 m + i, byte tb
#pragma unroll
      for (int i = 0; i < 8; i++) blk[(m * 8 + i) * 4 + tb] = (uint8_t)(int8_t)q[i];
      if ((tq & 1) == 0) reinterpret_cast<int*>(blk + 260)[tq >> 1] = s;
      if (tq == 0) *reinterpret_cast<float*>(blk + 256) = dd;
    }
  }
}

// Dword i of the lane's block in LDS (its 144 / 176 / 210 bytes at `o`;
// 210-byte blocks of odd lanes start 2 bytes past a dword).
template <int T>
__device__ inline uint32_t gblk_u32(const uint32_t* lds, int o, int i) {
  if constexpr (T == kGgmlQ6) return lds_u32(lds, o + 4 * i);
  else return lds[(o >> 2) + i];
}

// Transpose of 8 dwords D (32 bytes): o[l] holds bytes l, 8 + l, 16 + l,
// 24 + l -- byte (l & 3) of D[l >> 2], D[2 + (l >> 2)], D[4 + ...], D[6 + ...].
// Byte selects (v_perm: selector bytes 0-3 pick the second operand's bytes,
// 4-7 the first's), two per result: first the byte pairs of D[h], D[2 + h]
// and of D[4 + h], D[6 + h], then the pairs side by side.
__device__ inline void gtr8(const uint32_t (&D)[8], uint32_t (&o)[8]) {
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const uint32_t p01 = __builtin_amdgcn_perm(D[2 + h], D[h], 0x05010400u);
    const uint32_t p23 = __builtin_amdgcn_perm(D[2 + h], D[h], 0x07030602u);
    const uint32_t q01 = __builtin_amdgcn_perm(D[6 + h], D[4 + h], 0x05010400u);
    const uint32_t q23 = __builtin_amdgcn_perm(D[6 + h], D[4 + h], 0x07030602u);
    o[4 * h + 0] = __builtin_amdgcn_perm(q01, p01, 0x05040100u);
    o[4 * h + 1] = __builtin_amdgcn_perm(q01, p01, 0x07060302u);
    o[4 * h + 2] = __builtin_amdgcn_perm(q23, p23, 0x05040100u);
    o[4 * h + 3] = __builtin_amdgcn_perm(q23, p23, 0x07060302u);
  }
}

// a - 32 for four bytes a in 0..63, as signed bytes (no borrow across bytes).
__device__ inline uint32_t minus32(uint32_t a) {
  return ((a | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
}

// The integer parts of the lane's block against NT activation blocks (act at
// the block's position of token 0; tokens tokb apart): aux[t][8], sumi[t].
template <int T, int NT>
__device__ inline void ggml_block_ints(const uint32_t* lds, int o, const uint8_t* act, size_t tokb,
                                       int32_t (&aux)[NT][8], int32_t (&sumi)[NT], float& dw,
                                       float& dmw) {
#pragma unroll
  for (int t = 0; t < NT; t++) {
    sumi[t] = 0;
#pragma unroll
    for (int l = 0; l < 8; l++) aux[t][l] = 0;
  }
  if constexpr (T == kGgmlQ4 || T == kGgmlQ5) {
    const uint32_t h0 = gblk_u32<T>(lds, o, 0);
    dw = ggml_h2f(h0);
    dmw = ggml_h2f(h0 >> 16);
    uint32_t s12[3];
#pragma unroll
    for (int i = 0; i < 3; i++) s12[i] = gblk_u32<T>(lds, o, 1 + i);
    auto sb = [&](int i) { return (int)((s12[i >> 2] >> (8 * (i & 3))) & 0xFFu); };
    int sc[8], mn[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      if (j < 4) {
        sc[j] = sb(j) & 63;
        mn[j] = sb(j + 4) & 63;
      } else {
        sc[j] = (sb(j + 4) & 0xF) | ((sb(j - 4) >> 6) << 4);
        mn[j] = (sb(j + 4) >> 4) | ((sb(j) >> 6) << 4);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const int* bs = reinterpret_cast<const int*>(act + (size_t)t * tokb + 260);
      int s = 0;
      // |bs[2 j] + bs[2 j + 1]| < 2^12, mn < 64: 24-bit products
#pragma unroll
      for (int j = 0; j < 8; j++) s += __mul24(bs[2 * j] + bs[2 * j + 1], mn[j]);
      sumi[t] = s;
    }
    uint32_t HT[8];
    if constexpr (T == kGgmlQ5) {
      uint32_t H[8];
#pragma unroll
      for (int i = 0; i < 8; i++) H[i] = gblk_u32<T>(lds, o, 4 + i);
      gtr8(H, HT);
    }
    constexpr int QS = T == kGgmlQ4 ? 4 : 12;  // dword of qs[0]
    // one token: the four groups unrolled together; more tokens: one group
    // after the other (unrolled, their values would hold too many registers)
    constexpr int GU = NT == 1 ? 4 : 1;
#pragma unroll GU
    for (int g = 0; g < 4; g++) {  // 64-element groups: sub-blocks 2 g (low), 2 g + 1 (high)
      uint32_t D[8], WT[8];
#pragma unroll
      for (int i = 0; i < 8; i++) D[i] = gblk_u32<T>(lds, o, QS + 8 * g + i);
      gtr8(D, WT);
#pragma unroll
      for (int l = 0; l < 8; l++) {
        const uint32_t w = WT[l];
        uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
        if constexpr (T == kGgmlQ5) {
          const uint32_t h = HT[l];
          lo |= ((h >> (2 * g)) & 0x01010101u) << 4;
          hi |= ((h >> (2 * g + 1)) & 0x01010101u) << 4;
        }
#pragma unroll
        for (int t = 0; t < NT; t++) {
          const uint32_t* xt = reinterpret_cast<const uint32_t*>(act + (size_t)t * tokb);
          const int s0 = __builtin_amdgcn_sdot4((int)lo, (int)xt[(2 * g) * 8 + l], 0, false);
          const int s1 = __builtin_amdgcn_sdot4((int)hi, (int)xt[(2 * g + 1) * 8 + l], 0, false);
          // 24-bit products (full-rate): |s| < 2^13, sc < 64
          aux[t][l] += __mul24(sc[2 * g], s0) + __mul24(sc[2 * g + 1], s1);
        }
      }
    }
  } else {  // Q6_K: ql[128] qh[64] scales[16] d
    dw = ggml_h2f(gblk_u32<T>(lds, o, 52));  // bytes 208..209
    dmw = 0.0f;
    int sc[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t w = gblk_u32<T>(lds, o, 48 + i);
#pragma unroll
      for (int k = 0; k < 4; k++) sc[4 * i + k] = (int)(int8_t)((w >> (8 * k)) & 0xFFu);
    }
    // the halves likewise; a half's scales are picked without indexing
    constexpr int HU = NT == 1 ? 2 : 1;
#pragma unroll HU
    for (int n = 0; n < 2; n++) {  // 128-element halves
      int scn[8];
#pragma unroll
      for (int i = 0; i < 8; i++) scn[i] = n ? sc[8 + i] : sc[i];
      uint32_t L0[8], L1[8], H[8], T0[8], T1[8], TH[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        L0[i] = gblk_u32<T>(lds, o, 16 * n + i);
        L1[i] = gblk_u32<T>(lds, o, 16 * n + 8 + i);
        H[i] = gblk_u32<T>(lds, o, 32 + 8 * n + i);
      }
      gtr8(L0, T0);
      gtr8(L1, T1);
      gtr8(H, TH);
#pragma unroll
      for (int l = 0; l < 8; l++) {
        const uint32_t t0 = T0[l], t1 = T1[l], th = TH[l];
        uint32_t A[4];
        A[0] = minus32((t0 & 0x0F0F0F0Fu) | ((th & 0x03030303u) << 4));
        A[1] = minus32((t1 & 0x0F0F0F0Fu) | (((th >> 2) & 0x03030303u) << 4));
        A[2] = minus32(((t0 >> 4) & 0x0F0F0F0Fu) | (((th >> 4) & 0x03030303u) << 4));
        A[3] = minus32(((t1 >> 4) & 0x0F0F0F0Fu) | (((th >> 6) & 0x03030303u) << 4));
#pragma unroll
        for (int s = 0; s < 4; s++) {  // group m = 4 n + s: sub-blocks 2 m, 2 m + 1
          const int m = 4 * n + s;
#pragma unroll
          for (int t = 0; t < NT; t++) {
            const uint32_t* xt = reinterpret_cast<const uint32_t*>(act + (size_t)t * tokb);
            const int xv = (int)xt[m * 8 + l];
            const int s0 = __builtin_amdgcn_sdot4((int)(A[s] & 0x0000FFFFu), xv, 0, false);
            const int s1 = __builtin_amdgcn_sdot4((int)(A[s] & 0xFFFF0000u), xv, 0, false);
            aux[t][l] += __mul24(scn[2 * s], s0) + __mul24(scn[2 * s + 1], s1);  // |s| < 2^14
          }
        }
      }
    }
  }
}

}  // namespace qr

namespace qr {

// The GEMV: persistent waves, one tile in flight per wave, NT tokens.  The
// start-up, three forms (XM):
//   kXmRegs (one token, d <= 256 G, Q4_K / Q5_K): one asm block per thread
//            loads its G groups of 8 activation values and issues the wave's
//            first tile DMA behind them, then waits for the values only; the
//            workgroup quantizes from registers while the tiles land, and
//            the workgroup needs no LDS for the fp32 activation.
//   kXmLds   (activations up to kXsMax): the fp32 activation is first moved
//            into LDS by DMA, then each wave's first tile DMA is issued, and
//            the quantizer waits only for the activation (the wave's
//            operations complete in issue order).
//   kXmLate  (larger activations): it is read and quantized before the first
//            tile is requested.
enum { kXmRegs = 0, kXmLds = 1, kXmLate = 2 };

// Q4_K with the register start-up fits four workgroups to a CU by LDS; at
// most 128 registers a lane keep four waves on each SIMD.
template <int T, int NT, int XM, int G = 1>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(T == kGgmlQ4 && XM == kXmRegs ? 4 : 1)))
void k_gemv_ggml(GemvArgs g) {
  constexpr bool XS = XM == kXmLds;
  extern __shared__ __align__(16) uint8_t smem[];
  if (g.eidx) {  // pair mode: this workgroup row's expert, activation row and output row
    const int p = blockIdx.y;
    const int e = g.eidx[p];
    if (e < 0 || e >= g.E) return;  // uniform, before any barrier
    g.W += (size_t)e * g.eslice;
    g.X += (size_t)(p / g.xk) * g.xstride;
    g.Y += (size_t)p * g.ystride;
  }
  constexpr int BB = GgmlFmt<T>::kBytes, NDMA = GgmlFmt<T>::kDma;
  constexpr size_t SB = (size_t)NDMA * 1024;
  const int nb = g.d >> 8, RB = 64 / nb;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int rl = lane / nb, b = lane - rl * nb;
  const bool lane_on = rl < RB;
  const size_t rb = (size_t)nb * BB;
  const size_t tokb = q8k_tok_bytes(g.d);
  const int ntiles = (g.n + RB - 1) / RB;
  const int tstep = gridDim.x * 4;
  int tile = blockIdx.x * 4 + wave;
  const size_t xsb = XS ? blk_xs_bytes(g.d, NT) : 0;
  float* xs = reinterpret_cast<float*>(smem);
  uint8_t* act = smem + xsb;
  uint8_t* slot = act + align16((size_t)NT * tokb) + (size_t)wave * SB;
  const uint32_t* slot32 = reinterpret_cast<const uint32_t*>(slot);
  auto dma = [&](int t) {
    if (t >= ntiles) return;
    const int rows = min(RB, g.n - t * RB);
    tile_dma<NDMA>(g.W + (size_t)t * RB * rb, slot, rows * (int)rb, lane);
  };
  if constexpr (XM == kXmRegs) {
    static_assert(NT == 1 && (T == kGgmlQ4 || T == kGgmlQ5), "register start-up");
    const int tid = threadIdx.x;
    const float* xp[G];
#pragma unroll
    for (int k = 0; k < G; k++) {
      const int gi = tid + 256 * k;
      xp[k] = g.X + 8 * (size_t)(gi < (g.d >> 3) ? gi : 0);
    }
    float4 v[2 * G];
    const bool has = tile < ntiles;
    if (has) {
      const int rows = min(RB, g.n - tile * RB);
      const int valid = rows * (int)rb;
      const uint8_t* tb = g.W + (size_t)tile * RB * rb;
      const uint8_t* src[NDMA];
#pragma unroll
      for (int k = 0; k < NDMA; k++) {
        const int off = k * 1024 + lane * 16;
        src[k] = tb + (off < valid ? off : 0);
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      tiled_pro_asm<NDMA, G>(xp, src, lds_u32addr(slot), v);
    } else {
      tiled_x_asm<G>(xp, v);
    }
    quantize_q8k_regs<G>(v, g.d, act, tid);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    if (!has) return;  // no barriers below
  } else if constexpr (XS) {
    stage_act_dma(g.X, (size_t)g.xstride, NT, g.d, smem, wave, lane);
    const bool has = tile < ntiles;
    dma(tile);
    if (has) wait_vmcnt<NDMA>();  // this wave's share of the activation has landed
    else wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();  // ... and every wave's
    quantize_q8k_lds(xs, (size_t)g.d, NT, g.d, act, wave, 4, lane);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    if (!has) return;  // no barriers below
  } else {
    // the activation first (every wave quantizes its share), then the stream
    quantize_q8k_lds(g.X, (size_t)g.xstride, NT, g.d, act, wave, 4, lane);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    if (tile >= ntiles) return;  // no barriers below
    dma(tile);
  }
  const uint8_t* actb = act + (size_t)b * kQ8kBlk;
  for (;;) {
    wait_vmcnt<0>();
    const int cur = tile;
    int32_t aux[NT][8], sumi[NT];
    float dw, dmw;
    ggml_block_ints<T, NT>(slot32, lane * BB, actb, tokb, aux, sumi, dw, dmw);
    tile += tstep;
    dma(tile);  // waits for the slot's reads, then refills it
    float S[NT][8], F[NT], tv[NT][8], u[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const float yd = *reinterpret_cast<const float*>(actb + (size_t)t * tokb + 256);
      const float d = dw * yd;
#pragma unroll
      for (int l = 0; l < 8; l++) tv[t][l] = d * (float)aux[t][l];
      u[t] = 0.0f;
      if constexpr (T != kGgmlQ6) u[t] = (dmw * yd) * (float)sumi[t];
      // stage 0 (block 0 of a row): from 0.0f, as the reference's sums start
#pragma unroll
      for (int l = 0; l < 8; l++) S[t][l] = 0.0f + tv[t][l];
      F[t] = 0.0f;
      if constexpr (T != kGgmlQ6) F[t] = F[t] - u[t];
    }
    // stage k: lane k of a row adds its block onto lane k - 1's running sums;
    // by induction lane k holds the exact prefix over blocks 0 .. k
    for (int k = 1; k < nb; k++) {
#pragma unroll
      for (int t = 0; t < NT; t++) {
#pragma unroll
        for (int l = 0; l < 8; l++) S[t][l] = wave_shr1f(S[t][l]) + tv[t][l];
        F[t] = wave_shr1f(F[t]);
        if constexpr (T != kGgmlQ6) F[t] = F[t] - u[t];
      }
    }
    const int row = cur * RB + rl;
    if (lane_on && row < g.n && b == nb - 1) {
#pragma unroll
      for (int t = 0; t < NT; t++) {
        float y = F[t];
#pragma unroll
        for (int l = 0; l < 8; l++) y += S[t][l];
        g.Y[(size_t)t * g.ystride + row] = g.R ? g.R[row] + y : y;
      }
    }
    if (tile >= ntiles) break;
  }
}

// quantize_row_q8_K into ggml's block_q8_K (292 bytes: f32 d, i8 qs[256],
// i16 bsums[16]); one wave per block.
__global__ __launch_bounds__(256) void k_quantize_q8k(const float* __restrict__ x,
                                                      uint8_t* __restrict__ y, long nblocks) {
  __shared__ __align__(16) uint8_t buf[4][kQ8kBlk];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const long blk = (long)blockIdx.x * 4 + wave;
  if (blk >= nblocks) return;  // whole waves; no barriers
  quantize_q8k_lds(x + blk * 256, 256, 1, 256, buf[wave], 0, 1, lane);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  uint8_t* out = y + blk * 292;
  const uint8_t* b = buf[wave];
#pragma unroll
  for (int k = 0; k < 4; k++) {  // element e = lane + 64 k back from the transposed layout
    const int e = lane + 64 * k;
    out[4 + e] = b[((e >> 5) * 8 + (e & 7)) * 4 + ((e & 31) >> 3)];
  }
  if (lane < 16) {
    const int s = reinterpret_cast<const int*>(b + 260)[lane];
    out[260 + 2 * lane] = (uint8_t)(s & 0xFF);
    out[261 + 2 * lane] = (uint8_t)((s >> 8) & 0xFF);
  }
  if (lane == 0) {
    const uint32_t dbits = __builtin_bit_cast(uint32_t, *reinterpret_cast<const float*>(b + 256));
    for (int i = 0; i < 4; i++) out[i] = (uint8_t)(dbits >> (8 * i));
  }
}

__global__ __launch_bounds__(256) void k_ggml_dequant_rows(const uint8_t* __restrict__ src,
                                                           int type, size_t row_bytes, int nrows,
                                                           int n, float* __restrict__ out) {
  const long total = (long)nrows * n;
  for (long gi = (long)blockIdx.x * blockDim.x + threadIdx.x; gi < total;
       gi += (long)gridDim.x * blockDim.x) {
    const int r = (int)(gi / n), e = (int)(gi - (long)r * n);
    out[gi] = ggml_deq_elem(src + (size_t)r * row_bytes, type, e);
  }
}

}  // namespace qr
