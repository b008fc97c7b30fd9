// qr_stream.h -- the wave-tile engine of the streaming quantized GEMV.
//
// A workgroup is kStreamWaves independent waves; each wave owns a "tile" of
// RW consecutive weight rows at a time -- one contiguous byte range of the
// matrix -- and walks tiles with a stride of the whole grid.  Lane l's unit
// slots (unit 64 i + l of a tile, i < kUPL) sit at the same (row, unit)
// position in every tile, so each lane quantizes the one to kUPL activation
// blocks it will ever use into registers once, at kernel start, while its
// first tile's weight loads are in flight: no shared activation, no workgroup
// barrier.  Per tile a wave
//   1. has the tile's weight bytes in registers,
//   2. computes one fp32 term (and int32 sum) per 32-element unit, 64 units
//      per instruction with lane = unit, into its own LDS slice [NT][RW][TS],
//   3. issues the next tile's loads,
//   4. adds each row's terms in unit order, one lane per (token, row).
// Direct formats (Q4_K, Q5_K: every sub-block 16-byte aligned) load each
// lane's header and sub-block straight from HBM.  Staged formats (Q8_0 34-byte
// and Q6_K 210-byte blocks) load the tile's byte range in 16-byte chunks,
// 1 KB per instruction, and extract blocks from an LDS copy.
#pragma once

#include "qr_gemv.h"

namespace qr {

constexpr int kStreamWaves = 4;  // waves per workgroup
constexpr int kUPL = 4;          // unit slots per lane and tile
constexpr int kCPL = 8;          // 16-byte chunks per lane and tile (staged formats)

template <int TYPE>
struct IsDirect {
  static constexpr bool value = (TYPE == QR_T_Q4_K || TYPE == QR_T_Q5_K);
};

struct TileShape {
  int U;   // units per row
  int RW;  // rows per wave tile; 0 when the row does not fit one tile
  int TS;  // LDS stride of one row's terms, in floats (16-byte aligned rows)
  int rb;  // bytes per row
  int SL;  // term slots per unit (q8_slots: 9 for the Q8_0 lane orders)
};

// Rows per tile: as many whole rows as kUPL unit slots per lane cover, and for
// staged formats as many as kCPL chunks per lane hold with the up to 15 bytes
// of misalignment in front and the slack dword that unaligned LDS reads touch.
__host__ __device__ inline TileShape tile_shape(int type, int d, int q8o = kQ8Seq) {
  TileShape s;
  s.SL = q8_slots(type, q8o);
  s.U = qr_units(type, d);
  s.rb = (int)qr_wrow_bytes(type, d);
  s.TS = ((s.U + 3) & ~3) + 4;
  int rw = s.U > 0 ? (64 * kUPL) / s.U : 0;
  if (!(type == QR_T_Q4_K || type == QR_T_Q5_K) && s.rb > 0) {
    const int r2 = (kCPL * 1024 - 19) / s.rb;
    rw = rw < r2 ? rw : r2;
  }
  s.RW = rw;
  return s;
}

// Bytes of one wave's LDS slice: the term rows ([nt][RW][SL][TS] floats),
// then (staged formats) the staged tile.
__host__ __device__ inline size_t wave_terms_bytes(int nt, const TileShape& s) {
  return align16((size_t)nt * s.RW * s.SL * s.TS * 4);
}
__host__ __device__ inline size_t wave_slice_bytes(int type, int nt, const TileShape& s) {
  const bool direct = type == QR_T_Q4_K || type == QR_T_Q5_K;
  return wave_terms_bytes(nt, s) + (direct ? 0 : (size_t)kCPL * 1024);
}

// LDS of a streaming kernel: kStreamWaves wave slices.
struct StreamLds {
  size_t slice, total;
};
__host__ __device__ inline StreamLds stream_lds(int type, int nt, const TileShape& s) {
  StreamLds L;
  L.slice = wave_slice_bytes(type, nt, s);
  L.total = (size_t)kStreamWaves * L.slice;
  return L;
}

// Order this wave's LDS accesses: everything before is complete before
// anything after starts (LDS serves a wave's instructions in order; this also
// stops the compiler from moving LDS accesses across it).
__device__ inline void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Registers holding one tile's weight bytes.
template <int TYPE, bool DIRECT = IsDirect<TYPE>::value>
struct TileRegs;

template <int TYPE>
struct TileRegs<TYPE, true> {
  uint4 hdr[kUPL];
  uint4 qs[kUPL];
  uint32_t qh[kUPL];
};

template <int TYPE>
struct TileRegs<TYPE, false> {
  uint4 c[kCPL];
};

// Lane-constant slot coordinates: slot i of a lane is unit fu = 64 i + lane of
// the tile, i.e. row fu / U, unit fu % U.
struct Slots {
  int row[kUPL];
  int u[kUPL];
};
__device__ inline Slots make_slots(int U, int lane) {
  Slots s;
#pragma unroll
  for (int i = 0; i < kUPL; i++) {
    const int fu = i * 64 + lane;
    s.row[i] = fu / U;
    s.u[i] = fu - s.row[i] * U;
  }
  return s;
}

// 16 weight bytes read once, with the non-temporal hint (the weight stream
// is the first L2 gives up, so the activation stays cached).
typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
__device__ inline uint4 ld_nt16(const uint8_t* p) {
  const u32x4_nt v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ inline uint32_t ld_nt4(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}

// Load tile rows [r0, r0 + RWt) of matrix W ([rows][rb], `total` bytes).
template <int TYPE>
__device__ inline void load_tile(const uint8_t* __restrict__ W, size_t total, int r0, int RWt,
                                 const TileShape& sh, const Slots& sl, int lane,
                                 TileRegs<TYPE>& R) {
  if constexpr (IsDirect<TYPE>::value) {
    constexpr int BB = TYPE == QR_T_Q4_K ? QR_Q4K_BYTES : QR_Q5K_BYTES;
#pragma unroll
    for (int i = 0; i < kUPL; i++) {
      if (sl.row[i] < RWt) {
        const uint8_t* blk =
            W + (size_t)(r0 + sl.row[i]) * sh.rb + (size_t)(sl.u[i] >> 3) * BB;
        const int s = sl.u[i] & 7;
        R.hdr[i] = ld_nt16(blk);
        if constexpr (TYPE == QR_T_Q4_K) {
          R.qs[i] = ld_nt16(blk + 16 + 16 * s);
          R.qh[i] = 0;
        } else {
          R.qs[i] = ld_nt16(blk + 48 + 16 * s);
          R.qh[i] = ld_nt4(blk + 16 + 4 * s);
        }
      } else {
        R.hdr[i] = make_uint4(0, 0, 0, 0);
        R.qs[i] = make_uint4(0, 0, 0, 0);
        R.qh[i] = 0;
      }
    }
  } else {
    const size_t gs = (size_t)r0 * sh.rb;
    const size_t ge = gs + (size_t)RWt * sh.rb;
    const size_t a0 = gs & ~(size_t)15;
#pragma unroll
    for (int j = 0; j < kCPL; j++) {
      const size_t off = a0 + (size_t)(j * 64 + lane) * 16;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (off < ge) {
        if (off + 16 <= total) {
          v = ld_nt16(W + off);
        } else {  // the matrix ends inside this chunk: no load leaves it
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
      }
      R.c[j] = v;
    }
  }
}

// Direct formats from a tile staged in LDS (byte 0 = matrix byte r0 * rb, which
// is 16-byte aligned for these formats): the same registers as load_tile.
template <int TYPE>
__device__ inline void load_tile_lds(const uint8_t* stage, int r0, int RWt, const TileShape& sh,
                                     const Slots& sl, TileRegs<TYPE>& R) {
  (void)r0;
  if constexpr (IsDirect<TYPE>::value) {
    constexpr int BB = TYPE == QR_T_Q4_K ? QR_Q4K_BYTES : QR_Q5K_BYTES;
#pragma unroll
    for (int i = 0; i < kUPL; i++) {
      if (sl.row[i] < RWt) {
        const uint8_t* blk = stage + (size_t)sl.row[i] * sh.rb + (size_t)(sl.u[i] >> 3) * BB;
        const int s = sl.u[i] & 7;
        R.hdr[i] = *reinterpret_cast<const uint4*>(blk);
        if constexpr (TYPE == QR_T_Q4_K) {
          R.qs[i] = *reinterpret_cast<const uint4*>(blk + 16 + 16 * s);
          R.qh[i] = 0;
        } else {
          R.qs[i] = *reinterpret_cast<const uint4*>(blk + 48 + 16 * s);
          R.qh[i] = *reinterpret_cast<const uint32_t*>(blk + 16 + 4 * s);
        }
      } else {
        R.hdr[i] = make_uint4(0, 0, 0, 0);
        R.qs[i] = make_uint4(0, 0, 0, 0);
        R.qh[i] = 0;
      }
    }
  }
}

// Staged formats: copy the tile's chunks into the wave's stage area.
template <int TYPE>
__device__ inline void stage_regs(const TileRegs<TYPE>& R, uint32_t* stage, int lane) {
  if constexpr (!IsDirect<TYPE>::value) {
#pragma unroll
    for (int j = 0; j < kCPL; j++) reinterpret_cast<uint4*>(stage)[j * 64 + lane] = R.c[j];
  }
}

// quantize_row_q8_0 (src/quant.c:143-158) of one 32-float block x (16-byte
// aligned) into registers: amax is a max (order-free), d = amax / 127 and
// 1 / d are correctly rounded IEEE divisions, rintf rounds ties to even like
// lrintf, and the scale goes through the truncating fp16 routine.  PERM packs
// each 8-element group as [x0 x2 x4 x6 | x1 x3 x5 x7] (the Q4_K nibble order).
struct ActBlock {
  uint32_t q[8];
  float bd;  // h2f(f2h(d))
  int bs;    // sum of the 32 int8 values
};

template <bool PERM>
__device__ inline ActBlock quantize_block(const float* __restrict__ x) {
  float v[32];
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const float4 f = reinterpret_cast<const float4*>(x)[k];
    v[4 * k] = f.x;
    v[4 * k + 1] = f.y;
    v[4 * k + 2] = f.z;
    v[4 * k + 3] = f.w;
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; i++) {
    const float av = __builtin_fabsf(v[i]);
    amax = av > amax ? av : amax;
  }
  const float dd = amax / 127.0f;
  const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
  int q[32];
  int s = 0;
#pragma unroll
  for (int i = 0; i < 32; i++) {
    q[i] = (int)(int8_t)(int)__builtin_rintf(v[i] * id);
    s += q[i];
  }
  ActBlock a;
#pragma unroll
  for (int g = 0; g < 4; g++) {
    const int* p = q + 8 * g;
    if (PERM) {
      a.q[2 * g] = pack4(p[0], p[2], p[4], p[6]);
      a.q[2 * g + 1] = pack4(p[1], p[3], p[5], p[7]);
    } else {
      a.q[2 * g] = pack4(p[0], p[1], p[2], p[3]);
      a.q[2 * g + 1] = pack4(p[4], p[5], p[6], p[7]);
    }
  }
  a.bd = qr_h2f(qr_f2h(dd));
  a.bs = s;
  return a;
}

// The activation blocks of a lane's slots for NT activation rows.  NS = 1
// when every slot has the same unit (U divides 64), else one per slot.
template <int NT, int NS>
struct LaneAct {
  ActBlock a[NT][NS];
};

template <int TYPE, int NT, int NS>
__device__ inline void quantize_lane_act(const float* __restrict__ X, size_t xstride,
                                         const Slots& sl, int RW, LaneAct<NT, NS>& A) {
#pragma unroll
  for (int i = 0; i < NS; i++) {
    if (sl.row[i] < RW) {
#pragma unroll
      for (int t = 0; t < NT; t++)
        A.a[t][i] = quantize_block<TYPE == QR_T_Q4_K>(X + (size_t)t * xstride + (size_t)sl.u[i] * 32);
    }
  }
}

// The same activation blocks, each quantized once per wave: lane u < U
// quantizes block u of x (global or LDS) into the wave's LDS area ab
// (48 bytes per block: 32 int8, bd, bs), then every lane gathers the blocks
// of its slots.  U blocks instead of 64 x kUPL.
//
// Four adjacent lanes share a block, 8 elements each (amax and the integer sum
// reduce across the quad with DPP; the operations are quantize_block's).
template <int TYPE, int NS>
__device__ inline void quantize_lane_act_wave(const float* __restrict__ X, const Slots& sl, int RW,
                                              int U, uint8_t* ab, int lane, LaneAct<1, NS>& A) {
  constexpr bool PERM = TYPE == QR_T_Q4_K;
  for (int base = 0; base < 4 * U; base += 64) {
    const int gi = base + lane;
    const bool live = gi < 4 * U;
    const int u = gi >> 2, part = gi & 3;
    float v[8];
    if (live) {
      const float4* p = reinterpret_cast<const float4*>(X + (size_t)u * 32 + part * 8);
      const float4 f0 = p[0], f1 = p[1];
      v[0] = f0.x; v[1] = f0.y; v[2] = f0.z; v[3] = f0.w;
      v[4] = f1.x; v[5] = f1.y; v[6] = f1.z; v[7] = f1.w;
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
    float o = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, amax), 0xB1, 0xF, 0xF, false));
    amax = o > amax ? o : amax;
    o = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, amax), 0x4E, 0xF, 0xF, false));
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
    s += __builtin_amdgcn_update_dpp(0, s, 0xB1, 0xF, 0xF, false);
    s += __builtin_amdgcn_update_dpp(0, s, 0x4E, 0xF, 0xF, false);
    if (live) {
      uint8_t* ob = ab + (size_t)u * 48;
      *reinterpret_cast<uint2*>(ob + part * 8) =
          PERM ? make_uint2(pack4(q[0], q[2], q[4], q[6]), pack4(q[1], q[3], q[5], q[7]))
               : make_uint2(pack4(q[0], q[1], q[2], q[3]), pack4(q[4], q[5], q[6], q[7]));
      if (part == 0)
        *reinterpret_cast<uint2*>(ob + 32) =
            make_uint2(__builtin_bit_cast(uint32_t, qr_h2f(qr_f2h(dd))), (uint32_t)s);
    }
  }
  wave_lds_sync();
#pragma unroll
  for (int i = 0; i < NS; i++) {
    if (sl.row[i] < RW) {
      const uint4* o = reinterpret_cast<const uint4*>(ab + (size_t)sl.u[i] * 48);
      const uint4 q0 = o[0], q1 = o[1], c = o[2];
      ActBlock& a = A.a[0][i];
      a.q[0] = q0.x; a.q[1] = q0.y; a.q[2] = q0.z; a.q[3] = q0.w;
      a.q[4] = q1.x; a.q[5] = q1.y; a.q[6] = q1.z; a.q[7] = q1.w;
      a.bd = __builtin_bit_cast(float, c.x);
      a.bs = (int)c.y;
    }
  }
}

// Terms of every valid slot into terms[t][row][u] (t < NT).  `stage` is the
// staged tile whose byte 0 is matrix byte (r0 * rb) & ~15.  Optional acc
// receives the int32 unit sums ([NT][n][U]).  Q8_0 in a lane order (Q8O)
// writes the unit's 8 lane sums and da * db into terms[t][row][k][u] instead.
template <int TYPE, int NT, int NS, int Q8O = kQ8Seq>
__device__ inline void tile_terms(const TileRegs<TYPE>& R, const Slots& sl, int RWt, int r0,
                                  const TileShape& sh, const LaneAct<NT, NS>& A,
                                  const uint32_t* stage, float* terms, int32_t* acc, int n) {
  const int lds_base = (int)(((size_t)r0 * sh.rb) & 15);
#pragma unroll
  for (int i = 0; i < kUPL; i++) {
    if (sl.row[i] < RWt) {
      const int ai = NS == 1 ? 0 : i;
      const int u = sl.u[i];
      float tv[NT];
      int32_t is[NT];
      if constexpr (IsDirect<TYPE>::value) {
        const int s = u & 7;
        const uint32_t sbyte = ((s < 4 ? R.hdr[i].y : R.hdr[i].z) >> (8 * (s & 3))) & 0xFFu;
#pragma unroll
        for (int t = 0; t < NT; t++) {
          const ActBlock& a = A.a[t][ai];
          int isum;
          if constexpr (TYPE == QR_T_Q4_K) isum = dot_q4_regs(R.qs[i], a.q);
          else isum = dot_q5_regs(R.qs[i], R.qh[i], a.q);
          tv[t] = term_q45(R.hdr[i].x, sbyte, isum, a.bs, a.bd);
          is[t] = isum;
        }
      } else if constexpr (TYPE == QR_T_Q6_K) {
        const int o = lds_base + sl.row[i] * sh.rb + (u >> 3) * QR_Q6K_BYTES;
        const int s = u & 7;
        const uint4 ql = make_uint4(lds_u32(stage, o + 16 * s), lds_u32(stage, o + 16 * s + 4),
                                    lds_u32(stage, o + 16 * s + 8), lds_u32(stage, o + 16 * s + 12));
        const uint2 qh = make_uint2(lds_u32(stage, o + 128 + 8 * s), lds_u32(stage, o + 132 + 8 * s));
        const int scale = (int)(int8_t)(lds_u32(stage, o + 192 + s) & 0xFFu);
        const uint32_t dh = lds_u32(stage, o + 208) & 0xFFFFu;
#pragma unroll
        for (int t = 0; t < NT; t++) {
          const ActBlock& a = A.a[t][ai];
          const int isum = dot_q6_regs_raw(ql, qh, a.q) - 32 * a.bs;
          tv[t] = term_q6(scale, dh, isum, a.bd);
          is[t] = isum;
        }
      } else {  // Q8_0
        const int o = lds_base + sl.row[i] * sh.rb + u * QR_Q8_BYTES;
        const uint32_t dh = lds_u32(stage, o) & 0xFFFFu;
        uint32_t w[8];
#pragma unroll
        for (int k = 0; k < 8; k++) w[k] = lds_u32(stage, o + 2 + 4 * k);
#pragma unroll
        for (int t = 0; t < NT; t++) {
          const ActBlock& a = A.a[t][ai];
          if constexpr (Q8O != kQ8Seq) {
            int l[8];
            q8_lanes(w, a.q, l);
            float* sp = terms + ((t * sh.RW + sl.row[i]) * 9) * sh.TS + u;
            int isum = 0;
#pragma unroll
            for (int k = 0; k < 8; k++) {
              sp[k * sh.TS] = (float)l[k];
              isum += l[k];
            }
            sp[8 * sh.TS] = qr_h2f(dh) * a.bd;  // fp16_to_fp32(a.d) * fp16_to_fp32(b.d)
            tv[t] = 0.0f;
            is[t] = isum;
          } else {
            const int isum = dot_q8_regs(w, a.q);
            tv[t] = term_q8(dh, isum, a.bd);
            is[t] = isum;
          }
        }
      }
#pragma unroll
      for (int t = 0; t < NT; t++) {
        if (q8_slots(TYPE, Q8O) == 1) terms[(t * sh.RW + sl.row[i]) * sh.TS + u] = tv[t];
        if (acc) acc[((size_t)t * n + r0 + sl.row[i]) * sh.U + u] = is[t];
      }
    }
  }
}

// Sequential sum of one row's U terms from 0.0f, unit 0 first (the fp32
// accumulation of every reference dot, src/quant.c:279-285, 384-400,
// 422-434); `tp` is 16-byte aligned.  The LDS reads of 32 terms are issued
// before their adds, so the add chain waits on LDS once per 32 terms.
__device__ inline float row_sum_seq(const float* tp, int U) {
  float s = 0.0f;
  int u = 0;
  for (; u + 32 <= U; u += 32) {
    float4 v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = *reinterpret_cast<const float4*>(tp + u + 4 * k);
#pragma unroll
    for (int k = 0; k < 8; k++) {
      s += v[k].x;
      s += v[k].y;
      s += v[k].z;
      s += v[k].w;
    }
  }
  for (; u + 4 <= U; u += 4) {
    const float4 v = *reinterpret_cast<const float4*>(tp + u);
    s += v.x;
    s += v.y;
    s += v.z;
    s += v.w;
  }
  for (; u < U; u++) s += tp[u];
  return s;
}

// Lane accumulator k of a row in a Q8_0 lane order (`tp` = the row's [9][ts]
// slots, 16-byte aligned, ts a multiple of 4): acc over units 0..U-1, the
// slot reads four units at a time.
template <int Q8O>
__device__ inline float q8_chain(const float* tp, int ts, int U, int k) {
  const float* f = tp + k * ts;
  const float* dd = tp + 8 * ts;
  float acc = 0.0f;
  int u = 0;
  for (; u + 4 <= U; u += 4) {
    const float4 fv = *reinterpret_cast<const float4*>(f + u);
    const float4 dv = *reinterpret_cast<const float4*>(dd + u);
    acc = q8_lane_update<Q8O>(fv.x, dv.x, acc);
    acc = q8_lane_update<Q8O>(fv.y, dv.y, acc);
    acc = q8_lane_update<Q8O>(fv.z, dv.z, acc);
    acc = q8_lane_update<Q8O>(fv.w, dv.w, acc);
  }
  for (; u < U; u++) acc = q8_lane_update<Q8O>(f[u], dd[u], acc);
  return acc;
}

}  // namespace qr
