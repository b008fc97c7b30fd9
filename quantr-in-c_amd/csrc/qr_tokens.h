// qr_tokens.h -- device helpers of the MoE layer at T > 1 shared by several
// kernels: the quantized activation records the grouped expert products read,
// and the deterministic token -> expert dispatch of one workgroup.
#pragma once

#include "qr_gemv.h"

namespace qr {

// Activation record of one 32-element block in HBM, 48 bytes:
// [32 int8 | bd f32 | (float)bs f32 | bs i32 | pad], bd = h2f(f2h(d)) and bs
// the block's integer sum; PERM stores each 8-element group as
// [x0 x2 x4 x6 | x1 x3 x5 x7] (the K-quant nibble order).
constexpr int kXQ = 48;

// quantize_row_q8_0 (src/quant.c:143-158) of one 8-element group v[] of a
// 32-element block whose four groups sit in four adjacent lanes (the quad):
// amax and the integer sum reduce across the quad with DPP; d = amax / 127
// and 1 / d are correctly rounded; rintf rounds ties to even like lrintf.
// Returns the group's packed int8 (PERM: [x0 x2 x4 x6 | x1 x3 x5 x7]), the
// block's stored scale bd = h2f(f2h(d)) and integer sum bs.  Every lane of
// the quad must call.
template <bool PERM>
__device__ inline void quant8_core(const float (&v)[8], uint2* q8, float* bd, int* bs) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float av = __builtin_fabsf(v[i]);
    amax = av > amax ? av : amax;
  }
  auto xor1 = [](int q) { return __builtin_amdgcn_update_dpp(0, q, 0xB1, 0xF, 0xF, false); };
  auto xor2 = [](int q) { return __builtin_amdgcn_update_dpp(0, q, 0x4E, 0xF, 0xF, false); };
  float o = __builtin_bit_cast(float, xor1(__builtin_bit_cast(int, amax)));
  amax = o > amax ? o : amax;
  o = __builtin_bit_cast(float, xor2(__builtin_bit_cast(int, amax)));
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
  s += xor1(s);
  s += xor2(s);
  if (PERM) *q8 = make_uint2(pack4(q[0], q[2], q[4], q[6]), pack4(q[1], q[3], q[5], q[7]));
  else *q8 = make_uint2(pack4(q[0], q[1], q[2], q[3]), pack4(q[4], q[5], q[6], q[7]));
  *bd = qr_h2f(qr_f2h(dd));
  *bs = s;
}

// Store one group's share of a block's record (part = the group's index in
// the block; part 0 also writes the scale and sums).
__device__ inline void record_store(uint8_t* rec, int part, uint2 q8, float bd, int bs) {
  *reinterpret_cast<uint2*>(rec + part * 8) = q8;
  if (part == 0) {
    float* f = reinterpret_cast<float*>(rec + 32);
    f[0] = bd;
    f[1] = (float)bs;
    reinterpret_cast<int*>(rec + 40)[0] = bs;
  }
}

// Group gi of nrows rows of `cols` floats (row r at x + r * xstride) into
// the records at out: four adjacent lanes per block (gi & 3 = the part).
// Lanes past the end compute on zeros and store nothing.
template <bool PERM>
__device__ inline void quant_rows_group(const float* __restrict__ x, int xstride, int nrows,
                                        int cols, uint8_t* __restrict__ out, long gi) {
  const int U = cols >> 5;
  const long total = (long)nrows * U * 4;
  const bool live = gi < total;
  const long blk = live ? gi >> 2 : 0;
  const int part = (int)(gi & 3);
  const long r = blk / U;
  const int u = (int)(blk - r * U);
  float v[8];
  if (live) {
    const float4* p = reinterpret_cast<const float4*>(x + r * xstride + u * 32 + part * 8);
    const float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = 0.0f;
  }
  uint2 q8;
  float bd;
  int bs;
  quant8_core<PERM>(v, &q8, &bd, &bs);
  if (live) record_store(out + blk * kXQ, part, q8, bd, bs);
}

// ---------------------------------------------------------------------------
// Dispatch by one workgroup of kDispThreads threads, E <= 256: a histogram of
// the P (token, slot) pairs by expert, exclusive scans of the counts and of
// the `tile`-pair work items per expert, and a stable permutation (pairs of
// one expert keep their order): perm[offsets[e] + i] = the i-th pair of e,
// inv[p] = its position (-1 for an index outside 0..E-1).  `idx` may point
// to global or LDS memory.
//
// Wave w owns the pairs of one contiguous range (ranges in wave order), so a
// pair's position is offsets[e] + (pairs of e in the ranges of waves before
// w) + (pairs of e before it in w's range): the first term and the second
// come from per-wave counts, the third from a running per-wave count and the
// wave's ballots over each 64 pairs.
// ---------------------------------------------------------------------------
constexpr int kDispThreads = 1024;
constexpr int kDispWaves = kDispThreads / 64;

__device__ inline void dispatch_wg(const int32_t* idx, int P, int E, int tile,
                                   int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                                   int32_t* __restrict__ tiles, int32_t* __restrict__ perm,
                                   int32_t* __restrict__ inv) {
  __shared__ int cnt[256];
  __shared__ int wcnt[kDispWaves][256];  // the wave's counts, then its running position
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int per = ((P + kDispWaves - 1) / kDispWaves + 63) & ~63;  // whole rounds of 64
  const int p0 = wave * per, p1 = min(P, p0 + per);
  for (int i = tid; i < kDispWaves * 256; i += kDispThreads) (&wcnt[0][0])[i] = 0;
  __syncthreads();
  // the indices are read four rounds at a time, so their loads overlap
  for (int b = p0; b < p1; b += 4 * 64) {  // wave-uniform
    int ev[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int p = b + 64 * k + lane;
      ev[k] = p < p1 ? idx[p] : -1;
    }
#pragma unroll
    for (int k = 0; k < 4; k++)
      if (ev[k] >= 0 && ev[k] < E) atomicAdd(&wcnt[wave][ev[k]], 1);  // a count: order-free
  }
  __syncthreads();
  for (int e = tid; e < E; e += kDispThreads) {
    int c = 0;
#pragma unroll
    for (int w = 0; w < kDispWaves; w++) c += wcnt[w][e];
    cnt[e] = c;
  }
  __syncthreads();
  if (wave == 0) {
    // exclusive scans of the counts and of the tiles per expert: lane l owns
    // experts 4l .. 4l+3, then an inclusive scan across the wave; the first
    // position of expert e goes back to cnt[e]
    int c[4], tl[4], cs = 0, ts = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int e = 4 * lane + i;
      c[i] = e < E ? cnt[e] : 0;
      tl[i] = (c[i] + tile - 1) / tile;
      cs += c[i];
      ts += tl[i];
    }
    int ci = cs, ti = ts;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(ci, o), w = __shfl_up(ti, o);
      if (lane >= o) {
        ci += v;
        ti += w;
      }
    }
    int acc = ci - cs, tacc = ti - ts;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int e = 4 * lane + i;
      if (e < E) {
        cnt[e] = acc;
        counts[e] = c[i];
        offsets[e] = acc;
        if (tiles) tiles[e] = tacc;
      }
      acc += c[i];
      tacc += tl[i];
    }
    if (lane == 63) {
      offsets[E] = ci;
      if (tiles) tiles[E] = ti;
    }
  }
  __syncthreads();
  // each wave's first position per expert
  for (int e = tid; e < E; e += kDispThreads) {
    int run = cnt[e];
#pragma unroll
    for (int w = 0; w < kDispWaves; w++) {
      const int c = wcnt[w][e];
      wcnt[w][e] = run;
      run += c;
    }
  }
  __syncthreads();
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int b = p0; b < p1; b += 4 * 64) {  // wave-uniform
    int ev[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int p = b + 64 * r + lane;
      ev[r] = p < p1 ? idx[p] : -1;
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {  // rounds of 64 pairs, in order
      const int p = b + 64 * r + lane;
      const int e = ev[r] < E ? ev[r] : -1;
      const bool valid = e >= 0;
      // lanes of this round holding the same expert: match the 8 expert bits
      uint64_t peers = __ballot(valid);
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const bool bit = valid && ((e >> k) & 1);
        const uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
      }
      const int rank = __popcll(peers & lt);
      if (valid) {
        const int pos = wcnt[wave][e] + rank;
        perm[pos] = p;
        inv[p] = pos;
      } else if (p < p1) {
        inv[p] = -1;
      }
      // the wave's LDS operations complete in order: every lane's read above
      // precedes the first lane's update, which the next round's reads see
      if (valid && rank == 0) wcnt[wave][e] += __popcll(peers);
    }
  }
}

}  // namespace qr
