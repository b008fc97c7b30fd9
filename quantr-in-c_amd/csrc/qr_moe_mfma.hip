// qr_moe_mfma.hip -- grouped expert products on int8 MFMA for experts that
// receive many tokens (the MoE layer at large T).
//
// A work item is (64 weight rows of one expert) x (up to 32 dispatched
// (token, slot) pairs of that expert).  The K loop walks the row one "stage"
// at a time -- one K-quant super-block, or 8 Q8_0 blocks -- staging the 64
// rows' bytes (both matrices in gate/up mode), the pairs' quantized
// activation blocks, and each (row, unit)'s fp32 scale and min into LDS.
// Each 32-element unit is one v_mfma_i32_16x16x32_i8: a 16 x 16 tile of exact
// int32 unit sums (16 rows x 16 pairs per wave, two such column tiles).  The
// epilogue forms the reference's fp32 term of every (row, pair, unit) --
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
#include "qr_gemv.h"
#include "qr_internal.h"

namespace qr {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kXQ = 48;   // activation record: [32 int8 | bd f32 | (float)bs f32 | bs i32 | pad]
constexpr int kMR = 64;   // weight rows per workgroup (16 per wave)
constexpr int kMT = 32;   // pairs per workgroup (two MFMA column tiles)

// ---------------------------------------------------------------------------
// Activation rows -> quantized records in HBM (quantize_row_q8_0,
// src/quant.c:143-158, four lanes per 32-element block).
// ---------------------------------------------------------------------------
template <bool PERM>
__global__ __launch_bounds__(256) void k_quant_rows(const float* __restrict__ x, int xstride,
                                                   int nrows, int cols, uint8_t* __restrict__ out) {
  const int U = cols >> 5;
  const long total = (long)nrows * U * 4;
  const long gi = (long)blockIdx.x * 256 + threadIdx.x;
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
  if (!live) return;
  uint8_t* rec = out + blk * kXQ;
  uint32_t w0, w1;
  if (PERM) {
    w0 = pack4(q[0], q[2], q[4], q[6]);
    w1 = pack4(q[1], q[3], q[5], q[7]);
  } else {
    w0 = pack4(q[0], q[1], q[2], q[3]);
    w1 = pack4(q[4], q[5], q[6], q[7]);
  }
  *reinterpret_cast<uint2*>(rec + part * 8) = make_uint2(w0, w1);
  if (part == 0) {
    float* f = reinterpret_cast<float*>(rec + 32);
    f[0] = qr_h2f(qr_f2h(dd));
    f[1] = (float)s;
    reinterpret_cast<int*>(rec + 40)[0] = s;
  }
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

// Spread the four nibbles of a 16-bit value to the low nibbles of 4 bytes.
__device__ inline uint32_t nib16_to_bytes(uint32_t x) {
  uint32_t t = (x | (x << 8)) & 0x00FF00FFu;
  return (t | (t << 4)) & 0x0F0F0F0Fu;
}
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
  } else if constexpr (TYPE == QR_T_Q6_K) {
    const uint32_t w = lds_u32(wl, o + 16 * s + 4 * kg);
    const uint32_t h = lds_u32(wl, o + 128 + 8 * s + 2 * kg) & 0xFFFFu;
    lo = (w & 0x0F0F0F0Fu) | (nib16_to_bytes(h & 0x3333u) << 4);
    hi = ((w >> 4) & 0x0F0F0F0Fu) | (nib16_to_bytes((h >> 2) & 0x3333u) << 4);
  } else {  // Q8_0: block s, bytes 2 + 8 kg .. +7
    lo = lds_u32(wl, o + QR_Q8_BYTES * s + 2 + 8 * kg);
    hi = lds_u32(wl, o + QR_Q8_BYTES * s + 6 + 8 * kg);
  }
  return (long)((uint64_t)lo | ((uint64_t)hi << 32));
}

// fp32 scale (and min) of unit s of a staged row.
template <int TYPE>
__device__ inline void unit_scale(const uint32_t* wl, int o, int s, float* sc, float* mn) {
  if constexpr (TYPE == QR_T_Q4_K || TYPE == QR_T_Q5_K) {
    const uint32_t h0 = wl[o >> 2];
    const uint32_t sbyte = (wl[(o + 4 + s) >> 2] >> (8 * ((4 + s) & 3))) & 0xFFu;
    *sc = (float)(sbyte & 63u) * qr_h2f(h0 & 0xFFFFu);
    *mn = (float)(sbyte >> 6) * qr_h2f(h0 >> 16);
  } else if constexpr (TYPE == QR_T_Q6_K) {
    const int scale = (int)(int8_t)(lds_u32(wl, o + 192 + s) & 0xFFu);
    *sc = (float)scale * qr_h2f(lds_u32(wl, o + 208) & 0xFFFFu);
    *mn = 0.0f;
  } else {
    *sc = qr_h2f(lds_u32(wl, o + QR_Q8_BYTES * s) & 0xFFFFu);
    *mn = 0.0f;
  }
}

// ---------------------------------------------------------------------------
// The grouped MFMA kernel.
// ---------------------------------------------------------------------------
struct MfmaArgs {
  const uint8_t* W1;      // [E][rows][rb] (up in gate/up mode)
  const uint8_t* W2;      // [E][rows][rb] (gate in gate/up mode)
  size_t slice;           // bytes per expert
  size_t wtotal;          // bytes of each weight tensor
  int rows, cols, E, K;
  const uint8_t* XQ;      // activation records [xrows][cols/32][kXQ]
  int x_by_token;         // activation row of dispatch position p: perm[p] / K, else p
  const int32_t* offsets; // dispatch (tile = kMT)
  const int32_t* perm;
  const int32_t* tiles;
  float* Y;               // [P][ystride], row = dispatch position
  int ystride;
};

template <int TYPE, bool GATEUP>
__global__ __launch_bounds__(256) void k_expert_mfma(MfmaArgs a) {
  constexpr int NMAT = GATEUP ? 2 : 1;
  constexpr int SLOT = MF<TYPE>::kSlot;
  constexpr int NCH = MF<TYPE>::kChunks;
  constexpr int NLOAD = (NMAT * kMR * NCH + 255) / 256;
  constexpr int ACT_TOK = 8 * kXQ + 16;  // LDS stride of one pair's 8 records
  __shared__ __align__(16) uint32_t wl[NMAT * kMR * SLOT / 4];
  __shared__ __align__(16) float scl[NMAT][8][kMR];
  __shared__ __align__(16) float mnl[NMAT][8][kMR];
  __shared__ __align__(16) uint8_t act[kMT * ACT_TOK];
  __shared__ int xrow[kMT];
  __shared__ int whead[NMAT * kMR];  // misaligned head bytes of each row's stage

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
  const int p0 = a.offsets[e] + (item - a.tiles[e]) * kMT;
  const int np = min(kMT, a.offsets[e + 1] - p0);
  if (np <= 0) return;  // uniform
  const int r0 = blockIdx.x * kMR;
  const int nr = min(kMR, a.rows - r0);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int kg = lane >> 4, ln = lane & 15;
  const int U = TYPE == QR_T_Q8_0 ? a.cols / 32 : (a.cols / 256) * 8;
  const size_t rb = qr_wrow_bytes(TYPE, a.cols);
  const int nstage = (U + 7) / 8;
  if (tid < kMT) {
    int xr = 0;
    if (tid < np) xr = a.x_by_token ? a.perm[p0 + tid] / a.K : p0 + tid;
    xrow[tid] = xr;
  }

  float acc[NMAT][2][4];
#pragma unroll
  for (int m = 0; m < NMAT; m++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int i = 0; i < 4; i++) acc[m][j][i] = 0.0f;

  uint4 wreg[NLOAD];
  uint4 areg[3];
  __syncthreads();  // xrow
  // global loads of stage st into registers
  auto load_stage = [&](int st) {
#pragma unroll
    for (int q = 0; q < NLOAD; q++) {
      const int c = tid + 256 * q;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (c < NMAT * kMR * NCH) {
        const int m = c / (kMR * NCH);
        const int rem = c - m * kMR * NCH;
        const int rr = rem / NCH, ch = rem - rr * NCH;
        if (rr < nr) {
          const size_t base = (size_t)e * a.slice + (size_t)(r0 + rr) * rb;
          const size_t start = base + (size_t)st * MF<TYPE>::kStage;
          const size_t end = base + min((size_t)(st + 1) * MF<TYPE>::kStage, rb);
          const size_t off = (start & ~(size_t)15) + (size_t)ch * 16;
          const uint8_t* W = m == 0 ? a.W1 : a.W2;
          if (off < end) {
            if (off + 16 <= a.wtotal) {
              v = *reinterpret_cast<const uint4*>(W + off);
            } else {  // the tensor ends inside this chunk: no load leaves it
              uint32_t w[4];
#pragma unroll
              for (int k = 0; k < 4; k++) {
                const size_t o = off + 4 * k;
                if (o + 4 <= a.wtotal) w[k] = *reinterpret_cast<const uint32_t*>(W + o);
                else if (o + 2 <= a.wtotal) w[k] = *reinterpret_cast<const uint16_t*>(W + o);
                else w[k] = 0;
              }
              v = make_uint4(w[0], w[1], w[2], w[3]);
            }
          }
        }
      }
      wreg[q] = v;
    }
    // activation records of the stage's units: 24 16-byte chunks per pair
#pragma unroll
    for (int q = 0; q < 3; q++) {
      const int c = tid + 256 * q;  // < 768 = kMT * 24
      const int tt = c / 24, ch = c - tt * 24;
      uint4 v = make_uint4(0, 0, 0, 0);
      const int u0 = st * 8 + (ch * 16) / kXQ;
      if (tt < np && u0 < U) {
        const uint8_t* rec = a.XQ + ((size_t)xrow[tt] * (a.cols / 32) + (size_t)st * 8) * kXQ;
        v = reinterpret_cast<const uint4*>(rec)[ch];
      }
      areg[q] = v;
    }
  };

  load_stage(0);
  for (int st = 0; st < nstage; st++) {
    __syncthreads();  // previous stage's LDS reads are done
#pragma unroll
    for (int q = 0; q < NLOAD; q++) {
      const int c = tid + 256 * q;
      if (c < NMAT * kMR * NCH) {
        const int m = c / (kMR * NCH);
        const int rem = c - m * kMR * NCH;
        const int rr = rem / NCH, ch = rem - rr * NCH;
        reinterpret_cast<uint4*>(wl)[((m * kMR + rr) * SLOT) / 16 + ch] = wreg[q];
        if (ch == 0) {
          const size_t start = (size_t)e * a.slice + (size_t)(r0 + rr) * rb +
                               (size_t)st * MF<TYPE>::kStage;
          whead[m * kMR + rr] = (int)(start & 15);
        }
      }
    }
#pragma unroll
    for (int q = 0; q < 3; q++) {
      const int c = tid + 256 * q;
      const int tt = c / 24, ch = c - tt * 24;
      *reinterpret_cast<uint4*>(act + tt * ACT_TOK + ch * 16) = areg[q];
    }
    __syncthreads();
    if (st + 1 < nstage) load_stage(st + 1);
    // scales and mins of the stage's (row, unit)s
    const int su = min(8, U - st * 8);
    for (int i = tid; i < NMAT * kMR * 8; i += 256) {
      const int m = i / (kMR * 8);
      const int rem = i - m * kMR * 8;
      const int s = rem / kMR, rr = rem - s * kMR;
      float sc = 0.0f, mn = 0.0f;
      if (s < su && rr < nr) {
        const int o = (m * kMR + rr) * SLOT + whead[m * kMR + rr];
        unit_scale<TYPE>(wl, o, s, &sc, &mn);
      }
      scl[m][s][rr] = sc;
      mnl[m][s][rr] = mn;
    }
    __syncthreads();

    const int rw = wave * 16 + ln;  // this lane's A row (within the 64)
    for (int s = 0; s < su; s++) {
      long A[NMAT];
#pragma unroll
      for (int m = 0; m < NMAT; m++) {
        const int o = (m * kMR + rw) * SLOT + whead[m * kMR + rw];
        A[m] = unit_a<TYPE>(wl, o, s, kg);
      }
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const uint8_t* rec = act + (16 * j + ln) * ACT_TOK + s * kXQ;
        const uint2 bq = *reinterpret_cast<const uint2*>(rec + 8 * kg);
        const long B = (long)((uint64_t)bq.x | ((uint64_t)bq.y << 32));
        const float bd = *reinterpret_cast<const float*>(rec + 32);
        const float bsf = *reinterpret_cast<const float*>(rec + 36);
        const int bs = *reinterpret_cast<const int*>(rec + 40);
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
          const v4i zero = {0, 0, 0, 0};
          const v4i D = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[m], B, zero, 0, 0, 0);
          const float4 sc4 = *reinterpret_cast<const float4*>(&scl[m][s][wave * 16 + 4 * kg]);
          const float4 mn4 = *reinterpret_cast<const float4*>(&mnl[m][s][wave * 16 + 4 * kg]);
          const float scv[4] = {sc4.x, sc4.y, sc4.z, sc4.w};
          const float mnv[4] = {mn4.x, mn4.y, mn4.z, mn4.w};
#pragma unroll
          for (int i = 0; i < 4; i++) {
            float term;
            if constexpr (MF<TYPE>::kMin) {
              term = (scv[i] * (float)D[i] - mnv[i] * bsf) * bd;
            } else if constexpr (TYPE == QR_T_Q6_K) {
              term = scv[i] * (float)(D[i] - 32 * bs) * bd;
            } else {
              term = (float)D[i] * scv[i] * bd;
            }
            acc[m][j][i] += term;
          }
        }
      }
    }
  }

  // outputs: rows r0 + 16 wave + 4 kg + i, pairs 16 j + ln
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int tt = 16 * j + ln;
    if (tt >= np) continue;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int rr = wave * 16 + 4 * kg + i;
      if (rr >= nr) continue;
      float out = acc[0][j][i];
      if constexpr (GATEUP) out = qr_silu(acc[0][j][i]) * acc[1][j][i];
      a.Y[(size_t)(p0 + tt) * a.ystride + r0 + rr] = out;
    }
  }
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

template <int TYPE, bool GATEUP>
static hipError_t mfma_launch_t(const MfmaArgs& a, int items, hipStream_t st) {
  dim3 grid((a.rows + kMR - 1) / kMR, items);
  if (grid.x == 0 || grid.y == 0) return hipSuccess;
  hipLaunchKernelGGL((k_expert_mfma<TYPE, GATEUP>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t expert_mfma_launch(int type, bool gateup, const uint8_t* W1, const uint8_t* W2,
                              size_t slice, int E, int K, int rows, int cols, const uint8_t* XQ,
                              int x_by_token, const int32_t* offsets, const int32_t* perm,
                              const int32_t* tiles, float* Y, int ystride, int items,
                              hipStream_t st) {
  MfmaArgs a;
  a.W1 = W1;
  a.W2 = W2;
  a.slice = slice;
  a.wtotal = slice * (size_t)E;
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
  switch (type) {
    case QR_T_Q4_K: return gateup ? mfma_launch_t<QR_T_Q4_K, true>(a, items, st)
                                  : mfma_launch_t<QR_T_Q4_K, false>(a, items, st);
    case QR_T_Q5_K: return gateup ? mfma_launch_t<QR_T_Q5_K, true>(a, items, st)
                                  : mfma_launch_t<QR_T_Q5_K, false>(a, items, st);
    case QR_T_Q6_K: return gateup ? mfma_launch_t<QR_T_Q6_K, true>(a, items, st)
                                  : mfma_launch_t<QR_T_Q6_K, false>(a, items, st);
    case QR_T_Q8_0: return gateup ? mfma_launch_t<QR_T_Q8_0, true>(a, items, st)
                                  : mfma_launch_t<QR_T_Q8_0, false>(a, items, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qr
