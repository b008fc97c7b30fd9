// qr_gemv.hip -- quantized decode GEMV for gfx950:  y[t][r] = W[r] . x[t]
// for W in Q8_0 / Q4_K / Q5_K / Q6_K (the reference's block layouts, streamed
// straight from HBM), x fp32 quantized to Q8_0 inside the kernel, t < NT.
//
// Semantics: matmul_q_fused (src/quant.c:441-523): one Q8_0 quantization of x
// per call, then per row the fused dot in the reference's order: int32 sums per
// 32-element unit, one fp32 term per unit, the terms added sequentially from
// 0.0f.  Results are bit-identical to the reference's -std=c99 build (Q8_0,
// Q5_K, Q6_K) and to the corrected Q4_K dot.
//
// Work split: a workgroup owns R consecutive rows (one contiguous byte range
// of W).  Its waves sweep the rows' units 64 at a time (lane = unit), compute
// each unit's int32 sum with v_dot4_i32_i8 and its fp32 term, and park the
// term in LDS; then R*NT threads add their row's terms in unit order.
#include "qr_gemv.h"
#include "qr_internal.h"

namespace qr {

constexpr int kWg = 256;

struct GemvArgs {
  const uint8_t* W;      // [n][row_bytes], 16-byte aligned
  const float* X;        // [nt][xstride]
  float* Y;              // [nt][ystride]
  int n, d;
  int xstride, ystride;
  int rows_per_wg;
  int32_t* acc;          // optional [nt][n][units] int32 unit sums
  int32_t* accb;         // optional [nt][units] activation block sums
};

// LDS layout: act q | act bd | act bs | terms | staged tile.
__host__ __device__ inline size_t gemv_lds_layout(int type, int d, int nt, int R, size_t* o_bd,
                                                  size_t* o_bs, size_t* o_terms, size_t* o_tile) {
  const int nxb = d / 32;
  const int U = qr_units(type, d);
  size_t off = align16((size_t)nt * nxb * 32);
  *o_bd = off;
  off = align16(off + (size_t)nt * nxb * 4);
  *o_bs = off;
  off = align16(off + (size_t)nt * nxb * 4);
  *o_terms = off;
  off = align16(off + (size_t)nt * R * (U + 1) * 4);
  *o_tile = off;
  if (type == QR_T_Q8_0 || type == QR_T_Q6_K) off += stage_bytes((size_t)R * qr_wrow_bytes(type, d));
  return off;
}

template <int TYPE, int NT>
__global__ __launch_bounds__(kWg) void k_gemv(GemvArgs g) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int d = g.d;
  const int U = qr_units(TYPE, d);
  const int nxb = d >> 5;
  const size_t rb = qr_wrow_bytes(TYPE, d);
  const int r0 = blockIdx.x * g.rows_per_wg;
  const int R = min(g.rows_per_wg, g.n - r0);
  if (R <= 0) return;

  size_t o_bd, o_bs, o_terms, o_tile;
  gemv_lds_layout(TYPE, d, NT, g.rows_per_wg, &o_bd, &o_bs, &o_terms, &o_tile);
  UnitSrc S;
  S.act.q = reinterpret_cast<int8_t*>(smem);
  S.act.bd = reinterpret_cast<float*>(smem + o_bd);
  S.act.bs = reinterpret_cast<int32_t*>(smem + o_bs);
  S.tile = reinterpret_cast<const uint32_t*>(smem + o_tile);
  S.nxb = nxb;
  float* terms = reinterpret_cast<float*>(smem + o_terms);
  const int tstride = U + 1;

  const size_t gstart = (size_t)r0 * rb;
  int lds_base = 0;
  if constexpr (!Fmt<TYPE>::kDirect) {
    stage_tile(g.W, (size_t)g.n * rb, gstart, gstart + (size_t)R * rb,
               reinterpret_cast<uint32_t*>(smem + o_tile));
    lds_base = (int)(gstart & 15);
  }
  quantize_act_lds<Fmt<TYPE>::kPerm>(g.X, (size_t)g.xstride, nullptr, NT, NT, d, S.act);
  __syncthreads();

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nwaves = blockDim.x >> 6;
  const int total_units = R * U;
  for (int fu = wave * 64 + lane; fu < total_units; fu += nwaves * 64) {
    const int row = fu / U;
    const int u = fu - row * U;
    float tv[NT];
    int32_t is[NT];
    unit_terms<TYPE, NT>(g.W + gstart + (size_t)row * rb, lds_base + row * (int)rb, u, S, 0, tv,
                         is);
#pragma unroll
    for (int t = 0; t < NT; t++) {
      terms[((size_t)t * g.rows_per_wg + row) * tstride + u] = tv[t];
      if (g.acc) g.acc[((size_t)t * g.n + r0 + row) * U + u] = is[t];
    }
    if (g.accb && blockIdx.x == 0 && row == 0) {
#pragma unroll
      for (int t = 0; t < NT; t++) g.accb[(size_t)t * U + u] = S.act.bs[t * nxb + u];
    }
  }
  __syncthreads();

  for (int i = threadIdx.x; i < R * NT; i += blockDim.x) {
    const int t = i / R, row = i - t * R;
    g.Y[(size_t)t * g.ystride + r0 + row] =
        row_sum(terms + ((size_t)t * g.rows_per_wg + row) * tstride, U);
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
size_t gemv_lds_bytes(int type, int d, int nt, int R) {
  size_t a, b, c, e;
  return gemv_lds_layout(type, d, nt, R, &a, &b, &c, &e);
}

// Rows per workgroup: enough workgroups to cover the 256 CUs several times,
// at most 16 units per thread, and an LDS footprint that leaves room for
// several workgroups per CU.
int gemv_rows_per_wg(int type, int n, int d, int nt) {
  const int U = qr_units(type, d);
  int R = 64;
  while (R > 1 && ((n + R - 1) / R < 1024 || (size_t)R * U > 16 * kWg)) R >>= 1;
  while (R > 1 && gemv_lds_bytes(type, d, nt, R) > 48 * 1024) R >>= 1;
  return R;
}

template <int TYPE, int NT>
static hipError_t launch_t(const GemvArgs& a, hipStream_t st) {
  const size_t lds = gemv_lds_bytes(TYPE, a.d, NT, a.rows_per_wg);
  const int U = qr_units(TYPE, a.d);
  int threads = ((a.rows_per_wg * U + 63) / 64) * 64;
  threads = threads < 64 ? 64 : (threads > kWg ? kWg : threads);
  const int grid = (a.n + a.rows_per_wg - 1) / a.rows_per_wg;
  if (lds > 64 * 1024) return hipErrorInvalidValue;  // dynamic LDS without an opt-in
  hipLaunchKernelGGL((k_gemv<TYPE, NT>), dim3(grid), dim3(threads), lds, st, a);
  return hipGetLastError();
}

template <int TYPE>
static hipError_t launch_nt(const GemvArgs& a, int nt, hipStream_t st) {
  switch (nt) {
    case 1: return launch_t<TYPE, 1>(a, st);
    case 2: return launch_t<TYPE, 2>(a, st);
    case 3: return launch_t<TYPE, 3>(a, st);
    case 4: return launch_t<TYPE, 4>(a, st);
    case 8: return launch_t<TYPE, 8>(a, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t gemv_launch(int type, const void* W, const float* X, float* Y, int n, int d, int nt,
                       int xstride, int ystride, int32_t* acc, int32_t* accb, hipStream_t st) {
  GemvArgs a;
  a.W = static_cast<const uint8_t*>(W);
  a.X = X;
  a.Y = Y;
  a.n = n;
  a.d = d;
  a.xstride = xstride;
  a.ystride = ystride;
  a.rows_per_wg = gemv_rows_per_wg(type, n, d, nt);
  a.acc = acc;
  a.accb = accb;
  switch (type) {
    case QR_T_Q4_K: return launch_nt<QR_T_Q4_K>(a, nt, st);
    case QR_T_Q5_K: return launch_nt<QR_T_Q5_K>(a, nt, st);
    case QR_T_Q6_K: return launch_nt<QR_T_Q6_K>(a, nt, st);
    case QR_T_Q8_0: return launch_nt<QR_T_Q8_0>(a, nt, st);
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------
// fp32 GEMV in the reference's accumulation orders (router logits and F32
// weights):  out[t][r] = sum_j W[r][j] * x[t][j].
//   SEQ    matmul_ref (src/kernels.c:18-28) and matmul_q_fused's F32 rows
//          (src/quant.c:455-462): j ascending, multiply then add.
//   AVX2   matmul_omp built -mavx2 -mfma (src/kernels.c:50-65): lane k keeps
//          the FMA chain over j = 8i + k; lanes added 0..7 into 0.0f; then a
//          multiply-add tail for d % 8.
//   AVX512 matmul_omp built -mavx512f (src/kernels.c:38-49): 16 FMA chains,
//          GCC's _mm512_reduce_add_ps tree (upper 8 + lower 8, upper 4 +
//          lower 4, [0]+[2] and [1]+[3], then their sum), then the tail.
// One thread per chain; the LANES chains of one row sit in adjacent lanes.
// ---------------------------------------------------------------------------
template <int LANES>
__global__ __launch_bounds__(256) void k_gemv_f32(const float* __restrict__ W,
                                                  const float* __restrict__ X,
                                                  float* __restrict__ Y, int n, int d, int nt,
                                                  int xstride, int ystride) {
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int k = (int)(gid % LANES);
  const long rt = gid / LANES;  // (token, row) pair
  const bool live = rt < (long)n * nt;
  const int t = live ? (int)(rt / n) : 0;
  const int r = live ? (int)(rt - (long)t * n) : 0;
  const float* w = W + (size_t)r * d;
  const float* x = X + (size_t)t * xstride;
  if constexpr (LANES == 1) {
    if (!live) return;
    float s = 0.0f;
    for (int j = 0; j < d; j++) s += w[j] * x[j];
    Y[(size_t)t * ystride + r] = s;
  } else {
    const int dm = d - d % LANES;
    float acc = 0.0f;
    if (live)
      for (int j = k; j < dm; j += LANES) acc = __builtin_fmaf(w[j], x[j], acc);
    float v[LANES];
    const int base = (int)(threadIdx.x & 63) - k;
#pragma unroll
    for (int i = 0; i < LANES; i++) v[i] = __shfl(acc, base + i);
    if (!live || k != 0) return;
    float s = 0.0f;
    if constexpr (LANES == 8) {
#pragma unroll
      for (int i = 0; i < 8; i++) s += v[i];
    } else {
      float t8[8], t4[4];
#pragma unroll
      for (int i = 0; i < 8; i++) t8[i] = v[8 + i] + v[i];
#pragma unroll
      for (int i = 0; i < 4; i++) t4[i] = t8[4 + i] + t8[i];
      const float a02 = t4[0] + t4[2];
      const float a13 = t4[1] + t4[3];
      s += a02 + a13;
    }
    for (int j = dm; j < d; j++) s += w[j] * x[j];
    Y[(size_t)t * ystride + r] = s;
  }
}

hipError_t gemv_f32_launch(int order, const float* W, const float* X, float* Y, int n, int d,
                           int nt, int xstride, int ystride, hipStream_t st) {
  const int lanes = order == QR_ORDER_SEQ ? 1 : order == QR_ORDER_AVX2 ? 8 : 16;
  const long total = (long)n * nt * lanes;
  const int threads = 256;
  const long grid = (total + threads - 1) / threads;
  if (grid == 0) return hipSuccess;
  switch (lanes) {
    case 1:
      hipLaunchKernelGGL(k_gemv_f32<1>, dim3((unsigned)grid), dim3(threads), 0, st, W, X, Y, n, d,
                         nt, xstride, ystride);
      break;
    case 8:
      hipLaunchKernelGGL(k_gemv_f32<8>, dim3((unsigned)grid), dim3(threads), 0, st, W, X, Y, n, d,
                         nt, xstride, ystride);
      break;
    default:
      hipLaunchKernelGGL(k_gemv_f32<16>, dim3((unsigned)grid), dim3(threads), 0, st, W, X, Y, n,
                         d, nt, xstride, ystride);
      break;
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// quantize_row_q8_0 (src/quant.c:143-158) to block_q8_0 bytes in HBM, one
// thread per 32-element block: the activation quantizer's drop-in and the
// Q8_0 weight quantizer.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_quantize_q8_0(const float* __restrict__ x,
                                                       uint8_t* __restrict__ y, long nblocks) {
  const long b = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const float* p = x + b * 32;
  float v[32];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; j++) {
    v[j] = p[j];
    const float av = __builtin_fabsf(v[j]);
    amax = av > amax ? av : amax;
  }
  const float dd = amax / 127.0f;
  const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
  const uint32_t dh = qr_f2h(dd);
  uint8_t* o = y + b * QR_Q8_BYTES;
  o[0] = (uint8_t)(dh & 0xFFu);
  o[1] = (uint8_t)(dh >> 8);
#pragma unroll
  for (int j = 0; j < 32; j++) o[2 + j] = (uint8_t)(int8_t)(int)__builtin_rintf(v[j] * id);
}

hipError_t quantize_q8_0_launch(const float* x, void* y, long nblocks, hipStream_t st) {
  if (nblocks <= 0) return hipSuccess;
  const int threads = 256;
  const long grid = (nblocks + threads - 1) / threads;
  hipLaunchKernelGGL(k_quantize_q8_0, dim3((unsigned)grid), dim3(threads), 0, st, x,
                     static_cast<uint8_t*>(y), nblocks);
  return hipGetLastError();
}

}  // namespace qr
