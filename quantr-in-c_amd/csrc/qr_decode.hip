// qr_decode.hip -- quantr-in-c's single-token decode step (forward_runtime,
// src/runtime.c:94-288) on gfx950, bit-exact with the reference's arithmetic:
//
//   x  = dequantize_row(token embedding)                 src/runtime.c:108-113
//   per layer:
//     xb = rmsnorm_ref(x, rms_att)                        src/kernels.c:170-180
//     q, k, v = Wq xb, Wk xb, Wv xb     (matmul_q)         src/runtime.c:124-126
//     apply_rope(q, k)                                     src/runtime.c:19-41
//     K[pos], V[pos] = k, v             (fp32 or Q8_0 rows)
//     att[h][t] = dot_ref(q_h, K[t]_h) / sqrt(head_dim)    src/runtime.c:136-160
//     att[h] = softmax_ref(att[h])                         src/runtime.c:162-168
//     o_h[i] = sum over t, in order, of att[h][t] V[t]_h[i] src/runtime.c:170-193
//     x += Wo o;  xb = rmsnorm_ref(x, rms_ffn)             src/runtime.c:195-200
//     x += MoE(xb)                                         src/runtime.c:202-269
//   logits = wcls rmsnorm_ref(x, rms_final)               src/runtime.c:286-287
//
// The sums the reference forms one term at a time (rmsnorm's sum of squares,
// softmax's denominator, each attention output element over the positions)
// are formed the same way here: one lane adds the terms in order, while other
// lanes produce the terms (squares, exponentials, attention-weighted values)
// into LDS ahead of it.  The cos / sin of RoPE come from a table the decoder
// builds at set-up with the host C library's powf / cosf / sinf, the
// functions apply_rope calls, for every position of the cache.
#include <cmath>
#include <cstring>
#include <vector>

#include "qr_common.h"
#include "qr_ggml_elem.h"
#include "qr_internal.h"
#include "qr_norm.h"

namespace qr {

// ---------------------------------------------------------------------------
// Element e of a row of `type` (dequantize_row, src/quant.c:160-240; a
// llama.cpp-layout K-quant row through ggml's dequantize_row_q*_K).
// ---------------------------------------------------------------------------
__device__ inline float deq_elem(const uint8_t* __restrict__ row, int type, int e) {
  if (type & QR_GGML) return ggml_deq_elem(row, type & ~(int)QR_GGML, e);
  if (type == QR_T_F32) return reinterpret_cast<const float*>(row)[e];
  if (type == QR_T_Q8_0) {
    const uint8_t* b = row + (size_t)(e >> 5) * QR_Q8_BYTES;
    const float d = qr_h2f((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    return (float)(int8_t)b[2 + (e & 31)] * d;
  }
  const int i = e >> 8, j = (e & 255) >> 5, l = e & 31;
  if (type == QR_T_Q6_K) {
    const uint8_t* b = row + (size_t)i * QR_Q6K_BYTES;
    const float d = qr_h2f((uint32_t)b[208] | ((uint32_t)b[209] << 8));
    const float sc = (float)(int8_t)b[192 + j] * d;
    const int ql = (b[(j * 32 + l) >> 1] >> ((l & 1) * 4)) & 0xF;
    const int qh = (b[128 + ((j * 32 + l) >> 2)] >> (((j * 32 + l) & 3) * 2)) & 3;
    return (float)((ql | (qh << 4)) - 32) * sc;
  }
  // Q4_K / Q5_K
  const int bb = type == QR_T_Q4_K ? QR_Q4K_BYTES : QR_Q5K_BYTES;
  const uint8_t* b = row + (size_t)i * bb;
  const float d = qr_h2f((uint32_t)b[0] | ((uint32_t)b[1] << 8));
  const float dmin = qr_h2f((uint32_t)b[2] | ((uint32_t)b[3] << 8));
  const float sc = (float)(b[4 + j] & 63) * d;
  const float m = (float)(b[4 + j] >> 6) * dmin;
  const int qs0 = type == QR_T_Q4_K ? 16 : 48;
  int q = (b[qs0 + ((j * 32 + l) >> 1)] >> ((l & 1) * 4)) & 0xF;
  if (type == QR_T_Q5_K) q |= ((b[16 + ((j * 32 + l) >> 3)] >> ((j * 32 + l) & 7)) & 1) << 4;
  return (float)q * sc - m;
}

// out[r][e] = element e of row r (nrows rows of row_bytes; whole blocks of n;
// unknown types give zeros, as dequantize_row does).
__global__ __launch_bounds__(256) void k_dequant_rows(const uint8_t* __restrict__ src, int type,
                                                      size_t row_bytes, int nrows, int n,
                                                      float* __restrict__ out) {
  const long total = (long)nrows * n;
  for (long gi = (long)blockIdx.x * blockDim.x + threadIdx.x; gi < total;
       gi += (long)gridDim.x * blockDim.x) {
    const int r = (int)(gi / n), e = (int)(gi - (long)r * n);
    const bool known = type == QR_T_F32 || type == QR_T_Q8_0 || type == QR_T_Q4_K ||
                       type == QR_T_Q5_K || type == QR_T_Q6_K;
    out[gi] = known ? deq_elem(src + (size_t)r * row_bytes, type, e) : 0.0f;
  }
}

// The embedding row of the state's token (src/runtime.c:108-113); workgroup
// t takes token t of a batch (state st[2 t], row x + t n).
__global__ __launch_bounds__(256) void k_embed(const uint8_t* __restrict__ tab, int type,
                                               size_t row_bytes, const int32_t* __restrict__ st,
                                               int n, float* __restrict__ x) {
  const int token = st[2 * blockIdx.x];
  x += (size_t)blockIdx.x * n;
  const uint8_t* row = tab + (size_t)token * row_bytes;
  for (int e = threadIdx.x; e < n; e += blockDim.x) x[e] = deq_elem(row, type, e);
}

// ---------------------------------------------------------------------------
// Sequential sums.  The reference adds n terms one at a time (rmsnorm's sum
// of squares, softmax's denominator, each attention value); the decode step
// does the same, the terms produced in parallel beforehand: one whole wave
// for a single sum (seq_sum_wave, qr_common.h: the terms in registers, the
// running sum passed lane to lane), one lane per attention element for the
// value sums (read from LDS 32 adds ahead of their use).

// ---------------------------------------------------------------------------
// rmsnorm_ref (src/kernels.c:170-180), optionally after x += add (the
// residual of src/runtime.c:196-198).  Every thread loads its share of x (and
// add, w) at once, the squares go to LDS, wave 0 adds them in order, the
// workgroup scales from registers.  n <= kNormMax; VEC: n % 4 == 0.
// Workgroup r normalizes row r of a batch (x, add, o advanced by r n).
// ---------------------------------------------------------------------------
constexpr int kNormMax = 8192;
constexpr int kNormThreads = 512;
constexpr int kNormPer = kNormMax / 4 / kNormThreads;  // float4 per thread

template <bool VEC>
__global__ __launch_bounds__(kNormThreads) void k_rmsnorm(float* __restrict__ x,
                                                          const float* __restrict__ add,
                                                          const float* __restrict__ w, int n,
                                                          float* __restrict__ o) {
  __shared__ __align__(16) float sq[kNormMax];
  __shared__ float scale_s;
  x += (size_t)blockIdx.x * n;
  o += (size_t)blockIdx.x * n;
  if (add) add += (size_t)blockIdx.x * n;
  if constexpr (VEC) {
    const int n4 = n >> 2;
    float4* x4 = reinterpret_cast<float4*>(x);
    float4 xv[kNormPer], wv[kNormPer], av[kNormPer];
#pragma unroll
    for (int j = 0; j < kNormPer; j++) {
      const int i4 = threadIdx.x + j * kNormThreads;
      if (i4 < n4) {
        xv[j] = x4[i4];
        wv[j] = reinterpret_cast<const float4*>(w)[i4];
        if (add) av[j] = reinterpret_cast<const float4*>(add)[i4];
      }
    }
#pragma unroll
    for (int j = 0; j < kNormPer; j++) {
      const int i4 = threadIdx.x + j * kNormThreads;
      if (i4 < n4) {
        if (add) {
          xv[j].x = xv[j].x + av[j].x;
          xv[j].y = xv[j].y + av[j].y;
          xv[j].z = xv[j].z + av[j].z;
          xv[j].w = xv[j].w + av[j].w;
          x4[i4] = xv[j];
        }
        float4 q;
        q.x = xv[j].x * xv[j].x;
        q.y = xv[j].y * xv[j].y;
        q.z = xv[j].z * xv[j].z;
        q.w = xv[j].w * xv[j].w;
        reinterpret_cast<float4*>(sq)[i4] = q;
      }
    }
    __syncthreads();
    if (threadIdx.x < 64) {  // wave 0
      const float ss = seq_sum_wave<64>(sq, n, (int)threadIdx.x);
      if (threadIdx.x == 0) scale_s = rms_scale(ss, n);
    }
    __syncthreads();
    const float scale = scale_s;
#pragma unroll
    for (int j = 0; j < kNormPer; j++) {
      const int i4 = threadIdx.x + j * kNormThreads;
      if (i4 < n4) {
        float4 r;
        r.x = wv[j].x * (xv[j].x * scale);
        r.y = wv[j].y * (xv[j].y * scale);
        r.z = wv[j].z * (xv[j].z * scale);
        r.w = wv[j].w * (xv[j].w * scale);
        reinterpret_cast<float4*>(o)[i4] = r;
      }
    }
  } else {
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      float xi = x[i];
      if (add) {
        xi = xi + add[i];
        x[i] = xi;
      }
      sq[i] = xi * xi;
    }
    __syncthreads();
    if (threadIdx.x < 64) {  // wave 0
      const float ss = seq_sum_wave<64>(sq, n, (int)threadIdx.x);
      if (threadIdx.x == 0) scale_s = rms_scale(ss, n);
    }
    __syncthreads();
    const float scale = scale_s;
    for (int i = threadIdx.x; i < n; i += blockDim.x) o[i] = w[i] * (x[i] * scale);
  }
}

hipError_t rmsnorm_launch(float* x, const float* add, const float* w, int n, float* o,
                          hipStream_t s, int rows = 1) {
  const bool vec = (n & 3) == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                                     reinterpret_cast<uintptr_t>(o) |
                                     reinterpret_cast<uintptr_t>(add)) & 15) == 0;
  if (vec)
    hipLaunchKernelGGL(k_rmsnorm<true>, dim3(rows), dim3(kNormThreads), 0, s, x, add, w, n, o);
  else
    hipLaunchKernelGGL(k_rmsnorm<false>, dim3(rows), dim3(kNormThreads), 0, s, x, add, w, n, o);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// apply_rope (src/runtime.c:19-41) of q (qd) and k (the first kvd of its
// pairs) with the position's cos / sin, then the K and V rows of the
// position: fp32 copies or quantize_row_q8_0 (src/quant.c:143-158) blocks.
// ---------------------------------------------------------------------------

__device__ inline void q8_block_store(const float* __restrict__ v, uint8_t* __restrict__ out) {
  float amax = 0.0f;
  for (int j = 0; j < 32; j++) {
    const float av = __builtin_fabsf(v[j]);
    amax = av > amax ? av : amax;
  }
  const float dd = amax / 127.0f;
  const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
  const uint32_t dh = qr_f2h(dd);
  out[0] = (uint8_t)(dh & 0xFFu);
  out[1] = (uint8_t)(dh >> 8);
  for (int j = 0; j < 32; j++) out[2 + j] = (uint8_t)(int8_t)(int)__builtin_rintf(v[j] * id);
}

// Where position t's row of one layer's K or V cache lives: pages of `page`
// positions, logical page t / page at physical page ptab[t / page].
struct KvView {
  const uint8_t* base;  // K or V pages
  const int32_t* ptab;  // this layer's page table
  int page;             // a power of two
  int page_shift;       // log2(page)
  size_t row_bytes;
  int kv_type;
  __device__ const uint8_t* row(int t) const {
    const int pp = ptab[t >> page_shift];
    return base + (((size_t)pp << page_shift) + (size_t)(t & (page - 1))) * row_bytes;
  }
};

// One 32-element block of a position's row as kv_cache_type 1 stores it: each
// value by the reference's truncating fp32_to_fp16 (src/runtime.c:74-79),
// written as four 16-byte stores.
__device__ inline void f16_block_store(const float* vals, uint8_t* dst) {
  uint4* d4 = reinterpret_cast<uint4*>(dst);
#pragma unroll
  for (int j = 0; j < 4; j++) {
    uint4 w;
    w.x = qr_f2h(vals[8 * j]) | (qr_f2h(vals[8 * j + 1]) << 16);
    w.y = qr_f2h(vals[8 * j + 2]) | (qr_f2h(vals[8 * j + 3]) << 16);
    w.z = qr_f2h(vals[8 * j + 4]) | (qr_f2h(vals[8 * j + 5]) << 16);
    w.w = qr_f2h(vals[8 * j + 6]) | (qr_f2h(vals[8 * j + 7]) << 16);
    d4[j] = w;
  }
}

// Element col of a cache row as the attention reads it (kv_get_element,
// src/runtime.c:87-92, for fp32 and fp16 rows; qs * d for Q8_0 rows).
template <int KVT>
__device__ inline float kv_value(const uint8_t* row, int col) {
  if constexpr (KVT == QR_KV_Q8_0) {
    const uint8_t* blk = row + (size_t)(col >> 5) * QR_Q8_BYTES;
    return (float)(int8_t)blk[2 + (col & 31)] * qr_h2f(*reinterpret_cast<const uint16_t*>(blk));
  } else if constexpr (KVT == QR_KV_F16) {
    return qr_h2f(reinterpret_cast<const uint16_t*>(row)[col]);
  } else {
    return reinterpret_cast<const float*>(row)[col];
  }
}

// npos = st[1] + 1 when the position comes from device state (a captured
// decode step), else the argument.
__device__ inline int npos_of(const int32_t* st, int npos) { return st ? st[1] + 1 : npos; }

// One thread per q pair (threads 0 .. qd/2 - 1), then one per 32-element
// block of k and of v (2 kvd / 32 threads): k's pairs rotate in registers,
// then the block is stored as fp32 or as a quantize_row_q8_0 block.  grid
// (ceil((qd / 2 + 2 kvd / 32) / 256), tokens): blockIdx.y takes token t of a
// batch (q + t qd, k and v + t kvd, state st[2 t]).
__global__ __launch_bounds__(256) void k_rope_kv(float* __restrict__ q, const float* __restrict__ k,
                                                 const float* __restrict__ v,
                                                 const float* __restrict__ rope,
                                                 const int32_t* __restrict__ st, int qd, int kvd,
                                                 KvView K, uint8_t* __restrict__ vbase) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  q += (size_t)blockIdx.y * qd;
  k += (size_t)blockIdx.y * kvd;
  v += (size_t)blockIdx.y * kvd;
  const int pos = st[2 * blockIdx.y + 1];
  const float* cs = rope + (size_t)pos * qd;
  const int np = qd >> 1, nb = kvd >> 5;
  if (g < np) {
    const float2 c2 = reinterpret_cast<const float2*>(cs)[g];
    const float2 q2 = reinterpret_cast<const float2*>(q)[g];
    float2 r;
    r.x = q2.x * c2.x - q2.y * c2.y;
    r.y = q2.x * c2.y + q2.y * c2.x;
    reinterpret_cast<float2*>(q)[g] = r;
    return;
  }
  const int b = g - np;
  if (b >= 2 * nb) return;
  const bool isv = b >= nb;
  const int bi = isv ? b - nb : b;
  float vals[32];
  const float4* src = reinterpret_cast<const float4*>((isv ? v : k) + 32 * bi);
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const float4 f = src[j];
    vals[4 * j] = f.x;
    vals[4 * j + 1] = f.y;
    vals[4 * j + 2] = f.z;
    vals[4 * j + 3] = f.w;
  }
  if (!isv) {
    const float4* c4 = reinterpret_cast<const float4*>(cs + 32 * bi);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float4 c = c4[j];  // cos, sin of two pairs
      const float k0 = vals[4 * j], k1 = vals[4 * j + 1], k2 = vals[4 * j + 2], k3 = vals[4 * j + 3];
      vals[4 * j] = k0 * c.x - k1 * c.y;
      vals[4 * j + 1] = k0 * c.y + k1 * c.x;
      vals[4 * j + 2] = k2 * c.z - k3 * c.w;
      vals[4 * j + 3] = k2 * c.w + k3 * c.z;
    }
  }
  uint8_t* krow = const_cast<uint8_t*>(K.row(pos));
  uint8_t* row = isv ? vbase + (size_t)(krow - K.base) : krow;
  if (K.kv_type == QR_KV_Q8_0) {
    q8_block_store(vals, row + (size_t)bi * QR_Q8_BYTES);
  } else if (K.kv_type == QR_KV_F16) {
    f16_block_store(vals, row + (size_t)bi * 64);
  } else {
    float4* dst = reinterpret_cast<float4*>(reinterpret_cast<float*>(row) + 32 * bi);
#pragma unroll
    for (int j = 0; j < 8; j++)
      dst[j] = make_float4(vals[4 * j], vals[4 * j + 1], vals[4 * j + 2], vals[4 * j + 3]);
  }
}

// Rows [t0, t0 + n) of one layer's K and V caches from fp32 values
// (src [n][kvd]): fp32 copies, truncated halves or quantize_row_q8_0 blocks.
// One thread per 32-element block.
__global__ __launch_bounds__(256) void k_kv_write(const float* __restrict__ ksrc,
                                                  const float* __restrict__ vsrc, int t0, int n,
                                                  int kvd, KvView K, uint8_t* __restrict__ vbase) {
  const int nb = kvd / 32;
  const long total = 2L * n * nb;
  for (long g = (long)blockIdx.x * blockDim.x + threadIdx.x; g < total;
       g += (long)gridDim.x * blockDim.x) {
    const bool isv = g >= (long)n * nb;
    const long r = isv ? g - (long)n * nb : g;
    const int t = (int)(r / nb), b = (int)(r - (long)t * nb);
    const float* src = (isv ? vsrc : ksrc) + (size_t)t * kvd + 32 * b;
    uint8_t* krow = const_cast<uint8_t*>(K.row(t0 + t));
    uint8_t* row = isv ? vbase + (size_t)(krow - K.base) : krow;
    if (K.kv_type == QR_KV_Q8_0 || K.kv_type == QR_KV_F16) {
      float vals[32];
      for (int j = 0; j < 32; j++) vals[j] = src[j];
      if (K.kv_type == QR_KV_Q8_0) q8_block_store(vals, row + (size_t)b * QR_Q8_BYTES);
      else f16_block_store(vals, row + (size_t)b * 64);
    } else {
      float* dst = reinterpret_cast<float*>(row) + 32 * b;
      for (int j = 0; j < 32; j++) dst[j] = src[j];
    }
  }
}

// ---------------------------------------------------------------------------
// Attention (src/runtime.c:136-193).
// ---------------------------------------------------------------------------
constexpr int kHdMax = 512;          // the reference's own bound (kh_buf[512], src/runtime.c:145)
constexpr size_t kDecLdsMax = 160 * 1024;

// att[h][t] = dot_ref(q_h, K[t]_kvh) * inv_sqrt for the kv_mul query heads of
// kv head blockIdx.y and positions [64 blockIdx.x, +64): the K tile is
// dequantized once into LDS (rows padded to hd + 4 floats), then one thread
// per (head, position) adds the hd products in order; a thread runs the
// chains of heads m and m + 4 side by side, which share the K row.  Dynamic
// LDS: (64 (hd + 4) + kv_mul hd) floats.
//
// ROPE (the decode step, one token): q and k arrive unrotated and this
// kernel does k_rope_kv's work as well -- each workgroup rotates its query
// heads while staging them, and the workgroup whose tile holds the current
// position rotates kv head blockIdx.y's k, stores its K and V blocks in the
// cache rows of that position and puts the K row (as the cache holds it) in
// its LDS tile directly.
constexpr int kScTile = 64;

struct RopeArgs {
  const float* rope;  // [cap][q_dim] (cos, sin) pairs
  const float* k;     // [kv_dim] unrotated
  const float* v;     // [kv_dim]
  uint8_t* vbase;     // V pages (same layout as K's)
  int qd;
};

template <bool ROPE>
__global__ __launch_bounds__(256) void k_attn_scores(const float* __restrict__ q, KvView K,
                                                     const int32_t* __restrict__ st, int npos_arg,
                                                     int kv_mul, int hd, float inv_sqrt,
                                                     int att_stride, float* __restrict__ att,
                                                     RopeArgs R) {
  extern __shared__ __align__(16) float sm[];
  // blockIdx.z: token t of a batch (q + t n_heads hd, att + t n_heads att_stride, st + 2 t)
  const int nh = gridDim.y * kv_mul;
  q += (size_t)blockIdx.z * nh * hd;
  att += (size_t)blockIdx.z * nh * att_stride;
  if (st) st += 2 * blockIdx.z;
  const int npos = npos_of(st, npos_arg);
  const int t0 = blockIdx.x * kScTile;
  if (t0 >= npos) return;
  const int kvh = blockIdx.y;
  const int ks = hd + 4;
  float* kt = sm;
  float* qs = sm + kScTile * ks;
  const int nt = min(kScTile, npos - t0);
  // ROPE: the current position's row within this tile, else -1
  const int cur = ROPE ? npos - 1 - t0 : -1;
  const float* cs = ROPE ? R.rope + (size_t)(npos - 1) * R.qd : nullptr;
  for (int i = threadIdx.x * 4; i < kv_mul * hd; i += blockDim.x * 4) {
    const size_t e = (size_t)kvh * kv_mul * hd + i;
    float4 a = *reinterpret_cast<const float4*>(q + e);
    if constexpr (ROPE) {  // k_rope_kv's rotation of two pairs
      const float4 c = *reinterpret_cast<const float4*>(cs + e);
      const float4 r = a;
      a.x = r.x * c.x - r.y * c.y;
      a.y = r.x * c.y + r.y * c.x;
      a.z = r.z * c.z - r.w * c.w;
      a.w = r.z * c.w + r.w * c.z;
    }
    *reinterpret_cast<float4*>(qs + i) = a;
  }
  if (ROPE && cur >= 0 && cur < kScTile && (int)threadIdx.x < 2 * (hd / 32)) {
    // block b of kv head kvh's k (rotated) or v, at the current position
    const int nbh = hd / 32;
    const bool isv = (int)threadIdx.x >= nbh;
    const int b = isv ? (int)threadIdx.x - nbh : (int)threadIdx.x;
    const size_t e = (size_t)kvh * hd + 32 * b;
    float vals[32];
    const float4* src = reinterpret_cast<const float4*>((isv ? R.v : R.k) + e);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float4 f = src[j];
      vals[4 * j] = f.x;
      vals[4 * j + 1] = f.y;
      vals[4 * j + 2] = f.z;
      vals[4 * j + 3] = f.w;
    }
    if (!isv) {
      const float4* c4 = reinterpret_cast<const float4*>(cs + e);
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const float4 c = c4[j];
        const float k0 = vals[4 * j], k1 = vals[4 * j + 1], k2 = vals[4 * j + 2], k3 = vals[4 * j + 3];
        vals[4 * j] = k0 * c.x - k1 * c.y;
        vals[4 * j + 1] = k0 * c.y + k1 * c.x;
        vals[4 * j + 2] = k2 * c.z - k3 * c.w;
        vals[4 * j + 3] = k2 * c.w + k3 * c.z;
      }
    }
    uint8_t* krow = const_cast<uint8_t*>(K.row(npos - 1));
    uint8_t* row = isv ? R.vbase + (size_t)(krow - K.base) : krow;
    float* dst = kt + cur * ks + 32 * b;
    if (K.kv_type == QR_KV_Q8_0) {
      uint8_t* blk = row + (size_t)(kvh * nbh + b) * QR_Q8_BYTES;
      q8_block_store(vals, blk);
      if (!isv) {  // the row as the cache holds it
        const float d = qr_h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
#pragma unroll
        for (int j = 0; j < 32; j++) dst[j] = (float)(int8_t)blk[2 + j] * d;
      }
    } else if (K.kv_type == QR_KV_F16) {
      f16_block_store(vals, row + (size_t)(kvh * nbh + b) * 64);
      if (!isv) {
#pragma unroll
        for (int j = 0; j < 32; j++) dst[j] = qr_h2f(qr_f2h(vals[j]));
      }
    } else {
      float* out = reinterpret_cast<float*>(row) + (size_t)kvh * hd + 32 * b;
#pragma unroll
      for (int j = 0; j < 32; j++) {
        out[j] = vals[j];
        if (!isv) dst[j] = vals[j];
      }
    }
  }
  if (K.kv_type == QR_KV_Q8_0) {
    const int bpr = hd / 32;
    for (int j = threadIdx.x; j < nt * bpr; j += blockDim.x) {
      const int tt = j / bpr, b = j - tt * bpr;
      if (ROPE && tt == cur) continue;  // staged above
      const uint16_t* hw =
          reinterpret_cast<const uint16_t*>(K.row(t0 + tt) + (size_t)(kvh * bpr + b) * QR_Q8_BYTES);
      uint32_t u[17];
#pragma unroll
      for (int w = 0; w < 17; w++) u[w] = hw[w];
      const float d = qr_h2f(u[0]);
      float* dst = kt + tt * ks + 32 * b;
#pragma unroll
      for (int w = 0; w < 8; w++) {
        float4 f;
        f.x = (float)(int8_t)(u[1 + 2 * w] & 0xFFu) * d;
        f.y = (float)(int8_t)(u[1 + 2 * w] >> 8) * d;
        f.z = (float)(int8_t)(u[2 + 2 * w] & 0xFFu) * d;
        f.w = (float)(int8_t)(u[2 + 2 * w] >> 8) * d;
        *reinterpret_cast<float4*>(dst + 4 * w) = f;
      }
    }
  } else if (K.kv_type == QR_KV_F16) {
    for (int j = threadIdx.x * 4; j < nt * hd; j += blockDim.x * 4) {
      const int tt = j / hd, i = j - tt * hd;
      if (ROPE && tt == cur) continue;  // staged above
      const uint2 w = *reinterpret_cast<const uint2*>(
          reinterpret_cast<const uint16_t*>(K.row(t0 + tt)) + (size_t)kvh * hd + i);
      float4 f;
      f.x = qr_h2f(w.x & 0xFFFFu);
      f.y = qr_h2f(w.x >> 16);
      f.z = qr_h2f(w.y & 0xFFFFu);
      f.w = qr_h2f(w.y >> 16);
      *reinterpret_cast<float4*>(kt + tt * ks + i) = f;
    }
  } else {
    for (int j = threadIdx.x * 4; j < nt * hd; j += blockDim.x * 4) {
      const int tt = j / hd, i = j - tt * hd;
      if (ROPE && tt == cur) continue;  // staged above
      *reinterpret_cast<float4*>(kt + tt * ks + i) = *reinterpret_cast<const float4*>(
          reinterpret_cast<const float*>(K.row(t0 + tt)) + (size_t)kvh * hd + i);
    }
  }
  __syncthreads();
  const int P = kv_mul * kScTile;
  for (int p = threadIdx.x; p < P; p += 2 * blockDim.x) {
    const int m = p / kScTile, tt = p - m * kScTile;
    const bool two = p + (int)blockDim.x < P;  // head m + 4, same position
    const float* kr = kt + tt * ks;
    const float* q0 = qs + m * hd;
    const float* q1 = q0 + 4 * hd;
    float s0 = 0.0f, s1 = 0.0f;
    if (two) {
      for (int i = 0; i < hd; i += 4) {
        const float4 kv = *reinterpret_cast<const float4*>(kr + i);
        const float4 a = *reinterpret_cast<const float4*>(q0 + i);
        const float4 c = *reinterpret_cast<const float4*>(q1 + i);
        s0 += a.x * kv.x;
        s1 += c.x * kv.x;
        s0 += a.y * kv.y;
        s1 += c.y * kv.y;
        s0 += a.z * kv.z;
        s1 += c.z * kv.z;
        s0 += a.w * kv.w;
        s1 += c.w * kv.w;
      }
    } else {
      for (int i = 0; i < hd; i += 4) {
        const float4 kv = *reinterpret_cast<const float4*>(kr + i);
        const float4 a = *reinterpret_cast<const float4*>(q0 + i);
        s0 += a.x * kv.x;
        s0 += a.y * kv.y;
        s0 += a.z * kv.z;
        s0 += a.w * kv.w;
      }
    }
    if (tt < nt) {
      att[(size_t)(kvh * kv_mul + m) * att_stride + t0 + tt] = s0 * inv_sqrt;
      if (two) att[(size_t)(kvh * kv_mul + m + 4) * att_stride + t0 + tt] = s1 * inv_sqrt;
    }
  }
}

// softmax_ref (src/kernels.c:191-207) of one head's scores, then
// o_h[c] = sum over t = 0 .. npos-1, in order, of att[h][t] * V[t]_kvh[c]
// (src/runtime.c:182-190: each product rounded, then added), for kValCols
// elements c of head blockIdx.y.  grid (hd / kValCols, n_heads), 512 threads.
//
//  1. The scores go to LDS; their max over the workgroup (a max is exact, so
//     its order does not matter; seeded with the first score, strict '>');
//     the exponentials in parallel, in place.
//  2. Lane 0 adds the exponentials in order (the softmax denominator) while
//     waves 1, 2, 3 and 5 start loading the V values of the first two
//     position blocks.
//  3. Waves 1, 2, 3 and 5 form the products (e[t] * inv) * v of a block of kValBlk
//     positions into LDS, element-major (one ds_read_b128 gives an element
//     four consecutive positions), while lanes 0..31 of wave 0 add the
//     previous block's products in position order.  Each block's V loads are
//     issued two blocks ahead of their use.  Waves 4, 6 and 7 only help in
//     step 1.
// Dynamic LDS: npos floats (the exponentials), then ceil(npos / page) ints
// (this layer's page table).  att is only read.
constexpr int kValCols = 32;
constexpr int kValBlk = 256;
constexpr int kValPitch = kValBlk + 4;
constexpr int kSvThreads = 512;
constexpr int kAttnMaxPos = 22528;  // exponentials (LDS) beside the product buffers

// Producer threads (four waves) take position pid of a block: the raw V
// values of their kValCols elements.
constexpr int kSvProd = 256;
constexpr int kSvPer = kValBlk / kSvProd;
struct SvRegs {
  uint32_t r[kSvPer][kValCols];  // Q8_0: [0] = d, [1..8] = the 32 qs bytes; fp16: [0..15] =
                                 // the 32 halves in pairs; fp32: the values
};

// V.row(t) with the page table read from LDS (pt), so that a row's address
// does not wait on a global load.
__device__ inline const uint8_t* kv_row_lds(const KvView& V, const int32_t* pt, int t) {
  return V.base + (((size_t)pt[t >> V.page_shift] << V.page_shift) + (size_t)(t & (V.page - 1))) *
                      V.row_bytes;
}

// Every producer loads (positions past the end read the last row and are
// ignored): with no branch around them the loads' count is static, so a later
// use waits only for its own loads.
template <int KVT>
__device__ inline void sv_load(SvRegs& R, const KvView& V, const int32_t* pt, int b, int npos,
                               int pid, int kvh, int hd, int c0) {
  const int e0 = kvh * hd + c0;
#pragma unroll
  for (int u = 0; u < kSvPer; u++) {
    const int t = min(b * kValBlk + pid + u * kSvProd, npos - 1);
    const uint8_t* row = kv_row_lds(V, pt, t);
    if constexpr (KVT == QR_KV_Q8_0) {
      const uint8_t* blk = row + (size_t)(e0 >> 5) * QR_Q8_BYTES;
      R.r[u][0] = *reinterpret_cast<const uint16_t*>(blk);
      __builtin_memcpy(&R.r[u][1], blk + 2, 32);  // 2-byte aligned
    } else if constexpr (KVT == QR_KV_F16) {
      const uint4* f = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(row) + e0);
#pragma unroll
      for (int j = 0; j < kValCols / 8; j++) {
        const uint4 w = f[j];
        R.r[u][4 * j] = w.x;
        R.r[u][4 * j + 1] = w.y;
        R.r[u][4 * j + 2] = w.z;
        R.r[u][4 * j + 3] = w.w;
      }
    } else {
      const uint4* f = reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(row) + e0);
#pragma unroll
      for (int j = 0; j < kValCols / 4; j++) {
        const uint4 w = f[j];
        R.r[u][4 * j] = w.x;
        R.r[u][4 * j + 1] = w.y;
        R.r[u][4 * j + 2] = w.z;
        R.r[u][4 * j + 3] = w.w;
      }
    }
  }
}

template <int KVT>
__device__ inline void sv_produce(const SvRegs& R, int b, int npos, int pid,
                                  const float* __restrict__ e, float inv, float* __restrict__ pb) {
#pragma unroll
  for (int u = 0; u < kSvPer; u++) {
    const int tt = pid + u * kSvProd;
    const int t = b * kValBlk + tt;
    const float at = t < npos ? e[t] * inv : 0.0f;  // softmax_ref's x[i] *= inv
    if constexpr (KVT == QR_KV_Q8_0) {
      const float d = qr_h2f(R.r[u][0]);
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const uint32_t w = R.r[u][1 + j];
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const float v = (float)(int8_t)((w >> (8 * q)) & 0xFFu) * d;
          pb[(4 * j + q) * kValPitch + tt] = at * v;
        }
      }
    } else if constexpr (KVT == QR_KV_F16) {
#pragma unroll
      for (int c = 0; c < kValCols; c++)
        pb[c * kValPitch + tt] = at * qr_h2f((R.r[u][c >> 1] >> (16 * (c & 1))) & 0xFFFFu);
    } else {
#pragma unroll
      for (int c = 0; c < kValCols; c++) pb[c * kValPitch + tt] = at * __uint_as_float(R.r[u][c]);
    }
  }
}

__device__ inline void sv_chain(const float* __restrict__ pb, int cnt, float& acc) {
  static_assert(kValBlk == 256, "block of the unrolled sum");
  if (cnt == kValBlk) {
    add256_lds(pb, acc);
  } else {
    for (int tt = 0; tt < cnt; tt++) acc += pb[tt];
  }
}

template <int KVT>
__global__ __launch_bounds__(kSvThreads) void k_attn_sv(const float* __restrict__ att,
                                                        int att_stride,
                                                        KvView V, const int32_t* __restrict__ st,
                                                        int npos_arg, int lds_cap, int kv_mul,
                                                        int hd, float* __restrict__ out) {
  extern __shared__ __align__(16) float e[];
  __shared__ __align__(16) float prod[2][kValCols * kValPitch];
  __shared__ float red[kSvThreads / 64];
  __shared__ float inv_s;
  // blockIdx.z: token t of a batch (att + t n_heads att_stride, out + t n_heads hd, st + 2 t)
  att += (size_t)blockIdx.z * gridDim.y * att_stride;
  out += (size_t)blockIdx.z * gridDim.y * hd;
  if (st) st += 2 * blockIdx.z;
  const int npos = npos_of(st, npos_arg);
  int32_t* pt = reinterpret_cast<int32_t*>(e + lds_cap);
  for (int i = threadIdx.x; i < (npos + V.page - 1) / V.page; i += kSvThreads) pt[i] = V.ptab[i];
  const int h = blockIdx.y;
  const int c0 = blockIdx.x * kValCols;
  const int kvh = h / kv_mul;
  const float* a = att + (size_t)h * att_stride;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // producers: waves 1, 2, 3 and 5 (pid 0..255); wave 4 would share wave 0's
  // SIMD (a workgroup's waves go to the SIMDs in turn) and slow its chain
  const int pw = wave < 4 ? wave - 1 : wave - 2;
  const int pid = pw * 64 + lane;
  const bool producer = wave != 0 && wave != 4 && pid < kSvProd;
  const ExpTab tab = qr_expf_tab();

  // 1. scores -> LDS and their max; eight loads in flight per thread
  float mx = a[0];
  for (int base = 0; base < npos; base += 8 * kSvThreads) {
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = a[min(base + k * kSvThreads + (int)threadIdx.x, npos - 1)];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int i = base + k * kSvThreads + threadIdx.x;
      if (i < npos) {
        e[i] = v[k];
        mx = v[k] > mx ? v[k] : mx;
      }
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float v = __shfl_xor(mx, o);
    mx = v > mx ? v : mx;
  }
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int w = 1; w < kSvThreads / 64; w++) mx = red[w] > mx ? red[w] : mx;
  // every lane runs the same number of rounds (qr_expf_w reads other lanes)
  const int rounds = (npos + kSvThreads - 1) / kSvThreads;
  for (int r = 0; r < rounds; r++) {
    const int i = r * kSvThreads + threadIdx.x;
    const float v = i < npos ? e[i] : 0.0f;
    const float ev = qr_expf_w(v - mx, tab);
    if (i < npos) e[i] = ev;
  }
  __syncthreads();

  // 2. the denominator; the first V loads
  SvRegs A, B;
  if (producer) {
    sv_load<KVT>(A, V, pt, 0, npos, pid, kvh, hd, c0);
    sv_load<KVT>(B, V, pt, 1, npos, pid, kvh, hd, c0);
  } else if (wave == 0) {
    const float den = seq_sum_wave<64>(e, npos, lane);
    if (lane == 0) inv_s = 1.0f / den;
  }
  __syncthreads();
  const float inv = inv_s;

  // 3. products two blocks ahead of the loads, one block ahead of the adds.
  // The adding wave and the producing waves run separate loops that pass
  // the same barriers in the same number (each wave takes one side): the
  // producers' loop then holds only unconditional loads, so each product
  // waits for its own block's loads alone.
  const int nblk = (npos + kValBlk - 1) / kValBlk;
  float acc = 0.0f;
  if (producer) {
    sv_produce<KVT>(A, 0, npos, pid, e, inv, prod[0]);
    sv_load<KVT>(A, V, pt, 2, npos, pid, kvh, hd, c0);
  }
  __syncthreads();
  if (wave == 0) {
    for (int b = 0; b < nblk; b += 2) {
      if (lane < kValCols) sv_chain(prod[0] + lane * kValPitch, min(kValBlk, npos - b * kValBlk), acc);
      __syncthreads();
      if (b + 1 >= nblk) break;
      if (lane < kValCols)
        sv_chain(prod[1] + lane * kValPitch, min(kValBlk, npos - (b + 1) * kValBlk), acc);
      __syncthreads();
    }
  } else if (producer) {
    for (int b = 0; b < nblk; b += 2) {
      sv_produce<KVT>(B, b + 1, npos, pid, e, inv, prod[1]);
      sv_load<KVT>(B, V, pt, b + 3, npos, pid, kvh, hd, c0);
      __syncthreads();
      if (b + 1 >= nblk) break;
      sv_produce<KVT>(A, b + 2, npos, pid, e, inv, prod[0]);
      sv_load<KVT>(A, V, pt, b + 4, npos, pid, kvh, hd, c0);
      __syncthreads();
    }
  } else {
    for (int b = 0; b < nblk; b += 2) {
      __syncthreads();
      if (b + 1 >= nblk) break;
      __syncthreads();
    }
  }
  if (wave == 0 && lane < kValCols) out[(size_t)h * hd + c0 + lane] = acc;
}

// The same attention values for a prompt chunk: many queries (tokens) over
// contexts that are short at first.  Workgroup (head blockIdx.x, token
// blockIdx.y of a batch: att + (t n_heads + h) att_stride, out + (t n_heads +
// h) hd, state st[2 t]); lane c < hd owns output column c and runs its chain
// over the positions itself, reading V straight from the cache (the rows of
// a kv head are shared by its query heads and by the chunk's tokens, so they
// come from L2).  softmax_ref as in k_attn_sv: the max over the workgroup,
// the exponentials in parallel, lane 0 adds them in order; then each
// position's weight e_t * inv once into LDS.  o[c] = sum over t in order of
// (e_t * inv) * v_t[c], each product rounded, then added.  Dynamic LDS:
// lds_cap floats.
template <int KVT>
__global__ __launch_bounds__(512) void k_attn_sv_rows(const float* __restrict__ att,
                                                      int att_stride, KvView V,
                                                      const int32_t* __restrict__ st, int lds_cap,
                                                      int kv_mul, int hd, float* __restrict__ out) {
  extern __shared__ __align__(16) float e[];
  __shared__ float red[8];
  __shared__ float inv_s;
  // the chunk's last token first: its chain is the longest (causal), so the
  // longest workgroups are dispatched first and the short ones fill in
  const int nh = gridDim.x, h = blockIdx.x, z = gridDim.y - 1 - blockIdx.y;
  att += ((size_t)z * nh + h) * att_stride;
  out += ((size_t)z * nh + h) * hd;
  const int npos = st[2 * z + 1] + 1;
  const int nthr = blockDim.x, tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const ExpTab tab = qr_expf_tab();
  float mx = att[0];
  for (int i = tid; i < npos; i += nthr) {
    const float v = att[i];
    e[i] = v;
    mx = v > mx ? v : mx;
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float v = __shfl_xor(mx, o);
    mx = v > mx ? v : mx;
  }
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = red[0];
  for (int w = 1; w < (nthr >> 6); w++) mx = red[w] > mx ? red[w] : mx;
  // every lane runs the same number of rounds (qr_expf_w reads other lanes)
  const int rounds = (npos + nthr - 1) / nthr;
  for (int r = 0; r < rounds; r++) {
    const int i = r * nthr + tid;
    const float v = i < npos ? e[i] : 0.0f;
    const float ev = qr_expf_w(v - mx, tab);
    if (i < npos) e[i] = ev;
  }
  __syncthreads();
  if (tid == 0) inv_s = 1.0f / seq_sum_lds_short(e, npos);
  __syncthreads();
  const float inv = inv_s;
  for (int i = tid; i < npos; i += nthr) e[i] = e[i] * inv;  // softmax_ref's x[i] *= inv
  __syncthreads();
  if (tid >= hd) return;
  const int col = (h / kv_mul) * hd + tid;
  float acc = 0.0f;
  constexpr int U = 32;  // positions whose values are loaded ahead of their adds
  int t = 0;
  // groups of U positions at t % U == 0 lie in one page when U <= page (both
  // powers of two): one page-table read per group, the rows' addresses then
  // known without waiting on a scalar load each
  if (V.page >= U) {
    for (; t + U <= npos; t += U) {
      const uint8_t* row0 = V.row(t);
      float v[U];
#pragma unroll
      for (int u = 0; u < U; u++) {
        v[u] = kv_value<KVT>(row0 + (size_t)u * V.row_bytes, col);
      }
#pragma unroll
      for (int u = 0; u < U; u++) acc += e[t + u] * v[u];
    }
  }
  for (; t + 8 <= npos; t += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      // one address per wave: the page table by scalar loads
      v[u] = kv_value<KVT>(V.row(t + u), col);
    }
#pragma unroll
    for (int u = 0; u < 8; u++) acc += e[t + u] * v[u];
  }
  for (; t < npos; t++) {
    acc += e[t] * kv_value<KVT>(V.row(t), col);
  }
  out[tid] = acc;
}

// The same attention values with the query heads of one kv head together:
// workgroup (kv head blockIdx.x, token blockIdx.y) of kv_mul hd threads,
// thread j hd + c = query head blockIdx.x kv_mul + j, column c.  Each head's softmax runs as in
// k_attn_sv_rows (its max, exponentials, denominator by the head's first
// thread, x *= inv); then the values in groups of kSgGrp positions: the
// group's V values of the kv head are loaded into registers one group ahead,
// dequantized into LDS once per workgroup, and every thread adds
// e_j[t] * v[t][c] in position order -- the chains of k_attn_sv_rows, with
// each V value read from L2 once per kv head instead of once per query head.
// Dynamic LDS: kv_mul rows of ecap floats rounded up to 4 (the
// exponentials), 2 x kSgGrp x hd
// floats (the value tiles), ceil(ecap / page) ints (the page table).
// kv_mul hd threads (a multiple of 64, at most 1024); NPER = kSgGrp / kv_mul
// values per thread and group (kv_mul 4 or 8).
constexpr int kSgGrp = 32;
template <int KVT, int NPER>
__global__ __launch_bounds__(1024) void k_attn_sv_gqa(const float* __restrict__ att,
                                                     int att_stride, KvView V,
                                                     const int32_t* __restrict__ st, int ecap,
                                                     int kv_mul, int hd,
                                                     float* __restrict__ out) {
  extern __shared__ __align__(16) float sm[];
  __shared__ float red[16];
  __shared__ float inv_s[16];
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int wave = tid >> 6, lane = tid & 63;
  // the chunk's last token first: its chains are the longest (causal), so
  // the longest workgroups are dispatched first and the short ones fill in
  const int kvh = blockIdx.x, z = gridDim.y - 1 - blockIdx.y;
  const int nh = gridDim.x * kv_mul;
  const int j = tid / hd, c = tid - j * hd;
  const int h = kvh * kv_mul + j;
  const int wph = hd >> 6;  // waves per head
  const float* a = att + ((size_t)z * nh + h) * att_stride;
  const int npos = st[2 * z + 1] + 1;
  const int es = (ecap + 3) & ~3;  // 16-byte aligned rows (float4 reads)
  float* e = sm + (size_t)j * es;
  float* vs = sm + (size_t)kv_mul * es;  // [2][kSgGrp][hd]
  int32_t* pt = reinterpret_cast<int32_t*>(vs + 2 * kSgGrp * hd);
  const int npg = (npos + V.page - 1) / V.page;
  for (int i = tid; i < npg; i += nthr) pt[i] = V.ptab[i];
  const ExpTab tab = qr_expf_tab();
  float mx = a[0];
  for (int i = c; i < npos; i += hd) {
    const float v = a[i];
    e[i] = v;
    mx = v > mx ? v : mx;
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float v = __shfl_xor(mx, o);
    mx = v > mx ? v : mx;
  }
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = red[j * wph];
  for (int w = 1; w < wph; w++) mx = red[j * wph + w] > mx ? red[j * wph + w] : mx;
  // every lane runs the same number of rounds (qr_expf_w reads other lanes)
  const int rounds = (npos + hd - 1) / hd;
  for (int r = 0; r < rounds; r++) {
    const int i = r * hd + c;
    const float v = i < npos ? e[i] : 0.0f;
    const float ev = qr_expf_w(v - mx, tab);
    if (i < npos) e[i] = ev;
  }
  __syncthreads();
  if (c == 0) inv_s[j] = 1.0f / seq_sum_lds_short(e, npos);
  __syncthreads();
  const float inv = inv_s[j];
  for (int i = c; i < npos; i += hd) e[i] = e[i] * inv;  // softmax_ref's x[i] *= inv
  // (the barrier of the first group below orders these writes before the adds)

  // value k of a group: position g0 + (tid + nthr k) / hd, column (tid + nthr k) % hd
  const size_t col0 = (size_t)kvh * hd;
  uint32_t rq[NPER], rd[NPER];
  auto load = [&](int g0) {
#pragma unroll
    for (int k = 0; k < NPER; k++) {
      const int idx = tid + nthr * k;
      const int u = idx / hd, cc = idx - u * hd;
      const int t = min(g0 + u, npos - 1);  // past the end: reload the last row
      const uint8_t* row = kv_row_lds(V, pt, t);
      if constexpr (KVT == QR_KV_Q8_0) {
        const uint8_t* blk = row + ((col0 + cc) >> 5) * QR_Q8_BYTES;
        rd[k] = *reinterpret_cast<const uint16_t*>(blk);
        rq[k] = (uint32_t)blk[2 + ((col0 + cc) & 31)];
      } else if constexpr (KVT == QR_KV_F16) {
        rq[k] = reinterpret_cast<const uint16_t*>(row)[col0 + cc];
      } else {
        rq[k] = reinterpret_cast<const uint32_t*>(row)[col0 + cc];
      }
    }
  };
  __syncthreads();  // the page table
  load(0);
  float acc = 0.0f;
  int buf = 0;
  for (int g0 = 0; g0 < npos; g0 += kSgGrp) {
    float* vb = vs + buf * kSgGrp * hd;
#pragma unroll
    for (int k = 0; k < NPER; k++) {
      const int idx = tid + nthr * k;
      float v;
      if constexpr (KVT == QR_KV_Q8_0) v = (float)(int8_t)(uint8_t)rq[k] * qr_h2f((uint16_t)rd[k]);
      else if constexpr (KVT == QR_KV_F16) v = qr_h2f(rq[k]);
      else v = __uint_as_float(rq[k]);
      vb[idx] = v;  // [u][cc] = idx
    }
    __syncthreads();
    if (g0 + kSgGrp < npos) load(g0 + kSgGrp);
    const int n = min(kSgGrp, npos - g0);
    if (n == kSgGrp) {
#pragma unroll
      for (int u = 0; u < kSgGrp; u++) acc += e[g0 + u] * vb[u * hd + c];
    } else {
      for (int u = 0; u < n; u++) acc += e[g0 + u] * vb[u * hd + c];
    }
    buf ^= 1;
  }
  out[((size_t)z * nh + h) * hd + c] = acc;
}

// Whether k_attn_sv_gqa takes a chunk whose positions stop below ecap.
inline size_t sv_gqa_lds(int ecap, int kv_mul, int hd, int page) {
  return ((size_t)kv_mul * ((ecap + 3) & ~3) + 2 * (size_t)kSgGrp * hd) * 4 +
         (size_t)((ecap + page - 1) / page) * 4;
}
// k_attn_sv_gqa's static LDS (red[16] and inv_s[16]): the dynamic part may
// take only what it leaves of the CU's 160 KiB.
constexpr size_t kSvGqaStatic = 2 * 16 * sizeof(float);
inline bool sv_gqa_ok(int ecap, int kv_mul, int hd, int page) {
  // kv_mul 1 and 2 (16 and 32 values per thread and group) would spill
  return (kv_mul == 4 || kv_mul == 8) && hd % 64 == 0 && kv_mul * hd <= 1024 && ecap >= 1 &&
         sv_gqa_lds(ecap, kv_mul, hd, page) + kSvGqaStatic <= kDecLdsMax;
}
template <int KVT, int NPER>
std::atomic<bool>* gqa_opt() {
  static std::atomic<bool> f[64];
  return f;
}
template <int KVT, int NPER>
hipError_t gqa_launch(dim3 g, int threads, size_t lds, hipStream_t s, const float* att,
                      int att_stride, const KvView& V, const int32_t* st, int ecap, int kv_mul,
                      int hd, float* out) {
  if (lds > 64 * 1024) {
    const hipError_t e = lds_opt_in((const void*)k_attn_sv_gqa<KVT, NPER>, gqa_opt<KVT, NPER>());
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((k_attn_sv_gqa<KVT, NPER>), g, dim3(threads), lds, s, att, att_stride, V, st,
                     ecap, kv_mul, hd, out);
  return hipGetLastError();
}
template <int KVT>
hipError_t gqa_launch_kv(dim3 g, size_t lds, hipStream_t s, const float* att, int att_stride,
                         const KvView& V, const int32_t* st, int ecap, int kv_mul, int hd,
                         float* out) {
  const int threads = kv_mul * hd;
  if (kv_mul == 8)
    return gqa_launch<KVT, 4>(g, threads, lds, s, att, att_stride, V, st, ecap, kv_mul, hd, out);
  return gqa_launch<KVT, 8>(g, threads, lds, s, att, att_stride, V, st, ecap, kv_mul, hd, out);
}

// ecap: the chunk's positions end (every token's npos <= ecap).
hipError_t sv_rows_launch(const float* att, int att_stride, const KvView& V, const int32_t* st,
                          int lds_cap, int n_heads, int kv_mul, int hd, float* out, int tokens,
                          hipStream_t s, int ecap = 0) {
  if (ecap > 0 && sv_gqa_ok(ecap, kv_mul, hd, V.page)) {
    const dim3 g(n_heads / kv_mul, tokens);
    const size_t l = sv_gqa_lds(ecap, kv_mul, hd, V.page);
    if (V.kv_type == QR_KV_Q8_0)
      return gqa_launch_kv<QR_KV_Q8_0>(g, l, s, att, att_stride, V, st, ecap, kv_mul, hd, out);
    if (V.kv_type == QR_KV_F16)
      return gqa_launch_kv<QR_KV_F16>(g, l, s, att, att_stride, V, st, ecap, kv_mul, hd, out);
    return gqa_launch_kv<QR_KV_F32>(g, l, s, att, att_stride, V, st, ecap, kv_mul, hd, out);
  }
  const dim3 grid(n_heads, tokens);
  const int threads = ((hd + 63) / 64) * 64;
  const size_t lds = (size_t)lds_cap * 4;
  if (V.kv_type == QR_KV_Q8_0)
    hipLaunchKernelGGL(k_attn_sv_rows<QR_KV_Q8_0>, grid, dim3(threads), lds, s, att, att_stride, V,
                       st, lds_cap, kv_mul, hd, out);
  else if (V.kv_type == QR_KV_F16)
    hipLaunchKernelGGL(k_attn_sv_rows<QR_KV_F16>, grid, dim3(threads), lds, s, att, att_stride, V,
                       st, lds_cap, kv_mul, hd, out);
  else
    hipLaunchKernelGGL(k_attn_sv_rows<QR_KV_F32>, grid, dim3(threads), lds, s, att, att_stride, V,
                       st, lds_cap, kv_mul, hd, out);
  return hipGetLastError();
}

// k_attn_sv's dynamic LDS for a cache of cap positions in pages of `page`,
// and whether it fits beside the kernel's static LDS.
inline size_t sv_lds_bytes(int cap, int page) {
  return (size_t)cap * 4 + (size_t)((cap + page - 1) / page) * 4;
}
hipError_t sv_launch(const float* att, int att_stride, const KvView& V, const int32_t* st,
                     int npos, int lds_cap, int n_heads, int kv_mul, int hd, float* out,
                     hipStream_t s, int tokens = 1) {
  const dim3 grid(hd / kValCols, n_heads, tokens);
  const size_t lds = sv_lds_bytes(lds_cap, V.page);
  if (V.kv_type == QR_KV_Q8_0)
    hipLaunchKernelGGL(k_attn_sv<QR_KV_Q8_0>, grid, dim3(kSvThreads), lds, s, att, att_stride, V,
                       st, npos, lds_cap, kv_mul, hd, out);
  else if (V.kv_type == QR_KV_F16)
    hipLaunchKernelGGL(k_attn_sv<QR_KV_F16>, grid, dim3(kSvThreads), lds, s, att, att_stride, V,
                       st, npos, lds_cap, kv_mul, hd, out);
  else
    hipLaunchKernelGGL(k_attn_sv<QR_KV_F32>, grid, dim3(kSvThreads), lds, s, att, att_stride, V,
                       st, npos, lds_cap, kv_mul, hd, out);
  return hipGetLastError();
}

inline bool sv_lds_ok(int cap, int page) {
  const size_t stat = sizeof(float) * (2 * kValCols * kValPitch + kSvThreads / 64 + 1);
  return sv_lds_bytes(cap, page) + stat <= kDecLdsMax;
}

}  // namespace qr

// ===========================================================================
// Host side.
// ===========================================================================
using namespace qr;

struct qr_decoder {
  qr_ctx* ctx = nullptr;
  int device = 0;
  int dim = 0, nh = 0, nkv = 0, hd = 0, nl = 0, vocab = 0, cap = 0;
  int qd = 0, kvd = 0, kv_mul = 0;
  const void* tok_embd = nullptr;
  uint32_t tok_type = 0;
  size_t tok_row = 0;
  const float* rms_final = nullptr;
  const void* wcls = nullptr;
  uint32_t wcls_type = 0;
  std::vector<qr_layer> layers;
  int kv_type = QR_KV_Q8_0, order = QR_ORDER_SEQ, page = 0, ppl = 0, flags = 0;
  size_t row_bytes = 0;
  uint8_t* kc = nullptr;  // K pages, all layers
  uint8_t* vc = nullptr;  // V pages, all layers
  size_t layer_pages_bytes = 0;
  int32_t* ptab = nullptr;  // [layer][ppl]
  float* rope = nullptr;    // [cap][qd]
  int32_t* st = nullptr;    // token, pos
  float *x = nullptr, *xb = nullptr, *xb2 = nullptr, *q = nullptr, *k = nullptr, *v = nullptr;
  float *ao = nullptr, *att = nullptr;
  uint8_t* moe_base = nullptr;  // MoE scratch, carved per layer
  void* mem = nullptr;  // activations, state, page table, RoPE table, MoE scratch
  size_t sc_lds = 0;    // k_attn_scores' dynamic LDS
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  float* graph_logits = nullptr;
  float* graph_xout = nullptr;
  int calls = 0;
  // prefill workspace (the first qr_decoder_prefill allocates it): chunk
  // activations of up to pcap tokens, the prompt's states, MFMA records and
  // dispatch lists, MoE scratch
  void* pmem = nullptr;
  int pcap = 0;
  float *px = nullptr, *pxb = nullptr, *pxb2 = nullptr, *pq = nullptr, *pk = nullptr;
  float *pv = nullptr, *pao = nullptr, *patt = nullptr;
  int32_t* pst = nullptr;   // [cap][2]: token, position of every prompt position
  uint8_t* prec = nullptr;  // activation records [pcap][max(dim, q_dim) / 32]
  int32_t *poff = nullptr, *pperm = nullptr, *ptiles = nullptr;
  uint8_t* pmoe = nullptr;
  const float* prec_src = nullptr;  // the rows prec holds records of (nullptr: none)
  int prec_perm = 0;
  // per layer: the v matrix in the Q6_K / Q8_0 tiled layout when the decode
  // step runs q / k and v in one normalising launch (k_gemv_norm2), else
  // null; row-major v matrices are tiled into wvt (owned) at creation
  std::vector<const void*> wv_tiled;
  std::vector<int> wv_tiled_type;
  uint8_t* wvt = nullptr;
};

namespace {

std::atomic<bool> g_sc_opt[64];
std::atomic<bool> g_sc_opt_r[64];
std::atomic<bool> g_sm_opt[64];
std::atomic<bool> g_sm_opt2[64];
std::atomic<bool> g_sm_opt3[64];
std::atomic<bool> g_rows_opt[64];
std::atomic<bool> g_rows_opt2[64];
std::atomic<bool> g_rows_opt3[64];

#define DEC_HIP(call, what)                                                        \
  do {                                                                             \
    hipError_t e_ = (call);                                                        \
    if (e_ != hipSuccess) return set_error(QR_ERR_HIP, "%s: %s", what, hipGetErrorString(e_)); \
  } while (0)

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

KvView kv_view(const qr_decoder* d, int layer, bool values) {
  KvView K;
  K.base = (values ? d->vc : d->kc) + (size_t)layer * d->layer_pages_bytes;
  K.ptab = d->ptab + (size_t)layer * d->ppl;
  K.page = d->page;
  K.page_shift = __builtin_ctz((unsigned)d->page);
  K.row_bytes = d->row_bytes;
  K.kv_type = d->kv_type;
  return K;
}

// out[n] = W x for one token: matmul_q (src/runtime.c:58-70): fp32 weights
// go through the build's KernelOps.matmul order, quantized ones through the
// fused GEMV with the build's Q8_0 dot order, llama.cpp-layout K-quants
// through ggml's Q8_K dot.
// R (quantized weights only): y = R + W x, the residual add in the GEMV's
// store (y may be R).
hipError_t matmul_q_dev(const void* w, uint32_t type, int order, const float* x, float* y, int n,
                        int dd, hipStream_t s, const float* R = nullptr) {
  if (type == QR_T_F32) {
    if (R) return hipErrorInvalidValue;
    return gemv_f32_launch(order, static_cast<const float*>(w), x, y, n, dd, 1, dd, n, s);
  }
  if (type & QR_GGML)
    return gemv_ggml_launch((int)(type & ~(uint32_t)QR_GGML), w, x, y, n, dd, 1, dd, n, s, R);
  if (type & QR_TILED)
    return gemv_tiled_launch((int)(type & ~(uint32_t)QR_TILED), w, x, y, n, dd, 1, dd, n, s,
                             order, R);
  return gemv_launch((int)type, order, w, x, y, n, dd, 1, dd, n, nullptr, nullptr, s, R);
}

// x += W v in the GEMV's store where the type allows it (every quantized
// layout): true; else the caller adds W v to x itself.
inline bool residual_gemv(uint32_t type) { return type != QR_T_F32; }

// The attention RMSNorm formed inside the q (and k) GEMV's launch
// (qr_norm.h): a tiled Q4_K / Q5_K wq, aligned norm weights and residual.
inline bool norm_in_q(const qr_decoder* d, const qr_layer& L) {
  if (!(L.wq_type & QR_TILED) || (L.wq_type & QR_GGML)) return false;
  const int base = (int)(L.wq_type & ~(uint32_t)QR_TILED);
  return gemv_tiled_norm_ok(base, d->dim) &&
         (reinterpret_cast<uintptr_t>(L.rms_att) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(d->x) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(d->xb) & 15) == 0;
}

// wq and wk as one matrix of qd + kvd rows: the same type and width, wk's
// bytes right after wq's (in the tiled layout, wq a whole number of tiles,
// so the two tilings concatenate into the tiling of the stacked rows), and
// the decoder's k buffer right after q -- one GEMV launch instead of two.
static bool qk_stacked(const qr_decoder* d, const qr_layer& L) {
  if (L.wq_type != L.wk_type || L.wq_type == QR_T_F32 || !L.wq || !L.wk) return false;
  if (d->k != d->q + d->qd) return false;
  const int base = (int)(L.wq_type & ~(uint32_t)(QR_TILED | QR_GGML));
  if ((L.wq_type & QR_TILED) && d->qd % (64 / (d->dim >> 8)) != 0) return false;
  const size_t qbytes = qr_wrow_bytes(base, d->dim) * (size_t)d->qd;
  return static_cast<const uint8_t*>(L.wk) == static_cast<const uint8_t*>(L.wq) + qbytes;
}

// The decode step's kernels, in order, on stream s (the state holds the
// token and the position).
// The dense FFN's SwiGLU (src/runtime.c:278-280): g = silu(u) * g with u the
// w1 (SiLU slot) rows and g the w3 rows.
__global__ __launch_bounds__(256) void k_swiglu(const float* __restrict__ u, float* __restrict__ g,
                                                long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    g[i] = qr_silu(u[i]) * g[i];
}

// x += y (the dense FFN's residual, src/runtime.c:282-284), n a multiple of 4.
__global__ __launch_bounds__(256) void k_add4(float* __restrict__ x, const float* __restrict__ y,
                                              long n4) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (long)gridDim.x * blockDim.x) {
    float4 a = reinterpret_cast<float4*>(x)[i];
    const float4 b = reinterpret_cast<const float4*>(y)[i];
    a.x += b.x;
    a.y += b.y;
    a.z += b.z;
    a.w += b.w;
    reinterpret_cast<float4*>(x)[i] = a;
  }
}

// A layer without experts (moe.n_experts == 0) has the dense SwiGLU FFN of
// forward_runtime (src/runtime.c:270-284): w1 = moe.up (ffn_up, the SiLU
// slot), w3 = moe.gate (ffn_gate), w2 = moe.down (ffn_down).
inline bool is_dense(const qr_layer& L) { return L.moe.n_experts == 0; }

// Its scratch for T tokens: the w1 rows, the w3 rows (then hb) and w2's output.
inline size_t dense_scratch_bytes(const qr_moe_layer& M, int T) {
  return (size_t)T * (2 * (size_t)M.hidden + (size_t)M.dim) * 4;
}

hipError_t enqueue_step(qr_decoder* d, float* logits, float* xout, hipStream_t s) {
  hipError_t e;
  const int dim = d->dim;
  hipLaunchKernelGGL(k_embed, dim3(1), dim3(256), 0, s,
                     static_cast<const uint8_t*>(d->tok_embd), (int)d->tok_type, d->tok_row,
                     d->st, dim, d->x);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const float inv_sqrt = 1.0f / sqrtf((float)d->hd);
  // a layer output not yet added to x (an fp32 down or wo matrix, whose
  // GEMV has no residual store): the next norm adds it
  const float* pend = nullptr;
  for (int l = 0; l < d->nl; l++) {
    const qr_layer& L = d->layers[l];
    const bool stacked = qk_stacked(d, L);
    const bool vdone = !pend && stacked && d->wv_tiled[l] && norm_in_q(d, L);
    if (vdone) {
      // the norm, q / k and v in one launch, xb stored for the rest
      const int base = (int)(L.wq_type & ~(uint32_t)QR_TILED);
      if ((e = gemv_norm2_launch(base, L.wq, d->q, d->qd + d->kvd, d->wv_tiled_type[l],
                                 d->wv_tiled[l], d->v, d->kvd, d->x, L.rms_att, d->xb, dim, s)))
        return e;
    } else if (!pend && norm_in_q(d, L)) {
      // the norm inside the q (and stacked k) launch, xb stored for the rest
      const int base = (int)(L.wq_type & ~(uint32_t)QR_TILED);
      if ((e = gemv_tiled_norm_launch(base, L.wq, d->x, L.rms_att, d->xb, d->q,
                                      stacked ? d->qd + d->kvd : d->qd, dim, s)))
        return e;
      if (!stacked &&
          (e = matmul_q_dev(L.wk, L.wk_type, d->order, d->xb, d->k, d->kvd, dim, s)))
        return e;
    } else {
      if ((e = rmsnorm_launch(d->x, pend, L.rms_att, dim, d->xb, s))) return e;
      pend = nullptr;
      if (stacked) {
        if ((e = matmul_q_dev(L.wq, L.wq_type, d->order, d->xb, d->q, d->qd + d->kvd, dim, s)))
          return e;
      } else {
        if ((e = matmul_q_dev(L.wq, L.wq_type, d->order, d->xb, d->q, d->qd, dim, s))) return e;
        if ((e = matmul_q_dev(L.wk, L.wk_type, d->order, d->xb, d->k, d->kvd, dim, s))) return e;
      }
    }
    if (!vdone &&
        (e = matmul_q_dev(L.wv, L.wv_type, d->order, d->xb, d->v, d->kvd, dim, s)))
      return e;
    const KvView K = kv_view(d, l, false), V = kv_view(d, l, true);
    // RoPE, the position's K / V rows and the scores in one launch
    const RopeArgs R{d->rope, d->k, d->v, const_cast<uint8_t*>(V.base), d->qd};
    hipLaunchKernelGGL(k_attn_scores<true>, dim3((d->cap + kScTile - 1) / kScTile, d->nkv),
                       dim3(256), d->sc_lds, s, d->q, K, d->st, 0, d->kv_mul, d->hd, inv_sqrt,
                       d->cap, d->att, R);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if ((e = sv_launch(d->att, d->cap, V, d->st, 0, d->cap, d->nh, d->kv_mul, d->hd, d->ao, s)))
      return e;
    // x += wo . ao (src/runtime.c:196-198), in the GEMV's store where it can
    const float* fadd = nullptr;
    if (residual_gemv(L.wo_type)) {
      if ((e = matmul_q_dev(L.wo, L.wo_type, d->order, d->ao, d->x, dim, d->qd, s, d->x)))
        return e;
    } else {
      if ((e = matmul_q_dev(L.wo, L.wo_type, d->order, d->ao, d->xb2, dim, d->qd, s))) return e;
      fadd = d->xb2;
    }
    if (is_dense(L)) {
      const qr_moe_layer& M = L.moe;
      float* u = reinterpret_cast<float*>(d->moe_base);
      float* g = u + M.hidden;
      float* y = g + M.hidden;
      if ((e = rmsnorm_launch(d->x, fadd, L.rms_ffn, dim, d->xb, s))) return e;
      if ((e = matmul_q_dev(M.up, M.up_type, d->order, d->xb, u, M.hidden, dim, s))) return e;
      if ((e = matmul_q_dev(M.gate, M.gate_type, d->order, d->xb, g, M.hidden, dim, s))) return e;
      hipLaunchKernelGGL(k_swiglu, dim3((M.hidden + 255) / 256), dim3(256), 0, s, u, g,
                         (long)M.hidden);
      if ((e = hipGetLastError()) != hipSuccess) return e;
      if (residual_gemv(M.down_type)) {  // x += w2 . hb (src/runtime.c:282-284)
        if ((e = matmul_q_dev(M.down, M.down_type, d->order, g, d->x, dim, M.hidden, s, d->x)))
          return e;
      } else {
        if ((e = matmul_q_dev(M.down, M.down_type, d->order, g, y, dim, M.hidden, s))) return e;
        pend = y;
      }
      continue;
    }
    MoeScratch ms;
    moe_scratch_carve(d->moe_base, &L.moe, 1, &ms);
    if (!fadd && moe_t1_norm_ok(&L.moe, d->x, d->xb, L.rms_ffn, d->order)) {
      // the FFN norm inside the router's launch
      if ((e = moe_forward_launch(&L.moe, d->x, d->xb, 1, d->order, ms, s, QR_MOE_PATH_AUTO,
                                  L.rms_ffn)))
        return e;
    } else {
      if ((e = rmsnorm_launch(d->x, fadd, L.rms_ffn, dim, d->xb, s))) return e;
      if ((e = moe_forward_launch(&L.moe, d->x, d->xb, 1, d->order, ms, s))) return e;
    }
  }
  if ((e = rmsnorm_launch(d->x, pend, d->rms_final, dim, d->xb, s))) return e;
  if ((e = matmul_q_dev(d->wcls, d->wcls_type, d->order, d->xb, logits, d->vocab, dim, s)))
    return e;
  if (xout) {
    if ((e = hipMemcpyAsync(xout, d->x, (size_t)dim * 4, hipMemcpyDeviceToDevice, s))) return e;
  }
  return hipSuccess;
}

// A single-"expert" dispatch of T rows for the grouped MFMA product:
// offsets {0, T}, the identity permutation, tiles {0, ceil(T / tile)}; with
// tiles2, also {0, ceil(T / 32)} there (a chunk's products take 16- or
// 32-pair items by their row count).
__global__ __launch_bounds__(256) void k_rows_dispatch(int T, int tile, int32_t* off,
                                                       int32_t* perm, int32_t* tiles,
                                                       int32_t* tiles2) {
  for (int i = threadIdx.x; i < T; i += blockDim.x) perm[i] = i;
  if (threadIdx.x == 0) {
    off[0] = 0;
    off[1] = T;
    tiles[0] = 0;
    tiles[1] = (T + tile - 1) / tile;
    if (tiles2) {
      tiles2[0] = 0;
      tiles2[1] = (T + 31) / 32;
    }
  }
}

// y[t][.] = W x[t] for T rows of x (a prompt chunk), each row exactly as
// matmul_q_dev computes it for one token: fp32 weights through the build's
// order with all T rows at once; K-quant (row-major or tiled) and C99-order
// Q8_0 weights as one grouped int8 MFMA product (qr_moe_mfma.hip, the rows
// dispatched to a single "expert"), whose per-row terms and order are the
// fused dot's; Q8_0 in a lane order and llama.cpp-layout K-quants through the
// GEMV, four rows per launch.
// The records of x are quantized unless `records` says the previous call
// left those of the same x (and the same record order) in d->prec; the chunk's
// single-expert dispatch lists are written once per chunk (prefill_rows_setup).
// Pairs per work item of the T-row products: a dense matrix has one
// "expert", so the items are what spreads it over the CUs.  16 for chunks
// below 256 rows (128-token chunks: 71 ms for 512 prompt tokens against 75
// ms with 32-pair items) and for matrices of fewer than 2048 rows (wk / wv
// at a 512-token chunk: 15-17 against 19-21 us, their few row blocks need
// the items), 32 otherwise (wq / wo: 74-78 -> 42-46 us).
static int rows_tile(int T, int n) { return T >= 256 && n >= 2048 ? 32 : 16; }

hipError_t matmul_rows_dev(qr_decoder* d, const void* w, uint32_t type, const float* x, float* y,
                           int n, int dd, int T, hipStream_t s, bool records = false) {
  hipError_t e;
  if (type == QR_T_F32)
    return gemv_f32_launch(d->order, static_cast<const float*>(w), x, y, n, dd, T, dd, n, s);
  if (type & QR_GGML) {  // ggml's Q8_K dot, four rows per launch
    d->prec_src = nullptr;  // d->prec keeps no records of x
    for (int t0 = 0; t0 < T; t0 += 4) {
      const int nt = T - t0 < 4 ? T - t0 : 4;
      if ((e = gemv_ggml_launch((int)(type & ~(uint32_t)QR_GGML), w, x + (size_t)t0 * dd,
                                y + (size_t)t0 * n, n, dd, nt, dd, n, s)))
        return e;
    }
    return hipSuccess;
  }
  const bool tiled = (type & QR_TILED) != 0;
  const uint32_t base = type & ~(uint32_t)QR_TILED;
  const bool lanes = base == QR_T_Q8_0 && d->order != QR_ORDER_SEQ;
  // the MFMA products read row-major or Q4_K / Q5_K tiles; Q6_K / Q8_0 tiles
  // take the tiled GEMV four rows at a time
  const bool sq_tiles = tiled && (base == QR_T_Q6_K || base == QR_T_Q8_0);
  if (!lanes && !sq_tiles && T >= 2 && mfma_type_ok((int)base) && dd % 256 == 0 &&
      (dd >> 8) <= 64) {
    const int tile = rows_tile(T, n);
    const int perm = base != QR_T_Q8_0;
    if (!records || d->prec_src != x || d->prec_perm != perm) {
      if ((e = quant_rows_launch(x, dd, T, dd, perm != 0, d->prec, s))) return e;
      d->prec_src = x;
      d->prec_perm = perm;
    }
    const size_t slice = qr_wrow_bytes((int)base, dd) * (size_t)n;
    return expert_mfma_launch((int)base, false, static_cast<const uint8_t*>(w), nullptr, slice, 1,
                              1, n, dd, d->prec, 1, d->poff, d->pperm,
                              tile == 16 ? d->ptiles : d->ptiles + 2, y, n,
                              (T + tile - 1) / tile + 1, tile, nullptr, false, s, tiled);
  }
  for (int t0 = 0; t0 < T; t0 += 4) {
    const int nt = T - t0 < 4 ? T - t0 : 4;
    if (tiled)
      e = gemv_tiled_launch((int)base, w, x + (size_t)t0 * dd, y + (size_t)t0 * n, n, dd, nt, dd, n,
                            s, d->order);
    else
      e = gemv_launch((int)base, d->order, w, x + (size_t)t0 * dd, y + (size_t)t0 * n, n, dd, nt,
                      dd, n, nullptr, nullptr, s);
    if (e) return e;
  }
  return hipSuccess;
}

// One prompt chunk of T tokens (states st[2 T]) through every layer: the
// decode step's kernels with a token dimension, the projections as T-row
// products, the MoE layer at T tokens.  Leaves the chunk's residuals in px.
// pend: one past the chunk's last position.
hipError_t enqueue_prefill_chunk(qr_decoder* d, int T, const int32_t* st, int pend,
                                 hipStream_t s) {
  hipError_t e;
  const int dim = d->dim;
  // the chunk's single-expert dispatch of its T rows (in the items
  // matmul_rows_dev launches)
  hipLaunchKernelGGL(k_rows_dispatch, dim3(1), dim3(256), 0, s, T, 16, d->poff, d->pperm,
                     d->ptiles, d->ptiles + 2);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  d->prec_src = nullptr;
  hipLaunchKernelGGL(k_embed, dim3(T), dim3(256), 0, s, static_cast<const uint8_t*>(d->tok_embd),
                     (int)d->tok_type, d->tok_row, st, dim, d->px);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const float inv_sqrt = 1.0f / sqrtf((float)d->hd);
  for (int l = 0; l < d->nl; l++) {
    const qr_layer& L = d->layers[l];
    if ((e = rmsnorm_launch(d->px, nullptr, L.rms_att, dim, d->pxb, s, T))) return e;
    d->prec_src = nullptr;  // pxb has new rows: no records of them yet
    if ((e = matmul_rows_dev(d, L.wq, L.wq_type, d->pxb, d->pq, d->qd, dim, T, s))) return e;
    // k and v read the records q's product left (same rows, same order)
    if ((e = matmul_rows_dev(d, L.wk, L.wk_type, d->pxb, d->pk, d->kvd, dim, T, s, true))) return e;
    if ((e = matmul_rows_dev(d, L.wv, L.wv_type, d->pxb, d->pv, d->kvd, dim, T, s, true))) return e;
    const KvView K = kv_view(d, l, false), V = kv_view(d, l, true);
    hipLaunchKernelGGL(k_rope_kv, dim3((d->qd / 2 + 2 * (d->kvd / 32) + 255) / 256, T), dim3(256),
                       0, s, d->pq, d->pk, d->pv, d->rope, st, d->qd, d->kvd, K,
                       const_cast<uint8_t*>(V.base));
    if ((e = hipGetLastError()) != hipSuccess) return e;
    // position tiles up to the chunk's last position (not the cache's
    // capacity: tiles past a token's positions are dispatched only to
    // return), an odd count of them: workgroups go to the XCDs in turn, and an
    // even count would send every token's tile x to the same XCD -- the early
    // tiles, which every token has, to a few XCDs, the late ones, which few
    // tokens have, to the others
    hipLaunchKernelGGL(k_attn_scores<false>, dim3(((pend + kScTile - 1) / kScTile) | 1, d->nkv, T),
                       dim3(256), d->sc_lds, s, d->pq, K, st, 0, d->kv_mul, d->hd, inv_sqrt, d->cap,
                       d->patt, RopeArgs{});
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if ((e = sv_rows_launch(d->patt, d->cap, V, st, d->cap, d->nh, d->kv_mul, d->hd, d->pao, T,
                            s, pend)))
      return e;
    if ((e = matmul_rows_dev(d, L.wo, L.wo_type, d->pao, d->pxb2, dim, d->qd, T, s))) return e;
    if ((e = rmsnorm_launch(d->px, d->pxb2, L.rms_ffn, dim, d->pxb, s, T))) return e;
    if (is_dense(L)) {
      const qr_moe_layer& M = L.moe;
      const size_t th = (size_t)T * M.hidden;
      float* u = reinterpret_cast<float*>(d->pmoe);
      float* g = u + th;
      float* y = g + th;
      d->prec_src = nullptr;  // pxb has new rows
      if ((e = matmul_rows_dev(d, M.up, M.up_type, d->pxb, u, M.hidden, dim, T, s))) return e;
      if ((e = matmul_rows_dev(d, M.gate, M.gate_type, d->pxb, g, M.hidden, dim, T, s, true)))
        return e;
      hipLaunchKernelGGL(k_swiglu, dim3((unsigned)((th + 255) / 256)), dim3(256), 0, s, u, g,
                         (long)th);
      if ((e = hipGetLastError()) != hipSuccess) return e;
      d->prec_src = nullptr;
      if ((e = matmul_rows_dev(d, M.down, M.down_type, g, y, dim, M.hidden, T, s))) return e;
      const long n4 = (long)T * dim / 4;
      hipLaunchKernelGGL(k_add4, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, d->px, y, n4);
      if ((e = hipGetLastError()) != hipSuccess) return e;
      continue;
    }
    MoeScratch ms;
    moe_scratch_carve(d->pmoe, &L.moe, T, &ms);
    if ((e = moe_forward_launch(&L.moe, d->px, d->pxb, T, d->order, ms, s))) return e;
  }
  return hipSuccess;
}

__global__ void k_set_state(int32_t* st, int token, int pos) {
  if (threadIdx.x == 0) {
    st[0] = token;
    st[1] = pos;
  }
}

void drop_graph(qr_decoder* d) {
  if (d->exec) (void)hipGraphExecDestroy(d->exec);
  if (d->graph) (void)hipGraphDestroy(d->graph);
  d->exec = nullptr;
  d->graph = nullptr;
}

// Which layers run q / k and v in one normalising launch (k_gemv_norm2), and
// their v matrices in the Q6_K / Q8_0 tiled layout: the caller's when it
// passes them tiled, else a copy tiled here (the decode step reads it; the
// prompt's row products keep reading the caller's row-major matrix).
hipError_t plan_wv_tiled(qr_decoder* d, hipStream_t s) {
  d->wv_tiled.assign(d->nl, nullptr);
  d->wv_tiled_type.assign(d->nl, 0);
  std::vector<size_t> off(d->nl, (size_t)-1);
  size_t total = 0;
  for (int l = 0; l < d->nl; l++) {
    const qr_layer& L = d->layers[l];
    if (!qk_stacked(d, L) || !norm_in_q(d, L)) continue;
    const int qb = (int)(L.wq_type & ~(uint32_t)QR_TILED);
    const uint32_t vt = L.wv_type;
    const int vb = (int)(vt & ~(uint32_t)QR_TILED);
    if ((vt & QR_GGML) || (vb != QR_T_Q6_K && vb != QR_T_Q8_0)) continue;
    if (vb == QR_T_Q8_0 && d->order != QR_ORDER_SEQ) continue;  // tiles take the C99 order
    if (!gemv_norm2_ok(qb, vb, d->kvd, d->dim)) continue;
    d->wv_tiled_type[l] = vb;
    if (vt & QR_TILED) {
      d->wv_tiled[l] = L.wv;
    } else {
      off[l] = total;
      total += (qr_wrow_bytes(vb, d->dim) * (size_t)d->kvd + 255) & ~(size_t)255;
    }
  }
  if (!total) return hipSuccess;
  hipError_t e = hipMalloc((void**)&d->wvt, total);
  if (e != hipSuccess) return e;
  for (int l = 0; l < d->nl; l++) {
    if (off[l] == (size_t)-1) continue;
    uint8_t* dst = d->wvt + off[l];
    e = tile_pack_launch(d->wv_tiled_type[l], d->layers[l].wv, dst, d->kvd, d->dim, false, s);
    if (e != hipSuccess) return e;
    d->wv_tiled[l] = dst;
  }
  return hipSuccess;
}

int check_layer_weights(const qr_model* m, int l, int order) {
  const qr_layer& L = m->layers[l];
  const int hd = m->head_dim, qd = m->n_heads * hd, kvd = m->n_kv_heads * hd;
  if (!L.rms_att || !L.rms_ffn || !L.wq || !L.wk || !L.wv || !L.wo)
    return set_error(QR_ERR_INVALID, "qr_decoder_create: layer %d has a null tensor", l);
  int rc;
  if ((rc = gemv_check(L.wq_type, order, L.wq, qd, m->dim, "qr_decoder_create: wq"))) return rc;
  if ((rc = gemv_check(L.wk_type, order, L.wk, kvd, m->dim, "qr_decoder_create: wk"))) return rc;
  if ((rc = gemv_check(L.wv_type, order, L.wv, kvd, m->dim, "qr_decoder_create: wv"))) return rc;
  if ((rc = gemv_check(L.wo_type, order, L.wo, m->dim, qd, "qr_decoder_create: wo"))) return rc;
  if (is_dense(L)) {
    const qr_moe_layer& M = L.moe;
    if (!M.up || !M.gate || !M.down || M.hidden <= 0 || M.hidden % 4)
      return set_error(QR_ERR_INVALID, "qr_decoder_create: layer %d dense FFN (hidden %d)", l,
                       M.hidden);
    if ((rc = gemv_check(M.up_type, order, M.up, M.hidden, m->dim, "qr_decoder_create: ffn_up")))
      return rc;
    if ((rc = gemv_check(M.gate_type, order, M.gate, M.hidden, m->dim,
                         "qr_decoder_create: ffn_gate")))
      return rc;
    if ((rc = gemv_check(M.down_type, order, M.down, m->dim, M.hidden,
                         "qr_decoder_create: ffn_down")))
      return rc;
  } else if ((rc = moe_check(&L.moe, "qr_decoder_create: moe"))) {
    return rc;
  }
  if (L.moe.dim != m->dim)
    return set_error(QR_ERR_INVALID, "qr_decoder_create: layer %d moe.dim %d != dim %d", l,
                     L.moe.dim, m->dim);
  return QR_OK;
}

}  // namespace

namespace qr {
hipError_t rows_dispatch_launch(int T, int tile, int32_t* off, int32_t* perm, int32_t* tiles,
                                hipStream_t st) {
  hipLaunchKernelGGL(k_rows_dispatch, dim3(1), dim3(256), 0, st, T, tile, off, perm, tiles,
                     (int32_t*)nullptr);
  return hipGetLastError();
}
}  // namespace qr

extern "C" {

size_t qr_kv_row_bytes(int kv_type, int kv_dim) {
  if (kv_dim <= 0) return 0;
  if (kv_type == QR_KV_Q8_0) return kv_dim % 32 ? 0 : (size_t)(kv_dim / 32) * QR_Q8_BYTES;
  if (kv_type == QR_KV_F16) return kv_dim % 32 ? 0 : (size_t)kv_dim * 2;
  if (kv_type == QR_KV_F32) return (size_t)kv_dim * 4;
  return 0;
}

int qr_dequantize(qr_ctx* c, uint32_t type, const void* src, int rows, int n, float* out) {
  if (!c) return set_error(QR_ERR_INVALID, "qr_dequantize: null ctx");
  if (rows < 0 || n < 0) return set_error(QR_ERR_INVALID, "qr_dequantize: negative size");
  if ((long)rows * n == 0) return QR_OK;
  if (!out) return set_error(QR_ERR_INVALID, "qr_dequantize: null out");
  if (type & QR_GGML) {  // llama.cpp / ggml K-quant blocks
    const uint32_t base = type & ~(uint32_t)QR_GGML;
    if ((base != QR_T_Q4_K && base != QR_T_Q5_K && base != QR_T_Q6_K) || n % 256)
      return set_error(QR_ERR_INVALID, "qr_dequantize: ggml type %u, n=%d", base, n);
    if (!src) return set_error(QR_ERR_INVALID, "qr_dequantize: null src");
    DEC_HIP(hipSetDevice(ctx_device(c)), "hipSetDevice");
    DEC_HIP(ggml_dequant_launch((int)base, src, rows, n, out, ctx_stream(c)), "k_ggml_dequant_rows");
    return QR_OK;
  }
  const size_t rb = qr_row_bytes(type, n);
  const bool known = type == QR_T_F32 || type == QR_T_Q8_0 || type == QR_T_Q4_K ||
                     type == QR_T_Q5_K || type == QR_T_Q6_K;
  if (known && n % qr_block_elems((int)type))
    return set_error(QR_ERR_INVALID, "qr_dequantize: n=%d is not whole blocks", n);
  DEC_HIP(hipSetDevice(ctx_device(c)), "hipSetDevice");
  long grid = ((long)rows * n + 255) / 256;
  if (grid > 4096) grid = 4096;
  // no source (src/quant.c:161-164) or an unknown type: zeros
  hipLaunchKernelGGL(k_dequant_rows, dim3((unsigned)grid), dim3(256), 0, ctx_stream(c),
                     static_cast<const uint8_t*>(src), src ? (int)type : -1, rb, rows, n, out);
  DEC_HIP(hipGetLastError(), "k_dequant_rows");
  return QR_OK;
}

int qr_rmsnorm(qr_ctx* c, float* o, float* x, const float* add, const float* w, int n) {
  if (!c) return set_error(QR_ERR_INVALID, "qr_rmsnorm: null ctx");
  if (n <= 0 || n > kNormMax) return set_error(QR_ERR_INVALID, "qr_rmsnorm: n=%d (1..%d)", n, kNormMax);
  if (!o || !x || !w) return set_error(QR_ERR_INVALID, "qr_rmsnorm: null pointer");
  DEC_HIP(hipSetDevice(ctx_device(c)), "hipSetDevice");
  DEC_HIP(rmsnorm_launch(x, add, w, n, o, ctx_stream(c)), "k_rmsnorm");
  return QR_OK;
}

int qr_attention(qr_ctx* c, const float* q, const void* kc, const void* vc, const int32_t* ptab,
                 int page, int kv_type, int npos, int n_heads, int n_kv_heads, int head_dim,
                 float* att, float* out) {
  if (!c) return set_error(QR_ERR_INVALID, "qr_attention: null ctx");
  if (!q || !kc || !vc || !ptab || !att || !out)
    return set_error(QR_ERR_INVALID, "qr_attention: null pointer");
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads)
    return set_error(QR_ERR_INVALID, "qr_attention: heads %d / kv heads %d", n_heads, n_kv_heads);
  if (head_dim <= 0 || head_dim % kValCols || head_dim > kHdMax)
    return set_error(QR_ERR_INVALID, "qr_attention: head_dim %d (a multiple of 32, <= %d)",
                     head_dim, kHdMax);
  if (page <= 0 || (page & (page - 1)))
    return set_error(QR_ERR_INVALID, "qr_attention: page %d (a power of two)", page);
  const size_t rb = qr_kv_row_bytes(kv_type, n_kv_heads * head_dim);
  if (!rb) return set_error(QR_ERR_INVALID, "qr_attention: kv_type %d", kv_type);
  if (npos <= 0 || npos > kAttnMaxPos)
    return set_error(QR_ERR_INVALID, "qr_attention: npos %d (1..%d)", npos, kAttnMaxPos);
  if (!sv_lds_ok(npos, page))
    return set_error(QR_ERR_UNSUPPORTED, "qr_attention: %d positions in pages of %d", npos, page);
  if (!al16(kc) || !al16(vc)) return set_error(QR_ERR_INVALID, "qr_attention: cache alignment");
  const int kv_mul = n_heads / n_kv_heads;
  const size_t sc_lds = ((size_t)kScTile * (head_dim + 4) + (size_t)kv_mul * head_dim) * 4;
  if (sc_lds > kDecLdsMax) return set_error(QR_ERR_UNSUPPORTED, "qr_attention: head group too large");
  DEC_HIP(hipSetDevice(ctx_device(c)), "hipSetDevice");
  DEC_HIP(lds_opt_in((const void*)k_attn_scores<false>, g_sc_opt), "lds opt-in");
  DEC_HIP(lds_opt_in((const void*)k_attn_sv<QR_KV_Q8_0>, g_sm_opt), "lds opt-in");
  DEC_HIP(lds_opt_in((const void*)k_attn_sv<QR_KV_F32>, g_sm_opt2), "lds opt-in");
  DEC_HIP(lds_opt_in((const void*)k_attn_sv<QR_KV_F16>, g_sm_opt3), "lds opt-in");
  KvView K;
  K.base = static_cast<const uint8_t*>(kc);
  K.ptab = ptab;
  K.page = page;
  K.page_shift = __builtin_ctz((unsigned)page);
  K.row_bytes = rb;
  K.kv_type = kv_type;
  KvView V = K;
  V.base = static_cast<const uint8_t*>(vc);
  hipStream_t s = ctx_stream(c);
  const float inv_sqrt = 1.0f / sqrtf((float)head_dim);
  hipLaunchKernelGGL(k_attn_scores<false>, dim3((npos + kScTile - 1) / kScTile, n_kv_heads),
                     dim3(256), sc_lds, s, q, K, (const int32_t*)nullptr, npos, kv_mul, head_dim,
                     inv_sqrt, npos, att, RopeArgs{});
  DEC_HIP(hipGetLastError(), "k_attn_scores");
  DEC_HIP(sv_launch(att, npos, V, nullptr, npos, npos, n_heads, kv_mul, head_dim, out, s),
          "k_attn_sv");
  // the normalised weights, in place of the scores (the same softmax_ref)
  DEC_HIP(softmax_launch(att, n_heads, npos, s), "k_softmax");
  return QR_OK;
}

int qr_decoder_create(qr_ctx* c, const qr_model* m, int kv_type, int order, int page, int flags,
                      qr_decoder** out) {
  if (!out) return set_error(QR_ERR_INVALID, "qr_decoder_create: null out");
  *out = nullptr;
  if (!c || !m || !m->layers) return set_error(QR_ERR_INVALID, "qr_decoder_create: null argument");
  if (ctx_capturing(c))
    return set_error(QR_ERR_INVALID, "qr_decoder_create: not allowed while the stream is captured");
  if (order < QR_ORDER_SEQ || order > QR_ORDER_AVX512)
    return set_error(QR_ERR_INVALID, "qr_decoder_create: order %d", order);
  if (flags & ~QR_DEC_GRAPH) return set_error(QR_ERR_INVALID, "qr_decoder_create: flags %d", flags);
  const int dim = m->dim, nh = m->n_heads, nkv = m->n_kv_heads, hd = m->head_dim;
  if (dim <= 0 || dim > kNormMax || m->n_layers <= 0 || m->vocab <= 0 || m->seq_len <= 0)
    return set_error(QR_ERR_INVALID, "qr_decoder_create: dim %d, layers %d, vocab %d, seq_len %d",
                     dim, m->n_layers, m->vocab, m->seq_len);
  if (nh <= 0 || nkv <= 0 || nh % nkv)
    return set_error(QR_ERR_INVALID, "qr_decoder_create: heads %d / kv heads %d", nh, nkv);
  if (hd <= 0 || hd % kValCols || hd > kHdMax)
    return set_error(QR_ERR_INVALID, "qr_decoder_create: head_dim %d (a multiple of 32, <= %d)",
                     hd, kHdMax);
  const int qd = nh * hd, kvd = nkv * hd;
  if (m->seq_len > kAttnMaxPos)
    return set_error(QR_ERR_UNSUPPORTED, "qr_decoder_create: seq_len %d (<= %d)", m->seq_len,
                     kAttnMaxPos);
  const size_t rb = qr_kv_row_bytes(kv_type, kvd);
  if (!rb) return set_error(QR_ERR_INVALID, "qr_decoder_create: kv_type %d", kv_type);
  if (page <= 0) page = 256;
  if (page & (page - 1))
    return set_error(QR_ERR_INVALID, "qr_decoder_create: page %d (a power of two)", page);
  if (!sv_lds_ok(m->seq_len, page))
    return set_error(QR_ERR_UNSUPPORTED, "qr_decoder_create: seq_len %d in pages of %d",
                     m->seq_len, page);
  if (!m->tok_embd || !m->rms_final || !m->wcls)
    return set_error(QR_ERR_INVALID, "qr_decoder_create: null embedding / final norm / wcls");
  const uint32_t tok_base = m->tok_type & ~(uint32_t)QR_GGML;
  const bool tok_ggml = (m->tok_type & QR_GGML) != 0;
  const bool tok_known = tok_base == QR_T_Q4_K || tok_base == QR_T_Q5_K ||
                         tok_base == QR_T_Q6_K ||
                         (!tok_ggml && (tok_base == QR_T_F32 || tok_base == QR_T_Q8_0));
  if (!tok_known || dim % qr_block_elems((int)tok_base))
    return set_error(QR_ERR_INVALID, "qr_decoder_create: embedding type %u at dim %d", m->tok_type,
                     dim);
  int rc = gemv_check(m->wcls_type, order, m->wcls, m->vocab, dim, "qr_decoder_create: wcls");
  if (rc) return rc;
  for (int l = 0; l < m->n_layers; l++)
    if ((rc = check_layer_weights(m, l, order))) return rc;
  const int kv_mul = nh / nkv;
  const size_t sc_lds = ((size_t)kScTile * (hd + 4) + (size_t)kv_mul * hd) * 4;
  if (sc_lds > kDecLdsMax) return set_error(QR_ERR_UNSUPPORTED, "qr_decoder_create: head group too large");

  DEC_HIP(hipSetDevice(ctx_device(c)), "hipSetDevice");
  DEC_HIP(lds_opt_in((const void*)k_attn_scores<false>, g_sc_opt), "lds opt-in");
  DEC_HIP(lds_opt_in((const void*)k_attn_scores<true>, g_sc_opt_r), "lds opt-in");
  DEC_HIP(lds_opt_in((const void*)k_attn_sv<QR_KV_Q8_0>, g_sm_opt), "lds opt-in");
  DEC_HIP(lds_opt_in((const void*)k_attn_sv<QR_KV_F32>, g_sm_opt2), "lds opt-in");
  DEC_HIP(lds_opt_in((const void*)k_attn_sv<QR_KV_F16>, g_sm_opt3), "lds opt-in");
  DEC_HIP(lds_opt_in((const void*)k_attn_sv_rows<QR_KV_Q8_0>, g_rows_opt), "lds opt-in");
  DEC_HIP(lds_opt_in((const void*)k_attn_sv_rows<QR_KV_F32>, g_rows_opt2), "lds opt-in");
  DEC_HIP(lds_opt_in((const void*)k_attn_sv_rows<QR_KV_F16>, g_rows_opt3), "lds opt-in");
  qr_decoder* d = new (std::nothrow) qr_decoder();
  if (!d) return set_error(QR_ERR_NOMEM, "qr_decoder_create: host allocation");
  d->ctx = c;
  d->device = ctx_device(c);
  d->dim = dim;
  d->nh = nh;
  d->nkv = nkv;
  d->hd = hd;
  d->nl = m->n_layers;
  d->vocab = m->vocab;
  d->cap = m->seq_len;
  d->qd = qd;
  d->kvd = kvd;
  d->kv_mul = kv_mul;
  d->tok_embd = m->tok_embd;
  d->tok_type = m->tok_type;
  d->tok_row = qr_row_bytes(m->tok_type, dim);
  d->rms_final = m->rms_final;
  d->wcls = m->wcls;
  d->wcls_type = m->wcls_type;
  d->layers.assign(m->layers, m->layers + m->n_layers);
  d->kv_type = kv_type;
  d->order = order;
  d->page = page;
  d->ppl = (m->seq_len + page - 1) / page;
  d->flags = flags;
  d->row_bytes = rb;
  d->sc_lds = sc_lds;
  d->layer_pages_bytes = (size_t)d->ppl * page * rb;
  d->layer_pages_bytes = (d->layer_pages_bytes + 255) & ~(size_t)255;

  // one allocation: activations, state, page table, RoPE table, MoE scratch
  size_t moe_bytes = 0;
  for (int l = 0; l < d->nl; l++) {
    const qr_layer& L = d->layers[l];
    const size_t b = is_dense(L) ? dense_scratch_bytes(L.moe, 1) : moe_scratch_bytes(&L.moe, 1);
    if (b > moe_bytes) moe_bytes = b;
  }
  auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
  const size_t o_x = 0, o_xb = o_x + up(dim * 4), o_xb2 = o_xb + up(dim * 4);
  const size_t o_q = o_xb2 + up(dim * 4), o_k = o_q + up(qd * 4), o_v = o_k + up(qd * 4);
  const size_t o_ao = o_v + up(qd * 4), o_att = o_ao + up(qd * 4);
  const size_t o_st = o_att + up((size_t)nh * d->cap * 4), o_pt = o_st + 256;
  const size_t o_rope = o_pt + up((size_t)d->nl * d->ppl * 4);
  const size_t o_moe = o_rope + up((size_t)d->cap * qd * 4);
  const size_t total = o_moe + up(moe_bytes);
  hipError_t e = hipMalloc(&d->mem, total);
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&d->kc), d->layer_pages_bytes * d->nl);
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&d->vc), d->layer_pages_bytes * d->nl);
  if (e != hipSuccess) {
    qr_decoder_destroy(d);
    return set_error(QR_ERR_NOMEM, "qr_decoder_create: device allocation: %s", hipGetErrorString(e));
  }
  uint8_t* b = static_cast<uint8_t*>(d->mem);
  d->x = reinterpret_cast<float*>(b + o_x);
  d->xb = reinterpret_cast<float*>(b + o_xb);
  d->xb2 = reinterpret_cast<float*>(b + o_xb2);
  d->q = reinterpret_cast<float*>(b + o_q);
  d->k = reinterpret_cast<float*>(b + o_k);
  d->v = reinterpret_cast<float*>(b + o_v);
  d->ao = reinterpret_cast<float*>(b + o_ao);
  d->att = reinterpret_cast<float*>(b + o_att);
  d->st = reinterpret_cast<int32_t*>(b + o_st);
  d->ptab = reinterpret_cast<int32_t*>(b + o_pt);
  d->rope = reinterpret_cast<float*>(b + o_rope);
  d->moe_base = b + o_moe;  // sized for the largest layer, carved per layer

  // identity page table, RoPE table with the host C library's powf / cosf /
  // sinf (apply_rope, src/runtime.c:19-41): pair p of position t at
  // [t][2p], [t][2p + 1]
  std::vector<int32_t> pt((size_t)d->nl * d->ppl);
  for (int l = 0; l < d->nl; l++)
    for (int i = 0; i < d->ppl; i++) pt[(size_t)l * d->ppl + i] = i;
  const float base = m->rope_base > 0.0f ? m->rope_base : 10000.0f;
  std::vector<float> freq(qd / 2), tab((size_t)d->cap * qd);
  for (int i = 0; i < qd; i += 2) freq[i / 2] = powf(base, -((float)i / (float)hd));
  for (int t = 0; t < d->cap; t++)
    for (int i = 0; i < qd; i += 2) {
      const float theta = (float)t * freq[i / 2];
      tab[(size_t)t * qd + i] = cosf(theta);
      tab[(size_t)t * qd + i + 1] = sinf(theta);
    }
  hipStream_t s = ctx_stream(c);
  e = hipMemcpyAsync(d->ptab, pt.data(), pt.size() * 4, hipMemcpyHostToDevice, s);
  if (e == hipSuccess)
    e = hipMemcpyAsync(d->rope, tab.data(), tab.size() * 4, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = plan_wv_tiled(d, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) {
    qr_decoder_destroy(d);
    return set_error(QR_ERR_HIP, "qr_decoder_create: upload: %s", hipGetErrorString(e));
  }
  *out = d;
  return QR_OK;
}

int qr_decoder_destroy(qr_decoder* d) {
  if (!d) return QR_OK;
  (void)hipSetDevice(d->device);
  if (d->ctx) (void)hipStreamSynchronize(ctx_stream(d->ctx));
  drop_graph(d);
  if (d->kc) (void)hipFree(d->kc);
  if (d->vc) (void)hipFree(d->vc);
  if (d->mem) (void)hipFree(d->mem);
  if (d->pmem) (void)hipFree(d->pmem);
  if (d->wvt) (void)hipFree(d->wvt);
  delete d;
  return QR_OK;
}

int qr_decoder_set_pages(qr_decoder* d, const int32_t* table) {
  if (!d || !table) return set_error(QR_ERR_INVALID, "qr_decoder_set_pages: null argument");
  for (int l = 0; l < d->nl; l++) {
    std::vector<char> seen(d->ppl, 0);
    for (int i = 0; i < d->ppl; i++) {
      const int32_t p = table[(size_t)l * d->ppl + i];
      if (p < 0 || p >= d->ppl || seen[p])
        return set_error(QR_ERR_INVALID,
                         "qr_decoder_set_pages: layer %d is not a permutation of 0..%d", l,
                         d->ppl - 1);
      seen[p] = 1;
    }
  }
  DEC_HIP(hipSetDevice(d->device), "hipSetDevice");
  hipStream_t s = ctx_stream(d->ctx);
  DEC_HIP(hipMemcpyAsync(d->ptab, table, (size_t)d->nl * d->ppl * 4, hipMemcpyHostToDevice, s),
          "page table upload");
  DEC_HIP(hipStreamSynchronize(s), "hipStreamSynchronize");
  return QR_OK;
}

int qr_decoder_pages(const qr_decoder* d, int* pages_per_layer, int* page) {
  if (!d) return set_error(QR_ERR_INVALID, "qr_decoder_pages: null decoder");
  if (pages_per_layer) *pages_per_layer = d->ppl;
  if (page) *page = d->page;
  return QR_OK;
}

int qr_decoder_kv_write(qr_decoder* d, int layer, int pos0, int n, const float* k, const float* v) {
  if (!d || !k || !v) return set_error(QR_ERR_INVALID, "qr_decoder_kv_write: null argument");
  if (layer < 0 || layer >= d->nl || pos0 < 0 || n < 0 || pos0 + n > d->cap)
    return set_error(QR_ERR_INVALID, "qr_decoder_kv_write: layer %d, positions [%d, %d) of %d",
                     layer, pos0, pos0 + n, d->cap);
  if (n == 0) return QR_OK;
  DEC_HIP(hipSetDevice(d->device), "hipSetDevice");
  const KvView K = kv_view(d, layer, false), V = kv_view(d, layer, true);
  long grid = (2L * n * (d->kvd / 32) + 255) / 256;
  if (grid > 4096) grid = 4096;
  hipLaunchKernelGGL(k_kv_write, dim3((unsigned)grid), dim3(256), 0, ctx_stream(d->ctx), k, v,
                     pos0, n, d->kvd, K, const_cast<uint8_t*>(V.base));
  DEC_HIP(hipGetLastError(), "k_kv_write");
  return QR_OK;
}

int qr_decoder_kv_rows(const qr_decoder* d, int layer, int pos, const void** krow,
                       const void** vrow) {
  if (!d || !krow || !vrow) return set_error(QR_ERR_INVALID, "qr_decoder_kv_rows: null argument");
  if (layer < 0 || layer >= d->nl || pos < 0 || pos >= d->cap)
    return set_error(QR_ERR_INVALID, "qr_decoder_kv_rows: layer %d pos %d", layer, pos);
  // the page table is host-known only through set_pages; read it back
  int32_t pp = 0;
  DEC_HIP(hipSetDevice(d->device), "hipSetDevice");
  DEC_HIP(hipMemcpy(&pp, d->ptab + (size_t)layer * d->ppl + pos / d->page, 4,
                    hipMemcpyDeviceToHost),
          "page table read");
  const size_t off = (size_t)layer * d->layer_pages_bytes +
                     ((size_t)pp * d->page + (size_t)(pos % d->page)) * d->row_bytes;
  *krow = d->kc + off;
  *vrow = d->vc + off;
  return QR_OK;
}


// The prefill workspace for chunks of up to `chunk` tokens.
static int prefill_workspace(qr_decoder* d, int chunk) {
  if (d->pmem && d->pcap >= chunk) return QR_OK;
  if (d->pmem) {
    (void)hipStreamSynchronize(ctx_stream(d->ctx));
    (void)hipFree(d->pmem);
    d->pmem = nullptr;
    d->pcap = 0;
  }
  auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
  const size_t T = (size_t)chunk;
  size_t moe_bytes = 0;
  for (int l = 0; l < d->nl; l++) {
    const qr_layer& L = d->layers[l];
    const size_t b =
        is_dense(L) ? dense_scratch_bytes(L.moe, chunk) : moe_scratch_bytes(&L.moe, chunk);
    if (b > moe_bytes) moe_bytes = b;
  }
  // the widest input a row product quantizes: q (wo's input), x, or a dense
  // FFN's hidden rows (w2's input)
  int wide = d->qd > d->dim ? d->qd : d->dim;
  for (int l = 0; l < d->nl; l++)
    if (is_dense(d->layers[l]) && d->layers[l].moe.hidden > wide) wide = d->layers[l].moe.hidden;
  const size_t o_x = 0, o_xb = o_x + up(T * d->dim * 4), o_xb2 = o_xb + up(T * d->dim * 4);
  const size_t o_q = o_xb2 + up(T * d->dim * 4), o_k = o_q + up(T * d->qd * 4);
  const size_t o_v = o_k + up(T * d->kvd * 4), o_ao = o_v + up(T * d->kvd * 4);
  const size_t o_att = o_ao + up(T * d->qd * 4);
  const size_t o_st = o_att + up(T * d->nh * (size_t)d->cap * 4);
  const size_t o_rec = o_st + up((size_t)d->cap * 8);
  const size_t o_off = o_rec + up(T * (size_t)(wide / 32) * 48);
  const size_t o_perm = o_off + 256, o_tiles = o_perm + up(T * 4);
  const size_t o_moe = o_tiles + 256, total = o_moe + up(moe_bytes);
  void* p = nullptr;
  const hipError_t e = hipMalloc(&p, total);
  if (e != hipSuccess)
    return set_error(QR_ERR_NOMEM, "qr_decoder_prefill: workspace of %zu bytes: %s", total,
                     hipGetErrorString(e));
  uint8_t* b = static_cast<uint8_t*>(p);
  d->pmem = p;
  d->pcap = chunk;
  d->px = reinterpret_cast<float*>(b + o_x);
  d->pxb = reinterpret_cast<float*>(b + o_xb);
  d->pxb2 = reinterpret_cast<float*>(b + o_xb2);
  d->pq = reinterpret_cast<float*>(b + o_q);
  d->pk = reinterpret_cast<float*>(b + o_k);
  d->pv = reinterpret_cast<float*>(b + o_v);
  d->pao = reinterpret_cast<float*>(b + o_ao);
  d->patt = reinterpret_cast<float*>(b + o_att);
  d->pst = reinterpret_cast<int32_t*>(b + o_st);
  d->prec = b + o_rec;
  d->poff = reinterpret_cast<int32_t*>(b + o_off);
  d->pperm = reinterpret_cast<int32_t*>(b + o_perm);
  d->ptiles = reinterpret_cast<int32_t*>(b + o_tiles);
  d->pmoe = b + o_moe;
  return QR_OK;
}

int qr_decoder_prefill(qr_decoder* d, const int32_t* tokens, int n, int pos0, int chunk,
                       float* logits, float* x_out, int flags) {
  if (!d || (n > 0 && !tokens)) return set_error(QR_ERR_INVALID, "qr_decoder_prefill: null argument");
  if (n < 0 || pos0 < 0 || pos0 + n > d->cap)
    return set_error(QR_ERR_INVALID, "qr_decoder_prefill: positions [%d, %d) of %d", pos0,
                     pos0 + n, d->cap);
  if (flags & ~QR_PREFILL_ALL_LOGITS)
    return set_error(QR_ERR_INVALID, "qr_decoder_prefill: flags %#x", flags);
  if (chunk < 0 || chunk > QR_PREFILL_MAX_CHUNK)
    return set_error(QR_ERR_INVALID, "qr_decoder_prefill: chunk %d (1 .. %d, 0 for %d)", chunk,
                     QR_PREFILL_MAX_CHUNK, QR_PREFILL_CHUNK);
  if ((logits && !al16(logits)) || (x_out && !al16(x_out)))
    return set_error(QR_ERR_INVALID, "qr_decoder_prefill: output alignment");
  for (int i = 0; i < n; i++)
    if (tokens[i] < 0 || tokens[i] >= d->vocab)
      return set_error(QR_ERR_INVALID, "qr_decoder_prefill: token %d at %d (vocab %d)", tokens[i],
                       i, d->vocab);
  if (n == 0) return QR_OK;
  if (ctx_capturing(d->ctx))
    return set_error(QR_ERR_INVALID, "qr_decoder_prefill: not under stream capture");
  if (chunk == 0) chunk = QR_PREFILL_CHUNK;
  if (chunk > n) chunk = n;
  DEC_HIP(hipSetDevice(d->device), "hipSetDevice");
  int rc = prefill_workspace(d, chunk);
  if (rc) return rc;
  hipStream_t s = ctx_stream(d->ctx);
  // every prompt position's (token, position), uploaded once
  std::vector<int32_t> st((size_t)2 * n);
  for (int i = 0; i < n; i++) {
    st[2 * (size_t)i] = tokens[i];
    st[2 * (size_t)i + 1] = pos0 + i;
  }
  DEC_HIP(hipMemcpyAsync(d->pst, st.data(), st.size() * 4, hipMemcpyHostToDevice, s),
          "prefill state upload");
  DEC_HIP(hipStreamSynchronize(s), "hipStreamSynchronize");
  const int dim = d->dim;
  for (int c0 = 0; c0 < n; c0 += chunk) {
    const int T = n - c0 < chunk ? n - c0 : chunk;
    DEC_HIP(enqueue_prefill_chunk(d, T, d->pst + 2 * (size_t)c0, pos0 + c0 + T, s),
            "prefill chunk");
    const bool last = c0 + T == n;
    if (logits && (flags & QR_PREFILL_ALL_LOGITS)) {
      // final norm of every row (x itself is left as is), then the lm_head rows
      DEC_HIP(rmsnorm_launch(d->px, nullptr, d->rms_final, dim, d->pxb, s, T), "k_rmsnorm");
      DEC_HIP(matmul_rows_dev(d, d->wcls, d->wcls_type, d->pxb, logits + (size_t)c0 * d->vocab,
                              d->vocab, dim, T, s),
              "lm_head");
    } else if (logits && last) {
      float* xl = d->px + (size_t)(T - 1) * dim;
      DEC_HIP(rmsnorm_launch(xl, nullptr, d->rms_final, dim, d->pxb, s), "k_rmsnorm");
      DEC_HIP(matmul_q_dev(d->wcls, d->wcls_type, d->order, d->pxb, logits, d->vocab, dim, s),
              "lm_head");
    }
    if (last && x_out)
      DEC_HIP(hipMemcpyAsync(x_out, d->px + (size_t)(T - 1) * dim, (size_t)dim * 4,
                             hipMemcpyDeviceToDevice, s),
              "x_out copy");
  }
  return QR_OK;
}

int qr_decoder_forward(qr_decoder* d, int token, int pos, float* logits, float* x_out) {
  if (!d || !logits) return set_error(QR_ERR_INVALID, "qr_decoder_forward: null argument");
  if (token < 0 || token >= d->vocab)
    return set_error(QR_ERR_INVALID, "qr_decoder_forward: token %d (vocab %d)", token, d->vocab);
  if (pos < 0 || pos >= d->cap)
    return set_error(QR_ERR_INVALID, "qr_decoder_forward: pos %d (seq_len %d)", pos, d->cap);
  if (!al16(logits) || (x_out && !al16(x_out)))
    return set_error(QR_ERR_INVALID, "qr_decoder_forward: output alignment");
  DEC_HIP(hipSetDevice(d->device), "hipSetDevice");
  hipStream_t s = ctx_stream(d->ctx);
  if (ctx_capturing(d->ctx) && (d->flags & QR_DEC_GRAPH))
    return set_error(QR_ERR_INVALID, "qr_decoder_forward: a graph decoder cannot be captured");
  hipLaunchKernelGGL(k_set_state, dim3(1), dim3(64), 0, s, d->st, token, pos);
  DEC_HIP(hipGetLastError(), "k_set_state");
  d->calls++;
  if (!(d->flags & QR_DEC_GRAPH) || d->calls == 1) {
    // eager (the first call of a graph decoder also sets every kernel's
    // attributes outside capture)
    DEC_HIP(enqueue_step(d, logits, x_out, s), "decode step");
    return QR_OK;
  }
  if (!d->exec || d->graph_logits != logits || d->graph_xout != x_out) {
    drop_graph(d);
    DEC_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    const hipError_t e = enqueue_step(d, logits, x_out, s);
    hipGraph_t g = nullptr;
    const hipError_t e2 = hipStreamEndCapture(s, &g);
    if (e != hipSuccess || e2 != hipSuccess) {
      if (g) (void)hipGraphDestroy(g);
      return set_error(QR_ERR_HIP, "qr_decoder_forward: capture: %s",
                       hipGetErrorString(e != hipSuccess ? e : e2));
    }
    d->graph = g;
    DEC_HIP(hipGraphInstantiate(&d->exec, g, nullptr, nullptr, 0), "hipGraphInstantiate");
    d->graph_logits = logits;
    d->graph_xout = x_out;
  }
  DEC_HIP(hipGraphLaunch(d->exec, s), "hipGraphLaunch");
  return QR_OK;
}

}  // extern "C"
