// qr_norm.h -- rmsnorm_ref (src/kernels.c:170-180) inside the kernel that
// consumes its output: a GEMV's or the router's workgroup normalises the
// residual itself, while its own weight DMA is in flight, instead of waiting
// for a separate normalisation launch to finish.
//
//   ss = ((0 + x0*x0) + x1*x1) + ...      one lane, in element order
//   ss = ss / n + 1e-5f;  scale = 1 / sqrtf(ss)
//   o[j] = w[j] * (x[j] * scale)
//
// Every workgroup that runs it forms the same chain from the same values, so
// all of them hold the same o, bit for bit; one of them may also store o for
// later launches.
#pragma once

#include "qr_common.h"

namespace qr {

// The scale of rmsnorm_ref from the sum of squares.
__device__ inline float rms_scale(float ss, int n) {
  ss = ss / (float)n + 1e-5f;
  return 1.0f / sqrtf(ss);
}

// Widest row normalised inside a consumer kernel.
constexpr int kNormFuseMax = 4096;

// A thread's share of x and w: float4 j is element group tid + j * nthr.
template <int NP>
struct NormRegs {
  float4 x[NP], w[NP];
};

template <int NP>
__device__ inline void norm_load(const float* __restrict__ x, const float* __restrict__ w, int d,
                                 int tid, int nthr, NormRegs<NP>& r) {
  const int d4 = d >> 2;
#pragma unroll
  for (int j = 0; j < NP; j++) {
    const int i4 = tid + j * nthr;
    if (i4 < d4) {
      r.x[j] = reinterpret_cast<const float4*>(x)[i4];
      r.w[j] = reinterpret_cast<const float4*>(w)[i4];
    }
  }
}

// Barrier over LDS work only: vector memory operations (a weight tile's
// DMA) stay in flight across it.
__device__ inline void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
}

// The workgroup's normalisation of the loaded values: squares into xs (d
// floats of LDS), the chain by wave 0, then xs = o (and out = o where out
// is given).  slot: one float of LDS.  Every thread of the workgroup calls
// it; it ends with xs complete for all of them.
template <int NP>
__device__ inline void norm_finish(const NormRegs<NP>& r, int d, float* xs, float* slot, int tid,
                                   int nthr, float* __restrict__ out) {
  const int d4 = d >> 2;
  float4* xs4 = reinterpret_cast<float4*>(xs);
#pragma unroll
  for (int j = 0; j < NP; j++) {
    const int i4 = tid + j * nthr;
    if (i4 < d4) {
      float4 q;
      q.x = r.x[j].x * r.x[j].x;
      q.y = r.x[j].y * r.x[j].y;
      q.z = r.x[j].z * r.x[j].z;
      q.w = r.x[j].w * r.x[j].w;
      xs4[i4] = q;
    }
  }
  lds_barrier();
  if (tid < 64) {  // wave 0
    const float ss = seq_sum_wave<64>(xs, d, tid);
    if (tid == 0) *slot = rms_scale(ss, d);
  }
  lds_barrier();
  const float scale = *slot;
#pragma unroll
  for (int j = 0; j < NP; j++) {
    const int i4 = tid + j * nthr;
    if (i4 < d4) {
      float4 o;
      o.x = r.w[j].x * (r.x[j].x * scale);
      o.y = r.w[j].y * (r.x[j].y * scale);
      o.z = r.w[j].z * (r.x[j].z * scale);
      o.w = r.w[j].w * (r.x[j].w * scale);
      xs4[i4] = o;
      if (out) reinterpret_cast<float4*>(out)[i4] = o;
    }
  }
  lds_barrier();
}

}  // namespace qr
