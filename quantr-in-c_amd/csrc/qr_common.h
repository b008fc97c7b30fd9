// qr_common.h -- block formats and exact scalar numerics shared by the gfx950
// kernels of libqr_hip.so.
//
// Everything here is bit-exact with quantr-in-c's C99 code when compiled with
// -ffp-contract=off (the library's build flag): every float operation rounds
// once, in the written order, as the reference's -std=c99 build does.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// GGML type ids (src/quant.c:478-483).
#define QR_T_F32 0
#define QR_T_Q8_0 8
#define QR_T_Q4_K 12
#define QR_T_Q5_K 13
#define QR_T_Q6_K 14

#define QR_Q8_BYTES 34   // block_q8_0, include/quant.h:28-33
#define QR_Q4K_BYTES 144 // block_q4_K, include/quant.h:35-42
#define QR_Q5K_BYTES 176 // block_q5_K, include/quant.h:44-50
#define QR_Q6K_BYTES 210 // raw Q6_K block, src/quant.c:220-226

// fp16 bits -> fp32 by exponent rebias (include/quant.h:53-66).  Half
// subnormals keep exponent 0 and decode to mant * 2^-136, as in the reference.
// Branch-free: exponent 31 ORs in 0x7F800000, which (the shifted exponent's
// top three bits being clear) is the same as adding 0x70000000; exponents
// 1..30 add the 0x38000000 rebias; exponent 0 adds nothing.
__host__ __device__ inline float qr_h2f(uint32_t h) {
  const uint32_t w = (h & 0x7FFFu) << 13;
  const uint32_t e = h & 0x7C00u;
  const uint32_t adj = e == 0x7C00u ? 0x70000000u : (e != 0 ? 0x38000000u : 0u);
  return __builtin_bit_cast(float, (w + adj) | ((h & 0x8000u) << 16));
}

// Truncating fp32 -> fp16 bits (include/quant.h:68-77): exponents at or below
// zero flush to signed zero, at or above 31 saturate to infinity, the mantissa
// is cut, never rounded.
__host__ __device__ inline uint32_t qr_f2h(float f) {
  const uint32_t x = __builtin_bit_cast(uint32_t, f);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const int e = (int)((x >> 23) & 0xFFu) - 127 + 15;
  if (e <= 0) return sign;
  if (e >= 31) return sign | 0x7C00u;
  return sign | ((uint32_t)e << 10) | ((x >> 13) & 0x3FFu);
}

// expf, bit-exact with glibc's (the reference calls glibc expf in
// softmax_ref, src/kernels.c:200, and silu, src/runtime.c:16).  glibc >= 2.27
// uses the published ARM optimized-routines algorithm (Szabolcs Nagy): with
// N = 32, z = x*N/ln2 is split into an integer k and r = z - k, 2^(k/N) comes
// from a table of the correctly rounded 2^(i/N) with the exponent bits of
// i/N removed, and 2^(r/N) from a cubic, all in double, rounded once to float.
// glibc's x86-64 FMA build fuses the reduction r = x*N/ln2 - k and the cubic's
// multiply-adds; so does this, and with that every float input gives glibc's
// bits (an exhaustive CPU test compares all 2^32 inputs with the host libm).
// 2^(i/32) for i < 32, correctly rounded, with the exponent bits of i/32
// removed (the table of the published algorithm).
constexpr uint64_t kExpTab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

__host__ __device__ inline float qr_expf(float x) {
  constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
  constexpr double kShift = 0x1.8p+52;
  constexpr double kC0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
  constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
  constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  const uint32_t ux = __builtin_bit_cast(uint32_t, x);
  const uint32_t abstop = (ux >> 20) & 0x7FFu;
  if (abstop >= 0x42Bu) {  // |x| >= 88, inf or nan
    if (ux == 0xFF800000u) return 0.0f;         // -inf
    if (abstop >= 0x7F8u) return x + x;          // +inf, nan
    if (x > 0x1.62e42ep6f) return __builtin_bit_cast(float, 0x7F800000u);  // overflow
    if (x < -0x1.9fe368p6f) return 0.0f;         // underflow
  }
  const double xd = (double)x;
  const double z = kInvLn2N * xd;
  double kd = z + kShift;
  const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
  kd -= kShift;
  // glibc's FMA build contracts z - kd into one fused operation
  const double r = __builtin_fma(kInvLn2N, xd, -kd);
  const uint64_t t = kExpTab[ki % 32] + (ki << 47);
  const double s = __builtin_bit_cast(double, t);
  const double p = __builtin_fma(kC0, r, kC1);
  const double r2 = r * r;
  double y = __builtin_fma(kC2, r, 1.0);
  y = __builtin_fma(p, r2, y);
  y = y * s;
  return (float)y;
}

// silu(x) = x / (1 + expf(-x)) (src/runtime.c:15-17).
__host__ __device__ inline float qr_silu(float x) { return x / (1.0f + qr_expf(-x)); }

// The same expf with its table in registers: lane i < 32 of a VGPR pair holds
// kExpTab[i] and a lookup is a ds_bpermute.  A kernel loads the table once, at
// its start next to its other first loads, instead of paying a dependent
// memory round trip in every latency-critical expf.  qr_expf_w must be called
// with every lane of the wave active (a permute reads nothing from inactive
// lanes); its special cases are selects.
struct ExpTab {
  int lo, hi;
};
static __device__ const uint64_t kExpTabDev[32] = {
    kExpTab[0],  kExpTab[1],  kExpTab[2],  kExpTab[3],  kExpTab[4],  kExpTab[5],  kExpTab[6],
    kExpTab[7],  kExpTab[8],  kExpTab[9],  kExpTab[10], kExpTab[11], kExpTab[12], kExpTab[13],
    kExpTab[14], kExpTab[15], kExpTab[16], kExpTab[17], kExpTab[18], kExpTab[19], kExpTab[20],
    kExpTab[21], kExpTab[22], kExpTab[23], kExpTab[24], kExpTab[25], kExpTab[26], kExpTab[27],
    kExpTab[28], kExpTab[29], kExpTab[30], kExpTab[31]};
__device__ inline ExpTab qr_expf_tab() {
  const uint64_t v = kExpTabDev[threadIdx.x & 31];
  return ExpTab{(int)(uint32_t)v, (int)(uint32_t)(v >> 32)};
}
__device__ inline float qr_expf_w(float x, const ExpTab& T) {
  constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
  constexpr double kShift = 0x1.8p+52;
  constexpr double kC0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
  constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
  constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  const uint32_t ux = __builtin_bit_cast(uint32_t, x);
  const uint32_t abstop = (ux >> 20) & 0x7FFu;
  const double xd = (double)x;
  const double z = kInvLn2N * xd;
  double kd = z + kShift;
  const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
  kd -= kShift;
  const double r = __builtin_fma(kInvLn2N, xd, -kd);
  const int ti = (int)(ki & 31u) << 2;
  const uint32_t tlo = (uint32_t)__builtin_amdgcn_ds_bpermute(ti, T.lo);
  const uint32_t thi = (uint32_t)__builtin_amdgcn_ds_bpermute(ti, T.hi);
  const uint64_t t = (((uint64_t)thi << 32) | tlo) + (ki << 47);
  const double s = __builtin_bit_cast(double, t);
  const double p = __builtin_fma(kC0, r, kC1);
  const double r2 = r * r;
  double y = __builtin_fma(kC2, r, 1.0);
  y = __builtin_fma(p, r2, y);
  y = y * s;
  float res = (float)y;
  if (abstop >= 0x42Bu) {  // |x| >= 88, inf or nan
    if (ux == 0xFF800000u) res = 0.0f;                                        // -inf
    else if (abstop >= 0x7F8u) res = x + x;                                   // +inf, nan
    else if (x > 0x1.62e42ep6f) res = __builtin_bit_cast(float, 0x7F800000u);  // overflow
    else if (x < -0x1.9fe368p6f) res = 0.0f;                                  // underflow
  }
  return res;
}
__device__ inline float qr_silu_w(float x, const ExpTab& T) {
  return x / (1.0f + qr_expf_w(-x, T));
}

// Sequential fp32 sums of LDS values (one lane): 256 values per read batch,
// in two register buffers of 32 taken in turn, so the chain of adds does not
// wait on LDS.
__device__ inline void add32(const float4 (&v)[8], float& acc) {
#pragma unroll
  for (int k = 0; k < 8; k++) {
    acc += v[k].x;
    acc += v[k].y;
    acc += v[k].z;
    acc += v[k].w;
  }
}
__device__ inline void read32(const float* __restrict__ p, float4 (&v)[8]) {
#pragma unroll
  for (int k = 0; k < 8; k++) v[k] = *reinterpret_cast<const float4*>(p + 4 * k);
}
// 256 values (unrolled, so no buffer is carried across a loop iteration).
// The scheduling barriers keep each batch's reads where they are written, 32
// adds ahead of their use: left alone, the scheduler sinks them to just
// before the adds that need them and the chain waits on LDS every 8 adds.
__device__ inline void add256_lds(const float* __restrict__ p, float& s) {
  float4 A[8], B[8];
  read32(p, A);
#pragma unroll
  for (int t = 0; t < 256; t += 64) {
    read32(p + t + 32, B);
    __builtin_amdgcn_sched_barrier(0);
    add32(A, s);
    __builtin_amdgcn_sched_barrier(0);
    if (t + 64 < 256) read32(p + t + 64, A);
    __builtin_amdgcn_sched_barrier(0);
    add32(B, s);
    __builtin_amdgcn_sched_barrier(0);
  }
}
// The same sum in batches of 16 reads: fewer registers, for kernels that
// keep several workgroups per CU and sum short rows.
__device__ inline float seq_sum_lds_short(const float* __restrict__ p, int n) {
  float s = 0.0f;
  int i = 0;
  for (; i + 16 <= n; i += 16) {
    float4 v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) v[k] = *reinterpret_cast<const float4*>(p + i + 4 * k);
#pragma unroll
    for (int k = 0; k < 4; k++) {
      s += v[k].x;
      s += v[k].y;
      s += v[k].z;
      s += v[k].w;
    }
  }
  for (; i < n; i++) s += p[i];
  return s;
}


// The same sequential sum ((0 + p[0]) + p[1]) + ... + p[n - 1] by one whole
// wave: all 64 lanes call it and every lane gets the sum.  Lane L holds the
// SEG terms from SEG L on in registers; the running sum goes through lane L's
// terms and then moves one lane up (DPP wave shift), so the chain of adds
// reads registers only: 5.6-5.7 cycles per add at SEG = 64, against 7.1
// with the terms read from LDS in batches.  The last n % SEG terms go one per
// lane, the running sum moving a lane up with each add.  p: 16-byte aligned.
__device__ inline float wave_up1(float v) {
  const int b = __builtin_bit_cast(int, v);
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(b, b, 0x138, 0xF, 0xF, false));
}
template <int SEG>
__device__ inline float seq_sum_wave(const float* __restrict__ p, int n, int lane) {
  static_assert(SEG % 4 == 0 && SEG <= 64, "segments of whole float4s, at most one lane each");
  constexpr int V4 = SEG / 4;
  float s = 0.0f;
  const int nfull = n / SEG;
  for (int s0 = 0; s0 < nfull; s0 += 64) {
    const int nseg = min(64, nfull - s0);
    const float4* q =
        reinterpret_cast<const float4*>(p + (size_t)(s0 + (lane < nseg ? lane : 0)) * SEG);
    float4 v[V4];
#pragma unroll
    for (int k = 0; k < V4; k++) v[k] = q[k];
    float acc = s;
    for (int j = 0;;) {
#pragma unroll
      for (int k = 0; k < V4; k++) {
        acc += v[k].x;
        acc += v[k].y;
        acc += v[k].z;
        acc += v[k].w;
      }
      if (++j == nseg) break;
      acc = wave_up1(acc);
    }
    s = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), nseg - 1));
  }
  const int i0 = nfull * SEG, r = n - i0;  // r < SEG <= 64
  if (r > 0) {
    const float t = lane < r ? p[i0 + lane] : 0.0f;
    float acc = s + t;  // lane l: the sum through term i0 + l after step l
    for (int l = 1; l < r; l++) acc = wave_up1(acc) + t;
    s = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), r - 1));
  }
  return s;
}

__host__ __device__ inline int qr_block_elems(int type) { return type == QR_T_Q8_0 ? 32 : 256; }
__host__ __device__ inline int qr_block_bytes(int type) {
  return type == QR_T_Q8_0 ? QR_Q8_BYTES
       : type == QR_T_Q4_K ? QR_Q4K_BYTES
       : type == QR_T_Q5_K ? QR_Q5K_BYTES
       : type == QR_T_Q6_K ? QR_Q6K_BYTES : 4;
}
// Bytes per weight row, whole blocks only (src/quant.c:477-484).
__host__ __device__ inline size_t qr_wrow_bytes(int type, int d) {
  if (type == QR_T_F32) return (size_t)d * 4u;
  return (size_t)(d / qr_block_elems(type)) * (size_t)qr_block_bytes(type);
}
// 32-element integer units (= fp32 terms) per row.
__host__ __device__ inline int qr_units(int type, int d) {
  return type == QR_T_Q8_0 ? d / 32 : (d / 256) * 8;
}
