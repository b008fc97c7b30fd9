// qr_route.h -- the MoE router's exact arithmetic as device helpers shared by
// the T-token kernels (qr_moe.hip) and the one-token kernels (qr_moe_t1.hip):
// softmax_ref + top-K + renormalisation of one token by one wave, and the
// router logit chains in the reference build's accumulation orders.
#pragma once

#include "qr_common.h"

namespace qr {

constexpr float kMask = -1e9f;  // src/runtime.c:211, 221

// Maximum of v over the wave, in every lane: DPP butterflies inside each 16-lane
// row (quad xor 1, xor 2, half-row mirror, row mirror), then the four row
// maxima read with readlane.  A max, so the order of the steps is free.
__device__ inline float wave_max(float v) {
  auto step = [&](float o) { v = o > v ? o : v; };
  step(__builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
  step(__builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
  step(__builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)));
  step(__builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)));
  float m = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
#pragma unroll
  for (int r = 1; r < 4; r++) {
    const float o = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16 * r));
    m = o > m ? o : m;
  }
  return m;
}

__device__ inline void wave_lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Order-preserving keys of the non-NaN floats (-0 folded into +0): a larger
// float has a larger key; every float maps to a key >= 1 except the NaNs with
// all bits set (excluded by the callers).
__device__ inline uint32_t ord_key(float v) {
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ inline float unord_key(uint32_t k) {
  return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
__device__ inline uint32_t wave_max_u32(uint32_t v) {
  auto step = [&](uint32_t o) { v = o > v ? o : v; };
  step((uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  step((uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  step((uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  step((uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  uint32_t m = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
#pragma unroll
  for (int r = 1; r < 4; r++) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_readlane((int)v, 16 * r);
    m = o > m ? o : m;
  }
  return m;
}

// A wave's LDS routing row: the E exponentials (later the E 64-bit rank keys
// of route_rank_wg), then the E probabilities, then the winners of the argmax
// passes and their probabilities (slot order).
constexpr int kRouteRow = 512 + 256 + 32;  // floats
__device__ inline uint64_t* route_keys(float* pw) { return reinterpret_cast<uint64_t*>(pw); }
__device__ inline float* route_probs(float* pw) { return pw + 512; }
__device__ inline int* route_idx(float* pw) { return reinterpret_cast<int*>(pw + 768); }
__device__ inline float* route_wts(float* pw) { return pw + 784; }

// softmax_ref of one token's E logits (src/kernels.c:191-207) by one wave; `pw`
// is a wave-private LDS routing row, `tab` the expf table (qr_expf_tab).  Lane
// l gets the probabilities of e = l, l + 64, l + 128, l + 192 in pv (entries
// past E: -1e9f); `probs` (optional) receives the softmax.
__device__ inline void route_softmax(const float* __restrict__ lg, int E, float* pw, int lane,
                                     float* __restrict__ probs, const ExpTab& tab,
                                     float (&pv)[4]) {
  // the logits into registers with one batch of loads (E <= 256)
  float lv[4];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int e = lane + 64 * q;
    lv[q] = e < E ? lg[e] : 0.0f;
  }
  // max: seeded with x[0], strictly greater wins (src/kernels.c:192-197);
  // a max, so the lane split does not change it
  float mx = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lv[0]), 0));
#pragma unroll
  for (int q = 0; q < 4; q++)
    if (lane + 64 * q < E && lv[q] > mx) mx = lv[q];
  mx = wave_max(mx);
  float ev[4];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    ev[q] = 0.0f;
    if (64 * q >= E) break;  // uniform
    ev[q] = qr_expf_w(lv[q] - mx, tab);  // every lane
    if (lane + 64 * q < E) pw[lane + 64 * q] = ev[q];
  }
  wave_lds_fence();
  // sequential sum, e ascending (src/kernels.c:198-202), in lane 0: 32
  // exponentials per step, the next step's loads issued before this step's adds
  float inv = 0.0f;
  if (lane == 0) {
    float sum = 0.0f;
    const int e32 = E & ~31;
    float4 cur[8], nxt[8];
    if (e32 > 0) {
#pragma unroll
      for (int k = 0; k < 8; k++) cur[k] = *reinterpret_cast<const float4*>(pw + 4 * k);
    }
    for (int e = 0; e < e32; e += 32) {
      const bool more = e + 32 < e32;
      if (more) {
#pragma unroll
        for (int k = 0; k < 8; k++) nxt[k] = *reinterpret_cast<const float4*>(pw + e + 32 + 4 * k);
      }
#pragma unroll
      for (int k = 0; k < 8; k++) {
        sum += cur[k].x;
        sum += cur[k].y;
        sum += cur[k].z;
        sum += cur[k].w;
      }
      if (more) {
#pragma unroll
        for (int k = 0; k < 8; k++) cur[k] = nxt[k];
      }
    }
    for (int e = e32; e < E; e++) sum += pw[e];
    inv = 1.0f / sum;
  }
  inv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, inv), 0));
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int e = lane + 64 * q;
    pv[q] = kMask;
    if (e < E) {
      const float v = ev[q] * inv;
      pv[q] = v;
      if (probs) probs[e] = v;
    }
  }
  wave_lds_fence();  // every read of the exponentials is done
}

// The argmax passes (src/runtime.c:210-222) all reduce to one order: a scan
// from -1e9f with a strict '>' picks the first index holding the largest value
// among those above -1e9f (NaNs never win), i.e. the lowest index whose value
// equals (as a float: -0 == +0) the maximum; its own value is the weight, and
// the winner is masked with -1e9f for the next pass.  So pass k's winner is
// the entry of rank k under the key (ordered value, then lower index), and a
// pass with no candidate left yields index -1 with weight -1e9f.
__device__ inline uint64_t route_key(float p, int e) {
  return p > kMask ? ((uint64_t)ord_key(p) << 32) | (uint64_t)(0xFFFFu - (uint32_t)e) : 0ull;
}

// The first `npass` argmax passes by one wave from the probabilities pv (see
// route_softmax): per pass a wave max of the keys' value parts, then ballots
// for the lowest lane holding it, e block by e block.  Winners land in
// route_idx(pw)[0 .. npass) and route_wts(pw)[...].
__device__ inline void route_passes(float (&pv)[4], int E, int npass, float* pw, int lane) {
#pragma unroll 1
  for (int k = 0; k < npass; k++) {
    uint32_t key = 0;
#pragma unroll
    for (int q = 0; q < 4; q++)
      if (lane + 64 * q < E && pv[q] > kMask) {
        const uint32_t kq = ord_key(pv[q]);
        key = kq > key ? kq : key;
      }
    key = wave_max_u32(key);
    int win = -1;
    float wv = kMask;
    if (key != 0u) {
      const float m = unord_key(key);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint64_t bal = __ballot(lane + 64 * q < E && pv[q] > kMask && pv[q] == m);
        if (bal != 0ull) {
          const int l = __builtin_ctzll(bal);
          win = l + 64 * q;
          wv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pv[q]), l));
          break;
        }
      }
    }
    if (lane == 0) {
      route_idx(pw)[k] = win;
      route_wts(pw)[k] = wv;
    }
#pragma unroll
    for (int q = 0; q < 4; q++)
      if (win == lane + 64 * q) pv[q] = kMask;
  }
  wave_lds_fence();
}

// softmax + the first `npass` (<= K) argmax passes of one token by one wave.
__device__ inline void route_select(const float* __restrict__ lg, int E, int npass, float* pw,
                                    int lane, float* __restrict__ probs, const ExpTab& tab) {
  float pv[4];
  route_softmax(lg, E, pw, lane, probs, tab, pv);
  route_passes(pv, E, npass, pw, lane);
}

// Workgroup-parallel top-K, in two steps around the caller's barriers:
//   route_rank_keys  one wave (after route_softmax) writes the E keys and
//                    probabilities and clears the K winner slots;
//   -- barrier --
//   route_rank_wg    every thread of the workgroup (nthr >= E) counts, for
//                    candidate e = t / G, the keys above its own in its 1/G of
//                    the E keys (G = nthr / E rounded down to 1, 2 or 4), the G
//                    counts are added across adjacent lanes, and candidates of
//                    rank < K write themselves to their slot.
//   -- barrier --
__device__ inline void route_rank_keys(const float (&pv)[4], int E, int K, float* pw, int lane) {
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int e = lane + 64 * q;
    if (e < E) {
      route_keys(pw)[e] = route_key(pv[q], e);
      route_probs(pw)[e] = pv[q];
    }
  }
  if (lane < K) {
    route_idx(pw)[lane] = -1;
    route_wts(pw)[lane] = kMask;
  }
}
__device__ inline int route_rank_groups(int E, int nthr) {
  return nthr >= 4 * E ? 4 : nthr >= 2 * E ? 2 : 1;
}
template <int G>
__device__ inline void route_rank_wg_g(int E, int K, float* pw, int t, int nthr) {
  const int e = t / G, g = t % G;
  const bool live = e < E;
  const uint64_t* keys = route_keys(pw);
  const uint64_t mine = live ? keys[e] : ~0ull;
  // this thread counts the keys j = g, g + G, g + 2G, ...: the G threads of a
  // candidate read adjacent keys, so one read instruction touches G adjacent
  // 8-byte words (distinct LDS banks) and broadcasts each
  int c0 = 0, c1 = 0, c2 = 0, c3 = 0;
  int j = g;
  for (; j + 15 * G < E; j += 16 * G) {
    uint64_t k16[16];
#pragma unroll
    for (int u = 0; u < 16; u++) k16[u] = keys[j + u * G];
#pragma unroll
    for (int u = 0; u < 16; u += 4) {
      c0 += k16[u] > mine;
      c1 += k16[u + 1] > mine;
      c2 += k16[u + 2] > mine;
      c3 += k16[u + 3] > mine;
    }
  }
  for (; j < E; j += G) c0 += keys[j] > mine;
  int r = (c0 + c1) + (c2 + c3);
  if (G >= 2) r += __builtin_amdgcn_update_dpp(0, r, 0xB1, 0xF, 0xF, false);  // lane ^ 1
  if (G >= 4) r += __builtin_amdgcn_update_dpp(0, r, 0x4E, 0xF, 0xF, false);  // lane ^ 2
  if (live && g == 0 && mine != 0ull && r < K) {
    route_idx(pw)[r] = e;
    route_wts(pw)[r] = route_probs(pw)[e];
  }
  (void)nthr;
}
// Every thread of the workgroup must call (the DPP adds need whole waves).
__device__ inline void route_rank_wg(int E, int K, float* pw, int t, int nthr) {
  switch (route_rank_groups(E, nthr)) {
    case 4: route_rank_wg_g<4>(E, K, pw, t, nthr); break;
    case 2: route_rank_wg_g<2>(E, K, pw, t, nthr); break;
    default: route_rank_wg_g<1>(E, K, pw, t, nthr); break;
  }
}

// Renormalised routing weights w_k / sum(w), the sum sequential in slot order
// (src/runtime.c:224-230), written with the indices by lane 0 (from the
// routing row filled by route_select with K passes).
__device__ inline void route_write(const float* pw, int K, int lane, int32_t* __restrict__ idx,
                                   float* __restrict__ wts) {
  if (lane == 0) {
    const int* ri = reinterpret_cast<const int*>(pw + 768);
    const float* rw = pw + 784;
    float wsum = 0.0f;  // src/runtime.c:224-230
    for (int k = 0; k < K; k++) wsum += rw[k];
    for (int k = 0; k < K; k++) {
      idx[k] = ri[k];
      wts[k] = rw[k] / wsum;
    }
  }
}

// softmax_ref + top-K + renormalisation of one token by one wave; `pw` is a
// wave-private LDS routing row (kRouteRow floats).
__device__ inline void route_one(const float* __restrict__ lg, int E, int K, float* pw, int lane,
                                 float* __restrict__ probs, int32_t* __restrict__ idx,
                                 float* __restrict__ wts) {
  route_select(lg, E, K, pw, lane, probs, qr_expf_tab());
  route_write(pw, K, lane, idx, wts);
}

// FMA chain over j = k, k + LANES, ... < dm out of LDS, 16 steps' operands
// read before their FMAs.
template <int LANES>
__device__ inline float lds_chain(const float* w, const float* x, int k, int dm) {
  float acc = 0.0f;
  int j = k;
  for (; j + 15 * LANES < dm; j += 16 * LANES) {
    float wv[16], xv[16];
#pragma unroll
    for (int q = 0; q < 16; q++) {
      wv[q] = w[j + q * LANES];
      xv[q] = x[j + q * LANES];
    }
#pragma unroll
    for (int q = 0; q < 16; q++) acc = __builtin_fmaf(wv[q], xv[q], acc);
  }
  for (; j < dm; j += LANES) acc = __builtin_fmaf(w[j], x[j], acc);
  return acc;
}

}  // namespace qr
