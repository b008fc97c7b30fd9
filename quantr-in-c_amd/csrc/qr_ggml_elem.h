// qr_ggml_elem.h -- element access to llama.cpp / ggml K-quant rows
// (block_q4_K 144 B, block_q5_K 176 B, block_q6_K 210 B; ggml-common.h): the
// type ids and one element's dequantized value, for the GEMV's LDS layouts
// and for embedding rows stored in these layouts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qr {

// The reference's own ids of the three K-quants (include/qr_hip.h); the
// ggml layouts are told apart by a flag on top of them.
enum { kGgmlQ4 = 12, kGgmlQ5 = 13, kGgmlQ6 = 14 };

// IEEE half -> float (exact; v_cvt_f32_f16).
__device__ inline float ggml_h2f(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xFFFFu));
}

// dequantize_row_q{4,5,6}_K (ggml-quants.c) of element e of a row.
__device__ inline float ggml_deq_elem(const uint8_t* row, int type, int e) {
  const int i = e >> 8, r = e & 255;
  if (type == kGgmlQ4 || type == kGgmlQ5) {
    const uint8_t* blk = row + (size_t)i * (type == kGgmlQ4 ? 144 : 176);
    const float d = ggml_h2f(blk[0] | (blk[1] << 8)), mn = ggml_h2f(blk[2] | (blk[3] << 8));
    const uint8_t* s = blk + 4;
    const int g = r >> 6, half = (r >> 5) & 1, k = r & 31, j = 2 * g + half;
    int sc, m;
    if (j < 4) {
      sc = s[j] & 63;
      m = s[j + 4] & 63;
    } else {
      sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
      m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
    const uint8_t* qs = blk + (type == kGgmlQ4 ? 16 : 48);
    int q = half ? (qs[32 * g + k] >> 4) : (qs[32 * g + k] & 0xF);
    if (type == kGgmlQ5) q += (blk[16 + k] >> j) & 1 ? 16 : 0;
    const float d1 = d * (float)sc, m1 = mn * (float)m;
    return d1 * (float)q - m1;
  }
  const uint8_t* blk = row + (size_t)i * 210;
  const float d = ggml_h2f(blk[208] | (blk[209] << 8));
  const int n = r >> 7, rr = r & 127, s = rr >> 5, l = rr & 31;
  const uint8_t* ql = blk + 64 * n;
  const uint8_t* qh = blk + 128 + 32 * n;
  const int lo = (s & 1) ? ql[l + 32] : ql[l];
  const int nib = (s & 2) ? (lo >> 4) : (lo & 0xF);
  const int q = (int)(int8_t)(nib | (((qh[l] >> (2 * s)) & 3) << 4)) - 32;
  const int8_t sc = (int8_t)blk[192 + 8 * n + (l >> 4) + 2 * s];
  return d * (float)sc * (float)q;
}

}  // namespace qr
