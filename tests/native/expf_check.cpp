// expf_check.cpp -- test-only host helper: compiles the library's exact-expf
// restatement (quantr-in-c_amd/csrc/qr_common.h, the same source the gfx950
// kernels use) for the host and compares it with the C library's expf, which
// is what the reference calls (src/kernels.c:200, src/runtime.c:16).
//
// Built by __graft_entry__.build() into tests/native/libexpf_check.so.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "../../quantr-in-c_amd/csrc/qr_common.h"

extern "C" {

// Mismatches of qr_expf vs expf over float bit patterns [lo, hi) with a
// stride; NaN inputs are skipped.  The first mismatching input (bits) goes to
// *first (or 0xFFFFFFFF when none).
long long qrh_expf_mismatches(uint32_t lo, uint64_t hi, uint32_t stride, uint32_t* first) {
  long long bad = 0;
  uint32_t f0 = 0xFFFFFFFFu;
#pragma omp parallel for reduction(+ : bad) schedule(static)
  for (long long u = lo; u < (long long)hi; u += stride) {
    const uint32_t b = (uint32_t)u;
    float x;
    memcpy(&x, &b, 4);
    if (x != x) continue;
    const float a = expf(x), c = qr_expf(x);
    uint32_t ua, uc;
    memcpy(&ua, &a, 4);
    memcpy(&uc, &c, 4);
    if (ua != uc) {
      bad++;
#pragma omp critical
      if (b < f0) f0 = b;
    }
  }
  if (first) *first = f0;
  return bad;
}

void qrh_expf_batch(const float* x, float* y, long n) {
  for (long i = 0; i < n; i++) y[i] = qr_expf(x[i]);
}

void qrh_h2f_batch(const uint16_t* h, float* y, long n) {
  for (long i = 0; i < n; i++) y[i] = qr_h2f(h[i]);
}

void qrh_f2h_batch(const float* x, uint16_t* y, long n) {
  for (long i = 0; i < n; i++) y[i] = (uint16_t)qr_f2h(x[i]);
}

}  // extern "C"
