// The Metropolis threshold of tsa_arith.h, exhaustively.  Metropolis accepts when u < expf(x); the sweep
// kernels that draw their random numbers ahead test x >= T(u) instead, with T(u) = tsa_accept_threshold.  That
// is the same decision for every x exactly when (1) the restated expf is non-decreasing over the floats, so that
// {x : expf(x) > u} is every float from some least one up, and (2) T(u) is that least float: expf(T) > u and
// expf(next float below T) <= u.  (1) is checked over all 2^32 floats in value order, (2) for every uniform the
// kernels draw, u = k * 2^-24 for k = 0 .. 2^24 - 1.
// Build: g++ -O2 -fopenmp -ffp-contract=off -I treesa_gpu_amd/csrc tests/threshold_check.cpp
// Prints "drops bad_thresholds nan_thresholds" and exits 0 iff all three are 0.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include "tsa_arith.h"

// the float with value-order index i (0: -inf, ...; the floats from -inf to +inf, -0 and +0 once each)
static float by_value(int64_t i) {
  const int64_t nneg = 0x7F800000ll + 1;  // -inf .. -0 as bit patterns 0xFF800000 .. 0x80000000
  if (i < nneg) return tsa_ffrom((uint32_t)(0xFF800000ll - i));
  return tsa_ffrom((uint32_t)(i - nneg + 1));  // +denorm_min .. +inf (+0 equals -0 in value)
}

int main() {
  const int64_t n = 2 * (0x7F800000ll + 1) - 1;
  long long drops = 0;
#pragma omp parallel for reduction(+ : drops) schedule(static)
  for (int64_t i = 1; i < n; i++)
    if (tsa_expf(by_value(i)) < tsa_expf(by_value(i - 1))) drops++;
  long long bad = 0, nans = 0;
#pragma omp parallel for reduction(+ : bad, nans) schedule(static)
  for (int64_t k = 0; k < (1 << 24); k++) {
    const uint32_t r = (uint32_t)k << 8;
    const float u = (float)k * (1.0f / 16777216.0f);
    const float T = tsa_accept_threshold(r, TSA_EXP2_TABLE);
    if (T != T) {
      nans++;
      continue;
    }
    const float below = std::nextafter(T, -INFINITY);
    if (!(tsa_expf(T) > u) || tsa_expf(below) > u) bad++;
  }
  printf("%lld %lld %lld\n", drops, bad, nans);
  return drops == 0 && bad == 0 && nans == 0 ? 0 : 1;
}
