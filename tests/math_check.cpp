// Exhaustive comparison of tsa_math.h against the host libm (expf, exp2f, log2f on [1, 2]).
// Build: g++ -O2 -fopenmp -ffp-contract=off -I treesa_gpu_amd/csrc tests/math_check.cpp -o math_check
// Prints one line "expf_bad exp2f_bad log2_far log2_fixed lse_bad" and exits 0 iff expf_bad == exp2f_bad ==
// log2_far == lse_bad == 0 (log2_far counts inputs where the uncorrected core is more than 1 ulp from libm,
// which the 2-bit correction table could not express; log2_fixed is how many table entries are nonzero;
// lse_bad counts pairs where tsa_lse_f differs from max + log2f(1 + exp2f(min - max)) with this libm).
#include <cstdio>
#include <cstdlib>
#include <cmath>
#include <cstdint>
#include <vector>
#include "tsa_math.h"

// The reference's lse_f with this libm (csrc/common.h:125): max + log2f(1 + exp2f(min - max)).
static float lse_libm(float a, float b) {
  const float mx = a > b ? a : b, mn = a > b ? b : a;
  if (mx == -INFINITY) return mx;
  return mx + log2f(1.0f + exp2f(mn - mx));
}

int main(int argc, char** argv) {
  const uint64_t stride = argc > 1 ? strtoull(argv[1], nullptr, 10) : 1;  // 1 = every float
  long long bad_e = 0, bad_2 = 0, far = 0, fixed = 0;
#pragma omp parallel for reduction(+ : bad_e, bad_2) schedule(static)
  for (long long u = 0; u < 0x100000000ll; u += (long long)stride) {
    const float x = tsa_ffrom((uint32_t)u);
    const float g1 = expf(x), g2 = exp2f(x);
    const float m1 = tsa_expf(x), m2 = tsa_exp2f(x);
    if (tsa_fbits(g1) != tsa_fbits(m1) && !(std::isnan(g1) && std::isnan(m1))) bad_e++;
    if (tsa_fbits(g2) != tsa_fbits(m2) && !(std::isnan(g2) && std::isnan(m2))) bad_2++;
  }
  std::vector<uint32_t> fix(TSA_LOG2FIX_WORDS + TSA_LOG2MAP_WORDS, 0u);
#pragma omp parallel for reduction(+ : far, fixed) schedule(static)
  for (long long k = 0; k <= (1ll << 23); k++) {
    const float y = tsa_ffrom(0x3f800000u + (uint32_t)k);  // [1, 2], k = 2^23 is 2.0 (log2f_12 returns 1)
    const int32_t d = (int32_t)(tsa_fbits(log2f(y)) - tsa_fbits(k == (1ll << 23) ? 1.0f : tsa_log2f_core(y)));
    if (d != 0) fixed++;
    if (d > 1 || d < -1 || (k == (1ll << 23) && d != 0)) far++;
  }
  // the correction table and its summary bitmap, as the library builds them
  for (uint32_t k = 0; k < (1u << 23); k++) {
    const float y = tsa_ffrom(0x3f800000u + k);
    const int32_t d = (int32_t)(tsa_fbits(log2f(y)) - tsa_fbits(tsa_log2f_core(y)));
    const uint32_t code = d == 1 ? 1u : d == -1 ? 2u : 0u;
    fix[k >> 4] |= code << ((k & 15u) * 2u);
  }
  for (uint32_t w = 0; w < TSA_LOG2FIX_WORDS; w++)
    if (fix[w]) fix[TSA_LOG2FIX_WORDS + (w >> 5)] |= 1u << (w & 31u);
  // tsa_lse_f (table lookups through the bitmap, the exact shortcut below 2^-24) against the libm formula:
  // pairs on a grid of maxima and differences, dense around the shortcut's threshold d = -24
  uint64_t tab[32];
  for (int i = 0; i < 32; i++) tab[i] = tsa_exp2_tab_h[i];
  const TsaMathTabs T{tab, fix.data(), fix.data() + TSA_LOG2FIX_WORDS, tsa_log2_tab_h};
  const TsaMathTabs T0{tab, fix.data(), nullptr, tsa_log2_tab_h};
  long long bad_lse = 0;
#pragma omp parallel for reduction(+ : bad_lse) schedule(static)
  for (int ia = 0; ia < 4096; ia++) {
    uint32_t st = 0x9e3779b9u * (uint32_t)(ia + 1);
    const float a = ia == 0 ? -0.0f : ia == 1 ? INFINITY : ia == 2 ? -INFINITY : ia == 3 ? NAN
                  : ia < 2048 ? (float)(ia % 200) - 20.0f
                                                 : tsa_ffrom(0x3f000000u + (uint32_t)ia * 4093u) * 97.0f;
    for (int j = 0; j < 4096; j++) {
      st = st * 1664525u + 1013904223u;
      float d;
      if (j < 1024) d = -24.0f + (float)(j - 512) * 0x1p-10f;        // around the threshold
      else if (j < 1040) d = tsa_ffrom(tsa_fbits(-24.0f) + (uint32_t)(j - 1032));  // neighbours of -24
      else if (j == 1040) d = -INFINITY;
      else if (j == 1041) d = NAN;
      else if (j == 1042) d = 0.0f;
      else if (j == 1043) d = -0.0f;
      else d = -40.0f * (float)(st >> 8) * 0x1p-24f;
      const float b = a + d;
      // both argument orders (with a NaN operand the formula is not symmetric), the second without the
      // bitmap; NaN results compare as NaN (payloads are not specified)
      const float r0 = lse_libm(a, b), r1 = tsa_lse_f(a, b, T), q0 = lse_libm(b, a), q1 = tsa_lse_f(b, a, T0);
      if (std::isnan(r0) ? !std::isnan(r1) : tsa_fbits(r0) != tsa_fbits(r1)) bad_lse++;
      if (std::isnan(q0) ? !std::isnan(q1) : tsa_fbits(q0) != tsa_fbits(q1)) bad_lse++;
    }
  }
  printf("%lld %lld %lld %lld %lld\n", bad_e, bad_2, far, fixed, bad_lse);
  return (bad_e == 0 && bad_2 == 0 && far == 0 && bad_lse == 0) ? 0 : 1;
}
