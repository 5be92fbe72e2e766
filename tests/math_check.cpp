// Exhaustive comparison of tsa_math.h against the host libm (expf, exp2f, log2f on [1, 2]).
// Build: g++ -O2 -fopenmp -ffp-contract=off -I treesa_gpu_amd/csrc tests/math_check.cpp -o math_check
// Prints one line "expf_bad exp2f_bad log2_far log2_fixed" and exits 0 iff expf_bad == exp2f_bad ==
// log2_far == 0 (log2_far counts inputs where the uncorrected core is more than 1 ulp from libm, which
// the 2-bit correction table could not express; log2_fixed is how many table entries are nonzero).
#include <cstdio>
#include <cstdlib>
#include <cmath>
#include <cstdint>
#include "tsa_math.h"

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
#pragma omp parallel for reduction(+ : far, fixed) schedule(static)
  for (long long k = 0; k <= (1ll << 23); k++) {
    const float y = tsa_ffrom(0x3f800000u + (uint32_t)k);  // [1, 2], k = 2^23 is 2.0
    const int32_t d = (int32_t)(tsa_fbits(log2f(y)) - tsa_fbits(tsa_log2f_core(y)));
    if (d != 0) fixed++;
    if (d > 1 || d < -1 || (k == (1ll << 23) && d != 0)) far++;
  }
  printf("%lld %lld %lld %lld\n", bad_e, bad_2, far, fixed);
  return (bad_e == 0 && bad_2 == 0 && far == 0) ? 0 : 1;
}
