// The trace-row formatter (treesa_gpu_amd/host/tsa_fmt.h) against the C library's printf: for every precision
// 0..9, random doubles over all exponents, uniform values of the trace's ranges, exact ties at each precision
// (k / 2^j), signed zeros, values that round up across a power of ten, subnormals, the snprintf fallbacks
// (2^52 and above, infinities, NaN), and integers for fmt_int.  Prints the number of mismatches.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <random>
#include <vector>

#include "tsa_fmt.h"

static long bad = 0, checked = 0;

static void check(double x, int prec) {
  char a[512], b[512];
  const int n = tsa::fmt_fixed(a, x, prec);
  a[n] = 0;
  snprintf(b, sizeof b, "%.*f", prec, x);
  checked++;
  if (std::strcmp(a, b) != 0) {
    if (bad < 10) fprintf(stderr, "%.17g prec %d: %s vs %s\n", x, prec, a, b);
    bad++;
  }
}

int main() {
  std::mt19937_64 g(12345);
  std::vector<double> xs;
  for (int i = 0; i < 100000; i++) {  // random bit patterns: every exponent, both signs
    uint64_t u = g();
    double x;
    std::memcpy(&x, &u, 8);
    xs.push_back(x);
  }
  std::uniform_real_distribution<double> u01(0.0, 1.0);
  for (double hi : {1e-9, 1e-6, 1e-3, 1.0, 20.0, 300.0, 1e4, 1e6, 1e9, 1e12, 4.5e15})
    for (int i = 0; i < 10000; i++) {
      xs.push_back(hi * u01(g));
      xs.push_back(-hi * u01(g));
      xs.push_back((double)(float)(hi * u01(g)));  // float values widened, as lc and beta are
    }
  for (int j = 0; j <= 40; j++)  // exact ties and their neighbours
    for (int k = 0; k < 1000; k++) {
      const double x = std::ldexp((double)(2 * k + 1), -j);
      xs.push_back(x);
      xs.push_back(-x);
      xs.push_back(std::nextafter(x, 0.0));
      xs.push_back(std::nextafter(x, 1e300));
    }
  for (int p = 0; p <= 9; p++)  // rounding across a power of ten: 0.99995, 9.9999995, ...
    for (int d = 0; d <= 12; d++) {
      const double x = std::pow(10.0, d) - 0.5 * std::pow(10.0, -p);
      xs.push_back(x);
      xs.push_back(std::nextafter(x, 0.0));
      xs.push_back(std::nextafter(x, 1e300));
    }
  for (double x : {0.0, -0.0, 5e-324, -5e-324, 2.2250738585072014e-308, 4503599627370495.5, 4503599627370496.0,
                   -4503599627370496.0, 1e300, -1e300, std::numeric_limits<double>::infinity(),
                   -std::numeric_limits<double>::infinity(), std::numeric_limits<double>::quiet_NaN()})
    xs.push_back(x);
  for (double x : xs)
    for (int p = 0; p <= 9; p++) check(x, p);
  for (long long v : {0ll, 1ll, -1ll, 9ll, 10ll, -10ll, 2147483647ll, -2147483648ll, 9223372036854775807ll,
                      -9223372036854775807ll - 1}) {
    char a[32], b[32];
    const int n = tsa::fmt_int(a, v);
    a[n] = 0;
    snprintf(b, sizeof b, "%lld", v);
    checked++;
    if (std::strcmp(a, b) != 0) bad++;
  }
  for (int i = 0; i < 200000; i++) {
    const long long v = (long long)g() >> (g() % 64);
    char a[32], b[32];
    const int n = tsa::fmt_int(a, v);
    a[n] = 0;
    snprintf(b, sizeof b, "%lld", v);
    checked++;
    if (std::strcmp(a, b) != 0) bad++;
  }
  printf("%ld %ld\n", bad, checked);
  return 0;
}
