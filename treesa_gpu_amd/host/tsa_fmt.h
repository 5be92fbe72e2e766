// tsa_fmt.h -- printf's "%.Nf" and "%d", restated for the trace rows of the level loop.  The reference formats
// a row per level with snprintf inside its timed loop (csrc/treesa_gpu.cu:1830-1832); the device-side level
// loop has all of its rows only when the device is done, and formatting 100 of them with snprintf takes about
// 100 us.  These write the same characters in a fraction of that.
#pragma once
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>

namespace tsa {

// Writes x as printf("%.<prec>f", x) does (0 <= prec <= 9) at p, without a terminating NUL; returns the number
// of characters.  Exact: a finite double below 2^52 in magnitude is m * 2^-s with a 53-bit integer m and
// s >= 1, so x * 10^prec = m * 10^prec / 2^s, rounded from 128-bit integers to the nearest integer, ties to
// even (glibc rounds the exact binary value in the default rounding mode).  The sign is written whenever the
// sign bit is set, -0.0 and negative values that round to zero included, as printf does.  Larger magnitudes,
// infinities and NaN go to snprintf itself (at most 330 characters).
inline int fmt_fixed(char* p, double x, int prec) {
  static const uint64_t kPow10[10] = {1ull,      10ull,      100ull,      1000ull,      10000ull,
                                      100000ull, 1000000ull, 10000000ull, 100000000ull, 1000000000ull};
  const double a = std::fabs(x);
  if (!(a < 4503599627370496.0) || prec < 0 || prec > 9) {  // 2^52; NaN fails the comparison
    char b[400];
    const int n = snprintf(b, sizeof b, "%.*f", prec, x);
    std::memcpy(p, b, (size_t)n);
    return n;
  }
  int e = 0;
  const double f = std::frexp(a, &e);                 // a = f * 2^e, f in [0.5, 1) (0 for a == 0)
  const uint64_t m = (uint64_t)std::ldexp(f, 53);     // exact: f has at most 53 significant bits
  const int s = 53 - e;                               // a = m * 2^-s, s >= 1 since a < 2^52
  const uint64_t P = kPow10[prec];
  const unsigned __int128 N = (unsigned __int128)m * P;  // < 2^53 * 2^30
  unsigned __int128 q = 0;  // x * 10^prec rounded: up to 2^52 * 10^9
  if (s < 128) {
    q = N >> s;
    const unsigned __int128 r = N - (q << s), half = (unsigned __int128)1 << (s - 1);
    if (r > half || (r == half && (q & 1))) q++;
  }  // (s >= 128: N / 2^s < 2^83 / 2^128, far below one half)
  int n = 0;
  if (std::signbit(x)) p[n++] = '-';
  uint64_t ip = (uint64_t)(q / P), fp = (uint64_t)(q % P);
  char d[24];
  int k = 0;
  do {
    d[k++] = (char)('0' + ip % 10);
    ip /= 10;
  } while (ip);
  while (k) p[n++] = d[--k];
  if (prec > 0) {
    p[n++] = '.';
    for (int i = prec - 1; i >= 0; i--) {
      p[n + i] = (char)('0' + fp % 10);
      fp /= 10;
    }
    n += prec;
  }
  return n;
}

// printf("%d") / ("%lld"): the decimal digits of v, a '-' before them when negative.
inline int fmt_int(char* p, long long v) {
  int n = 0;
  unsigned long long u = (unsigned long long)v;
  if (v < 0) {
    p[n++] = '-';
    u = 0ull - u;
  }
  char d[24];
  int k = 0;
  do {
    d[k++] = (char)('0' + u % 10);
    u /= 10;
  } while (u);
  while (k) p[n++] = d[--k];
  return n;
}

}  // namespace tsa
