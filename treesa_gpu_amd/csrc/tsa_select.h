// tsa_select.h -- the level loop's selection score, computed identically by the host (g++) and by the
// device-side best tracking (hipcc).
//
// The reference scores every chain at every evaluated level in double with the host libm
// (csrc/treesa_gpu.cu:1737-1753) and keeps the lowest score over all levels and chains.  Here the score
// is evaluated with the restated double log2 / exp2 below (IEEE +, -, *, / and fma only; compiled with
// -ffp-contract=off) so that a kernel can select the best chain without a host round trip and the host
// level loop selects exactly the same chain.  Both functions are accurate to a few ulp of double; the
// score only orders chains, so its last bits matter only for ties, which both sides now break alike.
#pragma once
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define TSA_SEL_FN __host__ __device__ static inline
#else
#define TSA_SEL_FN static inline
#endif

TSA_SEL_FN uint64_t tsa_sel_bits(double x) {
  uint64_t u;
  memcpy(&u, &x, 8);
  return u;
}
TSA_SEL_FN double tsa_sel_from(uint64_t u) {
  double x;
  memcpy(&x, &u, 8);
  return x;
}
#if defined(__HIPCC__)
#define TSA_SEL_FMA(a, b, c) fma(a, b, c)
#else
#define TSA_SEL_FMA(a, b, c) __builtin_fma(a, b, c)
#endif

// 2^x: x = k + f with k = nearest integer, 2^f = e^(f ln 2) by its Taylor series to degree 14
// (|f ln 2| <= 0.347, remainder < 2e-18), then scaled by 2^k through the exponent bits.
TSA_SEL_FN double tsa_exp2d(double x) {
  if (x != x) return x;
  if (x >= 1024.0) return tsa_sel_from(0x7ff0000000000000ull);
  if (x < -1074.0) return 0.0;
  const double k = x >= 0 ? (double)(int64_t)(x + 0.5) : -(double)(int64_t)(-x + 0.5);
  const double t = (x - k) * 0x1.62e42fefa39efp-1;  // (x - k) ln 2
  double p = 1.0 / 87178291200.0;                    // 1/14!
  p = TSA_SEL_FMA(p, t, 1.0 / 6227020800.0);
  p = TSA_SEL_FMA(p, t, 1.0 / 479001600.0);
  p = TSA_SEL_FMA(p, t, 1.0 / 39916800.0);
  p = TSA_SEL_FMA(p, t, 1.0 / 3628800.0);
  p = TSA_SEL_FMA(p, t, 1.0 / 362880.0);
  p = TSA_SEL_FMA(p, t, 1.0 / 40320.0);
  p = TSA_SEL_FMA(p, t, 1.0 / 5040.0);
  p = TSA_SEL_FMA(p, t, 1.0 / 720.0);
  p = TSA_SEL_FMA(p, t, 1.0 / 120.0);
  p = TSA_SEL_FMA(p, t, 1.0 / 24.0);
  p = TSA_SEL_FMA(p, t, 1.0 / 6.0);
  p = TSA_SEL_FMA(p, t, 0.5);
  p = TSA_SEL_FMA(p, t, 1.0);
  p = TSA_SEL_FMA(p, t, 1.0);
  int ki = (int)k;
  // scale in two steps so that 2^k stays a normal double for k in [-1074, 1023]
  const int k1 = ki / 2, k2 = ki - k1;
  return p * tsa_sel_from((uint64_t)(k1 + 1023) << 52) * tsa_sel_from((uint64_t)(k2 + 1023) << 52);
}

// log2(x) for x > 0: x = 2^e m with m in [sqrt(1/2), sqrt(2)), log m = 2 atanh(s), s = (m-1)/(m+1),
// |s| <= 0.1716, series to s^27 (remainder < 1e-18).  0 -> -inf, negative / NaN -> NaN.
TSA_SEL_FN double tsa_log2d(double x) {
  if (x != x || x < 0) return tsa_sel_from(0x7ff8000000000000ull);
  if (x == 0) return tsa_sel_from(0xfff0000000000000ull);
  if (x == tsa_sel_from(0x7ff0000000000000ull)) return x;
  int e = 0;
  if (x < 0x1p-1022) {  // subnormal: scale into the normal range
    x *= 0x1p54;
    e = -54;
  }
  uint64_t u = tsa_sel_bits(x);
  e += (int)((u >> 52) & 0x7ff) - 1023;
  double m = tsa_sel_from((u & 0x000fffffffffffffull) | 0x3ff0000000000000ull);  // [1, 2)
  if (m > 0x1.6a09e667f3bcdp+0) {
    m *= 0.5;
    e += 1;
  }
  const double s = (m - 1.0) / (m + 1.0), s2 = s * s;
  double p = 1.0 / 27;
  p = TSA_SEL_FMA(p, s2, 1.0 / 25);
  p = TSA_SEL_FMA(p, s2, 1.0 / 23);
  p = TSA_SEL_FMA(p, s2, 1.0 / 21);
  p = TSA_SEL_FMA(p, s2, 1.0 / 19);
  p = TSA_SEL_FMA(p, s2, 1.0 / 17);
  p = TSA_SEL_FMA(p, s2, 1.0 / 15);
  p = TSA_SEL_FMA(p, s2, 1.0 / 13);
  p = TSA_SEL_FMA(p, s2, 1.0 / 11);
  p = TSA_SEL_FMA(p, s2, 1.0 / 9);
  p = TSA_SEL_FMA(p, s2, 1.0 / 7);
  p = TSA_SEL_FMA(p, s2, 1.0 / 5);
  p = TSA_SEL_FMA(p, s2, 1.0 / 3);
  p = TSA_SEL_FMA(p, s2, 1.0);
  return (double)e + (2.0 * s * p) * 0x1.71547652b82fep+0;
}

// Scoring parameters of the level loop.
struct TsaSelect {
  int mode, slicing, select_sc;
  double sc_target, sc_weight;
};

// Population energy |S| + lcost + sc_weight * max(0, sc - sc_target) (csrc/treesa_gpu.cu:1751-1753).
TSA_SEL_FN double tsa_energyE(float lc, int sc, int ns, const TsaSelect& S) {
  const double over = (double)sc - S.sc_target;
  return (double)ns + (double)lc + S.sc_weight * (over > 0.0 ? over : 0.0);
}

// Selection score, lower is better (csrc/treesa_gpu.cu:1737-1748): slicing -> feasibility first, then the
// total cost; --select-sc -> sc excess first; tc mode -> log2(2^tc + w (2^sc - 2^sc_target)); float modes
// -> the population energy.
TSA_SEL_FN double tsa_score(float lc, int sc, int ns, const TsaSelect& S) {
  const double over = (double)sc - S.sc_target;
  if (S.slicing) return (double)ns + (double)lc + 1000.0 * (over > 0.0 ? over : 0.0);
  if (S.select_sc) return 4096.0 * (over > 0.0 ? over : 0.0) + (double)lc;
  if (S.mode == 0) {
    const double tc = (double)lc;
    if ((double)sc <= S.sc_target || S.sc_weight <= 0) return tc;
    const double pen = tsa_log2d(S.sc_weight) + (double)sc + tsa_log2d(1.0 - tsa_exp2d(S.sc_target - (double)sc));
    const double mx = tc > pen ? tc : pen, mn = tc > pen ? pen : tc;
    return mx + tsa_log2d(1.0 + tsa_exp2d(mn - mx));
  }
  return tsa_energyE(lc, sc, ns, S);
}
