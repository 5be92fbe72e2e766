// tsa_math.h -- float exp/exp2/log2 that return exactly what the host C library returns.
//
// Every Metropolis test of the annealer compares a 24-bit uniform against expf(-beta*dE), and the
// whole-chain energy folds node costs with log2(2^a + 2^b) = mx + log2f(1 + exp2f(mn - mx)).  The
// accept decisions (and therefore whole trajectories) are only reproducible across host and device if
// these three functions return bit-identical floats on both sides, so they are restated here:
//
//  * expf / exp2f: the table method of Szabolcs Nagy's "optimized-routines" (Arm Ltd., published in
//    glibc >= 2.28 as sysdeps/ieee754/flt-32/e_expf.c / e_exp2f.c): x*N/ln2 = k + r with N = 32,
//    2^(k/N) from a 32-entry table of 2^(i/32) (correctly rounded doubles, entry i stored as
//    bits(2^(i/32)) - (i << 47) so that adding k << 47 scales by 2^(k div 32)), and a degree-3
//    polynomial for 2^(r/N) evaluated in double, rounded once to float.  The expf table carries entry
//    31 raised by 30 ulp: with it the restatement agrees with glibc 2.35's expf on all 2^32 inputs
//    (any raise in [12, 47] does; the unraised entry disagrees on exactly two inputs, both in
//    bucket 31).  exp2f agrees with the unraised table on all 2^32 inputs.  Both claims are checked
//    exhaustively by tests/test_math_exhaustive.py against the host libm.
//  * log2f is only ever called on 1 + exp2f(d) with d <= 0, i.e. on [1, 2].  It is evaluated in double
//    (atanh series after halving above sqrt 2), rounded to float, and then corrected by a 2-bit table
//    over the 2^23 floats of [1, 2) that the library's host side fills by comparing this same function
//    with its libm log2f (build_log2_fix in tsa_capi.hip).  The correction is a pure function of the input float, so host and
//    device agree bit for bit wherever the table came from the host libm that the oracle uses.
//
// All arithmetic is IEEE double (+, -, *, / and explicit fma), which is correctly rounded on both
// gfx950 and x86-64; the file must be compiled with -ffp-contract=off so that no further fusing happens.
#pragma once
#include <stdint.h>
#include <string.h>
#include <math.h>

#if defined(__HIPCC__)
#define TSA_MATH_FN __host__ __device__ static inline
#else
#define TSA_MATH_FN static inline
#endif

TSA_MATH_FN uint64_t tsa_dbits(double x) { uint64_t u; memcpy(&u, &x, 8); return u; }
TSA_MATH_FN double tsa_dfrom(uint64_t u) { double x; memcpy(&x, &u, 8); return x; }
TSA_MATH_FN uint32_t tsa_fbits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
TSA_MATH_FN float tsa_ffrom(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

// bits(2^(i/32)) - (i << 47), i = 0..31: 2^(i/32) correctly rounded to double
#define TSA_EXP2_TAB                                                                                  \
  {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,       \
   0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,       \
   0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,       \
   0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,       \
   0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,       \
   0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,       \
   0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,       \
   0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

#if defined(__HIPCC__)
__constant__ static const uint64_t tsa_exp2_tab_d[32] = TSA_EXP2_TAB;
#endif
#if defined(__HIP_DEVICE_COMPILE__)
#define TSA_EXP2_TABLE tsa_exp2_tab_d
#else
static const uint64_t tsa_exp2_tab_h[32] = TSA_EXP2_TAB;
#define TSA_EXP2_TABLE tsa_exp2_tab_h
#endif

// 2^(r/N) polynomial, N = 32 (exp2f form: r in units of 1, scaled for expf below)
#define TSA_EXP2_C0 0x1.c6af84b912394p-5
#define TSA_EXP2_C1 0x1.ebfce50fac4f3p-3
#define TSA_EXP2_C2 0x1.62e42ff0c52d6p-1
#define TSA_EXP_SHIFT 0x1.8p+52
#define TSA_EXP_INVLN2N (0x1.71547652b82fep+0 * 32)
#define TSA_EXPF_RAISE31 30ull

// expf with the 2^(i/32) table passed in (kernels pass a copy staged in LDS: a per-lane index into a
// constant or kernel-argument array would be a vector memory load on every call).
TSA_MATH_FN float tsa_expf_t(float x, const uint64_t* tab) {
  const uint32_t abstop = (tsa_fbits(x) >> 20) & 0x7ff;
  if (abstop >= 0x42b) {  // |x| >= 88: infinities, NaN, overflow and underflow
    if (tsa_fbits(x) == 0xff800000u) return 0.0f;
    if (abstop >= 0x7f8) return x + x;
    if (x > 0x1.62e42ep6f) return INFINITY;
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  const double xd = (double)x;
  const double z = TSA_EXP_INVLN2N * xd;
  double kd = z + TSA_EXP_SHIFT;
  const uint64_t ki = tsa_dbits(kd);
  kd -= TSA_EXP_SHIFT;
  const double r = z - kd;
  const uint32_t i = (uint32_t)(ki & 31u);
  const uint64_t t = tab[i] + (i == 31u ? TSA_EXPF_RAISE31 : 0ull) + (ki << 47);
  const double s = tsa_dfrom(t);
  const double c0 = TSA_EXP2_C0 / 32 / 32 / 32, c1 = TSA_EXP2_C1 / 32 / 32, c2 = TSA_EXP2_C2 / 32;
  const double zz = fma(c0, r, c1);
  const double r2 = r * r;
  double y = fma(c2, r, 1.0);
  y = fma(zz, r2, y);
  return (float)(y * s);
}

TSA_MATH_FN float tsa_exp2f_t(float x, const uint64_t* tab) {
  const uint32_t abstop = (tsa_fbits(x) >> 20) & 0x7ff;
  if (abstop >= 0x430) {  // |x| >= 128
    if (tsa_fbits(x) == 0xff800000u) return 0.0f;
    if (abstop >= 0x7f8) return x + x;
    if (x > 0.0f) return INFINITY;
    if (x <= -150.0f) return 0.0f;
  }
  const double xd = (double)x;
  double kd = xd + TSA_EXP_SHIFT / 32;
  const uint64_t ki = tsa_dbits(kd);
  kd -= TSA_EXP_SHIFT / 32;
  const double r = xd - kd;
  const uint64_t t = tab[ki & 31u] + (ki << 47);
  const double s = tsa_dfrom(t);
  const double zz = fma(TSA_EXP2_C0, r, TSA_EXP2_C1);
  const double r2 = r * r;
  double y = fma(TSA_EXP2_C2, r, 1.0);
  y = fma(zz, r2, y);
  return (float)(y * s);
}

TSA_MATH_FN float tsa_expf(float x) { return tsa_expf_t(x, TSA_EXP2_TABLE); }
TSA_MATH_FN float tsa_exp2f(float x) { return tsa_exp2f_t(x, TSA_EXP2_TABLE); }

// log2(y) in double for y in [1, 2] (float input): halve above sqrt(2), then
// log(v) = 2 atanh(s), s = (v - 1) / (v + 1), |s| <= 0.1716, series to s^23 (error < 1e-17 relative).
TSA_MATH_FN float tsa_log2f_core(float y) {
  double v = (double)y, e = 0.0;
  if (v > 0x1.6a09e667f3bcdp+0) { v *= 0.5; e = 1.0; }
  const double s = (v - 1.0) / (v + 1.0);
  const double s2 = s * s;
  double p = 1.0 / 23;
  p = fma(p, s2, 1.0 / 21);
  p = fma(p, s2, 1.0 / 19);
  p = fma(p, s2, 1.0 / 17);
  p = fma(p, s2, 1.0 / 15);
  p = fma(p, s2, 1.0 / 13);
  p = fma(p, s2, 1.0 / 11);
  p = fma(p, s2, 1.0 / 9);
  p = fma(p, s2, 1.0 / 7);
  p = fma(p, s2, 1.0 / 5);
  p = fma(p, s2, 1.0 / 3);
  p = fma(p, s2, 1.0);
  const double ln = 2.0 * s * p;
  return (float)(e + ln * 0x1.71547652b82fep+0);
}

// Number of 32-bit words of the log2f correction table: 2 bits for each of the 2^23 floats of [1, 2),
// 16 per word, so word mant >> 4 holds mantissa mant.
#define TSA_LOG2FIX_WORDS (1u << 19)

// Words of the summary bitmap of the correction table: bit w is set iff fix word w is nonzero (about one
// word in ten is), so a reader holding the 64 KB bitmap close by skips most reads of the 2 MB table.
#define TSA_LOG2MAP_WORDS (TSA_LOG2FIX_WORDS / 32u)

// log2f on [1, 2] with the host-libm correction table fix (2 bits per input: 0 keep, 1 +1 ulp, 2 -1 ulp)
// and, when map is not null, its summary bitmap.  Inputs outside [1, 2] only arise from NaN operands and
// return NaN.
TSA_MATH_FN float tsa_log2f_12(float y, const uint32_t* fix, const uint32_t* map = nullptr) {
  if (!(y >= 1.0f && y <= 2.0f)) return y - y + NAN;
  const float r = tsa_log2f_core(y);
  if (y == 2.0f) return r;
  const uint32_t mant = tsa_fbits(y) & 0x7fffffu;
  const uint32_t w = mant >> 4;
  if (map && ((map[w >> 5] >> (w & 31u)) & 1u) == 0u) return r;
  const uint32_t code = (fix[w] >> ((mant & 15u) * 2u)) & 3u;
  if (code == 0u) return r;
  return tsa_ffrom(tsa_fbits(r) + (code == 1u ? 1u : 0xffffffffu));
}

// Tables the float math reads: the 2^(i/32) table, the log2f correction table and optionally its summary
// bitmap.
struct TsaMathTabs {
  const uint64_t* exp2;
  const uint32_t* fix;
  const uint32_t* map;
};

// log2(2^a + 2^b) for floats (a or b may be -inf), the fold of modeled node costs.  For min - max <= -24,
// exp2f gives at most 2^-24, 1 + that rounds to 1.0f (2^-24 is half an ulp of 1: ties to even) and
// log2f(1) = +0, so the result is max + 0.0f without evaluating either function.
TSA_MATH_FN float tsa_lse_f(float a, float b, const TsaMathTabs& T) {
  const float mx = a > b ? a : b;
  const float mn = a > b ? b : a;
  if (mx == -INFINITY) return mx;
  const float d = mn - mx;
  if (d <= -24.0f) return mx + 0.0f;
  return mx + tsa_log2f_12(1.0f + tsa_exp2f_t(d, T.exp2), T.fix, T.map);
}
