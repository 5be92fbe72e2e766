// The level loop's device-side selection score (tsa_select.h: tsa_exp2d / tsa_log2d series) against the
// reference's formula with the host libm's exp2 / log2 (csrc/treesa_gpu.cu:1737-1748).
//   1. ulp error of tsa_exp2d and tsa_log2d against libm over the arguments the score passes them:
//      exp2 of sc_target - sc and of mn - mx (all doubles of [-1100, 0] on a dense grid plus random ones),
//      log2 of sc_weight, of 1 - 2^d and of 1 + 2^d;
//   2. the tc-mode score of random populations (sc above the target, tc and penalties close): the largest
//      score difference in ulps, and whether the best chain (lowest score, first on ties) ever differs.
// Build: g++ -O2 -ffp-contract=off -I treesa_gpu_amd/csrc tests/select_check.cpp
// Prints one JSON line.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>
#include "tsa_select.h"

static int64_t ulps(double a, double b) {
  if (a == b) return 0;
  if (a != a || b != b) return INT64_MAX;
  int64_t ia, ib;
  memcpy(&ia, &a, 8);
  memcpy(&ib, &b, 8);
  if (ia < 0) ia = INT64_MIN - ia;
  if (ib < 0) ib = INT64_MIN - ib;
  return ia > ib ? ia - ib : ib - ia;
}

static double glibc_score(float lc, int sc, double sct, double w) {
  const double tc = (double)lc;
  if ((double)sc <= sct || w <= 0) return tc;
  const double pen = std::log2(w) + (double)sc + std::log2(1.0 - std::exp2(sct - (double)sc));
  const double mx = tc > pen ? tc : pen, mn = tc > pen ? pen : tc;
  return mx + std::log2(1.0 + std::exp2(mn - mx));
}

int main() {
  std::mt19937_64 rng(12345);
  std::uniform_real_distribution<double> U(0.0, 1.0);
  int64_t e_exp2 = 0, e_log2 = 0;
  long long n_exp2 = 0, n_log2 = 0;
  for (long long i = 0; i <= 11000000; i++) {  // dense grid of [-1100, 0]
    const double x = -1100.0 * (double)i / 11000000.0;
    e_exp2 = std::max(e_exp2, ulps(tsa_exp2d(x), std::exp2(x)));
    n_exp2++;
  }
  for (int i = 0; i < 4000000; i++) {
    const double x = -std::pow(2.0, -60.0 + 71.0 * U(rng));  // tiny to about -2048 in magnitude
    if (x >= -1100.0) {
      e_exp2 = std::max(e_exp2, ulps(tsa_exp2d(x), std::exp2(x)));
      n_exp2++;
    }
    const double d = -60.0 * U(rng);
    const double a = 1.0 - std::exp2(d), b = 1.0 + std::exp2(d), w = std::pow(10.0, -3.0 + 9.0 * U(rng));
    for (double y : {a, b, w}) {
      if (y > 0) {
        e_log2 = std::max(e_log2, ulps(tsa_log2d(y), std::log2(y)));
        n_log2++;
      }
    }
  }
  // populations: 128 chains, tc in [20, 60], sc a few above the target, sc_weight 1 or 4
  int64_t e_score = 0;
  long long pops = 0, best_diff = 0, close_pairs = 0;
  for (int p = 0; p < 20000; p++) {
    const double sct = 20.0 + (double)(p % 20), w = (p & 1) ? 1.0 : 4.0;
    TsaSelect S{0, 0, 0, sct, w};
    int bd = -1, bg = -1;
    double sd = INFINITY, sg = INFINITY;
    std::vector<double> g(128);
    for (int c = 0; c < 128; c++) {
      const float lc = (float)(20.0 + 40.0 * U(rng));
      const int sc = (int)sct + (int)(8 * U(rng)) - 2;
      const double a = tsa_score(lc, sc, 0, S), b = glibc_score(lc, sc, sct, w);
      e_score = std::max(e_score, ulps(a, b));
      g[c] = b;
      if (a < sd) { sd = a; bd = c; }
      if (b < sg) { sg = b; bg = c; }
    }
    for (int c = 0; c < 128; c++)
      if (c != bg && g[c] != sg && ulps(g[c], sg) <= 8) close_pairs++;
    pops++;
    best_diff += bd != bg;
  }
  printf("{\"exp2_max_ulp\": %lld, \"exp2_args\": %lld, \"log2_max_ulp\": %lld, \"log2_args\": %lld, "
         "\"score_max_ulp\": %lld, \"populations\": %lld, \"best_chain_differs\": %lld, "
         "\"glibc_near_ties_within_8ulp\": %lld}\n",
         (long long)e_exp2, n_exp2, (long long)e_log2, n_log2, (long long)e_score, pops, best_diff, close_pairs);
  return 0;
}
