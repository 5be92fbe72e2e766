// tsa_population.cpp -- the level loop's host arithmetic: the selection score of a chain, the population
// energy, and the ancestor lists of the two population schemes.  All in double with the host libm, as the
// reference's level loop computes them (csrc/treesa_gpu.cu:1737-1753, 1836-1869).
#include <algorithm>
#include <cmath>
#include <numeric>

#include "tsa_host.h"

namespace tsa {

double population_energy(const Scoring& S, float lc, int sc, int ns) {
  const double excess = std::max(0.0, (double)sc - S.sc_target);
  return (double)ns + (double)lc + S.sc_weight * excess;
}

double selection_score(const Scoring& S, float lc, int sc, int ns) {
  const double excess = std::max(0.0, (double)sc - S.sc_target);
  if (S.slicing) return (double)ns + (double)lc + 1000.0 * excess;  // feasible trees rank first
  if (S.select_sc) return 4096.0 * excess + (double)lc;             // the sc excess ranks first
  if (S.mode != 0) return population_energy(S, lc, sc, ns);
  // omeco's ScoreFunction 2^tc + w (2^sc - 2^sc_target) in log2: log2 of the sum of the two terms
  if (excess <= 0.0 || S.sc_weight <= 0) return (double)lc;
  const double tc = (double)lc;
  const double penalty = std::log2(S.sc_weight) + (double)sc + std::log2(1.0 - std::exp2(S.sc_target - (double)sc));
  const double big = tc > penalty ? tc : penalty, small = tc > penalty ? penalty : tc;
  return big + std::log2(1.0 + std::exp2(small - big));
}

std::vector<int> systematic_ancestors(const std::vector<double>& E, double db, double u) {
  const int n = (int)E.size();
  std::vector<int> anc(n, n - 1);
  if (n == 0) return anc;
  const double emin = *std::min_element(E.begin(), E.end());
  std::vector<double> w(n);
  double total = 0;
  for (int c = 0; c < n; c++) total += (w[c] = std::exp(-db * (E[c] - emin)));
  // chain c owns the cumulative interval [cum_before, cum_after) of the weights scaled to sum n; pointer j
  // sits at j + u
  double cum = 0;
  int j = 0;
  for (int c = 0; c < n && j < n; c++) {
    cum += w[c] / total * n;
    while (j < n && j + u < cum) anc[j++] = c;
  }
  return anc;
}

std::vector<int> truncation_ancestors(const std::vector<double>& E, double frac) {
  const int n = (int)E.size();
  std::vector<int> rank(n);
  std::iota(rank.begin(), rank.end(), 0);
  std::sort(rank.begin(), rank.end(), [&E](int a, int b) { return E[a] < E[b]; });
  std::vector<int> anc(n);
  std::iota(anc.begin(), anc.end(), 0);
  const int nrep = (int)(frac * n);
  for (int k = 0; k < nrep; k++) anc[rank[n - 1 - k]] = rank[k];
  return anc;
}

}  // namespace tsa
