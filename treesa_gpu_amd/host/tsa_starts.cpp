// tsa_starts.cpp -- start trees for the annealer, native: path trees along spectral orderings of the tensor
// graph (treesa_gpu/spectral.py:1-199 is the reference's numpy version) and the greedy contraction tree
// (the reference takes its greedy trees from omeco, treesa_gpu/driver.py:117-122).
//
// Spectral orderings.  Tensor graph: one vertex per tensor; a label held by k >= 2 tensors adds 1/(k-1) to
// each of their k(k-1)/2 pairs.  The lowest eigenvectors of its Laplacian L (after the constant one) give
// linear orderings with small cuts.  Up to 400 tensors the Laplacian is diagonalised densely; above, by a
// block Krylov method -- blocks of 4 vectors, so that a degenerate pair (the x- and y-waves of a square
// lattice) is found as a pair -- with full reorthogonalisation (twice) and a Rayleigh-Ritz step on the
// projected matrix.  Dense problems use Householder tridiagonalisation and implicit symmetric QR steps.  Candidate
// orderings sort the tensors by v . x for directions v in the plane of eigenvectors 1 and 2 (nangles angles in
// [0, pi)) and random unit directions in the span of 1..3, each ordering also reversed; the best few angles
// are refined by a halving step search.  Every candidate path tree is scored exactly with path_cost; the k
// best distinct orderings are returned.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>
#include <queue>
#include <set>
#include <unordered_set>

#include "tsa_host.h"

namespace tsa {

namespace {

// Dense column-major n x c block: column j at data[j * n].
struct Block {
  int n = 0, c = 0;
  std::vector<double> a;
  double* col(int j) { return a.data() + (size_t)j * n; }
  const double* col(int j) const { return a.data() + (size_t)j * n; }
};

double dot(const double* x, const double* y, int n) {
  double s = 0.0;
  for (int i = 0; i < n; i++) s += x[i] * y[i];
  return s;
}

// Weighted tensor graph as a symmetric adjacency list (i < j pairs kept once) and degrees.
struct Graph {
  int n = 0;
  std::vector<int> r, c;
  std::vector<double> w, deg;
};

Graph tensor_graph(const Network& I) {
  Graph G;
  G.n = I.m;
  std::vector<std::vector<int>> holders(I.nlab);
  for (int t = 0; t < I.m; t++)
    for (int l : I.tensors[t]) holders[l].push_back(t);
  std::vector<std::pair<uint64_t, double>> acc;
  for (const auto& ts : holders) {
    const int k = (int)ts.size();
    if (k < 2) continue;
    const double wk = 1.0 / (k - 1);
    for (int a = 0; a < k; a++)
      for (int b = a + 1; b < k; b++) {
        const uint32_t x = (uint32_t)std::min(ts[a], ts[b]), y = (uint32_t)std::max(ts[a], ts[b]);
        acc.emplace_back(((uint64_t)x << 32) | y, wk);
      }
  }
  std::sort(acc.begin(), acc.end(), [](const auto& p, const auto& q) { return p.first < q.first; });
  G.deg.assign(G.n, 0.0);
  for (size_t i = 0; i < acc.size();) {
    size_t j = i;
    double s = 0.0;
    while (j < acc.size() && acc[j].first == acc[i].first) s += acc[j++].second;
    const int x = (int)(acc[i].first >> 32), y = (int)(acc[i].first & 0xFFFFFFFFu);
    G.r.push_back(x);
    G.c.push_back(y);
    G.w.push_back(s);
    G.deg[x] += s;
    G.deg[y] += s;
    i = j;
  }
  return G;
}

void lap_mul(const Graph& G, const double* x, double* y) {
  for (int i = 0; i < G.n; i++) y[i] = G.deg[i] * x[i];
  for (size_t e = 0; e < G.w.size(); e++) {
    y[G.r[e]] -= G.w[e] * x[G.c[e]];
    y[G.c[e]] -= G.w[e] * x[G.r[e]];
  }
}

// Eigen-decomposition of the symmetric n x n matrix A (row-major; on return its columns are the eigenvectors)
// with the eigenvalues in ascending order in d.  Householder reduction to tridiagonal form by symmetric
// rank-2 updates, then implicit symmetric QR steps with Wilkinson shifts and Givens rotations on the
// tridiagonal, the transformations accumulated (Golub and Van Loan, Matrix Computations, 8.3).
void sym_eig(int n, std::vector<double>& A, std::vector<double>& d) {
  auto a = [&](int i, int j) -> double& { return A[(size_t)i * n + j]; };
  std::vector<double> Qm((size_t)n * n, 0.0);
  auto q = [&](int i, int j) -> double& { return Qm[(size_t)i * n + j]; };
  for (int i = 0; i < n; i++) q(i, i) = 1.0;
  std::vector<double> v(n), p(n), w(n);
  for (int k = 0; k + 2 < n; k++) {
    // Householder vector for x = A[k+1.., k]: (I - beta v v^T) x = alpha e1
    const int len = n - k - 1;
    double xn = 0.0;
    for (int i = 0; i < len; i++) xn += a(k + 1 + i, k) * a(k + 1 + i, k);
    xn = std::sqrt(xn);
    if (xn == 0.0) continue;
    const double x0 = a(k + 1, k), alpha = x0 >= 0.0 ? -xn : xn;
    for (int i = 0; i < len; i++) v[i] = a(k + 1 + i, k);
    v[0] -= alpha;
    double vv = 0.0;
    for (int i = 0; i < len; i++) vv += v[i] * v[i];
    if (vv == 0.0) continue;
    const double beta = 2.0 / vv;
    // p = beta B v with B = A[k+1.., k+1..]; w = p - (beta p.v / 2) v; B -= v w^T + w v^T
    for (int i = 0; i < len; i++) {
      double s = 0.0;
      for (int j = 0; j < len; j++) s += a(k + 1 + i, k + 1 + j) * v[j];
      p[i] = beta * s;
    }
    double pv = 0.0;
    for (int i = 0; i < len; i++) pv += p[i] * v[i];
    for (int i = 0; i < len; i++) w[i] = p[i] - 0.5 * beta * pv * v[i];
    for (int i = 0; i < len; i++)
      for (int j = 0; j < len; j++) a(k + 1 + i, k + 1 + j) -= v[i] * w[j] + w[i] * v[j];
    a(k + 1, k) = a(k, k + 1) = alpha;
    for (int i = 1; i < len; i++) a(k + 1 + i, k) = a(k, k + 1 + i) = 0.0;
    // Q <- Q (I - beta v v^T) on columns k+1..
    for (int r = 0; r < n; r++) {
      double s = 0.0;
      for (int j = 0; j < len; j++) s += q(r, k + 1 + j) * v[j];
      s *= beta;
      for (int j = 0; j < len; j++) q(r, k + 1 + j) -= s * v[j];
    }
  }
  d.assign(n, 0.0);
  std::vector<double> e(n, 0.0);  // e[i]: T[i][i+1]
  for (int i = 0; i < n; i++) d[i] = a(i, i);
  for (int i = 0; i + 1 < n; i++) e[i] = a(i, i + 1);
  // implicit QR on the unreduced blocks of the tridiagonal, from the bottom
  int hi = n - 1, guard = 0;
  while (hi > 0 && guard < 60 * n) {
    if (std::fabs(e[hi - 1]) <= 1e-15 * (std::fabs(d[hi - 1]) + std::fabs(d[hi]))) {
      e[hi - 1] = 0.0;
      hi--;
      continue;
    }
    int lo = hi - 1;
    while (lo > 0 && std::fabs(e[lo - 1]) > 1e-15 * (std::fabs(d[lo - 1]) + std::fabs(d[lo]))) lo--;
    guard++;
    // Wilkinson shift from the trailing 2 x 2 block
    const double t = (d[hi - 1] - d[hi]) / 2.0, b2 = e[hi - 1] * e[hi - 1];
    const double mu = d[hi] - b2 / (t + (t >= 0.0 ? 1.0 : -1.0) * std::sqrt(t * t + b2));
    double x = d[lo] - mu, z = e[lo];
    for (int k = lo; k < hi; k++) {
      // Givens rotation zeroing z against x in rows / columns k, k+1
      const double r = std::hypot(x, z), c = x / r, s = -z / r;
      if (k > lo) e[k - 1] = r;
      const double dk = d[k], dk1 = d[k + 1], ek = e[k];
      d[k] = c * c * dk - 2.0 * c * s * ek + s * s * dk1;
      d[k + 1] = s * s * dk + 2.0 * c * s * ek + c * c * dk1;
      e[k] = c * s * (dk - dk1) + (c * c - s * s) * ek;
      if (k + 1 < hi) {
        x = e[k];
        z = -s * e[k + 1];
        e[k + 1] = c * e[k + 1];
      }
      for (int r2 = 0; r2 < n; r2++) {
        const double qa = q(r2, k), qb = q(r2, k + 1);
        q(r2, k) = c * qa - s * qb;
        q(r2, k + 1) = s * qa + c * qb;
      }
    }
  }
  // ascending order, eigenvectors with them (columns of A)
  std::vector<int> idx(n);
  std::iota(idx.begin(), idx.end(), 0);
  std::stable_sort(idx.begin(), idx.end(), [&](int x1, int y1) { return d[x1] < d[y1]; });
  std::vector<double> d2(n);
  for (int j = 0; j < n; j++) {
    d2[j] = d[idx[j]];
    for (int i = 0; i < n; i++) a(i, j) = q(i, idx[j]);
  }
  d.swap(d2);
}

// Normal deviates from a splitmix64 stream (Box-Muller).
struct Normal {
  uint64_t s;
  explicit Normal(uint64_t seed) : s(seed) {}
  double uniform() {
    s += 0x9e3779b97f4a7c15ull;
    return ((double)(splitmix64(s) >> 11) + 0.5) * 0x1p-53;
  }
  double operator()() {
    const double u = uniform(), v = uniform();
    return std::sqrt(-2.0 * std::log(u)) * std::cos(2.0 * M_PI * v);
  }
};

}  // namespace

std::vector<double> laplacian_vectors(const Network& I, int k, uint64_t seed, std::vector<double>* evals) {
  const Graph G = tensor_graph(I);
  const int n = G.n;
  k = std::min(k, std::max(1, n - 2));
  std::vector<double> V((size_t)n * k, 0.0);
  std::vector<double> dv;
  if (n <= 400) {  // dense: the whole Laplacian
    std::vector<double> A((size_t)n * n, 0.0);
    for (int i = 0; i < n; i++) A[(size_t)i * n + i] = G.deg[i];
    for (size_t e = 0; e < G.w.size(); e++) {
      A[(size_t)G.r[e] * n + G.c[e]] -= G.w[e];
      A[(size_t)G.c[e] * n + G.r[e]] -= G.w[e];
    }
    sym_eig(n, A, dv);
    for (int i = 0; i < n; i++)
      for (int j = 0; j < k; j++) V[(size_t)i * k + j] = A[(size_t)i * n + j + 1];
    if (evals) evals->assign(dv.begin() + 1, dv.begin() + 1 + k);
    return V;
  }
  // block Krylov: blocks of bs vectors, steps blocks, Q orthonormal, LQ = L Q
  const int bs = 4, steps = std::max(2, std::min(n / bs, 200));
  Normal rnd(seed ^ 0x5bd1e995u);
  Block X{n, bs, std::vector<double>((size_t)n * bs)};
  for (auto& x : X.a) x = rnd();
  Block Q{n, 0, {}}, LQ{n, 0, {}};
  Q.a.reserve((size_t)n * bs * steps);
  LQ.a.reserve((size_t)n * bs * steps);
  std::vector<double> coef;
  for (int st = 0; st < steps; st++) {
    for (int rep = 0; rep < 2; rep++) {  // X -= Q (Q^T X), twice
      coef.assign((size_t)Q.c * X.c, 0.0);
#pragma omp parallel for schedule(static)
      for (int q = 0; q < Q.c; q++)
        for (int j = 0; j < X.c; j++) coef[(size_t)q * X.c + j] = dot(Q.col(q), X.col(j), n);
#pragma omp parallel for schedule(static)
      for (int i = 0; i < n; i++)
        for (int j = 0; j < X.c; j++) {
          double s = 0.0;
          for (int q = 0; q < Q.c; q++) s += Q.a[(size_t)q * n + i] * coef[(size_t)q * X.c + j];
          X.a[(size_t)j * n + i] -= s;
        }
    }
    // modified Gram-Schmidt inside the block; columns that vanish are dropped
    Block Y{n, 0, {}};
    for (int j = 0; j < X.c; j++) {
      std::vector<double> v(X.col(j), X.col(j) + n);
      const double n0 = std::sqrt(dot(v.data(), v.data(), n));
      for (int q = 0; q < Y.c; q++) {
        const double p = dot(Y.col(q), v.data(), n);
        for (int i = 0; i < n; i++) v[i] -= p * Y.col(q)[i];
      }
      const double nv = std::sqrt(dot(v.data(), v.data(), n));
      if (nv <= 1e-10 || nv <= 1e-10 * n0) continue;
      for (int i = 0; i < n; i++) v[i] /= nv;
      Y.a.insert(Y.a.end(), v.begin(), v.end());
      Y.c++;
    }
    if (Y.c == 0) break;
    Block LY{n, Y.c, std::vector<double>((size_t)n * Y.c)};
    for (int j = 0; j < Y.c; j++) lap_mul(G, Y.col(j), LY.col(j));
    Q.a.insert(Q.a.end(), Y.a.begin(), Y.a.end());
    Q.c += Y.c;
    LQ.a.insert(LQ.a.end(), LY.a.begin(), LY.a.end());
    LQ.c += LY.c;
    X = LY;
  }
  // Rayleigh-Ritz: T = Q^T L Q, symmetrised
  const int c = Q.c;
  std::vector<double> T((size_t)c * c);
#pragma omp parallel for schedule(dynamic, 4)
  for (int p = 0; p < c; p++)
    for (int q = 0; q < c; q++) T[(size_t)p * c + q] = dot(Q.col(p), LQ.col(q), n);
  for (int p = 0; p < c; p++)
    for (int q = p + 1; q < c; q++) {
      const double s = 0.5 * (T[(size_t)p * c + q] + T[(size_t)q * c + p]);
      T[(size_t)p * c + q] = T[(size_t)q * c + p] = s;
    }
  sym_eig(c, T, dv);
  const int kk = std::min(k, c - 1);
#pragma omp parallel for schedule(static)
  for (int i = 0; i < n; i++)
    for (int j = 0; j < kk; j++) {
      double s = 0.0;
      for (int q = 0; q < c; q++) s += Q.a[(size_t)q * n + i] * T[(size_t)q * c + j + 1];
      V[(size_t)i * k + j] = s;
    }
  if (evals) evals->assign(dv.begin() + 1, dv.begin() + 1 + kk);
  return V;
}

std::pair<double, int> path_cost(const Network& I, const std::vector<int>& order) {
  const int m = (int)order.size();
  if (m < 2) return {0.0, I.largest_tensor()};
  std::vector<int> pos(m);
  for (int i = 0; i < m; i++) pos[order[i]] = i;
  std::vector<int> first(I.nlab, -1), last(I.nlab, -1);
  for (int t = 0; t < m; t++)
    for (int l : I.tensors[t]) {
      const int p = pos[t];
      if (first[l] < 0 || p < first[l]) first[l] = p;
      if (last[l] < 0 || p > last[l]) last[l] = p;
    }
  // alive[i]: labels of the prefix order[0..i-1] that are needed after it; newc[i]: labels first seen at i
  std::vector<long long> diff(m + 2, 0), newc(m, 0);
  for (int l = 0; l < I.nlab; l++) {
    if (first[l] < 0) continue;
    const int f = first[l], la = I.is_open[l] ? m : last[l];
    newc[f]++;
    diff[f + 1]++;
    diff[la + 1]--;
  }
  std::vector<long long> alive(m + 1, 0);
  long long run = 0;
  for (int i = 0; i <= m; i++) {
    run += diff[i];
    alive[i] = run;
  }
  // step i = 1..m-1 contracts the prefix (or, for i = 1, the leaf order[0]) with tensor order[i]; for
  // dimension-2 indices its cost is the size of the union of the two label sets
  std::vector<long long> cost(m - 1);
  {
    std::vector<int> u(I.tensors[order[0]]);
    u.insert(u.end(), I.tensors[order[1]].begin(), I.tensors[order[1]].end());
    std::sort(u.begin(), u.end());
    cost[0] = std::unique(u.begin(), u.end()) - u.begin();
  }
  for (int i = 2; i < m; i++) cost[i - 1] = alive[i] + newc[i];
  long long sc = I.largest_tensor();
  for (int i = 2; i <= m; i++) sc = std::max(sc, alive[i]);
  const long long cm = *std::max_element(cost.begin(), cost.end());
  double s = 0.0;
  for (long long x : cost) s += std::exp2((double)(x - cm));
  return {(double)cm + std::log2(s), (int)sc};
}

std::vector<uint32_t> path_tree(const std::vector<int>& order) {
  const int m = (int)order.size();
  std::vector<uint32_t> ch(m - 1);
  for (int i = 0; i < m - 1; i++) {
    const uint32_t left = i == 0 ? (uint32_t)order[0] : (uint32_t)(m + i - 1);
    ch[i] = left | ((uint32_t)order[i + 1] << 16);
  }
  return ch;
}

std::vector<SpectralOrder> spectral_search(const Network& I, const std::vector<double>& V, int d,
                                           const std::vector<double>& rdirs, int k, int nangles) {
  const int n = I.m;
  std::vector<SpectralOrder> out;
  if (n < 3) {
    std::vector<int> o(n);
    std::iota(o.begin(), o.end(), 0);
    out.push_back({0.0, I.largest_tensor(), o});
    return out;
  }
  struct Cand {
    double tc;
    int sc;
    std::vector<int> order;
    double th;  // angle of its direction's (v1, v2) components (NaN with one eigenvector)
  };
  std::vector<Cand> cands;
  std::set<std::vector<int>> seen;
  // sort by x = V dir (stable), score the ordering and its reverse; the best new tc (INFINITY if both seen)
  auto score = [&](const std::vector<double>& dir) -> double {
    std::vector<double> x(n, 0.0);
    for (int i = 0; i < n; i++)
      for (int j = 0; j < d; j++) x[i] += V[(size_t)i * d + j] * dir[j];
    std::vector<int> o(n);
    std::iota(o.begin(), o.end(), 0);
    std::stable_sort(o.begin(), o.end(), [&](int a, int b) { return x[a] < x[b]; });
    const double th = d >= 2 ? std::atan2(dir[1], dir[0]) : NAN;
    double best = INFINITY;
    for (int rev = 0; rev < 2; rev++) {
      std::vector<int> oo = o;
      if (rev) std::reverse(oo.begin(), oo.end());
      if (!seen.insert(oo).second) continue;
      const auto tcsc = path_cost(I, oo);
      cands.push_back({tcsc.first, tcsc.second, oo, th});
      best = std::min(best, tcsc.first);
    }
    return best;
  };
  auto plane = [&](double th) {
    std::vector<double> v(d, 0.0);
    v[0] = std::cos(th);
    v[1] = std::sin(th);
    return v;
  };
  if (d >= 2) {
    for (int a = 0; a < nangles; a++) score(plane(M_PI * a / nangles));
    for (size_t r = 0; d >= 3 && r + (size_t)d <= rdirs.size(); r += (size_t)d)
      score(std::vector<double>(rdirs.begin() + (long)r, rdirs.begin() + (long)r + d));
  } else {
    score(std::vector<double>(1, 1.0));
  }
  auto by_cost = [](const Cand& a, const Cand& b) { return a.tc < b.tc || (a.tc == b.tc && a.sc < b.sc); };
  if (d >= 2 && nangles > 0) {
    // refine the angle in the (v1, v2) plane around the directions of the three best candidates by a halving
    // step search: on square lattices the best ordering is one wave with a small tilt
    std::vector<Cand> sorted = cands;
    std::stable_sort(sorted.begin(), sorted.end(), by_cost);
    std::vector<double> starts;
    for (const Cand& c : sorted) {
      bool fresh = true;
      for (double t0 : starts) fresh = fresh && std::fabs(c.th - t0) > 1e-9;
      if (fresh) starts.push_back(c.th);
      if (starts.size() == 3) break;
    }
    for (double th0 : starts) {
      double th = th0, step = M_PI / nangles / 2, cur = INFINITY;
      for (const Cand& c : cands)
        if (std::fabs(c.th - th0) < 1e-9) cur = std::min(cur, c.tc);
      for (int it = 0; it < 8; it++) {
        bool improved = false;
        for (double dth : {-step, step}) {
          const double t = score(plane(th + dth));
          if (t < cur - 1e-9) {
            cur = t;
            th += dth;
            improved = true;
            break;
          }
        }
        if (!improved) step /= 2;
      }
    }
  }
  std::stable_sort(cands.begin(), cands.end(), by_cost);
  for (size_t i = 0; i < cands.size() && (int)out.size() < k; i++)
    out.push_back({cands[i].tc, cands[i].sc, cands[i].order});
  return out;
}

std::vector<SpectralOrder> spectral_orders(const Network& I, int k, int nangles, int nrandom, uint64_t seed) {
  const int n = I.m;
  if (n < 3) return spectral_search(I, {}, 0, {}, k, nangles);
  const int d = std::min(3, std::max(1, n - 2));
  const std::vector<double> V = laplacian_vectors(I, d, seed, nullptr);
  // random unit directions in the span of eigenvectors 1..3
  std::vector<double> rdirs;
  Normal rnd(seed * 0x9e3779b97f4a7c15ull + 12345u);
  for (int r = 0; d >= 3 && r < nrandom; r++) {
    double v[3], nv = 0.0;
    for (double& x : v) {
      x = rnd();
      nv += x * x;
    }
    nv = std::sqrt(nv);
    for (double x : v) rdirs.push_back(x / nv);
  }
  return spectral_search(I, V, d, rdirs, k, nangles);
}

// Greedy contraction: repeatedly contract the pair of tensors that share a label and give the smallest
// result (outer product of the two smallest when nothing is shared); run 0 breaks ties by discovery order,
// the others at random.  The tree with the lowest tc over nrepeat runs.
namespace {

struct GreedyRun {
  std::vector<uint32_t> ch;
  double tc;
};

GreedyRun greedy_once(const Network& I, uint64_t seed, bool random_ties) {
  const int m = I.m;
  std::vector<std::vector<int>> sets(2 * m - 1);
  for (int t = 0; t < m; t++) sets[t] = I.tensors[t];
  std::vector<int> cnt(I.nlab);
  for (int l = 0; l < I.nlab; l++) cnt[l] = I.occurrences(l);
  std::vector<std::set<int>> holders(I.nlab);
  for (int t = 0; t < m; t++)
    for (int l : sets[t]) holders[l].insert(t);
  auto result = [&](int a, int b) {
    std::vector<int> u;
    std::set_union(sets[a].begin(), sets[a].end(), sets[b].begin(), sets[b].end(), std::back_inserter(u));
    std::vector<int> o;
    for (int l : u) {
      const int inside = (int)std::binary_search(sets[a].begin(), sets[a].end(), l) +
                         (int)std::binary_search(sets[b].begin(), sets[b].end(), l);
      if (I.is_open[l] || cnt[l] - inside > 0) o.push_back(l);
    }
    return o;
  };
  struct Item {
    int size;
    double tie;
    long long tick;
    int a, b;
    bool operator>(const Item& o) const {
      if (size != o.size) return size > o.size;
      if (tie != o.tie) return tie > o.tie;
      return tick > o.tick;
    }
  };
  std::priority_queue<Item, std::vector<Item>, std::greater<Item>> heap;
  long long tick = 0;
  uint64_t rs = seed;
  auto push = [&](int a, int b) {
    if (a > b) std::swap(a, b);
    double tie = 0.0;
    if (random_ties) {
      rs += 0x9e3779b97f4a7c15ull;
      tie = (double)(splitmix64(rs) >> 11) * 0x1p-53;
    }
    heap.push({(int)result(a, b).size(), tie, tick++, a, b});
  };
  for (int l = 0; l < I.nlab; l++) {
    const std::vector<int> hs(holders[l].begin(), holders[l].end());
    for (size_t i = 0; i < hs.size(); i++)
      for (size_t j = i + 1; j < hs.size(); j++) push(hs[i], hs[j]);
  }
  std::vector<char> alive(2 * m - 1, 0);
  for (int t = 0; t < m; t++) alive[t] = 1;
  int nalive = m, nxt = m;
  std::vector<uint32_t> ch;
  std::vector<double> costs;
  while (nalive > 1) {
    int a = -1, b = -1;
    while (!heap.empty()) {
      const Item it = heap.top();
      heap.pop();
      if (alive[it.a] && alive[it.b]) {
        a = it.a;
        b = it.b;
        break;
      }
    }
    if (a < 0) {  // disconnected: outer product of the two smallest
      std::vector<int> al;
      for (int t = 0; t < nxt; t++)
        if (alive[t]) al.push_back(t);
      std::stable_sort(al.begin(), al.end(), [&](int x, int y) {
        return sets[x].size() < sets[y].size() || (sets[x].size() == sets[y].size() && x < y);
      });
      a = al[0];
      b = al[1];
    }
    std::vector<int> out = result(a, b);
    std::vector<int> u;
    std::set_union(sets[a].begin(), sets[a].end(), sets[b].begin(), sets[b].end(), std::back_inserter(u));
    costs.push_back((double)u.size());
    for (int l : u) {
      cnt[l] -= (int)std::binary_search(sets[a].begin(), sets[a].end(), l) +
                (int)std::binary_search(sets[b].begin(), sets[b].end(), l);
      holders[l].erase(a);
      holders[l].erase(b);
    }
    for (int l : out) {
      cnt[l]++;
      holders[l].insert(nxt);
    }
    sets[nxt] = out;
    alive[a] = alive[b] = 0;
    alive[nxt] = 1;
    ch.push_back((uint32_t)a | ((uint32_t)b << 16));
    std::set<int> nb;
    for (int l : out) nb.insert(holders[l].begin(), holders[l].end());
    nb.erase(nxt);
    for (int t : nb) push(t, nxt);
    nxt++;
    nalive--;
  }
  const double cm = *std::max_element(costs.begin(), costs.end());
  double s = 0.0;
  for (double x : costs) s += std::exp2(x - cm);
  return {ch, cm + std::log2(s)};
}

}  // namespace

std::vector<uint32_t> greedy_tree(const Network& I, int nrepeat, uint64_t seed, double* tc) {
  GreedyRun best{{}, INFINITY};
  for (int r = 0; r < std::max(1, nrepeat); r++) {
    GreedyRun g = greedy_once(I, splitmix64(seed * 1000003ull + (uint64_t)r), r > 0);
    if (g.tc < best.tc) best = std::move(g);
  }
  if (tc) *tc = best.tc;
  return best.ch;
}

}  // namespace tsa
