// ref_harness.cpp -- driver around the reference's own CPU port (csrc/cpu_ref.h + csrc/common.h,
// compiled from /root/reference by oracle/Makefile into oracle/_ref/ref_harness).  TEST INFRASTRUCTURE
// ONLY: it produces the golden fixtures under tests/golden/ and can serve as bench.py's CPU baseline.
//
// It sets chains up the way the reference's --check mode does (csrc/treesa_gpu.cu:2008-2039): chain c
// starts from tree c % K of the tree file (or, with --random-trees, from the Julia random tree seeded
// splitmix64(seed * 1000003 + c), csrc/treesa_gpu.cu:1608), leaf labels from the instance, internal labels
// from the topology, an optional fixed random slice set per chain (csrc/treesa_gpu.cu:1621-1627), then
// runs levels x niters sweeps of ref_par_sweep or ref_optimize_subtree with the global sweep counter
// lev * niters + it, and prints one JSON object with every chain's final children, a hash of its label
// sets and its proposal / accept counts.  --chain0 c0 runs chain slots c0 .. c0 + chains - 1 (a slot fixes
// the chain's start tree and its random streams), so that any part of a larger population can be sampled.
#include <algorithm>
#include <chrono>
#include <cinttypes>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <numeric>
#include <random>
#include <string>
#include <vector>

#include "cpu_ref.h"

float h_lse_tab[64];

static uint64_t sm64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ULL;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
  return x ^ (x >> 31);
}

static std::vector<float> betas_of(const std::string& s) {
  std::vector<float> b;
  double a, st, e;
  if (sscanf(s.c_str(), "%lf:%lf:%lf", &a, &st, &e) == 3) {
    const long n = (long)std::floor((e - a) / st + 1e-9) + 1;
    for (long i = 0; i < n; i++) b.push_back((float)(a + i * st));
    return b;
  }
  const char* p = s.c_str();
  while (*p) {
    char* q;
    const double x = strtod(p, &q);
    if (q == p) break;
    b.push_back((float)x);
    p = q;
    while (*p == ',' || *p == ' ') p++;
  }
  return b;
}

static void rand_tree(int m, uint64_t seed, std::vector<int>& L, std::vector<int>& R) {
  std::mt19937_64 rng(seed);
  int next = m;
  std::function<int(const std::vector<int>&)> go = [&](const std::vector<int>& xs) -> int {
    const int n = (int)xs.size();
    if (n == 1) return xs[0];
    std::vector<char> side(n);
    int ones = 0;
    for (int i = 0; i < n; i++) ones += (side[i] = (char)(rng() & 1));
    if (ones == 0 || ones == n) {
      const int i = (int)(rng() % n);
      side[i] = !side[i];
    }
    std::vector<int> a, b;
    for (int i = 0; i < n; i++) (side[i] ? a : b).push_back(xs[i]);
    const int l = go(a), r = go(b), v = next++;
    L[v] = l;
    R[v] = r;
    return v;
  };
  std::vector<int> all(m);
  std::iota(all.begin(), all.end(), 0);
  go(all);
}

int main(int argc, char** argv) {
  std::string inst, tree, betas = "0.2:0.7:7", order = "par";
  int chains = 4, chain0 = 0, niters = 4, mode = 0, random_slices = 0, par_follow = 0, par_band = 0, timing = 0, threads = 1;
  bool random_trees = false;
  double sc_target = 24, sc_weight = 1;
  uint64_t seed = 7;
  double gm[6] = {11.9e15, 1.6e13, 6, 6, 8, 4e-6};
  double hm[9] = {4e-6, 1.23e13, 5.44e-14, 7.68e-15, 6.37e-14, 2.02e-16, 1.77e-13, 14, 1e-12};
  for (int i = 1; i < argc; i++) {
    std::string a = argv[i];
    auto nx = [&]() -> std::string {
      if (i + 1 >= argc) { fprintf(stderr, "missing value for %s\n", a.c_str()); exit(1); }
      return argv[++i];
    };
    if (a == "-i") inst = nx();
    else if (a == "--tree") tree = nx();
    else if (a == "--random-trees") random_trees = true;
    else if (a == "--chains") chains = std::stoi(nx());
    else if (a == "--chain0") chain0 = std::stoi(nx());
    else if (a == "--niters") niters = std::stoi(nx());
    else if (a == "--betas") betas = nx();
    else if (a == "--order") order = nx();
    else if (a == "--mode") { std::string s = nx(); mode = s == "gpu" ? 1 : s == "h100" ? 2 : 0; }
    else if (a == "--seed") seed = std::stoull(nx());
    else if (a == "--sc-target") sc_target = std::stod(nx());
    else if (a == "--sc-weight") sc_weight = std::stod(nx());
    else if (a == "--random-slices") random_slices = std::stoi(nx());
    else if (a == "--par-follow") par_follow = 1;
    else if (a == "--par-band") par_band = std::stoi(nx());
    else if (a == "--timing") timing = 1;
    else if (a == "--threads") threads = std::max(1, std::stoi(nx()));
    else { fprintf(stderr, "unknown argument %s\n", a.c_str()); return 1; }
  }
  for (int d = 0; d < 64; d++) h_lse_tab[d] = (float)std::log2(1.0 + std::exp2(-(double)d));
  FILE* f = fopen(inst.c_str(), "r");
  if (!f) { fprintf(stderr, "cannot open %s\n", inst.c_str()); return 1; }
  int m, nlab;
  if (fscanf(f, "%d %d", &m, &nlab) != 2) return 1;
  std::vector<std::vector<int>> ixs(m);
  for (int i = 0; i < m; i++) {
    int k;
    if (fscanf(f, "%d", &k) != 1) return 1;
    ixs[i].resize(k);
    for (int j = 0; j < k; j++)
      if (fscanf(f, "%d", &ixs[i][j]) != 1) return 1;
    std::sort(ixs[i].begin(), ixs[i].end());
  }
  int ny = 0;
  std::vector<int> iy;
  if (fscanf(f, "%d", &ny) == 1) {
    iy.resize(ny);
    for (int j = 0; j < ny; j++)
      if (fscanf(f, "%d", &iy[j]) != 1) return 1;
  }
  fclose(f);
  std::vector<int> total(nlab, 0);
  std::vector<char> open(nlab, 0);
  for (auto& ix : ixs)
    for (int l : ix) total[l]++;
  for (int l : iy) open[l] = 1;

  std::vector<std::vector<int>> tl, tr;  // trees from file
  if (!tree.empty()) {
    FILE* g = fopen(tree.c_str(), "r");
    if (!g) { fprintf(stderr, "cannot open %s\n", tree.c_str()); return 1; }
    for (;;) {
      std::vector<int> L(2 * m - 1, -1), R(2 * m - 1, -1);
      int got = 0;
      for (int i = 0; i < m - 1; i++) {
        int a, b;
        if (fscanf(g, "%d %d", &a, &b) != 2) break;
        L[m + i] = a;
        R[m + i] = b;
        got++;
      }
      if (got == 0) break;
      if (got != m - 1) { fprintf(stderr, "truncated tree\n"); return 1; }
      tl.push_back(L);
      tr.push_back(R);
    }
    fclose(g);
  }
  const std::vector<float> bs = betas_of(betas);
  Params P{};
  P.m = m;
  P.nint = m - 1;
  P.sc_target = (float)sc_target;
  P.sc_weight = (float)sc_weight;
  const uint64_t key = sm64(seed);
  P.key0 = (uint32_t)key;
  P.key1 = (uint32_t)(key >> 32);
  P.par_follow = par_follow;
  P.par_band = par_band;
  P.lpeak = (float)std::log2(gm[0]);
  P.lbw = (float)std::log2(gm[1]);
  P.m0 = (int)gm[2];
  P.n0 = (int)gm[3];
  P.k0 = (int)gm[4];
  P.llaunch = (float)std::log2(gm[5]);
  P.v2_l3launch = (float)std::log2(3 * hm[0]);
  P.v2_lperm2 = (float)std::log2(2 / hm[1]);
  P.v2_lcc_bit = (float)std::log2(hm[2]);
  P.v2_lcc_cell = (float)std::log2(hm[3]);
  P.v2_ltc_bit = (float)std::log2(hm[4]);
  P.v2_ltc_pad = (float)std::log2(hm[5]);
  P.v2_ltc_out = (float)std::log2(hm[6]);
  P.v2_small_rank = (int)hm[7];
  P.v2_lsmall_cell = (float)std::log2(hm[8]);

  // chains are independent: with --threads N their records are built and swept under OpenMP, and --timing
  // reports the wall time of the sweep phase of all of them (one thread: the sum over chains)
  std::vector<RefTree> trees(chains);
  std::vector<long long> nprop(chains, 0), nacc(chains, 0);
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
  for (int k = 0; k < chains; k++) {
    const int c = chain0 + k;
    RefTree& T = trees[k];
    T.m = m;
    T.left.assign(2 * m - 1, -1);
    T.right.assign(2 * m - 1, -1);
    if (random_trees) rand_tree(m, sm64(seed * 1000003ULL + c), T.left, T.right);
    else {
      T.left = tl[c % tl.size()];
      T.right = tr[c % tr.size()];
    }
    T.labels.resize(2 * m - 1);
    T.sliced.assign(nlab, 0);
    if (random_slices > 0) {
      std::mt19937_64 rng(sm64(seed * 7919ULL + c));
      for (int j = 0; j < random_slices; j++) T.sliced[(int)(rng() % nlab)] = 1;
    }
    // topology labels bottom-up (internal ids are in post-order, children first): each node keeps its
    // subtree's (label, occurrences) pairs, sorted by label, merged from its children's; a label whose every
    // occurrence lies in the subtree (and that is not open) is dropped, and the node's set is what is left
    std::vector<std::vector<std::pair<int, int>>> occ(2 * m - 1);
    for (int i = 0; i < m; i++) {
      T.labels[i] = ixs[i];
      for (int l : ixs[i]) {
        if (!occ[i].empty() && occ[i].back().first == l) occ[i].back().second++;
        else occ[i].push_back({l, 1});
      }
    }
    std::vector<int> post;
    std::vector<int> stack{2 * m - 2};
    while (!stack.empty()) {  // reverse of a right-first pre-order = post-order
      const int v = stack.back();
      stack.pop_back();
      if (v < m) continue;
      post.push_back(v);
      stack.push_back(T.left[v]);
      stack.push_back(T.right[v]);
    }
    std::reverse(post.begin(), post.end());
    for (int v : post) {
      const auto& a = occ[T.left[v]];
      const auto& b = occ[T.right[v]];
      auto& o = occ[v];
      size_t i = 0, j = 0;
      while (i < a.size() || j < b.size()) {
        std::pair<int, int> x;
        if (j == b.size() || (i < a.size() && a[i].first < b[j].first)) x = a[i++];
        else if (i == a.size() || b[j].first < a[i].first) x = b[j++];
        else x = {a[i].first, a[i++].second + b[j++].second};
        if (x.second < total[x.first] || open[x.first]) o.push_back(x);
      }
      for (const auto& x : o) T.labels[v].push_back(x.first);
    }
    for (int v = m; v < 2 * m - 1; v++) std::vector<std::pair<int, int>>().swap(occ[v]);
  }
  const auto t0 = std::chrono::steady_clock::now();
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
  for (int k = 0; k < chains; k++) {
    const int c = chain0 + k;
    RefTree& T = trees[k];
    long long np = 0, na = 0;
    for (size_t lev = 0; lev < bs.size(); lev++)
      for (int it = 0; it < niters; it++) {
        const uint32_t sw = (uint32_t)(lev * niters + it);
        if (order == "par") {
          if (mode == 0) ref_par_sweep<0>(T, bs[lev], sw, (uint32_t)c, P, np, na);
          else if (mode == 1) ref_par_sweep<1>(T, bs[lev], sw, (uint32_t)c, P, np, na);
          else ref_par_sweep<2>(T, bs[lev], sw, (uint32_t)c, P, np, na);
        } else {
          if (mode == 0) ref_optimize_subtree<0>(T, 2 * m - 2, bs[lev], sw, (uint32_t)c, P, np, na);
          else if (mode == 1) ref_optimize_subtree<1>(T, 2 * m - 2, bs[lev], sw, (uint32_t)c, P, np, na);
          else ref_optimize_subtree<2>(T, 2 * m - 2, bs[lev], sw, (uint32_t)c, P, np, na);
        }
      }
    nprop[k] = np;
    nacc[k] = na;
  }
  const double secs = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  long long tot_prop = 0;
  printf("{\"chains\": [");
  for (int k = 0; k < chains; k++) {
    const RefTree& T = trees[k];
    tot_prop += nprop[k];
    // FNV-1a over the internal label sets as 64-bit words (W = ceil(nlab / 64)), node by node
    const int W = (nlab + 63) / 64;
    uint64_t h = 1469598103934665603ULL;
    for (int v = m; v < 2 * m - 1; v++) {
      std::vector<uint64_t> w(W, 0);
      for (int l : T.labels[v]) w[l >> 6] |= 1ULL << (l & 63);
      for (uint64_t x : w)
        for (int b = 0; b < 8; b++) {
          h ^= (x >> (8 * b)) & 0xFF;
          h *= 1099511628211ULL;
        }
    }
    printf("%s{\"chain\": %d, \"nprop\": %lld, \"nacc\": %lld, \"labels_fnv\": \"%016" PRIx64 "\", \"children\": [",
           k ? ", " : "", chain0 + k, nprop[k], nacc[k], h);
    for (int v = m; v < 2 * m - 1; v++) printf("%s%d,%d", v > m ? "," : "", T.left[v], T.right[v]);
    printf("]}");
  }
  printf("]");
  if (timing) printf(", \"seconds\": %.6f, \"proposals\": %lld, \"threads\": %d", secs, tot_prop, threads);
  printf("}\n");
  return 0;
}
