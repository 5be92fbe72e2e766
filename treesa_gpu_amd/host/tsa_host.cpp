// tsa_host.cpp -- host layer of the TreeSA drop-in: readers, tree set-up, double-precision checks.
// Behaviour (formats, messages, algorithms) follows the reference's host code in csrc/treesa_gpu.cu as
// cited per function; label sets are 64-bit words here.
#include "tsa_host.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <numeric>
#include <random>

namespace tsa {

static int popc(uint64_t x) { return __builtin_popcountll(x); }

Inst make_instance(int m, int nlab, const std::vector<std::vector<int>>& ixs, const std::vector<int>& iy) {
  Inst I;
  I.m = m;
  I.nlab = nlab;
  I.ixs = ixs;
  I.iy = iy;
  I.total.assign(nlab > 0 ? nlab : 0, 0);
  I.in_iy.assign(nlab > 0 ? nlab : 0, 0);
  for (auto& ix : I.ixs) {
    std::sort(ix.begin(), ix.end());
    if (std::adjacent_find(ix.begin(), ix.end()) != ix.end())
      throw InputError("repeated label inside one tensor is not supported");
    for (int l : ix) {
      if (l < 0 || l >= nlab) throw InputError("label out of range");
      I.total[l]++;
    }
  }
  for (int l : I.iy) {
    if (l < 0 || l >= nlab) throw InputError("label out of range");
    I.in_iy[l] = 1;
  }
  return I;
}

Inst read_instance(const std::string& path) {
  FILE* f = fopen(path.c_str(), "r");
  if (!f) throw InputError("cannot open " + path);
  int m = 0, nlab = 0;
  if (fscanf(f, "%d %d", &m, &nlab) != 2 || m < 0 || nlab < 0) {
    fclose(f);
    throw InputError("bad header");
  }
  std::vector<std::vector<int>> ixs(m);
  for (int i = 0; i < m; i++) {
    int k;
    if (fscanf(f, "%d", &k) != 1 || k < 0) {
      fclose(f);
      throw InputError("bad tensor line");
    }
    for (int j = 0; j < k; j++) {
      int l;
      if (fscanf(f, "%d", &l) != 1) {
        fclose(f);
        throw InputError("bad tensor line");
      }
      ixs[i].push_back(l);
    }
  }
  int ny = 0;
  std::vector<int> iy;
  if (fscanf(f, "%d", &ny) != 1) ny = 0;
  for (int j = 0; j < ny; j++) {
    int l;
    if (fscanf(f, "%d", &l) != 1) {
      fclose(f);
      throw InputError("bad output line");
    }
    iy.push_back(l);
  }
  fclose(f);
  return make_instance(m, nlab, ixs, iy);
}

std::vector<std::vector<uint32_t>> read_trees(const std::string& path, int m) {
  std::vector<std::vector<uint32_t>> trees;
  FILE* f = fopen(path.c_str(), "r");
  if (!f) throw InputError("cannot open " + path);
  for (;;) {
    std::vector<uint32_t> ch(m - 1);
    int got = 0;
    for (int i = 0; i < m - 1; i++) {
      int l, r;
      if (fscanf(f, "%d %d", &l, &r) != 2) break;
      if (l < 0 || r < 0 || l > 0xFFFF || r > 0xFFFF) {
        fclose(f);
        throw InputError("bad tree file (node id out of range)");
      }
      ch[i] = (uint32_t)l | ((uint32_t)r << 16);
      got++;
    }
    if (got == 0) break;
    if (got != m - 1) {
      fclose(f);
      throw InputError("bad tree file (truncated tree " + std::to_string(trees.size()) + ")");
    }
    trees.push_back(std::move(ch));
  }
  fclose(f);
  if (trees.empty()) throw InputError("bad tree file (no tree)");
  return trees;
}

std::vector<float> parse_betas(const std::string& s) {
  std::vector<float> b;
  if (s.rfind("file:", 0) == 0) {
    FILE* f = fopen(s.c_str() + 5, "r");
    if (!f) throw InputError("cannot open betas file");
    double x;
    while (fscanf(f, "%lf", &x) == 1) b.push_back((float)x);
    fclose(f);
    return b;
  }
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

uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ULL;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
  return x ^ (x >> 31);
}

std::vector<uint32_t> random_tree(int m, uint64_t seed) {
  std::mt19937_64 rng(seed);
  std::vector<uint32_t> ch(m - 1);
  int next = m;
  std::function<int(const std::vector<int>&)> build = [&](const std::vector<int>& xs) -> int {
    const int n = (int)xs.size();
    if (n == 1) return xs[0];
    std::vector<char> mask(n);
    int cnt = 0;
    for (int i = 0; i < n; i++) {
      mask[i] = (char)(rng() & 1);
      cnt += mask[i];
    }
    if (cnt == 0 || cnt == n) {
      const int i = (int)(rng() % (uint64_t)n);
      mask[i] = !mask[i];
    }
    std::vector<int> a, b;
    for (int i = 0; i < n; i++) (mask[i] ? a : b).push_back(xs[i]);
    const int l = build(a), r = build(b);
    const int v = next++;
    ch[v - m] = (uint32_t)l | ((uint32_t)r << 16);
    return v;
  };
  std::vector<int> all(m);
  std::iota(all.begin(), all.end(), 0);
  build(all);
  return ch;
}

bool preorder(int m, const uint32_t* ch, std::vector<int>& order) {
  order.clear();
  std::vector<char> seen(2 * m - 1, 0);
  std::vector<int> st{2 * m - 2};
  int nseen = 0;
  while (!st.empty()) {
    const int v = st.back();
    st.pop_back();
    if (v < 0 || v >= 2 * m - 1 || seen[v]) return false;
    seen[v] = 1;
    nseen++;
    if (v >= m) {
      order.push_back(v);
      st.push_back((int)(ch[v - m] >> 16));
      st.push_back((int)(ch[v - m] & 0xFFFFu));
    }
  }
  return nseen == 2 * m - 1;
}

bool labels_from_topology(const Inst& I, int W, const uint32_t* ch, uint64_t* lab) {
  const int m = I.m, L = I.nlab;
  std::vector<int> order;
  if (!preorder(m, ch, order)) return false;
  // per-node occurrence counts, children before parents (reverse pre-order)
  std::vector<uint16_t> cnt((size_t)(m - 1) * L, 0);
  for (int k = (int)order.size() - 1; k >= 0; k--) {
    const int v = order[k];
    uint16_t* cv = &cnt[(size_t)(v - m) * L];
    for (int side = 0; side < 2; side++) {
      const int u = side ? (int)(ch[v - m] >> 16) : (int)(ch[v - m] & 0xFFFFu);
      if (u < m) {
        for (int l : I.ixs[u]) cv[l]++;
      } else {
        const uint16_t* cu = &cnt[(size_t)(u - m) * L];
        for (int l = 0; l < L; l++) cv[l] += cu[l];
      }
    }
    uint64_t* z = lab + (size_t)(v - m) * W;
    for (int w = 0; w < W; w++) z[w] = 0;
    for (int l = 0; l < L; l++)
      if (cv[l] > 0 && (cv[l] < I.total[l] || I.in_iy[l])) z[l >> 6] |= 1ull << (l & 63);
  }
  return true;
}

ModelLog2 model_log2(const ModelConsts& C) {
  ModelLog2 P;
  P.lpeak = (float)std::log2(C.gm[0]);
  P.lbw = (float)std::log2(C.gm[1]);
  P.m0 = (int)C.gm[2];
  P.n0 = (int)C.gm[3];
  P.k0 = (int)C.gm[4];
  P.llaunch = (float)std::log2(C.gm[5]);
  P.v2_l3launch = (float)std::log2(3 * C.h100[0]);
  P.v2_lperm2 = (float)std::log2(2 / C.h100[1]);
  P.v2_lcc_bit = (float)std::log2(C.h100[2]);
  P.v2_lcc_cell = (float)std::log2(C.h100[3]);
  P.v2_ltc_bit = (float)std::log2(C.h100[4]);
  P.v2_ltc_pad = (float)std::log2(C.h100[5]);
  P.v2_ltc_out = (float)std::log2(C.h100[6]);
  P.v2_small_rank = (int)C.h100[7];
  P.v2_lsmall_cell = (float)std::log2(C.h100[8]);
  return P;
}

static double gpu_time_d(int B, int M, int N, int K, const ModelLog2& P) {
  const double ops = std::exp2((double)(1 + B + std::max(M, P.m0) + std::max(N, P.n0) + std::max(K, P.k0)));
  const double bits = std::exp2((double)(B + M + K)) + std::exp2((double)(B + N + K)) + std::exp2((double)(B + M + N));
  return std::max(ops / std::exp2((double)P.lpeak), bits / std::exp2((double)P.lbw)) + std::exp2((double)P.llaunch);
}

static double h100_time_d(int B, int M, int N, int K, const ModelLog2& P) {
  auto e = [](float l) { return std::exp2((double)l); };
  if (B + M + N <= P.v2_small_rank) return e(P.v2_lsmall_cell) * std::exp2((double)(B + M + N + K));
  const double a = std::exp2((double)(B + M + K)), b = std::exp2((double)(B + N + K)), c = std::exp2((double)(B + M + N));
  const double moved = a + b + c;
  const double perm = e(P.v2_lperm2) * (a + b);
  double best = e(P.v2_lcc_bit) * moved + e(P.v2_lcc_cell) * std::exp2((double)(B + M + N + K));
  if (K >= 7 && std::max(M, N) >= 5) {
    const double tc = e(P.v2_ltc_bit) * moved +
                      e(P.v2_ltc_pad) * std::exp2((double)(B + std::max(M, 6) + std::max(N, 6) + std::max(K, 8))) +
                      e(P.v2_ltc_out) * c;
    best = std::min(best, tc);
  }
  return e(P.v2_l3launch) + perm + best;
}

HostEnergy host_energy(const Inst& I, int W, const ModelLog2& P, const uint64_t* lab, const uint32_t* ch,
                       const std::vector<uint64_t>& leaf, const uint64_t* S) {
  HostEnergy E;
  std::vector<uint64_t> nm(W, ~0ull);
  if (S)
    for (int w = 0; w < W; w++) {
      nm[w] = ~S[w];
      E.ns += popc(S[w]);
    }
  for (int i = 0; i < I.m; i++) {
    int z = 0;
    for (int w = 0; w < W; w++) z += popc(leaf[(size_t)i * W + w] & nm[w]);
    E.sc = std::max(E.sc, z);
  }
  double mx = -1e300;
  std::vector<double> tcs;
  for (int i = 0; i < I.m - 1; i++) {
    const int l = (int)(ch[i] & 0xFFFFu), r = (int)(ch[i] >> 16);
    const uint64_t* x = l >= I.m ? lab + (size_t)(l - I.m) * W : &leaf[(size_t)l * W];
    const uint64_t* y = r >= I.m ? lab + (size_t)(r - I.m) * W : &leaf[(size_t)r * W];
    const uint64_t* z = lab + (size_t)i * W;
    int B = 0, M = 0, N = 0, K = 0, sz = 0;
    for (int w = 0; w < W; w++) {
      const uint64_t a = x[w] & nm[w], b = y[w] & nm[w], c = z[w] & nm[w];
      B += popc(a & b & c);
      M += popc(a & ~b & c);
      N += popc(~a & b & c);
      K += popc(a & b & ~c);
      sz += popc(c);
    }
    const double t = B + M + N + K;
    tcs.push_back(t);
    mx = std::max(mx, t);
    E.sc = std::max(E.sc, sz);
    E.time += gpu_time_d(B, M, N, K, P);
    E.time2 += h100_time_d(B, M, N, K, P);
  }
  double s = 0;
  for (double t : tcs) s += std::exp2(t - mx);
  E.tc = mx + std::log2(s);
  return E;
}

int greedy_repair(const Inst& I, int W, const uint64_t* lab, const std::vector<uint64_t>& leaf, uint64_t* S,
                  double sc_target) {
  int added = 0;
  const int n = 2 * I.m - 1;
  auto set_of = [&](int v) -> const uint64_t* { return v < I.m ? &leaf[(size_t)v * W] : lab + (size_t)(v - I.m) * W; };
  std::vector<int> sizes(n);
  for (;;) {
    int scmax = 0;
    for (int v = 0; v < n; v++) {
      const uint64_t* a = set_of(v);
      int z = 0;
      for (int w = 0; w < W; w++) z += popc(a[w] & ~S[w]);
      sizes[v] = z;
      scmax = std::max(scmax, z);
    }
    if (scmax <= sc_target || scmax == 0) return added;
    std::vector<int> freq(I.nlab, 0);
    for (int v = 0; v < n; v++)
      if (sizes[v] == scmax) {
        const uint64_t* a = set_of(v);
        for (int l = 0; l < I.nlab; l++)
          if ((a[l >> 6] & ~S[l >> 6]) >> (l & 63) & 1u) freq[l]++;
      }
    const int best = (int)(std::max_element(freq.begin(), freq.end()) - freq.begin());
    S[best >> 6] |= 1ull << (best & 63);
    added++;
  }
}

std::vector<uint64_t> leaf_sets(const Inst& I, int W) {
  std::vector<uint64_t> leaf((size_t)I.m * W, 0);
  for (int i = 0; i < I.m; i++)
    for (int l : I.ixs[i]) leaf[(size_t)i * W + (l >> 6)] |= 1ull << (l & 63);
  return leaf;
}

int leaf_sc(const Inst& I) {
  int s = 0;
  for (auto& ix : I.ixs) s = std::max(s, (int)ix.size());
  return s;
}

void build_population(const Inst& I, const Geometry& G, const std::vector<std::vector<uint32_t>>& trees, int nchains,
                      uint64_t seed, const std::vector<uint64_t>& S0, int random_slices, std::vector<uint64_t>& pop) {
  pop.assign((size_t)G.chain_words * nchains, 0);
  const int K = (int)trees.size();
  const int nint = I.m - 1;
  bool ok = true;
  const int ninit = K > 0 ? std::min(K, nchains) : nchains;
#pragma omp parallel for schedule(dynamic, 16)
  for (int c = 0; c < ninit; c++) {
    uint64_t* base = &pop[(size_t)c * G.chain_words];
    const std::vector<uint32_t> ch = K == 0 ? random_tree(I.m, splitmix64(seed * 1000003ULL + c)) : trees[c];
    uint32_t* chw = reinterpret_cast<uint32_t*>(base + G.ch_off);
    std::copy(ch.begin(), ch.end(), chw);
    if (!labels_from_topology(I, G.W, ch.data(), base)) {
#pragma omp atomic write
      ok = false;
    }
  }
  if (!ok) throw InputError("invalid initial tree");
  (void)nint;
  for (int c = ninit; c < nchains; c++)
    std::copy(pop.begin() + (size_t)(c % K) * G.chain_words, pop.begin() + (size_t)(c % K + 1) * G.chain_words,
              pop.begin() + (size_t)c * G.chain_words);
  for (int c = 0; c < nchains; c++) {
    uint64_t* S = &pop[(size_t)c * G.chain_words + G.s_off];
    for (int w = 0; w < G.W; w++) S[w] = w < (int)S0.size() ? S0[w] : 0;
    if (random_slices > 0) {
      std::mt19937_64 rng(splitmix64(seed * 7919ULL + c));
      for (int k = 0; k < random_slices; k++) {
        const int l = (int)(rng() % (uint64_t)I.nlab);
        S[l >> 6] |= 1ull << (l & 63);
      }
    }
  }
}

}  // namespace tsa
