// tsa_host.cpp -- host layer of the TreeSA drop-in: file readers, start populations, double-precision checks.
//
// The formats, messages, random streams and formulas are the reference binary's (cited per function); the
// algorithms are this file's own: whitespace token readers, an explicit-stack random splitter, output
// labels by marking each label's tensors' ancestors up to the smallest subtree that holds all of them
// (Euler-tour intervals), and a word-wise repair loop.
#include "tsa_host.h"

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>

namespace tsa {

namespace {

int popcount(uint64_t x) { return __builtin_popcountll(x); }

// The whole file as whitespace-separated tokens, read front to back.
class Tokens {
 public:
  explicit Tokens(const std::string& path) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) throw InputError("cannot open " + path);
    char buf[1 << 16];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) text_.append(buf, n);
    fclose(f);
  }
  // Next token as an integer; false at the end or at a token that is not one (nothing consumed then).
  bool next_int(long& v) {
    const char* s = skip();
    if (!*s) return false;
    char* e = nullptr;
    errno = 0;
    const long x = strtol(s, &e, 10);
    if (e == s || errno != 0) return false;
    v = x;
    pos_ = (size_t)(e - text_.c_str());
    return true;
  }
  bool next_double(double& v) {
    const char* s = skip();
    if (!*s) return false;
    char* e = nullptr;
    const double x = strtod(s, &e);
    if (e == s) return false;
    v = x;
    pos_ = (size_t)(e - text_.c_str());
    return true;
  }

 private:
  const char* skip() {
    while (pos_ < text_.size() && isspace((unsigned char)text_[pos_])) pos_++;
    return text_.c_str() + pos_;
  }
  std::string text_;
  size_t pos_ = 0;
};

}  // namespace

int Network::largest_tensor() const {
  size_t s = 0;
  for (const auto& t : tensors) s = std::max(s, t.size());
  return (int)s;
}

Network make_network(int m, int nlab, std::vector<std::vector<int>> tensors, const std::vector<int>& outputs) {
  Network N;
  N.m = m;
  N.nlab = nlab < 0 ? 0 : nlab;
  N.holders.assign(N.nlab, {});
  N.is_open.assign(N.nlab, 0);
  for (int t = 0; t < (int)tensors.size(); t++) {
    std::vector<int>& labs = tensors[t];
    std::sort(labs.begin(), labs.end());
    for (size_t k = 0; k < labs.size(); k++) {
      if (k > 0 && labs[k] == labs[k - 1]) throw InputError("repeated label inside one tensor is not supported");
      if (labs[k] < 0 || labs[k] >= N.nlab) throw InputError("label out of range");
      N.holders[labs[k]].push_back(t);
    }
  }
  for (int l : outputs) {
    if (l < 0 || l >= N.nlab) throw InputError("label out of range");
    N.is_open[l] = 1;
  }
  N.tensors = std::move(tensors);
  N.outputs = outputs;
  return N;
}

Network read_network(const std::string& path) {
  Tokens tk(path);
  long m = 0, nlab = 0;
  if (!tk.next_int(m) || !tk.next_int(nlab) || m < 0 || nlab < 0 || m > (1 << 24)) throw InputError("bad header");
  std::vector<std::vector<int>> tensors((size_t)m);
  for (auto& t : tensors) {
    long k = 0;
    if (!tk.next_int(k) || k < 0) throw InputError("bad tensor line");
    t.resize((size_t)k);
    for (int& l : t) {
      long v;
      if (!tk.next_int(v)) throw InputError("bad tensor line");
      l = (int)v;
    }
  }
  std::vector<int> outputs;
  long ny = 0;
  if (tk.next_int(ny) && ny > 0) {
    outputs.resize((size_t)ny);
    for (int& l : outputs) {
      long v;
      if (!tk.next_int(v)) throw InputError("bad output line");
      l = (int)v;
    }
  }
  return make_network((int)m, (int)nlab, std::move(tensors), outputs);
}

std::vector<std::vector<uint32_t>> read_tree_file(const std::string& path, int m) {
  Tokens tk(path);
  std::vector<uint32_t> words;  // every complete "left right" pair, in file order
  for (;;) {
    long l, r;
    if (!tk.next_int(l) || !tk.next_int(r)) break;
    if (l < 0 || r < 0 || l > 0xFFFF || r > 0xFFFF) throw InputError("bad tree file (node id out of range)");
    words.push_back((uint32_t)l | ((uint32_t)r << 16));
  }
  const size_t per = (size_t)(m > 1 ? m - 1 : 1);
  if (words.size() % per != 0)
    throw InputError("bad tree file (truncated tree " + std::to_string(words.size() / per) + ")");
  if (words.empty()) throw InputError("bad tree file (no tree)");
  std::vector<std::vector<uint32_t>> trees;
  for (size_t k = 0; k < words.size(); k += per) trees.emplace_back(words.begin() + k, words.begin() + k + per);
  return trees;
}

std::vector<float> parse_schedule(const std::string& spec) {
  std::vector<float> out;
  if (spec.compare(0, 5, "file:") == 0) {
    FILE* f = fopen(spec.c_str() + 5, "rb");
    if (!f) throw InputError("cannot open betas file");
    fclose(f);
    Tokens tk(spec.substr(5));
    double x;
    while (tk.next_double(x)) out.push_back((float)x);
    return out;
  }
  // "a:step:b"
  const char* s = spec.c_str();
  char* e = nullptr;
  double v[3];
  int got = 0;
  for (; got < 3; got++) {
    v[got] = strtod(s, &e);
    if (e == s) break;
    s = e;
    if (got < 2) {
      if (*s != ':') {
        got++;
        break;
      }
      s++;
    }
  }
  if (got == 3) {
    const long n = (long)std::floor((v[2] - v[0]) / v[1] + 1e-9) + 1;
    for (long i = 0; i < n; i++) out.push_back((float)(v[0] + (double)i * v[1]));
    return out;
  }
  // "b1,b2,.."
  s = spec.c_str();
  for (;;) {
    const double x = strtod(s, &e);
    if (e == s) break;
    out.push_back((float)x);
    s = e;
    while (*s == ',' || *s == ' ') s++;
  }
  return out;
}

std::vector<uint32_t> random_tree(int m, uint64_t seed) {
  std::mt19937_64 rng(seed);
  std::vector<uint32_t> ch(m > 1 ? m - 1 : 0);
  // Explicit-stack form of the recursive split: a frame holds its members, the side it is building and the
  // id of its finished left part; a finished part hands its id to the frame below.
  struct Frame {
    std::vector<int> members, right;
    int stage;  // 0 not split yet, 1 left part pending, 2 right part pending
    int left;
  };
  std::vector<Frame> st;
  st.push_back({{}, {}, 0, -1});
  st.back().members.resize(m);
  for (int i = 0; i < m; i++) st.back().members[i] = i;
  int next_id = m, done = -1;
  while (!st.empty()) {
    Frame& f = st.back();
    if (done >= 0) {  // a part just finished
      if (f.stage == 1) {
        f.left = done;
        f.stage = 2;
        done = -1;
        std::vector<int> r = std::move(f.right);
        st.push_back({std::move(r), {}, 0, -1});
      } else {
        const int id = next_id++;
        ch[id - m] = (uint32_t)f.left | ((uint32_t)done << 16);
        done = id;
        st.pop_back();
      }
      continue;
    }
    const int n = (int)f.members.size();
    if (n == 1) {
      done = f.members[0];
      st.pop_back();
      continue;
    }
    std::vector<char> bit(n);
    int ones = 0;
    for (int i = 0; i < n; i++) ones += bit[i] = (char)(rng() & 1u);
    if (ones == 0 || ones == n) {
      const int i = (int)(rng() % (uint64_t)n);
      bit[i] ^= 1;
    }
    std::vector<int> left;
    for (int i = 0; i < n; i++) (bit[i] ? left : f.right).push_back(f.members[i]);
    f.stage = 1;
    st.push_back({std::move(left), {}, 0, -1});
  }
  return ch;
}

TreeShape tree_shape(int m, const uint32_t* ch) {
  TreeShape T;
  const int n = 2 * m - 1;
  if (m < 2) return T;
  T.parent.assign(n, -2);  // -2: not reached
  T.tin.assign(n, 0);
  T.tout.assign(n, 0);
  // iterative DFS from the root; a node is entered once, children pushed right then left (left first out)
  std::vector<int> stack{n - 1};
  T.parent[n - 1] = -1;
  std::vector<int> order;
  order.reserve(n);
  while (!stack.empty()) {
    const int v = stack.back();
    stack.pop_back();
    T.tin[v] = (int)order.size();
    order.push_back(v);
    if (v < m) continue;
    T.internal_preorder.push_back(v);
    const int kids[2] = {(int)(ch[v - m] >> 16), (int)(ch[v - m] & 0xFFFFu)};
    for (int u : kids) {
      if (u < 0 || u >= n || T.parent[u] != -2) return T;  // out of range, reached twice, or the root
      T.parent[u] = v;
      stack.push_back(u);
    }
  }
  if ((int)order.size() != n) return T;
  // the last descendant of v in tour order: walk the tour backwards, a node's tout is the max of its own tin
  // and its children's tout
  for (int k = n - 1; k >= 0; k--) {
    const int v = order[k];
    int t = T.tin[v];
    if (v >= m) t = std::max(T.tout[(int)(ch[v - m] & 0xFFFFu)], T.tout[(int)(ch[v - m] >> 16)]);
    T.tout[v] = t;
  }
  T.ok = true;
  return T;
}

bool topology_labels(const Network& N, int W, const uint32_t* ch, uint64_t* lab) {
  const int m = N.m;
  const TreeShape T = tree_shape(m, ch);
  if (!T.ok) return false;
  std::fill(lab, lab + (size_t)(m - 1) * W, 0ull);
  for (int l = 0; l < N.nlab; l++) {
    const std::vector<int>& hold = N.holders[l];
    if (hold.empty()) continue;
    // the smallest subtree holding every tensor of l spans the tour interval [lo, hi] of those leaves; an
    // internal node is an output of l iff it is a proper ancestor of one of them and does not span [lo, hi]
    // (or anywhere up to the root when l is open)
    int lo = T.tin[hold[0]], hi = lo;
    for (int t : hold) {
      lo = std::min(lo, T.tin[t]);
      hi = std::max(hi, T.tin[t]);
    }
    const uint64_t bit = 1ull << (l & 63);
    const int w = l >> 6;
    for (int t : hold) {
      for (int v = T.parent[t]; v >= 0; v = T.parent[v]) {
        if (!N.is_open[l] && T.tin[v] <= lo && hi <= T.tout[v]) break;  // holds all of l's tensors
        uint64_t& word = lab[(size_t)(v - m) * W + w];
        if (word & bit) break;  // marked from another tensor of l: so is the rest of the way up
        word |= bit;
      }
    }
  }
  return true;
}

ModelLog2 model_log2(const ModelConsts& C) {
  ModelLog2 P;
  auto lg = [](double x) { return (float)std::log2(x); };
  P.lpeak = lg(C.gm[0]);
  P.lbw = lg(C.gm[1]);
  P.m0 = (int)C.gm[2];
  P.n0 = (int)C.gm[3];
  P.k0 = (int)C.gm[4];
  P.llaunch = lg(C.gm[5]);
  P.v2_l3launch = lg(3 * C.h100[0]);  // three kernel launches per contraction
  P.v2_lperm2 = lg(2 / C.h100[1]);    // a permuted input is read and written once at the permutation bandwidth
  P.v2_lcc_bit = lg(C.h100[2]);
  P.v2_lcc_cell = lg(C.h100[3]);
  P.v2_ltc_bit = lg(C.h100[4]);
  P.v2_ltc_pad = lg(C.h100[5]);
  P.v2_ltc_out = lg(C.h100[6]);
  P.v2_small_rank = (int)C.h100[7];
  P.v2_lsmall_cell = lg(C.h100[8]);
  return P;
}

namespace {

// Label counts of one contraction (x, y) -> z on the sliced network: B in x, y and z; M in x and z only; N in
// y and z only; K in x and y only (contracted).
struct Counts {
  int B = 0, M = 0, N = 0, K = 0, Z = 0;
};

Counts contraction_counts(const uint64_t* x, const uint64_t* y, const uint64_t* z, const uint64_t* keep, int W) {
  Counts c;
  for (int w = 0; w < W; w++) {
    const uint64_t a = x[w] & keep[w], b = y[w] & keep[w], o = z[w] & keep[w];
    const uint64_t both = a & b;
    c.B += popcount(both & o);
    c.M += popcount(a & ~b & o);
    c.N += popcount(~a & b & o);
    c.K += popcount(both & ~o);
    c.Z += popcount(o);
  }
  return c;
}

double p2(double e) { return std::exp2(e); }

// GPU roofline model v1: max(flops / peak, bits moved / bandwidth) + launch, with the matrix dimensions
// padded to the tile minima; the constants enter as their float log2 (csrc/treesa_gpu.cu:1176-1180).
double gpu_model_seconds(const Counts& c, const ModelLog2& P) {
  const double flops = p2(1 + c.B + std::max(c.M, P.m0) + std::max(c.N, P.n0) + std::max(c.K, P.k0));
  const double bits = p2(c.B + c.M + c.K) + p2(c.B + c.N + c.K) + p2(c.B + c.M + c.N);
  return std::max(flops / p2(P.lpeak), bits / p2(P.lbw)) + p2(P.llaunch);
}

// Measured H100 model: tiny contractions cost per cell; otherwise three launches, the permutation of both
// inputs and the cheaper of the CUDA-core and the tensor-core kernels (the latter only for K >= 7 and a free
// dimension >= 5) (treesa_gpu/trees.py:100-149).
double h100_model_seconds(const Counts& c, const ModelLog2& P) {
  const int all = c.B + c.M + c.N + c.K;
  if (c.B + c.M + c.N <= P.v2_small_rank) return p2(P.v2_lsmall_cell) * p2(all);
  const double in1 = p2(c.B + c.M + c.K), in2 = p2(c.B + c.N + c.K), out = p2(c.B + c.M + c.N);
  const double moved = in1 + in2 + out;
  double kernel = p2(P.v2_lcc_bit) * moved + p2(P.v2_lcc_cell) * p2(all);
  if (c.K >= 7 && std::max(c.M, c.N) >= 5) {
    const double padded = p2(c.B + std::max(c.M, 6) + std::max(c.N, 6) + std::max(c.K, 8));
    kernel = std::min(kernel, p2(P.v2_ltc_bit) * moved + p2(P.v2_ltc_pad) * padded + p2(P.v2_ltc_out) * out);
  }
  return p2(P.v2_l3launch) + p2(P.v2_lperm2) * (in1 + in2) + kernel;
}

}  // namespace

HostEnergy host_energy(const Network& N, int W, const ModelLog2& P, const uint64_t* lab, const uint32_t* ch,
                       const std::vector<uint64_t>& leaf, const uint64_t* S) {
  HostEnergy E;
  std::vector<uint64_t> keep(W, ~0ull);
  if (S)
    for (int w = 0; w < W; w++) {
      keep[w] = ~S[w];
      E.ns += popcount(S[w]);
    }
  auto set_of = [&](int v) { return v < N.m ? &leaf[(size_t)v * W] : lab + (size_t)(v - N.m) * W; };
  for (int t = 0; t < N.m; t++) {
    int z = 0;
    for (int w = 0; w < W; w++) z += popcount(set_of(t)[w] & keep[w]);
    E.sc = std::max(E.sc, z);
  }
  const int nint = N.m - 1;
  std::vector<double> cost(nint);
  double top = -INFINITY;
  for (int i = 0; i < nint; i++) {
    const Counts c = contraction_counts(set_of((int)(ch[i] & 0xFFFFu)), set_of((int)(ch[i] >> 16)), lab + (size_t)i * W,
                                        keep.data(), W);
    cost[i] = (double)(c.B + c.M + c.N + c.K);
    top = std::max(top, cost[i]);
    E.sc = std::max(E.sc, c.Z);
    E.time += gpu_model_seconds(c, P);
    E.time2 += h100_model_seconds(c, P);
  }
  // log2 of the summed costs, scaled by the largest term
  double sum = 0;
  for (double x : cost) sum += std::exp2(x - top);
  E.tc = top + std::log2(sum);
  return E;
}

int greedy_repair(const Network& N, int W, const uint64_t* lab, const std::vector<uint64_t>& leaf, uint64_t* S,
                  double sc_target) {
  const int n = 2 * N.m - 1;
  auto set_of = [&](int v) { return v < N.m ? &leaf[(size_t)v * W] : lab + (size_t)(v - N.m) * W; };
  std::vector<int> size(n), tally((size_t)W * 64);
  int added = 0;
  for (;;) {
    int top = 0;
    for (int v = 0; v < n; v++) {
      int z = 0;
      const uint64_t* a = set_of(v);
      for (int w = 0; w < W; w++) z += popcount(a[w] & ~S[w]);
      size[v] = z;
      top = std::max(top, z);
    }
    if (top == 0 || (double)top <= sc_target) return added;
    std::fill(tally.begin(), tally.end(), 0);
    for (int v = 0; v < n; v++) {
      if (size[v] != top) continue;
      const uint64_t* a = set_of(v);
      for (int w = 0; w < W; w++)
        for (uint64_t x = a[w] & ~S[w]; x; x &= x - 1) tally[w * 64 + __builtin_ctzll(x)]++;
    }
    int pick = 0;
    for (int l = 1; l < N.nlab; l++)
      if (tally[l] > tally[pick]) pick = l;
    S[pick >> 6] |= 1ull << (pick & 63);
    added++;
  }
}

std::vector<uint64_t> leaf_sets(const Network& N, int W) {
  std::vector<uint64_t> leaf((size_t)N.m * W, 0ull);
  for (int t = 0; t < N.m; t++)
    for (int l : N.tensors[t]) leaf[(size_t)t * W + (l >> 6)] |= 1ull << (l & 63);
  return leaf;
}

void build_population(const Network& N, const Geometry& G, const std::vector<std::vector<uint32_t>>& trees,
                      int nchains, uint64_t seed, const std::vector<uint64_t>& S0, int random_slices,
                      std::vector<uint64_t>& pop) {
  pop.assign((size_t)G.chain_words * nchains, 0ull);
  const int K = (int)trees.size();
  // distinct start records: one per given tree, or one random tree per chain
  const int nrec = K > 0 ? std::min(K, nchains) : nchains;
  int bad = 0;
#pragma omp parallel for schedule(dynamic, 16) reduction(+ : bad)
  for (int c = 0; c < nrec; c++) {
    uint64_t* rec = &pop[(size_t)c * G.chain_words];
    const std::vector<uint32_t> ch = K > 0 ? trees[c] : random_tree(N.m, splitmix64(seed * 1000003ull + (uint64_t)c));
    if (ch.size() != (size_t)(N.m - 1) || !topology_labels(N, G.W, ch.data(), rec)) {
      bad++;
      continue;
    }
    std::memcpy(rec + G.ch_off, ch.data(), ch.size() * sizeof(uint32_t));
  }
  if (bad) throw InputError("invalid initial tree");
  for (int c = nrec; c < nchains; c++)
    std::memcpy(&pop[(size_t)c * G.chain_words], &pop[(size_t)(c % K) * G.chain_words], (size_t)G.chain_words * 8);
  for (int c = 0; c < nchains; c++) {
    uint64_t* S = &pop[(size_t)c * G.chain_words + G.s_off];
    for (int w = 0; w < G.W; w++) S[w] = w < (int)S0.size() ? S0[w] : 0ull;
    if (random_slices <= 0) continue;
    std::mt19937_64 g(splitmix64(seed * 7919ull + (uint64_t)c));
    for (int k = 0; k < random_slices; k++) {
      const int l = (int)(g() % (uint64_t)N.nlab);
      S[l >> 6] |= 1ull << (l & 63);
    }
  }
}

}  // namespace tsa
