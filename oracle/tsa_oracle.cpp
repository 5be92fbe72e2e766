// tsa_oracle.cpp -- CPU oracle for the TreeSA sweep path.  TEST INFRASTRUCTURE ONLY: tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg load it (liboracle.so via ctypes) as the
// checker; the product (libtreesa_hip.so, bin/treesa_gpu) never links or calls it.
//
// A restatement, with its own data structures, of the reference's CPU port of Julia TreeSA:
//   * label sets are sorted std::vector<int> per node (leaves included), membership by binary search;
//     sliced labels have log2 size 0 (csrc/cpu_ref.h:14-38);
//   * one proposal = the four-rule rotation of Julia optimize_subtree! (csrc/cpu_ref.h:87-126), scored
//     with tcscrw counts (mode tc) or the GPU / H100 time models (csrc/cpu_ref.h:40-85,
//     csrc/common.h:128-163) and accepted with Metropolis on glibc expf (csrc/common.h:224-229);
//   * pre-order sweep = the literal recursion (csrc/cpu_ref.h:122-125); par sweep = independent sets
//     applied one visit after the other (csrc/cpu_ref.h:128-182);
//   * the slice step and the whole-chain energy, which the reference runs only on the GPU
//     (csrc/treesa_gpu.cu:386-502), are mirrored here in the same 32-lane fold order;
//   * set-up: topology-derived output labels (csrc/treesa_gpu.cu:1149-1172), Julia random trees
//     (csrc/treesa_gpu.cu:1101-1123), the host double-precision energy (csrc/treesa_gpu.cu:1206-1244).
// Everything is built with -ffp-contract=off and calls the host libm, so float results are those of
// the reference's cpu_ref.h compiled on this host.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <functional>
#include <random>
#include <vector>

namespace {

using Set = std::vector<int>;  // sorted label ids

struct Inst {
  int m = 0, nlab = 0;
  std::vector<Set> ixs;
  std::vector<int> iy;
  std::vector<int> total;
  std::vector<char> open;
};

// Field order matches the Python side (tests/oracle.py).
struct OParams {
  int32_t mode;
  float sc_target, sc_weight;
  uint32_t key0, key1;
  int32_t slicing, slice_moves, slice_every, max_slices, par_follow, par_band;
  float lpeak, lbw, llaunch;
  int32_t m0, n0, k0;
  float v2_l3launch, v2_lperm2, v2_lcc_bit, v2_lcc_cell, v2_ltc_bit, v2_ltc_pad, v2_ltc_out, v2_lsmall_cell;
  int32_t v2_small_rank;
  int32_t leaf_sc;
};

struct Layout {
  int W, ch_off, s_off, chain_words;
};

float g_lse[64];
bool g_lse_ready = false;
void ensure_lse() {
  if (g_lse_ready) return;
  for (int d = 0; d < 64; d++) g_lse[d] = (float)std::log2(1.0 + std::exp2(-(double)d));
  g_lse_ready = true;
}

// ---- random numbers and hashes -------------------------------------------------------------------
struct R4 {
  uint32_t a, b, c, d;
};
R4 philox10(R4 x, uint32_t k0, uint32_t k1) {
  for (int round = 0; round < 10; round++) {
    const uint64_t p = (uint64_t)x.a * 0xD2511F53ull, q = (uint64_t)x.c * 0xCD9E8D57ull;
    x = R4{(uint32_t)(q >> 32) ^ x.b ^ k0, (uint32_t)q, (uint32_t)(p >> 32) ^ x.d ^ k1, (uint32_t)p};
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return x;
}
uint32_t fmix(uint32_t h) {
  h = (h ^ (h >> 16)) * 0x85EBCA6Bu;
  h = (h ^ (h >> 13)) * 0xC2B2AE35u;
  return h ^ (h >> 16);
}
uint64_t smix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// ---- energy arithmetic (floats exactly as the reference's shared header) ----------------------------
float lse_int(int a, int b) {
  const int hi = std::max(a, b);
  const int d = std::min(std::abs(a - b), 63);
  return (float)hi + g_lse[d];
}
float lse_flt(float a, float b) {
  const float hi = a > b ? a : b, lo = a > b ? b : a;
  if (hi == -INFINITY) return hi;
  return hi + log2f(1.0f + exp2f(lo - hi));
}
// Rounding variants for perturbation experiments (oracle_set_variant): bit 0 evaluates the energy fold's lse
// in double and rounds once (an equally accurate float lse whose last bit differs from the libm form now and
// then), bit 1 does the same in the float energy models of the sweeps; bits 2 and 3 instead move the
// results of exp2f and log2f in the fold (bit 2) or in the models (bit 3) by one ulp up or down, each with
// probability 1/4 by a hash of the operand and g_noise_seed: a device whose exp2f / log2f stay within one ulp
// but round differently from libm; bit 4 moves the Metropolis expf result by -2..2 ulp the same way (accept()).
// 0 (the default) is the reference's arithmetic on this host.
int g_variant = 0;
uint32_t g_noise_seed = 0;
float lse_dbl(float a, float b) {
  const float hi = a > b ? a : b, lo = a > b ? b : a;
  if (hi == -INFINITY) return hi;
  return (float)((double)hi + std::log2(1.0 + std::exp2((double)lo - (double)hi)));
}
float nudge(float x, float operand, uint32_t salt) {
  uint32_t u;
  std::memcpy(&u, &operand, 4);
  const uint32_t h = fmix(u ^ (g_noise_seed * 0x9E3779B9u) ^ salt);
  if ((h & 3u) == 1u) return std::nextafter(x, INFINITY);
  if ((h & 3u) == 2u) return std::nextafter(x, -INFINITY);
  return x;
}
float lse_noisy(float a, float b) {
  const float hi = a > b ? a : b, lo = a > b ? b : a;
  if (hi == -INFINITY) return hi;
  const float d = lo - hi, e = nudge(exp2f(d), d, 0x51u), s = 1.0f + e;
  return hi + nudge(log2f(s), s, 0xA7u);
}
float lse_fold(float a, float b) {
  return (g_variant & 4) ? lse_noisy(a, b) : (g_variant & 1) ? lse_dbl(a, b) : lse_flt(a, b);
}
float lse_model(float a, float b) {
  return (g_variant & 8) ? lse_noisy(a, b) : (g_variant & 2) ? lse_dbl(a, b) : lse_flt(a, b);
}
float model_lt(int mode, int B, int M, int N, int K, const OParams& P) {
  if (mode == 1) {
    const float lops = (float)(1 + B + std::max(M, P.m0) + std::max(N, P.n0) + std::max(K, P.k0)) - P.lpeak;
    const float lbits = lse_model(lse_model((float)(B + M + K), (float)(B + N + K)), (float)(B + M + N)) - P.lbw;
    return lse_model(lops > lbits ? lops : lbits, P.llaunch);
  }
  if (B + M + N <= P.v2_small_rank) return P.v2_lsmall_cell + (float)(B + M + N + K);
  const float la = (float)(B + M + K), lb = (float)(B + N + K), lc = (float)(B + M + N);
  const float lab = lse_model(la, lb), lmv = lse_model(lab, lc);
  float best = lse_model(P.v2_lcc_bit + lmv, P.v2_lcc_cell + (float)(B + M + N + K));
  if (K >= 7 && std::max(M, N) >= 5) {
    const float t = lse_model(lse_model(P.v2_ltc_bit + lmv, P.v2_ltc_pad + (float)(B + std::max(M, 6) + std::max(N, 6) +
                                                                                std::max(K, 8))),
                            P.v2_ltc_out + lc);
    if (t < best) best = t;
  }
  return lse_model(lse_model(P.v2_l3launch, P.v2_lperm2 + lab), best);
}
// Metropolis with the 24-bit uniform of r (csrc/common.h:224-229).  near (optional) is set when u lies within
// two ulp of expf(-beta dE): a decision that an expf rounding differently by up to two ulp could flip.  Variant
// bit 4 moves the expf result by up to two ulp at hash-chosen operands (perturbation experiments only).
bool accept(uint32_t r, float beta, float dE, bool* near = nullptr) {
  const float u = (float)(r >> 8) * (1.0f / 16777216.0f);
  const float x = -beta * dE;
  float e = expf(x);
  if (near && e > 0.0f && e < 1.0f) {
    const float lo = std::nextafter(std::nextafter(e, 0.0f), 0.0f), hi = std::nextafter(std::nextafter(e, 2.0f), 2.0f);
    if (u >= lo && u < hi) *near = true;
  }
  if (g_variant & 16) {
    uint32_t ux;
    std::memcpy(&ux, &x, 4);
    const uint32_t h = fmix(ux ^ (g_noise_seed * 0x85EBCA77u) ^ 0x3C6EF372u);
    const int k = (int)(h % 5u) - 2;  // -2 .. 2 ulp
    for (int i = 0; i < k; i++) e = std::nextafter(e, INFINITY);
    for (int i = 0; i > k; i--) e = std::nextafter(e, -INFINITY);
  }
  return u < e;
}

// ---- sets --------------------------------------------------------------------------------------------
bool in(const Set& s, int l) { return std::binary_search(s.begin(), s.end(), l); }
int live_size(const Set& s, const std::vector<char>& cut) {
  int n = 0;
  for (int l : s) n += cut[l] ? 0 : 1;
  return n;
}
// counts of contraction (x, y) -> z over unsliced labels: B, M, N from z, K from x
void contraction_counts(const Set& x, const Set& y, const Set& z, const std::vector<char>& cut, int& B, int& M, int& N,
                        int& K) {
  B = M = N = K = 0;
  for (int l : z) {
    if (cut[l]) continue;
    const bool a = in(x, l), b = in(y, l);
    if (a && b) B++;
    else if (a) M++;
    else if (b) N++;
  }
  for (int l : x)
    if (!cut[l] && in(y, l) && !in(z, l)) K++;
}
// Julia tcscrw without rw: tc = |z| + |{l in x : l in y, l not in z}| over unsliced labels
int tcscrw(const Set& x, const Set& y, const Set& z, const std::vector<char>& cut) {
  int tc = live_size(z, cut);
  for (int l : x)
    if (!cut[l] && in(y, l) && !in(z, l)) tc++;
  return tc;
}
float contraction_cost(int mode, const Set& x, const Set& y, const Set& z, const std::vector<char>& cut,
                       const OParams& P) {
  int B, M, N, K;
  contraction_counts(x, y, z, cut, B, M, N, K);
  if (mode == 0) return (float)(live_size(z, cut) + K);
  return model_lt(mode, B, M, N, K, P);
}

// ---- the tree -----------------------------------------------------------------------------------------
struct Tree {
  int m = 0, nlab = 0;
  std::vector<int> L, R;   // children, -1 for leaves
  std::vector<Set> lab;    // output labels of every node (leaves: their tensor)
  std::vector<char> cut;   // sliced labels
  bool leaf(int v) const { return L[v] < 0; }
};

struct Counter {
  long long prop = 0, acc = 0, visits = 0, phases = 0, sprop = 0, sacc = 0;
  bool near = false;  // a Metropolis decision within two ulp of expf happened
};

// One proposal at internal node v (csrc/cpu_ref.h:87-121).  Julia rules 1..4: pivot = left child for
// rules 1, 2 and right child for 3, 4; (a, b) are the pivot's children in rule order, c the other child;
// an accepted move contracts (a, c) first: the pivot's labels become those of (a, c) and b moves up.
void propose(Tree& T, int v, float beta, uint32_t sweep, uint32_t chain, const OParams& P, int mode, Counter& C) {
  const int l = T.L[v], r = T.R[v];
  const bool li = !T.leaf(l), ri = !T.leaf(r);
  if (!li && !ri) return;
  const R4 rn = philox10(R4{(uint32_t)v, sweep, chain, 0u}, P.key0, P.key1);
  int rule;  // 1..4
  if (li && ri) rule = 1 + (int)(rn.a >> 30);
  else if (li) rule = 1 + (int)(rn.a >> 31);
  else rule = 3 + (int)(rn.a >> 31);
  const int piv = rule <= 2 ? l : r, oth = rule <= 2 ? r : l;
  int a, b;
  if (rule == 1) { a = T.L[piv]; b = T.R[piv]; }
  else if (rule == 2) { a = T.R[piv]; b = T.L[piv]; }
  else if (rule == 3) { a = T.R[piv]; b = T.L[piv]; }
  else { a = T.L[piv]; b = T.R[piv]; }
  const Set &A = T.lab[a], &Bs = T.lab[b], &AB = T.lab[piv], &Cs = T.lab[oth], &D = T.lab[v];
  Set AC;  // labels of (a, c) that survive: in a or c, and in b or d
  for (int x : A)
    if (in(Bs, x) || in(D, x)) AC.push_back(x);
  for (int x : Cs)
    if (!in(A, x) && (in(Bs, x) || in(D, x))) AC.push_back(x);
  std::sort(AC.begin(), AC.end());
  float dtc;
  if (mode == 0) {
    const float before = lse_int(tcscrw(A, Bs, AB, T.cut), tcscrw(AB, Cs, D, T.cut));
    const float after = lse_int(tcscrw(A, Cs, AC, T.cut), tcscrw(AC, Bs, D, T.cut));
    dtc = after - before;
  } else {
    const float before = lse_flt(contraction_cost(mode, A, Bs, AB, T.cut, P), contraction_cost(mode, AB, Cs, D, T.cut, P));
    const float after = lse_flt(contraction_cost(mode, A, Cs, AC, T.cut, P), contraction_cost(mode, AC, Bs, D, T.cut, P));
    dtc = after - before;
  }
  const int sd = live_size(D, T.cut);
  const int sc0 = std::max(live_size(AB, T.cut), sd), sc1 = std::max(live_size(AC, T.cut), sd);
  const float w = ((float)std::max(sc0, sc1) > P.sc_target) ? P.sc_weight : 0.0f;
  const float dE = w * (float)(sc1 - sc0) + dtc;
  C.prop++;
  if (!accept(rn.b, beta, dE, &C.near)) return;
  C.acc++;
  // b and c trade places, keeping slots
  if (rule == 1) { T.R[piv] = oth; T.R[v] = b; }
  else if (rule == 2) { T.L[piv] = oth; T.R[v] = b; }
  else if (rule == 3) { T.L[piv] = oth; T.L[v] = b; }
  else { T.R[piv] = oth; T.L[v] = b; }
  T.lab[piv] = AC;
}

void preorder_sweep(Tree& T, int v, float beta, uint32_t sweep, uint32_t chain, const OParams& P, int mode, Counter& C) {
  if (T.leaf(v)) return;
  C.visits++;
  if (T.leaf(T.L[v]) && T.leaf(T.R[v])) return;
  propose(T, v, beta, sweep, chain, P, mode, C);
  const int nl = T.L[v], nr = T.R[v];
  preorder_sweep(T, nl, beta, sweep, chain, P, mode, C);
  preorder_sweep(T, nr, beta, sweep, chain, P, mode, C);
}

// Par order (csrc/cpu_ref.h:128-182): random priorities, then independent sets of nodes whose
// (priority, id) key beats their unvisited parent and internal children, applied one after the other.
void par_sweep(Tree& T, float beta, uint32_t sweep, uint32_t chain, const OParams& P, int mode, Counter& C) {
  const int m = T.m, n = 2 * m - 1;
  std::vector<int> up(n, -1);
  for (int v = m; v < n; v++) up[T.L[v]] = up[T.R[v]] = v;
  const uint32_t hs = fmix(sweep * 0x85EBCA77u + fmix(chain ^ P.key0));
  std::vector<uint32_t> pr(n, 0);
  for (int v = m; v < n; v++) pr[v] = (fmix((uint32_t)v * 0x9E3779B1u + hs) >> 16) | 1u;
  if (P.par_band > 0) {
    std::vector<int> depth(n, 0);  // depth at sweep start (root 0), by walking up the parent links
    for (int v = m; v < n; v++)
      for (int u = v; up[u] >= 0; u = up[u]) depth[v]++;
    const int Lb = P.par_band;
    for (int v = m; v < n; v++)
      pr[v] = ((uint32_t)((Lb - 1 - depth[v] % Lb) & 15) << 12) | (pr[v] & 0x0FFEu) | 1u;
  }
  auto key = [&](int u) { return (pr[u] << 16) | (uint32_t)u; };
  auto beats = [&](int u, uint32_t kv) { return u >= m && pr[u] != 0 && key(u) > kv; };
  std::vector<int> set;
  for (;;) {
    set.clear();
    for (int v = m; v < n; v++) {
      if (pr[v] == 0) continue;
      const uint32_t kv = key(v);
      if (up[v] >= 0 && beats(up[v], kv)) continue;
      if (beats(T.L[v], kv) || beats(T.R[v], kv)) continue;
      set.push_back(v);
    }
    if (set.empty()) break;
    C.phases++;
    for (int v : set) {
      const bool follow = (pr[v] & 1u) == 0;
      const int l0 = T.L[v], r0 = T.R[v];
      C.visits++;
      propose(T, v, beta, follow ? (sweep | 0x80000000u) : sweep, chain, P, mode, C);
      if (P.par_follow && !follow && (T.L[v] != l0 || T.R[v] != r0)) {
        const int pv = T.L[v] == l0 ? l0 : r0;
        if (pr[pv] == 0) pr[pv] = ((fmix(((uint32_t)pv * 0x9E3779B1u + hs) ^ 0x5BD1E995u) >> 16) & 0xFFFEu) | 2u;
      }
      for (int u : {T.L[v], T.R[v]}) {
        up[u] = v;
        if (u >= m) up[T.L[u]] = up[T.R[u]] = u;
      }
      pr[v] = 0;
    }
  }
}

// ---- whole-chain energy in the 32-lane fold order, and the slice step ----------------------------------
struct Eval {
  float lcost;
  int sc, sc_int, ncand, ns;
};

Eval eval_chain(const Tree& T, const OParams& P, int mode) {
  const int m = T.m, nint = m - 1;
  float acc[32];
  int best[32], nbest[32];
  for (int t = 0; t < 32; t++) {
    acc[t] = -INFINITY;
    best[t] = 0;
    nbest[t] = 0;
    for (int i = t; i < nint; i += 32) {
      const int v = m + i;
      int B, M, N, K;
      contraction_counts(T.lab[T.L[v]], T.lab[T.R[v]], T.lab[v], T.cut, B, M, N, K);
      const int Z = live_size(T.lab[v], T.cut);
      const float cost = mode == 0 ? (float)(Z + K) : model_lt(mode, B, M, N, K, P);
      acc[t] = lse_fold(acc[t], cost);
      if (Z > best[t]) { best[t] = Z; nbest[t] = 1; }
      else if (Z == best[t]) nbest[t]++;
    }
  }
  for (int o = 16; o > 0; o >>= 1) {
    float nxt[32];
    for (int t = 0; t < 32; t++) nxt[t] = lse_fold(acc[t], acc[t ^ o]);
    std::memcpy(acc, nxt, sizeof acc);
  }
  int scmax = 0;
  for (int t = 0; t < 32; t++) scmax = std::max(scmax, best[t]);
  int cnt = 0;
  for (int t = 0; t < 32; t++)
    if (best[t] == scmax) cnt += nbest[t];
  int ns = 0;
  if (P.slicing)
    for (int l = 0; l < T.nlab; l++) ns += T.cut[l] ? 1 : 0;
  Eval e;
  e.lcost = acc[0];
  e.sc_int = scmax;
  e.ncand = cnt;
  e.ns = ns;
  e.sc = std::max(scmax, P.leaf_sc);
  if (P.slicing && P.leaf_sc > scmax) {
    int ll = 0;
    for (int i = 0; i < m; i++) ll = std::max(ll, live_size(T.lab[i], T.cut));
    e.sc = std::max(scmax, ll);
  }
  return e;
}


float slice_energy(const Eval& e, const OParams& P) {
  const float pen = (float)e.sc > P.sc_target ? P.sc_weight * ((float)e.sc - P.sc_target) : 0.0f;
  return (float)e.ns + e.lcost + pen;
}

// k-th (0-based) label of s in increasing id order that is not sliced (cut_aware) / any label
int kth_label(const Set& s, const std::vector<char>& cut, int k) {
  for (int l : s) {
    if (cut[l]) continue;
    if (k-- == 0) return l;
  }
  return -1;
}

// The proposal of one slice move from the chain's evaluation cur and the word r1 (csrc/treesa_gpu.cu:
// 455-478): type 0 add, 1 remove, 2 swap, -1 no move; ladd / lrem the labels added / removed (-1: none).
int propose_slice(const Tree& T, const Eval& cur, const R4& r1, const OParams& P, int& ladd, int& lrem) {
  const int m = T.m, nint = m - 1;
  int type;
  if (cur.ns == 0) type = 0;
  else if (cur.ns >= P.max_slices) type = (r1.a >> 31) ? 1 : 2;
  else type = r1.a < 0x80000000u ? 0 : (r1.a < 0xC0000000u ? 1 : 2);
  ladd = -1;
  lrem = -1;
  if (type != 1 && cur.ncand > 0 && cur.sc_int > 0) {
    int rr = (int)(r1.b % (uint32_t)cur.ncand), node = -1;
    for (int i = 0; i < nint && node < 0; i++)
      if (live_size(T.lab[m + i], T.cut) == cur.sc_int && rr-- == 0) node = m + i;
    if (node >= 0) ladd = kth_label(T.lab[node], T.cut, (int)(r1.c % (uint32_t)cur.sc_int));
  }
  if (type != 0) {
    int k = (int)(r1.d % (uint32_t)cur.ns);
    for (int l = 0; l < T.nlab; l++)
      if (T.cut[l] && k-- == 0) { lrem = l; break; }
  }
  if (type == 2 && ladd < 0) type = 1;
  if (type == 0 && ladd < 0) return -1;
  return type;
}

// Slice moves after a sweep (mirror of csrc/treesa_gpu.cu:445-502): add a label of a largest internal
// tensor, remove a sliced label, or swap, Metropolis on E = |S| + lcost + sc penalty.
void slice_step(Tree& T, float beta, uint32_t sweep, uint32_t chain, const OParams& P, int mode, Counter& C) {
  Eval cur = eval_chain(T, P, mode);
  float Ecur = slice_energy(cur, P);
  for (int j = 0; j < P.slice_moves; j++) {
    const R4 r1 = philox10(R4{0x10000u + 2u * (uint32_t)j, sweep, chain, 0u}, P.key0, P.key1);
    const R4 r2 = philox10(R4{0x10001u + 2u * (uint32_t)j, sweep, chain, 0u}, P.key0, P.key1);
    int ladd, lrem;
    const int type = propose_slice(T, cur, r1, P, ladd, lrem);
    if (type < 0) continue;
    if (type != 1) T.cut[ladd] = 1;
    if (type != 0) T.cut[lrem] = 0;
    const Eval nxt = eval_chain(T, P, mode);
    const float Enew = slice_energy(nxt, P);
    C.sprop++;
    if (accept(r2.a, beta, Enew - Ecur, &C.near)) {
      C.sacc++;
      cur = nxt;
      Ecur = Enew;
    } else {
      if (type != 1) T.cut[ladd] = 0;
      if (type != 0) T.cut[lrem] = 1;
    }
  }
}

// ---- records <-> trees ---------------------------------------------------------------------------------
Set bits_to_set(const uint64_t* w, int W) {
  Set s;
  for (int k = 0; k < W; k++)
    for (uint64_t x = w[k]; x; x &= x - 1) s.push_back(k * 64 + __builtin_ctzll(x));
  return s;
}
void set_to_bits(const Set& s, uint64_t* w, int W) {
  for (int k = 0; k < W; k++) w[k] = 0;
  for (int l : s) w[l >> 6] |= 1ull << (l & 63);
}

Tree from_record(const Inst& I, const Layout& Lo, const uint64_t* rec, bool slicing) {
  Tree T;
  T.m = I.m;
  T.nlab = I.nlab;
  const int n = 2 * I.m - 1;
  T.L.assign(n, -1);
  T.R.assign(n, -1);
  T.lab.resize(n);
  for (int i = 0; i < I.m; i++) T.lab[i] = I.ixs[i];
  const uint32_t* ch = reinterpret_cast<const uint32_t*>(rec + Lo.ch_off);
  for (int i = 0; i < I.m - 1; i++) {
    T.L[I.m + i] = (int)(ch[i] & 0xFFFFu);
    T.R[I.m + i] = (int)(ch[i] >> 16);
    T.lab[I.m + i] = bits_to_set(rec + (size_t)i * Lo.W, Lo.W);
  }
  T.cut.assign(I.nlab + 64 * Lo.W, 0);
  if (slicing)
    for (int l = 0; l < I.nlab; l++) T.cut[l] = (char)((rec[Lo.s_off + (l >> 6)] >> (l & 63)) & 1u);
  return T;
}

void to_record(const Tree& T, const Layout& Lo, uint64_t* rec, bool slicing) {
  uint32_t* ch = reinterpret_cast<uint32_t*>(rec + Lo.ch_off);
  for (int i = 0; i < T.m - 1; i++) {
    ch[i] = (uint32_t)T.L[T.m + i] | ((uint32_t)T.R[T.m + i] << 16);
    set_to_bits(T.lab[T.m + i], rec + (size_t)i * Lo.W, Lo.W);
  }
  if (slicing) {
    for (int k = 0; k < Lo.W; k++) rec[Lo.s_off + k] = 0;
    for (int l = 0; l < T.nlab; l++)
      if (T.cut[l]) rec[Lo.s_off + (l >> 6)] |= 1ull << (l & 63);
  }
}

// Output labels from topology: l is an output of v iff it occurs in v's subtree and (occurs outside it
// or is open).  Returns false if ch is not a binary tree over all 2m-1 nodes rooted at 2m-2.
bool topo_labels(const Inst& I, const uint32_t* ch, std::vector<Set>& out) {
  const int m = I.m, n = 2 * m - 1;
  std::vector<int> order, stack{n - 1};
  std::vector<char> seen(n, 0);
  while (!stack.empty()) {
    const int v = stack.back();
    stack.pop_back();
    if (v < 0 || v >= n || seen[v]) return false;
    seen[v] = 1;
    order.push_back(v);
    if (v >= m) {
      stack.push_back((int)(ch[v - m] & 0xFFFFu));
      stack.push_back((int)(ch[v - m] >> 16));
    }
  }
  if ((int)order.size() != n) return false;
  // occurrence counts per subtree, children before parents (reverse of the DFS order)
  std::vector<std::vector<std::pair<int, int>>> occ(n);
  out.assign(n, Set());
  for (int k = n - 1; k >= 0; k--) {
    const int v = order[k];
    std::vector<std::pair<int, int>> mine;
    if (v < m) {
      for (int l : I.ixs[v]) mine.push_back({l, 1});
    } else {
      const auto& a = occ[(int)(ch[v - m] & 0xFFFFu)];
      const auto& b = occ[(int)(ch[v - m] >> 16)];
      size_t i = 0, j = 0;
      while (i < a.size() || j < b.size()) {
        if (j == b.size() || (i < a.size() && a[i].first < b[j].first)) mine.push_back(a[i++]);
        else if (i == a.size() || b[j].first < a[i].first) mine.push_back(b[j++]);
        else { mine.push_back({a[i].first, a[i].second + b[j].second}); i++; j++; }
      }
      for (auto& pc : mine)
        if (pc.second < I.total[pc.first] || I.open[pc.first]) out[v].push_back(pc.first);
    }
    occ[v] = std::move(mine);
  }
  return true;
}

// ---- the level loop (csrc/treesa_gpu.cu:1730-1933) -------------------------------------------------------
// Selection score and population energy in double with the host libm, as the reference's host loop
// evaluates them (csrc/treesa_gpu.cu:1737-1753).
struct Selector {
  int slicing, select_sc;
  double sct, w;
  double energy(float lc, int sc, int ns) const {
    return (double)ns + (double)lc + w * std::max(0.0, (double)sc - sct);
  }
  double score(int mode, float lc, int sc, int ns) const {
    if (slicing) return (double)ns + (double)lc + 1000.0 * std::max(0.0, (double)sc - sct);
    if (select_sc) return 4096.0 * std::max(0.0, (double)sc - sct) + (double)lc;
    if (mode != 0) return energy(lc, sc, ns);
    const double tc = (double)lc;
    if ((double)sc <= sct || w <= 0) return tc;
    // log2(2^tc + w (2^sc - 2^sct)), both terms in log2
    const double pen = std::log2(w) + (double)sc + std::log2(1.0 - std::exp2(sct - (double)sc));
    const double hi = std::max(tc, pen), lo = std::min(tc, pen);
    return hi + std::log2(1.0 + std::exp2(lo - hi));
  }
};

// Systematic resampling (csrc/treesa_gpu.cu:1837-1856): weights exp(-db (E - Emin)); one uniform u places
// nc equally spaced pointers j + u on the cumulative scaled weights.  margin (optional) receives the smallest
// |cumulative - (j + u)| met at a pointer decision.
void systematic(const std::vector<double>& E, double db, double u, std::vector<int>& anc, double* margin) {
  const int nc = (int)E.size();
  double lo = INFINITY;
  for (double e : E) lo = std::min(lo, e);
  std::vector<double> wt(nc);
  double tot = 0;
  for (int c = 0; c < nc; c++) {
    wt[c] = std::exp(-db * (E[c] - lo));
    tot += wt[c];
  }
  anc.assign(nc, nc - 1);
  double cum = 0, mg = INFINITY;
  int j = 0;
  for (int c = 0; c < nc; c++) {
    cum += wt[c] / tot * nc;
    for (; j < nc; j++) {
      mg = std::min(mg, std::fabs(cum - (j + u)));
      if (!(j + u < cum)) break;
      anc[j] = c;
    }
  }
  if (margin) *margin = mg;
}

// Truncation selection (csrc/treesa_gpu.cu:1857-1869): chains ordered by E with std::sort (the reference's
// unstable libstdc++ introsort), then the k-th worst becomes a copy of the k-th best for k < frac * nc.
void truncation(const std::vector<double>& E, double frac, std::vector<int>& anc, std::vector<int>* order) {
  const int nc = (int)E.size();
  std::vector<int> ix(nc);
  for (int c = 0; c < nc; c++) ix[c] = c;
  std::sort(ix.begin(), ix.end(), [&](int a, int b) { return E[a] < E[b]; });
  anc.resize(nc);
  for (int c = 0; c < nc; c++) anc[c] = c;
  const int nrep = (int)(frac * nc);
  for (int k = 0; k < nrep; k++) anc[ix[nc - 1 - k]] = ix[k];
  if (order) *order = ix;
}

bool same_tree(const Tree& a, const Tree& b) { return a.L == b.L && a.R == b.R && a.cut == b.cut; }

// Final slice repair (csrc/treesa_gpu.cu:1248-1274): while the largest masked tensor (leaves included)
// exceeds sct, cut the label that occurs in most of the largest tensors, lowest id on ties.
int repair_slices(Tree& T, double sct) {
  const int n = 2 * T.m - 1;
  int added = 0;
  for (;;) {
    std::vector<int> sz(n);
    int top = 0;
    for (int v = 0; v < n; v++) top = std::max(top, sz[v] = live_size(T.lab[v], T.cut));
    if (top == 0 || (double)top <= sct) return added;
    std::vector<int> hits(T.nlab, 0);
    for (int v = 0; v < n; v++)
      if (sz[v] == top)
        for (int l : T.lab[v])
          if (!T.cut[l]) hits[l]++;
    int pick = 0;
    for (int l = 1; l < T.nlab; l++)
      if (hits[l] > hits[pick]) pick = l;
    T.cut[pick] = 1;
    added++;
  }
}

// nsweeps sweeps of one chain (slot `chain`) from global sweep sweep0, slice steps after every sweep s with
// (s + 1) % slice_every == 0 when slice moves are on (csrc/treesa_gpu.cu:975-978).
void run_chain(Tree& T, const OParams& P, int order, float beta, uint32_t sweep0, int nsweeps, uint32_t chain,
               Counter& C) {
  for (int s = 0; s < nsweeps; s++) {
    const uint32_t sw = sweep0 + (uint32_t)s;
    if (order == 0) par_sweep(T, beta, sw, chain, P, P.mode, C);
    else preorder_sweep(T, 2 * T.m - 2, beta, sw, chain, P, P.mode, C);
    if (P.slicing && P.slice_moves > 0 && (sw + 1u) % (uint32_t)(P.slice_every > 0 ? P.slice_every : 1) == 0u)
      slice_step(T, beta, sw, chain, P, P.mode, C);
  }
}

// Host double-precision complexities of a tree on its sliced network (csrc/treesa_gpu.cu:1206-1244):
// out = {tc, sc, gpu_time, h100_time, |S|}.  gm / hm: the model constants as given on the command line.
void tree_host_energy(const Tree& T, const double* gm, const double* hm, double* out) {
  const int m = T.m;
  int sc = 0, ns = 0;
  for (int l = 0; l < T.nlab; l++) ns += T.cut[l] ? 1 : 0;
  for (int i = 0; i < m; i++) sc = std::max(sc, live_size(T.lab[i], T.cut));
  std::vector<double> t;
  double time = 0, time2 = 0;
  const float lpeak = (float)std::log2(gm[0]), lbw = (float)std::log2(gm[1]), lla = (float)std::log2(gm[5]);
  const float hl[9] = {(float)std::log2(3 * hm[0]), (float)std::log2(2 / hm[1]), (float)std::log2(hm[2]),
                       (float)std::log2(hm[3]),     (float)std::log2(hm[4]),     (float)std::log2(hm[5]),
                       (float)std::log2(hm[6]),     0.f,                         (float)std::log2(hm[8])};
  auto e2 = [](float l) { return std::exp2((double)l); };
  for (int v = m; v < 2 * m - 1; v++) {
    int B, M, N, K;
    contraction_counts(T.lab[T.L[v]], T.lab[T.R[v]], T.lab[v], T.cut, B, M, N, K);
    t.push_back((double)(B + M + N + K));
    sc = std::max(sc, live_size(T.lab[v], T.cut));
    const double ops = std::exp2((double)(1 + B + std::max(M, (int)gm[2]) + std::max(N, (int)gm[3]) + std::max(K, (int)gm[4])));
    const double bits = std::exp2((double)(B + M + K)) + std::exp2((double)(B + N + K)) + std::exp2((double)(B + M + N));
    time += std::max(ops / std::exp2((double)lpeak), bits / std::exp2((double)lbw)) + std::exp2((double)lla);
    if (B + M + N <= (int)hm[7]) {
      time2 += e2(hl[8]) * std::exp2((double)(B + M + N + K));
    } else {
      const double a = std::exp2((double)(B + M + K)), b = std::exp2((double)(B + N + K)), c = std::exp2((double)(B + M + N));
      double best = e2(hl[2]) * (a + b + c) + e2(hl[3]) * std::exp2((double)(B + M + N + K));
      if (K >= 7 && std::max(M, N) >= 5)
        best = std::min(best, e2(hl[4]) * (a + b + c) +
                                  e2(hl[5]) * std::exp2((double)(B + std::max(M, 6) + std::max(N, 6) + std::max(K, 8))) +
                                  e2(hl[6]) * c);
      time2 += e2(hl[0]) + e2(hl[1]) * (a + b) + best;
    }
  }
  double mx = -1e300;
  for (double x : t) mx = std::max(mx, x);
  double s = 0;
  for (double x : t) s += std::exp2(x - mx);
  out[0] = mx + std::log2(s);
  out[1] = sc;
  out[2] = time;
  out[3] = time2;
  out[4] = ns;
}

}  // namespace

// =========================================================================================================
// C API for the tests (ctypes)
// =========================================================================================================
extern "C" {

void* oracle_new(int m, int nlab, const int* offs, const int* labels, int ny, const int* iy) {
  ensure_lse();
  Inst* I = new Inst();
  I->m = m;
  I->nlab = nlab;
  I->ixs.resize(m);
  for (int i = 0; i < m; i++) {
    I->ixs[i].assign(labels + offs[i], labels + offs[i + 1]);
    std::sort(I->ixs[i].begin(), I->ixs[i].end());
  }
  I->iy.assign(iy, iy + ny);
  I->total.assign(nlab, 0);
  I->open.assign(nlab, 0);
  for (auto& s : I->ixs)
    for (int l : s) I->total[l]++;
  for (int l : I->iy) I->open[l] = 1;
  return I;
}

void oracle_free(void* h) { delete static_cast<Inst*>(h); }

uint64_t oracle_splitmix64(uint64_t x) { return smix64(x); }

// Perturbation experiments only: see g_variant (0 restores the reference's arithmetic).
void oracle_set_variant(int v, uint32_t noise_seed) {
  g_variant = v;
  g_noise_seed = noise_seed;
}

void oracle_philox(const uint32_t* ctr, uint32_t k0, uint32_t k1, uint32_t* out) {
  const R4 r = philox10(R4{ctr[0], ctr[1], ctr[2], ctr[3]}, k0, k1);
  out[0] = r.a;
  out[1] = r.b;
  out[2] = r.c;
  out[3] = r.d;
}

uint32_t oracle_par_pri(uint32_t v, uint32_t s, uint32_t c, uint32_t key0) {
  return (fmix(v * 0x9E3779B1u + fmix(s * 0x85EBCA77u + fmix(c ^ key0))) >> 16) | 1u;
}

void oracle_lse_table(float* out) {
  ensure_lse();
  std::memcpy(out, g_lse, sizeof g_lse);
}

// Julia random_exprtree: recursive random bipartition, internal nodes numbered in post-order from m
// (csrc/treesa_gpu.cu:1101-1123); rng = mt19937_64(seed).
void oracle_random_tree(int m, uint64_t seed, uint32_t* ch) {
  std::mt19937_64 rng(seed);
  int next = m;
  std::function<int(const std::vector<int>&)> split = [&](const std::vector<int>& xs) -> int {
    const int n = (int)xs.size();
    if (n == 1) return xs[0];
    std::vector<char> side(n);
    int ones = 0;
    for (int i = 0; i < n; i++) {
      side[i] = (char)(rng() & 1u);
      ones += side[i];
    }
    if (ones == 0 || ones == n) {
      const int i = (int)(rng() % (uint64_t)n);
      side[i] = !side[i];
    }
    std::vector<int> a, b;
    for (int i = 0; i < n; i++) (side[i] ? a : b).push_back(xs[i]);
    const int l = split(a), r = split(b);
    const int v = next++;
    ch[v - m] = (uint32_t)l | ((uint32_t)r << 16);
    return v;
  };
  std::vector<int> all(m);
  for (int i = 0; i < m; i++) all[i] = i;
  split(all);
}

// The fixed random slice set of chain c in --check mode: k labels drawn with
// mt19937_64(splitmix64(seed * 7919 + c)) % nlab (csrc/treesa_gpu.cu:1621-1627), OR-ed into S (W words).
void oracle_random_slices(int nlab, uint64_t seed, int c, int k, int W, uint64_t* S) {
  std::mt19937_64 rng(smix64(seed * 7919ull + (uint64_t)c));
  for (int j = 0; j < k; j++) {
    const int l = (int)(rng() % (uint64_t)nlab);
    if ((l >> 6) < W) S[l >> 6] |= 1ull << (l & 63);
  }
}

// Internal-node label sets of a tree in record word format; 0 ok, 1 invalid tree.
int oracle_labels(void* h, const uint32_t* ch, int W, uint64_t* lab) {
  const Inst& I = *static_cast<Inst*>(h);
  std::vector<Set> out;
  if (!topo_labels(I, ch, out)) return 1;
  for (int i = 0; i < I.m - 1; i++) set_to_bits(out[I.m + i], lab + (size_t)i * W, W);
  return 0;
}

// nsweeps sweeps of chains [c0, c0 + n) of a population (records back to back, record k = chain c0 + k),
// in place.  order 0 par, 1 pre-order.  Slice steps follow sweep s when slice_moves > 0 and
// (s + 1) % slice_every == 0.  stats[6]: proposals, accepts, phases, visits, slice proposals, slice
// accepts, 0.  Chains run in parallel with OpenMP.
int oracle_sweeps(void* h, const OParams* P, int W, int ch_off, int s_off, int chain_words, uint64_t* pop, int c0,
                  int n, int order, float beta, uint32_t sweep0, int nsweeps, long long* stats) {
  const Inst& I = *static_cast<Inst*>(h);
  const Layout Lo{W, ch_off, s_off, chain_words};
  long long sp = 0, sa = 0, sph = 0, sv = 0, ssp = 0, ssa = 0;
#pragma omp parallel for schedule(dynamic, 1) reduction(+ : sp, sa, sph, sv, ssp, ssa)
  for (int k = 0; k < n; k++) {
    uint64_t* rec = pop + (size_t)k * chain_words;
    Tree T = from_record(I, Lo, rec, P->slicing != 0);
    Counter C;
    run_chain(T, *P, order, beta, sweep0, nsweeps, (uint32_t)(c0 + k), C);
    to_record(T, Lo, rec, P->slicing != 0);
    sp += C.prop;
    sa += C.acc;
    sph += C.phases;
    sv += C.visits;
    ssp += C.sprop;
    ssa += C.sacc;
  }
  if (stats) {
    stats[0] = sp;
    stats[1] = sa;
    stats[2] = sph;
    stats[3] = sv;
    stats[4] = ssp;
    stats[5] = ssa;
  }
  return 0;
}

// Per-chain energy (lc, sc, ns) of n records in the 32-lane fold order of the device.
int oracle_energy(void* h, const OParams* P, int W, int ch_off, int s_off, int chain_words, const uint64_t* pop,
                  int n, float* lc, int* sc, int* ns) {
  const Inst& I = *static_cast<Inst*>(h);
  const Layout Lo{W, ch_off, s_off, chain_words};
#pragma omp parallel for schedule(dynamic, 4)
  for (int k = 0; k < n; k++) {
    const Tree T = from_record(I, Lo, pop + (size_t)k * chain_words, P->slicing != 0);
    const Eval e = eval_chain(T, *P, P->mode);
    lc[k] = e.lcost;
    sc[k] = e.sc;
    ns[k] = e.ns;
  }
  return 0;
}

// One record's chain evaluation (the fold the sweep kernels run) and the slice proposal the words r1 make
// from it: out = {type, ladd, lrem, sc_int, ncand, ns, sc}, *lcost the folded log2 cost.
int oracle_slice_propose(void* h, const OParams* P, int W, int ch_off, int s_off, int chain_words,
                         const uint64_t* rec, const uint32_t* r1, int* out, float* lcost) {
  const Inst& I = *static_cast<Inst*>(h);
  const Layout Lo{W, ch_off, s_off, chain_words};
  const Tree T = from_record(I, Lo, rec, P->slicing != 0);
  const Eval e = eval_chain(T, *P, P->mode);
  int ladd, lrem;
  out[0] = propose_slice(T, e, R4{r1[0], r1[1], r1[2], r1[3]}, *P, ladd, lrem);
  out[1] = ladd;
  out[2] = lrem;
  out[3] = e.sc_int;
  out[4] = e.ncand;
  out[5] = e.ns;
  out[6] = e.sc;
  *lcost = e.lcost;
  return 0;
}

// Host double-precision complexities of one record (csrc/treesa_gpu.cu:1206-1244): out = {tc, sc,
// gpu_time, h100_time, |S|}.  gm / hm: the model constants as given on the command line.
void oracle_host_energy(void* h, const double* gm, const double* hm, int W, int ch_off, int s_off, int chain_words,
                        const uint64_t* rec, int slicing, double* out) {
  const Inst& I = *static_cast<Inst*>(h);
  const Layout Lo{W, ch_off, s_off, chain_words};
  tree_host_energy(from_record(I, Lo, rec, slicing != 0), gm, hm, out);
}

// ---- the level loop -----------------------------------------------------------------------------------
// Inputs of oracle_anneal (field order matches tests/oracle.py).
struct OAnnealIn {
  int32_t nlev;
  int32_t order;       // 0 par, 1 pre-order
  int32_t scheme;      // 0 indep, 1 pa, 2 trunc
  int32_t eval_every;
  int32_t select_sc;
  int32_t pad;
  double trunc_frac, sc_target, sc_weight;
  uint64_t seed;
  const float* betas;      // nlev
  const int32_t* lmode;    // nlev: energy mode of every level (stage 2 continues the population in another)
  const int32_t* lniters;  // nlev: sweeps of every level
  const double* gm;        // model constants as given on the command line (6 and 9 values)
  const double* hm;
  // near-tie record (diagnostics; near_cap 0: off): every evaluated level's best chain whose score lies within
  // near_tol of the incumbent's after the level, as {level, chain, score, lc, host tc, host sc}
  double near_tol;
  int32_t near_cap;
  int32_t pad2;
  double* near_out;        // near_cap x 6 doubles
  int32_t* near_count;     // entries written (at most near_cap)
};

// What one level left (field order matches tests/oracle.py).
struct OLevel {
  int32_t evaluated, best, sc, ns, families, mode, resampled;
  float lc;
  double score, meanE, meanNs;
  double sel_margin;  // smallest gap between the level's best score and another tree's score, or the incumbent's
  double pop_margin;  // resampling: smallest |cumulative - pointer| (pa) or E gap between ranked neighbours (trunc)
  int32_t metropolis_near;  // chains with a Metropolis decision within two ulp of expf in this level's sweeps
  int32_t pad;
};

// The reference's run_anneal (csrc/treesa_gpu.cu:1756-1877) over the population pop (nc records, chain c in
// slot c), in place: per level a stage switch when its energy mode changes (the incumbent is rescored in the
// new energy from the host double energy of its record, 1790-1798), niters sweeps of every chain with the
// global sweep counter, then at evaluated levels (every eval_every-th, the last, and the one before a switch)
// the energies, the lowest score over chains (first index on ties) replacing the incumbent only when strictly
// lower (1810-1824), the trace row, and pa / trunc population steps except at the last level and before a
// switch (1836-1869; the pa uniform from mt19937_64(splitmix64(seed + 777))).  anc receives nlev x nc
// ancestor lists (identity where nothing was resampled).  best_rec: the incumbent's record as it was copied
// (maintained labels, children, S).  iout = {best_chain, nresample, staged, total_sweeps}; h1 = the stage-1
// incumbent's host energy {tc, sc, gpu_time, h100_time, |S|} when staged.
int oracle_anneal(void* h, const OParams* P0, int W, int ch_off, int s_off, int chain_words, uint64_t* pop, int nc,
                  const OAnnealIn* in, OLevel* lev_out, int32_t* anc, uint64_t* best_rec, int32_t* iout, double* h1) {
  const Inst& I = *static_cast<Inst*>(h);
  const Layout Lo{W, ch_off, s_off, chain_words};
  const bool sl = P0->slicing != 0;
  std::vector<Tree> trees(nc);
  for (int c = 0; c < nc; c++) trees[c] = from_record(I, Lo, pop + (size_t)c * chain_words, sl);
  Selector sel{P0->slicing, in->select_sc, in->sc_target, in->sc_weight};
  int mode = P0->mode;
  Tree best;
  bool have_best = false;
  double best_score = INFINITY;
  int best_chain = -1, nresample = 0, staged = 0;
  uint32_t sweeps = 0;
  std::vector<int> family(nc);
  for (int c = 0; c < nc; c++) family[c] = c;
  std::mt19937_64 prng(smix64(in->seed + 777));
  float beta_mark = in->nlev > 0 ? in->betas[0] : 0.f;
  std::vector<float> lc(nc);
  std::vector<int> sc(nc), ns(nc);
  for (int L = 0; L < in->nlev; L++) {
    OLevel& o = lev_out[L];
    std::memset(&o, 0, sizeof o);
    o.best = -1;
    int32_t* a = anc + (size_t)L * nc;
    for (int c = 0; c < nc; c++) a[c] = c;
    if (in->lmode[L] != mode) {
      double e[5];
      tree_host_energy(best, in->gm, in->hm, e);
      std::memcpy(h1, e, sizeof e);
      staged = 1;
      mode = in->lmode[L];
      best_score = sel.score(mode, (float)std::log2(mode == 1 ? e[2] : e[3]), (int)e[1], (int)e[4]);
      beta_mark = in->betas[L];
    }
    OParams P = *P0;
    P.mode = mode;
    const float beta = in->betas[L];
    const int nsw = in->lniters[L];
    int near_here = 0;
#pragma omp parallel for schedule(dynamic, 1) reduction(+ : near_here)
    for (int c = 0; c < nc; c++) {
      Counter C;
      run_chain(trees[c], P, in->order, beta, sweeps, nsw, (uint32_t)c, C);
      near_here += C.near ? 1 : 0;
    }
    o.metropolis_near = near_here;
    sweeps += (uint32_t)nsw;
    const bool last = L + 1 == in->nlev;
    const bool switching = !last && in->lmode[L + 1] != mode;
    o.mode = mode;
    if (!(L % in->eval_every == in->eval_every - 1 || last || switching)) continue;
    o.evaluated = 1;
#pragma omp parallel for schedule(dynamic, 4)
    for (int c = 0; c < nc; c++) {
      const Eval e = eval_chain(trees[c], P, mode);
      lc[c] = e.lcost;
      sc[c] = e.sc;
      ns[c] = e.ns;
    }
    std::vector<double> s(nc), E(nc);
    int bi = 0;
    double sumE = 0, sumNs = 0;
    for (int c = 0; c < nc; c++) {
      s[c] = sel.score(mode, lc[c], sc[c], ns[c]);
      E[c] = sel.energy(lc[c], sc[c], ns[c]);
      if (s[c] < s[bi]) bi = c;
      sumE += E[c];
      sumNs += ns[c];
    }
    double mg = std::isfinite(best_score) ? std::fabs(s[bi] - best_score) : INFINITY;
    for (int c = 0; c < nc; c++)
      if (c != bi && !(s[c] == s[bi] && same_tree(trees[c], trees[bi]))) mg = std::min(mg, s[c] - s[bi]);
    o.sel_margin = mg;
    if (s[bi] < best_score) {
      best_score = s[bi];
      best_chain = bi;
      best = trees[bi];
      have_best = true;
    }
    if (in->near_cap > 0 && std::fabs(s[bi] - best_score) <= in->near_tol && *in->near_count < in->near_cap) {
      double e[5];
      tree_host_energy(trees[bi], in->gm, in->hm, e);
      double* q = in->near_out + 6 * (size_t)(*in->near_count)++;
      q[0] = L;
      q[1] = bi;
      q[2] = s[bi];
      q[3] = lc[bi];
      q[4] = e[0];
      q[5] = e[1];
    }
    std::vector<int> seen(nc, 0);
    int nf = 0;
    for (int c = 0; c < nc; c++) nf += seen[family[c]]++ == 0;
    o.best = bi;
    o.score = s[bi];
    o.lc = lc[bi];
    o.sc = sc[bi];
    o.ns = ns[bi];
    o.families = nf;
    o.meanE = sumE / nc;
    o.meanNs = sumNs / nc;
    if (last || switching || in->scheme == 0) continue;
    std::vector<int> an;
    if (in->scheme == 1) {
      const double db = (double)(in->betas[L + 1] - beta_mark);  // float difference, as the reference
      beta_mark = in->betas[L + 1];
      const double u = std::uniform_real_distribution<double>(0, 1)(prng);
      systematic(E, db, u, an, &o.pop_margin);
    } else {
      std::vector<int> ix;
      truncation(E, in->trunc_frac, an, &ix);
      const int nrep = (int)(in->trunc_frac * nc);
      double g = INFINITY;
      for (int p = 0; p + 1 < nc; p++) {
        if (!(p < nrep || p + 1 >= nc - nrep)) continue;
        const int x = ix[p], y = ix[p + 1];
        if (E[x] == E[y] && same_tree(trees[x], trees[y])) continue;
        g = std::min(g, E[y] - E[x]);
      }
      o.pop_margin = g;
    }
    std::vector<Tree> next(nc);
    std::vector<int> fam(nc);
    for (int c = 0; c < nc; c++) {
      next[c] = trees[an[c]];
      fam[c] = family[an[c]];
      a[c] = an[c];
    }
    trees.swap(next);
    family.swap(fam);
    o.resampled = 1;
    nresample++;
  }
  for (int c = 0; c < nc; c++) to_record(trees[c], Lo, pop + (size_t)c * chain_words, sl);
  std::memset(best_rec, 0, (size_t)chain_words * 8);
  if (have_best) to_record(best, Lo, best_rec, true);
  iout[0] = best_chain;
  iout[1] = nresample;
  iout[2] = staged;
  iout[3] = (int32_t)sweeps;
  return 0;
}

// The final slice repair of a record's tree (labels from its topology, S from the record), S updated in
// place; returns the number of labels added.
int oracle_repair(void* h, int W, int ch_off, int s_off, int chain_words, uint64_t* rec, double sc_target) {
  const Inst& I = *static_cast<Inst*>(h);
  const Layout Lo{W, ch_off, s_off, chain_words};
  Tree T = from_record(I, Lo, rec, true);
  std::vector<Set> lab;
  if (!topo_labels(I, reinterpret_cast<const uint32_t*>(rec + ch_off), lab)) return -1;
  for (int v = I.m; v < 2 * I.m - 1; v++) T.lab[v] = lab[v];
  const int k = repair_slices(T, sc_target);
  for (int w = 0; w < W; w++) rec[s_off + w] = 0;
  for (int l = 0; l < I.nlab; l++)
    if (T.cut[l]) rec[s_off + (l >> 6)] |= 1ull << (l & 63);
  return k;
}

// The population steps alone, on given energies: pa with one uniform u, and trunc.
void oracle_systematic(const double* E, int nc, double db, double u, int32_t* anc) {
  std::vector<int> an;
  systematic(std::vector<double>(E, E + nc), db, u, an, nullptr);
  std::copy(an.begin(), an.end(), anc);
}
void oracle_truncation(const double* E, int nc, double frac, int32_t* anc) {
  std::vector<int> an;
  truncation(std::vector<double>(E, E + nc), frac, an, nullptr);
  std::copy(an.begin(), an.end(), anc);
}
// The selection score and the population energy of one chain, in double with the host libm.
double oracle_score(int mode, int slicing, int select_sc, double sct, double w, float lc, int sc, int ns, int energy) {
  const Selector S{slicing, select_sc, sct, w};
  return energy ? S.energy(lc, sc, ns) : S.score(mode, lc, sc, ns);
}
// FNV-1a (64-bit) of n bytes: the hash the reference harness prints for a chain's label sets.
uint64_t oracle_fnv64(const uint8_t* b, size_t n) {
  uint64_t h = 1469598103934665603ULL;
  for (size_t i = 0; i < n; i++) {
    h ^= b[i];
    h *= 1099511628211ULL;
  }
  return h;
}
// The pa uniforms of a run: the first n draws of uniform_real_distribution<double>(0, 1) over
// mt19937_64(splitmix64(seed + 777)) (csrc/treesa_gpu.cu:1786, 1846).
void oracle_pa_uniforms(uint64_t seed, int n, double* out) {
  std::mt19937_64 g(smix64(seed + 777));
  for (int i = 0; i < n; i++) out[i] = std::uniform_real_distribution<double>(0, 1)(g);
}

}  // extern "C"
