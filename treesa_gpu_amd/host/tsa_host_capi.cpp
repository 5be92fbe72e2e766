// tsa_host_capi.cpp -- C entry points of libtreesa_host.so: the host layer (tsa_host.h) for Python
// (treesa_gpu_amd/host.py: tests, bench.py set-up).  Errors return a negative status and copy the message
// into err.
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "tsa_host.h"

using namespace tsa;

static void put_err(char* err, int len, const std::string& msg) {
  if (err && len > 0) {
    strncpy(err, msg.c_str(), (size_t)len - 1);
    err[len - 1] = 0;
  }
}

extern "C" {

void* tsh_instance_load(const char* path, char* err, int errlen) {
  try {
    return new Network(read_network(path));
  } catch (const std::exception& e) {
    put_err(err, errlen, e.what());
    return nullptr;
  }
}

// offs: m+1 offsets into labels (tensor i = labels[offs[i] .. offs[i+1]))
void* tsh_instance_make(int m, int nlab, const int* offs, const int* labels, int ny, const int* iy, char* err,
                        int errlen) {
  try {
    std::vector<std::vector<int>> ixs(m);
    for (int i = 0; i < m; i++) ixs[i].assign(labels + offs[i], labels + offs[i + 1]);
    return new Network(make_network(m, nlab, ixs, std::vector<int>(iy, iy + ny)));
  } catch (const std::exception& e) {
    put_err(err, errlen, e.what());
    return nullptr;
  }
}

void tsh_instance_free(void* h) { delete static_cast<Network*>(h); }

int tsh_instance_info(void* h, int* m, int* nlab, int* lsc) {
  const Network& I = *static_cast<Network*>(h);
  *m = I.m;
  *nlab = I.nlab;
  *lsc = I.largest_tensor();
  return 0;
}

int tsh_instance_leaf(void* h, int W, uint64_t* out) {
  const Network& I = *static_cast<Network*>(h);
  const std::vector<uint64_t> lf = leaf_sets(I, W);
  memcpy(out, lf.data(), lf.size() * 8);
  return 0;
}

// Up to maxk trees into out (maxk * (m-1) words); returns K or -1.
int tsh_read_trees(const char* path, int m, uint32_t* out, int maxk, char* err, int errlen) {
  try {
    const auto t = read_tree_file(path, m);
    const int K = (int)t.size() < maxk ? (int)t.size() : maxk;
    for (int k = 0; k < K; k++) memcpy(out + (size_t)k * (m - 1), t[k].data(), (size_t)(m - 1) * 4);
    return (int)t.size();
  } catch (const std::exception& e) {
    put_err(err, errlen, e.what());
    return -1;
  }
}

// Returns the number of betas (only the first maxn are written) or -1.
int tsh_parse_betas(const char* spec, float* out, int maxn, char* err, int errlen) {
  try {
    const auto b = parse_schedule(spec);
    for (int i = 0; i < (int)b.size() && i < maxn; i++) out[i] = b[i];
    return (int)b.size();
  } catch (const std::exception& e) {
    put_err(err, errlen, e.what());
    return -1;
  }
}

uint64_t tsh_splitmix64(uint64_t x) { return splitmix64(x); }

void tsh_random_tree(int m, uint64_t seed, uint32_t* out) {
  const auto ch = random_tree(m, seed);
  memcpy(out, ch.data(), ch.size() * 4);
}

int tsh_labels(void* h, int W, const uint32_t* ch, uint64_t* lab) {
  return topology_labels(*static_cast<Network*>(h), W, ch, lab) ? 0 : 1;
}

int tsh_build_population(void* h, int W, int ch_off, int s_off, int chain_words, const uint32_t* trees, int K,
                         int nchains, uint64_t seed, const uint64_t* S0, int random_slices, uint64_t* pop, char* err,
                         int errlen) {
  try {
    const Network& I = *static_cast<Network*>(h);
    std::vector<std::vector<uint32_t>> t(K);
    for (int k = 0; k < K; k++) t[k].assign(trees + (size_t)k * (I.m - 1), trees + (size_t)(k + 1) * (I.m - 1));
    std::vector<uint64_t> s0(S0 ? S0 : nullptr, S0 ? S0 + W : nullptr);
    std::vector<uint64_t> out;
    build_population(I, Geometry{W, ch_off, s_off, chain_words}, t, nchains, seed, s0, random_slices, out);
    memcpy(pop, out.data(), out.size() * 8);
    return 0;
  } catch (const std::exception& e) {
    put_err(err, errlen, e.what());
    return -1;
  }
}

// out = {tc, sc, gpu_time, h100_time, |S|}; S may be null (no slicing).
int tsh_host_energy(void* h, int W, const double* gm, const double* h100, const uint64_t* lab, const uint32_t* ch,
                    const uint64_t* S, double* out) {
  const Network& I = *static_cast<Network*>(h);
  ModelConsts C;
  if (gm) memcpy(C.gm, gm, sizeof C.gm);
  if (h100) memcpy(C.h100, h100, sizeof C.h100);
  const HostEnergy E = host_energy(I, W, model_log2(C), lab, ch, leaf_sets(I, W), S);
  out[0] = E.tc;
  out[1] = E.sc;
  out[2] = E.time;
  out[3] = E.time2;
  out[4] = E.ns;
  return 0;
}

int tsh_greedy_repair(void* h, int W, const uint64_t* lab, uint64_t* S, double sc_target) {
  const Network& I = *static_cast<Network*>(h);
  return greedy_repair(I, W, lab, leaf_sets(I, W), S, sc_target);
}

// The level loop's host arithmetic (tsa_population.cpp) for tests.  scoring: {mode, slicing, select_sc};
// which: 0 selection score, 1 population energy.
double tsh_score(const int* scoring, double sc_target, double sc_weight, float lc, int sc, int ns, int which) {
  Scoring S;
  S.mode = scoring[0];
  S.slicing = scoring[1] != 0;
  S.select_sc = scoring[2] != 0;
  S.sc_target = sc_target;
  S.sc_weight = sc_weight;
  return which ? population_energy(S, lc, sc, ns) : selection_score(S, lc, sc, ns);
}

void tsh_systematic(const double* E, int n, double db, double u, int* anc) {
  const std::vector<int> a = systematic_ancestors(std::vector<double>(E, E + n), db, u);
  memcpy(anc, a.data(), (size_t)n * 4);
}

void tsh_truncation(const double* E, int n, double frac, int* anc) {
  const std::vector<int> a = truncation_ancestors(std::vector<double>(E, E + n), frac);
  memcpy(anc, a.data(), (size_t)n * 4);
}

// path_cost of an ordering: out = {tc, sc}.
int tsh_path_cost(void* h, const int* order, int m, double* out) {
  const Network& I = *static_cast<Network*>(h);
  if (m != I.m) return -1;
  const auto r = path_cost(I, std::vector<int>(order, order + m));
  out[0] = r.first;
  out[1] = r.second;
  return 0;
}

// Up to k spectral orderings: orders (k * m ints), tc[k], sc[k]; returns how many were written.
int tsh_spectral_orders(void* h, int k, int nangles, int nrandom, uint64_t seed, int* orders, double* tc, int* sc) {
  const Network& I = *static_cast<Network*>(h);
  const auto so = spectral_orders(I, k, nangles, nrandom, seed);
  for (size_t i = 0; i < so.size(); i++) {
    memcpy(orders + i * (size_t)I.m, so[i].order.data(), (size_t)I.m * 4);
    tc[i] = so[i].tc;
    sc[i] = so[i].sc;
  }
  return (int)so.size();
}

// spectral_search over caller-given eigenvectors (m x d) and random directions (ndirs x d); as above.
int tsh_spectral_search(void* h, const double* V, int d, const double* dirs, int ndirs, int k, int nangles,
                        int* orders, double* tc, int* sc) {
  const Network& I = *static_cast<Network*>(h);
  const auto so = spectral_search(I, std::vector<double>(V, V + (size_t)I.m * d), d,
                                  std::vector<double>(dirs, dirs + (size_t)ndirs * d), k, nangles);
  for (size_t i = 0; i < so.size(); i++) {
    memcpy(orders + i * (size_t)I.m, so[i].order.data(), (size_t)I.m * 4);
    tc[i] = so[i].tc;
    sc[i] = so[i].sc;
  }
  return (int)so.size();
}

// Laplacian eigenvectors 1..k (m * k doubles, row-major) and eigenvalues (k); returns the k computed.
int tsh_laplacian_vectors(void* h, int k, uint64_t seed, double* vecs, double* vals) {
  const Network& I = *static_cast<Network*>(h);
  std::vector<double> ev;
  const auto V = laplacian_vectors(I, k, seed, &ev);
  const int kk = (int)ev.size();
  memcpy(vecs, V.data(), V.size() * 8);
  memcpy(vals, ev.data(), (size_t)kk * 8);
  return kk;
}

// Greedy tree into out (m - 1 children words); tc receives its tc.
int tsh_greedy_tree(void* h, int nrepeat, uint64_t seed, uint32_t* out, double* tc) {
  const Network& I = *static_cast<Network*>(h);
  const auto ch = greedy_tree(I, nrepeat, seed, tc);
  memcpy(out, ch.data(), ch.size() * 4);
  return 0;
}

}  // extern "C"
