// tsa_host.h -- host layer of the TreeSA drop-in: the reference binary's file formats, the trees and label
// sets a population starts from, and the double-precision checks of a result.  No GPU dependency: it is
// compiled by g++ into libtreesa_host.so (tests) and into bin/treesa_gpu.
//
// Label sets are bitsets of 64-bit words, bit l % 64 of word l / 64 for label l.  Trees are children words,
// one uint32 per internal node i (node id m + i): left | right << 16, leaves 0..m-1, root 2m-2.
#pragma once
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace tsa {

// An input error; the binary prints its message and exits 1.
struct InputError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// A tensor network whose indices all have dimension 2.
struct Network {
  int m = 0;                               // input tensors
  int nlab = 0;                            // labels 0..nlab-1
  std::vector<std::vector<int>> tensors;   // labels of each tensor, ascending, no repeats
  std::vector<int> outputs;                // open labels (the network's output), as given
  std::vector<char> is_open;               // per label: 1 if open
  std::vector<std::vector<int>> holders;   // per label: the tensors holding it, ascending
  int occurrences(int l) const { return (int)holders[l].size(); }
  int largest_tensor() const;              // log2 size of the largest input tensor
};

// A network from label lists (sorted here; repeats and out-of-range labels are input errors with the
// reference's messages, csrc/treesa_gpu.cu:1058-1068).
Network make_network(int m, int nlab, std::vector<std::vector<int>> tensors, const std::vector<int>& outputs);

// Instance file: "m nlab", then m tensors "k l1 .. lk", then optionally "ny y1 .. yny"; whitespace-separated
// integers (csrc/treesa_gpu.cu:1035-1073).
Network read_network(const std::string& path);

// Tree file: K >= 1 trees of m-1 "left right" pairs each, one after the other; chain c starts from tree c % K
// (csrc/treesa_gpu.cu:1075-1097).
std::vector<std::vector<uint32_t>> read_tree_file(const std::string& path, int m);

// Inverse temperatures: "file:PATH" (whitespace-separated numbers), "a:step:b" (the Julia range a + i*step for
// i = 0 .. floor((b - a)/step + 1e-9), computed in double) or a list "b1,b2,..", each stored as float
// (csrc/treesa_gpu.cu:1300-1328).
std::vector<float> parse_schedule(const std::string& spec);

// The splitmix64 finalizer (Vigna); seeds every host-side random stream and the Philox key.
constexpr uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// Julia's random_exprtree: the tensors are split recursively by one random bit each (mt19937_64 seeded with
// seed; a split that leaves a side empty flips the bit of one random member), left part first; internal
// nodes get ids from m in post-order, so the root is 2m-2 (csrc/treesa_gpu.cu:1101-1123).
std::vector<uint32_t> random_tree(int m, uint64_t seed);

// Structure of one tree: parent links, Euler-tour intervals [tin, tout] (u is in v's subtree iff
// tin[v] <= tin[u] <= tout[v]) and a pre-order list of the internal nodes.  ok is false unless the
// children words form a binary tree over all 2m-1 nodes rooted at 2m-2 (every node reached exactly once;
// the reference's check, csrc/treesa_gpu.cu:1127-1145).
struct TreeShape {
  bool ok = false;
  std::vector<int> parent;     // -1 for the root
  std::vector<int> tin, tout;  // Euler-tour entry / last-descendant indices
  std::vector<int> internal_preorder;
};
TreeShape tree_shape(int m, const uint32_t* ch);

// Output-label sets of every internal node from the topology (W words per node, lab[(v-m)*W ..]): label l is
// an output of v iff v's subtree holds some of l's tensors but not all of them, or holds one and l is open
// (csrc/treesa_gpu.cu:1149-1172).  Returns false for an invalid tree.
bool topology_labels(const Network& N, int W, const uint32_t* ch, uint64_t* lab);

// Energy-model constants as given on the command line (defaults: csrc/treesa_gpu.cu:1292-1295).
struct ModelConsts {
  double gm[6] = {11.9e15, 1.6e13, 6, 6, 8, 4e-6};
  double h100[9] = {4e-6, 1.23e13, 5.44e-14, 7.68e-15, 6.37e-14, 2.02e-16, 1.77e-13, 14, 1e-12};
};

// The float log2 constants the kernels use (csrc/treesa_gpu.cu:1460-1474).
struct ModelLog2 {
  float lpeak, lbw, llaunch;
  int m0, n0, k0;
  float v2_l3launch, v2_lperm2, v2_lcc_bit, v2_lcc_cell, v2_ltc_bit, v2_ltc_pad, v2_ltc_out, v2_lsmall_cell;
  int v2_small_rank;
};
ModelLog2 model_log2(const ModelConsts& C);

// Complexities of one tree on its sliced network (label sets masked by ~S), in double.
struct HostEnergy {
  double tc = 0;     // log2 of the summed contraction costs (per slice)
  int sc = 0;        // log2 size of the largest tensor, inputs included (per slice)
  double time = 0;   // GPU roofline model, seconds (per slice)
  double time2 = 0;  // measured H100 model, seconds (per slice)
  int ns = 0;        // |S|
};
// lab: internal sets (nint * W words), leaf: input sets (m * W), S: the slice set or null
// (csrc/treesa_gpu.cu:1182-1244).
HostEnergy host_energy(const Network& N, int W, const ModelLog2& P, const uint64_t* lab, const uint32_t* ch,
                       const std::vector<uint64_t>& leaf, const uint64_t* S);

// Final slice repair: while the largest masked tensor (inputs and internal) exceeds sc_target, add to S the
// label held by the most of the largest tensors, the lowest id on ties (Julia's TreeSASlicer rule,
// csrc/treesa_gpu.cu:1248-1274).  Returns the number of labels added.
int greedy_repair(const Network& N, int W, const uint64_t* lab, const std::vector<uint64_t>& leaf, uint64_t* S,
                  double sc_target);

// Input label sets, W words per tensor.
std::vector<uint64_t> leaf_sets(const Network& N, int W);

// Record geometry (the C ABI's layout, include/treesa_hip.h).
struct Geometry {
  int W, ch_off, s_off, chain_words;
};

// Initial population (csrc/treesa_gpu.cu:1585-1630): chain c from trees[c % K] when K = trees.size() > 0,
// else from random_tree(m, splitmix64(seed * 1000003 + c)); label sets from the topology; S = S0, plus
// random_slices labels drawn with mt19937_64(splitmix64(seed * 7919 + c)) % nlab when random_slices > 0.
// Throws InputError("invalid initial tree") when a tree is not valid.
void build_population(const Network& N, const Geometry& G, const std::vector<std::vector<uint32_t>>& trees,
                      int nchains, uint64_t seed, const std::vector<uint64_t>& S0, int random_slices,
                      std::vector<uint64_t>& pop);

// ---- level-loop arithmetic (tsa_population.cpp) ----

// Scoring of a chain's energies (lc = log2 per-slice cost, sc, ns = |S|) at an evaluated level.
struct Scoring {
  int mode = 0;          // 0 tc, 1 gpu, 2 h100
  bool slicing = false;
  bool select_sc = false;
  double sc_target = 20.0, sc_weight = 1.0;
};
// Population energy |S| + lc + sc_weight * max(0, sc - sc_target) (csrc/treesa_gpu.cu:1751-1753).
double population_energy(const Scoring& S, float lc, int sc, int ns);
// Selection score, lower is better, in double with the host libm (csrc/treesa_gpu.cu:1737-1748): with
// slicing, feasibility (sc <= sc_target) first and then |S| + lc; with select_sc, the sc excess first and
// then lc; tc mode: log2(2^lc + sc_weight (2^sc - 2^sc_target)) when sc exceeds the target; the float modes:
// the population energy.
double selection_score(const Scoring& S, float lc, int sc, int ns);

// Systematic resampling of population annealing (csrc/treesa_gpu.cu:1837-1856): weights
// exp(-db (E - min E)) scaled to sum nc, pointers j + u for j = 0..nc-1 with one uniform u in [0, 1); chain j
// takes the ancestor whose cumulative weight interval holds pointer j.
std::vector<int> systematic_ancestors(const std::vector<double>& E, double db, double u);
// Truncation selection (csrc/treesa_gpu.cu:1857-1869): chains ranked by E (std::sort, ties as libstdc++'s
// introsort leaves them); the k-th worst is replaced by the k-th best for k < (int)(frac * nc).
std::vector<int> truncation_ancestors(const std::vector<double>& E, double frac);

// ---- start trees (tsa_starts.cpp) ----

// Exact (tc, sc) in log2 of the path tree that contracts the tensors in `order` left to right, in
// O(sum of tensor sizes): step i contracts the prefix's surviving labels with tensor order[i], and for
// dimension-2 indices its cost is the size of the union of the two label sets (treesa_gpu/spectral.py:97-131).
std::pair<double, int> path_cost(const Network& N, const std::vector<int>& order);

// Children words of that path tree: node m+0 = (order[0], order[1]), node m+i = (m+i-1, order[i+1]).
std::vector<uint32_t> path_tree(const std::vector<int>& order);

// Eigenvectors 1..k of the tensor graph's Laplacian (the lowest, constant one skipped), row-major m x k;
// evals (optional) receives their eigenvalues (treesa_gpu/spectral.py:20-92).
std::vector<double> laplacian_vectors(const Network& N, int k, uint64_t seed, std::vector<double>* evals);

struct SpectralOrder {
  double tc;
  int sc;
  std::vector<int> order;
};
// The candidate search over given eigenvectors V (m x d, row-major) and random unit directions rdirs
// (consecutive d-vectors): orderings along nangles directions in the (v1, v2) plane and along rdirs, each
// also reversed, then a halving-step angle search around the three best, every candidate scored with
// path_cost; the k best distinct orderings, best first (treesa_gpu/spectral.py:141-199).
std::vector<SpectralOrder> spectral_search(const Network& N, const std::vector<double>& V, int d,
                                           const std::vector<double>& rdirs, int k, int nangles);
// spectral_search over eigenvectors 1..3 of the tensor graph's Laplacian and nrandom seeded directions.
std::vector<SpectralOrder> spectral_orders(const Network& N, int k, int nangles, int nrandom, uint64_t seed);

// Greedy contraction tree: the lowest-tc tree of nrepeat runs that repeatedly contract the pair of tensors
// sharing a label with the smallest result (ties by discovery order in run 0, at random in the others);
// tc (optional) receives its tc.  The reference takes greedy trees from omeco (treesa_gpu/driver.py:117-122).
std::vector<uint32_t> greedy_tree(const Network& N, int nrepeat, uint64_t seed, double* tc);

}  // namespace tsa
