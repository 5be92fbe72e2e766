// tsa_host.h -- host layer of the TreeSA drop-in binary: file formats, tree set-up and the double-precision
// checks, with no GPU dependency (compiled by g++ into libtreesa_host.so and into bin/treesa_gpu).
#pragma once
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace tsa {

// An input error with the message the reference prints (the binary exits 1 with it).
struct InputError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// Instance file: "m nlab", m lines "k l1 .. lk", then "ny y1 .. yny" (csrc/treesa_gpu.cu:1035-1073).
struct Inst {
  int m = 0, nlab = 0;
  std::vector<std::vector<int>> ixs;  // sorted per tensor
  std::vector<int> iy;
  std::vector<int> total;             // occurrences of each label over all tensors
  std::vector<char> in_iy;            // label is open
};

Inst read_instance(const std::string& path);
Inst make_instance(int m, int nlab, const std::vector<std::vector<int>>& ixs, const std::vector<int>& iy);

// K >= 1 trees of m-1 "left right" lines each (csrc/treesa_gpu.cu:1077-1097); children word l | r << 16.
std::vector<std::vector<uint32_t>> read_trees(const std::string& path, int m);

// "file:PATH", "a:step:b" (inclusive, a + i*step in double) or "b1,b2,.." (csrc/treesa_gpu.cu:1300-1328).
std::vector<float> parse_betas(const std::string& spec);

uint64_t splitmix64(uint64_t x);

// Julia random_exprtree: recursive random bipartition with mt19937_64(seed), internal ids in post-order
// from m, root 2m-2 (csrc/treesa_gpu.cu:1101-1123).
std::vector<uint32_t> random_tree(int m, uint64_t seed);

// Pre-order list of internal nodes; false unless ch is a binary tree over all 2m-1 nodes rooted at 2m-2
// (csrc/treesa_gpu.cu:1127-1145).
bool preorder(int m, const uint32_t* ch, std::vector<int>& order);

// Output labels of every internal node from the topology, W 64-bit words per set: l is an output of v
// iff it occurs in v's subtree and (occurs outside it, or is open) (csrc/treesa_gpu.cu:1149-1172).
bool labels_from_topology(const Inst& I, int W, const uint32_t* ch, uint64_t* lab);

// Energy-model constants as given on the command line (csrc/treesa_gpu.cu:1292-1295).
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

struct HostEnergy {
  double tc = 0;     // log2 sum_v 2^tc(v) (per slice)
  int sc = 0;        // largest tensor, leaves included (per slice)
  double time = 0;   // GPU roofline model, seconds (per slice)
  double time2 = 0;  // measured H100 model, seconds (per slice)
  int ns = 0;        // |S|
};

// Complexities of one chain on the sliced network in double (csrc/treesa_gpu.cu:1182-1244).
HostEnergy host_energy(const Inst& I, int W, const ModelLog2& P, const uint64_t* lab, const uint32_t* ch,
                       const std::vector<uint64_t>& leaf, const uint64_t* S);

// While sc > sc_target, slice the label that occurs most often among the largest masked tensors, lowest
// id on ties (csrc/treesa_gpu.cu:1248-1274).  Returns the number of labels added to S.
int greedy_repair(const Inst& I, int W, const uint64_t* lab, const std::vector<uint64_t>& leaf, uint64_t* S,
                  double sc_target);

// Leaf label sets in W-word format.
std::vector<uint64_t> leaf_sets(const Inst& I, int W);
int leaf_sc(const Inst& I);

// Record geometry (the C ABI layout, include/treesa_hip.h).
struct Geometry {
  int W, ch_off, s_off, chain_words;
};

// Initial population (csrc/treesa_gpu.cu:1585-1630): chain c from trees[c % K] (K = trees.size() > 0) or
// from random_tree(m, splitmix64(seed * 1000003 + c)); labels from the topology; S = S0 plus, when
// random_slices > 0, random_slices labels drawn with mt19937_64(splitmix64(seed * 7919 + c)).
// Throws InputError("invalid initial tree") when a tree is not valid.
void build_population(const Inst& I, const Geometry& G, const std::vector<std::vector<uint32_t>>& trees,
                      int nchains, uint64_t seed, const std::vector<uint64_t>& S0, int random_slices,
                      std::vector<uint64_t>& pop);

// ---- start trees (tsa_starts.cpp) ----

// Exact (tc, sc) in log2 of the path tree that contracts the tensors in `order` left to right, in
// O(sum of tensor sizes): step i contracts the prefix's surviving labels with tensor order[i], and for
// dimension-2 indices its cost is the size of the union of the two label sets (treesa_gpu/spectral.py:97-131).
std::pair<double, int> path_cost(const Inst& I, const std::vector<int>& order);

// Children words of that path tree: node m+0 = (order[0], order[1]), node m+i = (m+i-1, order[i+1]).
std::vector<uint32_t> path_tree(const std::vector<int>& order);

// Eigenvectors 1..k of the tensor graph's Laplacian (the lowest, constant one skipped), row-major m x k;
// evals (optional) receives their eigenvalues (treesa_gpu/spectral.py:20-92).
std::vector<double> laplacian_vectors(const Inst& I, int k, uint64_t seed, std::vector<double>* evals);

struct SpectralOrder {
  double tc;
  int sc;
  std::vector<int> order;
};
// The candidate search over given eigenvectors V (m x d, row-major) and random unit directions rdirs
// (consecutive d-vectors): orderings along nangles directions in the (v1, v2) plane and along rdirs, each
// also reversed, then a halving-step angle search around the three best, every candidate scored with
// path_cost; the k best distinct orderings, best first (treesa_gpu/spectral.py:141-199).
std::vector<SpectralOrder> spectral_search(const Inst& I, const std::vector<double>& V, int d,
                                           const std::vector<double>& rdirs, int k, int nangles);
// spectral_search over eigenvectors 1..3 of the tensor graph's Laplacian and nrandom seeded directions.
std::vector<SpectralOrder> spectral_orders(const Inst& I, int k, int nangles, int nrandom, uint64_t seed);

// Greedy contraction tree: the lowest-tc tree of nrepeat runs that repeatedly contract the pair of tensors
// sharing a label with the smallest result (ties by discovery order in run 0, at random in the others);
// tc (optional) receives its tc.  The reference takes greedy trees from omeco (treesa_gpu/driver.py:117-122).
std::vector<uint32_t> greedy_tree(const Inst& I, int nrepeat, uint64_t seed, double* tc);

}  // namespace tsa
