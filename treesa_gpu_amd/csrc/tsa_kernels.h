// tsa_kernels.h -- kernel parameter block and launch entry points shared by tsa_kernels.hip and
// tsa_capi.hip (host side of the library).
#pragma once
#include <stdint.h>
#include <hip/hip_runtime.h>
#include "tsa_arith.h"

// Everything a kernel reads besides pointers, passed by value.
struct TsaKParams {
  int m, nint, W;              // leaves, internal nodes, 64-bit words per label set
  int ch_off, s_off, chain_words;
  int leaf_sc;
  int slicing, slice_moves, slice_every, max_slices;
  int par_follow, par_band;
  uint32_t key0, key1;
  TsaModel model;
  float lse[64];               // lse[d] = (float)log2(1 + 2^-d), 0 for d >= 53
};

// Statistic slots (the reference's d_stats order, csrc/treesa_gpu.cu:713-721).
enum { TSA_ST_PROP = 0, TSA_ST_ACC, TSA_ST_STEPS, TSA_ST_VISITS, TSA_ST_SPROP, TSA_ST_SACC, TSA_ST_BUSY, TSA_NSTAT };

// Words (64-bit) of per-wave LDS for the node arrays: pri, par, work list, uint16 per internal node.
static inline int tsa_node_words(int nint) { return (3 * ((nint + 3) & ~3) * 2 + 7) / 8; }

struct TsaLaunch {
  int W;             // template width: 1, 2, 4, 8, or 0 = runtime width
  int lds;           // 1: chain staged in LDS
  int wpb;           // waves (= chains) per workgroup
  int lds_words;     // LDS words per wave
};

// Host-side launchers (tsa_kernels.hip).  All return hipError_t of the launch.
hipError_t tsa_launch_sweeps(const TsaLaunch& L, int mode, int order, const TsaKParams& P, uint64_t* rec,
                             const uint64_t* leaf, const uint32_t* fix, int nchains, float beta, uint32_t sweep0,
                             int nsweeps, unsigned long long* stats, hipStream_t st);
hipError_t tsa_launch_energy(int Wt, int mode, const TsaKParams& P, const uint64_t* rec, const uint64_t* leaf,
                             const uint32_t* fix, int nchains, float* lc, int* sc, int* ns, hipStream_t st);
hipError_t tsa_launch_copy(const uint64_t* src, uint64_t* dst, const int* anc, int nchains, int chain_words,
                           hipStream_t st);
