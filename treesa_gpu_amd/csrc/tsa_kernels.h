// tsa_kernels.h -- kernel parameter block and launch entry points shared by tsa_kernels.hip and
// tsa_capi.hip (host side of the library).
#pragma once
#include <stdint.h>
#include <hip/hip_runtime.h>
#include "tsa_arith.h"
#include "tsa_select.h"

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
// Each counter is spread over TSA_STAT_SLOTS device words (slot = chain % TSA_STAT_SLOTS) so that thousands
// of waves do not serialize their atomics on one address; the host sums the slots.
#define TSA_STAT_SLOTS 64

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
struct TsaTrackState {
  double best_score;
  int best_chain, best_level;
};
struct TsaTraceRowD {  // same layout as tsa_trace_row_t
  float lc;
  int sc, ns, chain;
  double score, meanE, meanNs;
  unsigned long long ticks;
};
hipError_t tsa_launch_track(const float* lc, const int* sc, const int* ns, int nchains, const TsaSelect& S, int level,
                            const uint64_t* rec, int chain_words, TsaTrackState* st, TsaTraceRowD* trace,
                            uint64_t* best_rec, hipStream_t stream);
hipError_t tsa_launch_track_init(TsaTrackState* st, unsigned long long* ticks0, hipStream_t stream);
hipError_t tsa_launch_copy(const uint64_t* src, uint64_t* dst, const int* anc, int nchains, int chain_words,
                           hipStream_t st);
