// tsa_kernels.h -- kernel parameter block and launch entry points shared by tsa_kernels.hip and
// tsa_capi.hip (host side of the library).
#pragma once
#include <stdint.h>
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include "tsa_arith.h"
#include "tsa_select.h"

// Everything a kernel reads besides pointers, passed by value.
struct TsaKParams {
  int m, nint, W;              // leaves, internal nodes, 64-bit words per label set
  int ch_off, s_off, chain_words;
  int leaf_sc;
  int slicing, slice_moves, slice_every, max_slices;
  int par_follow, par_band;
  int helpers;                 // pre-order, one chain per workgroup: waves after the first draw the next sweep's
                               // Philox words and Metropolis thresholds while the first sweeps (0: none)
  int chain0;                  // k_sweep: the launch sweeps chains chain0 .. nchains - 1 (its grid covers those)
  uint32_t key0, key1;
  TsaModel model;
  float lse[64];               // lse[d] = (float)log2(1 + 2^-d), 0 for d >= 53
  // k_sweep with the chain staged in LDS: when ganc is set, chain c starts from the record of chain ganc[c] in
  // gsrc (a resampled population, read from the previous population's buffer; the launch's rec is the other
  // buffer, which receives the swept records)
  const uint64_t* gsrc;
  const int* ganc;
};

// Statistic slots (the reference's d_stats order, csrc/treesa_gpu.cu:713-721).
enum { TSA_ST_PROP = 0, TSA_ST_ACC, TSA_ST_STEPS, TSA_ST_VISITS, TSA_ST_SPROP, TSA_ST_SACC, TSA_ST_BUSY, TSA_NSTAT };
// Two more counters of the wide kernel with chunk summaries: chunk positions loaded by proposals and
// written by accepts.
enum { TSA_ST_CHUNKS = TSA_NSTAT, TSA_ST_XCHUNKS, TSA_NSTAT_ALL };
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
  int draw_waves;    // 1: pre-order sweeps run one chain per workgroup with helper waves that draw ahead
  int lds_max;       // dynamic LDS bytes a workgroup may have, less the kernel's static LDS
};

// Helper waves per workgroup of a pre-order sweep with draws made ahead (the workgroup fills a compute unit's
// four SIMDs), and the LDS words they add: two buffers (this sweep's and the next) of one Philox word and one
// threshold per internal node.
#define TSA_DRAW_HELPERS 3
static inline int tsa_draw_words(int nint) { return 2 * ((nint + 3) & ~3); }

// Per-chain energies a sweep launch also writes (lc == nullptr: none): the chain is evaluated by the sweep
// kernel right after its last sweep, while it is still staged, exactly as the energy kernel would.
// What a sweep launch leaves of its chains' energies: lc / sc / ns per chain (the sweep kernel folds them),
// or, with cost set, only every node's cost and masked size (cost / z + chain * nint4; k_fold folds them);
// with ch set, also a copy of every chain's children words (ch + chain * nint): a snapshot of the trees those
// energies describe, which the selection reads while the next sweep rewrites the records.
// Several levels in one par sweep launch (n > 0; not the level loop): level i has niters[i] sweeps at beta[i]
// (total sweeps in all), and after its last sweep every chain leaves its node costs, masked sizes and children
// words in cost[i] / z[i] / ch[i] (+ chain * nint4, nint4, nint; the snapshot slot that the level's fold and
// selection read; null: the level is not evaluated).  The chain stays staged from its first level to its last.
#define TSA_BLOCK_MAX 8
struct TsaBlock {
  int n, total;
  float beta[TSA_BLOCK_MAX];
  int niters[TSA_BLOCK_MAX];
  float* cost[TSA_BLOCK_MAX];
  uint16_t* z[TSA_BLOCK_MAX];
  uint32_t* ch[TSA_BLOCK_MAX];
};

struct TsaEnergyOut {
  float* lc;
  int* sc;
  int* ns;
  float* cost;
  uint16_t* z;
  uint32_t* ch;
  TsaBlock blk;  // (blk.n == 0: the launch is one level of nsweeps sweeps at beta)
};

struct TsaTrackPart;
struct TsaTraceRowD;
struct TsaTrackState;

// The level loop of independent chains run by one sweep launch (nlev > 0; nlev == 0: the launch's single
// beta and nsweeps).  Level l sweeps niters[l] >= 1 times at beta[l], the sweep counter running on across
// levels from sweep0.  After an evaluated level (eval[l] = e >= 0, its index among the launch's evaluated
// levels) every chain folds its energy into en_* [e * nchains + c], writes its tree (the record's words
// [ch_off, s_off + W)) into one of its two candidate slots (cand + (slot * nchains + c) * cand_words) and
// keeps that slot when its score beats the best it has had (own / bslot, per chain, read at the start of
// the launch and written at its end).  The last of a group of 256 chains to arrive reduces the group into
// part [e * ngroups + g], the last group the level, into trace[level0 + l], in the order k_track reduces.
// cnt: (ngroups + 1) arrival counters per evaluated level, zero before the launch and left zero after it.
struct TsaLevels {
  const float* beta;
  const int* niters;
  const int* eval;
  int nlev, total, level0;   // levels; sweeps over all of them; the trace row of level 0
  float* en_lc;
  int* en_sc;
  int* en_ns;
  unsigned* cnt;
  TsaTrackPart* part;
  uint64_t* cand;
  int cand_words;
  double* own;
  int* bslot;
  TsaTraceRowD* trace;
  TsaSelect S;
  int reset;  // 1: every chain starts with no best (own +inf, no slot) instead of reading own / bslot
  // a tracking session's start, made by chain 0's tracking wave before its first arrival (null: none): the
  // tracking state, the start tick, trace_words words of trace rows and best_words words of the best record
  // cleared
  TsaTrackState* tinit;
  unsigned long long* ticks0;
  int trace_words;
  uint64_t* best;
  int best_words;
};

// Copy n elements with nthr threads (this one is tid), U loads per thread in flight at once: a loop that
// stores each element before it loads the next waits a memory latency per element.
template <typename T, int U>
__device__ __forceinline__ void tsa_copy_inflight(T* dst, const T* __restrict__ src, int n, int tid, int nthr) {
  for (int i0 = tid; i0 < n; i0 += U * nthr) {
    T v[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int i = i0 + u * nthr;
      if (i < n) v[u] = src[i];
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int i = i0 + u * nthr;
      if (i < n) dst[i] = v[u];
    }
  }
}

// Host-side launchers (tsa_kernels.hip).  All return hipError_t of the launch.
hipError_t tsa_launch_sweeps(const TsaLaunch& L, int mode, int order, const TsaKParams& P, uint64_t* rec,
                             const uint64_t* leaf, const uint32_t* fix, int nchains, float beta, uint32_t sweep0,
                             int nsweeps, unsigned long long* stats, const TsaEnergyOut& eo, hipStream_t st,
                             hipEvent_t e0 = nullptr, hipEvent_t e1 = nullptr, const TsaLevels* lv = nullptr,
                             int* res = nullptr);
// With res set nothing is launched: *res = chains of the launch's kernel (the level loop's with lv set) that
// are resident on one compute unit at once.
// The same for the slicing kernel variants only (tsa_sweep_sliced.hip; tsa_launch_sweeps calls it when
// P.slicing is set).
hipError_t tsa_launch_sweeps_sliced(const TsaLaunch& L, int mode, int order, const TsaKParams& P, uint64_t* rec,
                                    const uint64_t* leaf, const uint32_t* fix, int nchains, float beta, uint32_t sweep0,
                                    int nsweeps, unsigned long long* stats, const TsaEnergyOut& eo, hipStream_t st,
                                    hipEvent_t e0, hipEvent_t e1, const TsaLevels* lv, int* res);
hipError_t tsa_launch_energy(int Wt, int mode, const TsaKParams& P, const uint64_t* rec, const uint64_t* leaf,
                             const uint32_t* fix, int nchains, float* lc, int* sc, int* ns, hipStream_t st);
// The fold of node costs a sweep launch left in cost / z (nchains * nint4 each) into lc / sc / ns.
hipError_t tsa_launch_fold(const TsaKParams& P, const uint64_t* rec, const uint64_t* leaf, const uint32_t* fix,
                           const float* cost, const uint16_t* z, int nchains, float* lc, int* sc, int* ns,
                           hipStream_t st);
// The same for several levels' snapshots in one launch, chains chain0 .. nchains - 1: level i folds cost[i] / z[i]
// into lc[i] / sc[i] / ns[i].
struct TsaFoldLevels {
  int n;
  const float* cost[TSA_BLOCK_MAX];
  const uint16_t* z[TSA_BLOCK_MAX];
  float* lc[TSA_BLOCK_MAX];
  int* sc[TSA_BLOCK_MAX];
  int* ns[TSA_BLOCK_MAX];
};
hipError_t tsa_launch_fold_levels(const TsaKParams& P, const uint64_t* rec, const uint64_t* leaf, const uint32_t* fix,
                                  const TsaFoldLevels& F, int chain0, int nchains, hipStream_t st);
struct TsaTrackState {
  double best_score;
  int best_chain, best_level;
  int snap;  // chain whose tree the last tracked level copied, -1 if none
};
struct TsaTraceRowD {  // same layout as tsa_trace_row_t
  float lc;
  int sc, ns, chain;
  double score, meanE, meanNs;
  unsigned long long ticks;
};
// Result of one selection workgroup (256 chains): best score and chain, sums of E and |S|.
struct TsaTrackPart {
  double score, sumE, sumNs;
  int idx;
};
// Levels of one selection launch, in level order: level i writes trace row lev[i] from the energies lc[i] /
// sc[i] / ns[i] of the trees whose children words are ch[i] (nint words per chain; null: the records' own).
struct TsaTrackLevels {
  int n;
  int lev[TSA_BLOCK_MAX];
  const float* lc[TSA_BLOCK_MAX];
  const int* sc[TSA_BLOCK_MAX];
  const int* ns[TSA_BLOCK_MAX];
  const uint32_t* ch[TSA_BLOCK_MAX];
};
// part: (L.n + 1) * ceil(nchains / 256) entries; done: L.n + 1 zeroed counters (left zero after every launch).
// When a level improves the best score, the chain's tree is copied into best_rec: its children words (from
// L.ch, when not null, else from rec) and its S words (from rec); label words are left as they are.  alone: the
// selection runs by itself between sweeps (workgroups of four waves that score a chain per lane at once) rather
// than beside a sweep (one wave per group, no LDS); the results are the same.
hipError_t tsa_launch_track_levels(const TsaTrackLevels& L, int nchains, const TsaSelect& S, const uint64_t* rec,
                                   int chain_words, int ch_off, int s_off, int W, int nint, TsaTrackState* st,
                                   TsaTraceRowD* trace, uint64_t* best_rec, TsaTrackPart* part, unsigned* done,
                                   hipStream_t stream, bool alone);
// One level: lc / sc / ns, trace row `level`, children words ch_snap.
hipError_t tsa_launch_track(const float* lc, const int* sc, const int* ns, int nchains, const TsaSelect& S, int level,
                            const uint64_t* rec, int chain_words, int ch_off, int s_off, int W, int nint,
                            const uint32_t* ch_snap, TsaTrackState* st, TsaTraceRowD* trace, uint64_t* best_rec,
                            TsaTrackPart* part, unsigned* done, hipStream_t stream, bool alone);
// After a level-loop launch (Lv: its levels, trace rows, candidate slots and the chains' own / bslot as the
// launch left them): the best over the launch's evaluated levels in level order (the lowest score, the first
// level on ties) against the session's best in st, which it replaces, and the best chain's kept tree (its
// slot's words: children words and S) into best_rec + ch_off.  One wave.  With O.h_st set it then writes the
// session's results as k_track_out does (the state, the start tick, the best tree and all O.row_words words of
// trace rows into mapped page-locked memory), so that the session's end needs no launch of its own.
struct TsaTrackOut {
  unsigned long long* h_st;  // null: no results written
  unsigned long long* h_t0;
  unsigned long long* h_tree;
  unsigned long long* h_rows;
  const unsigned long long* ticks0;
  int row_words;
};
hipError_t tsa_launch_level_best(const TsaLevels& Lv, int nchains, TsaTrackState* st, uint64_t* best_rec, int ch_off,
                                 const TsaTrackOut& O, hipStream_t stream);
hipError_t tsa_launch_track_init(TsaTrackState* st, unsigned long long* ticks0, unsigned long long* trace,
                                 int trace_words, unsigned long long* best, int best_words, hipStream_t stream);
// The set-up of a level-loop launch in one launch, each part optional: the level table copied from page-locked
// host memory (tab_src != nullptr: tab_words 32-bit words into tab_dst) and the arrival counters zeroed
// (cnt != nullptr: cnt_words 64-bit words).
struct TsaAnnealInit {
  const int* tab_src;
  int* tab_dst;
  int tab_words;
  unsigned long long* cnt;
  int cnt_words;
};
hipError_t tsa_launch_anneal_init(const TsaAnnealInit& A, hipStream_t stream);
// A tracking session's results into page-locked host memory in one launch (instead of one copy each): the
// tracking state (st_words 64-bit words), the start tick, the best record's tree (tree_words words from tree)
// and the trace rows (row_words words), and, when werr is not null, the wide path's error word.
hipError_t tsa_launch_track_out(const unsigned long long* st, int st_words, const unsigned long long* ticks0,
                                const unsigned long long* tree, int tree_words, const unsigned long long* rows,
                                int row_words, const unsigned* werr, unsigned long long* h_st,
                                unsigned long long* h_t0, unsigned long long* h_tree, unsigned long long* h_rows,
                                unsigned* h_werr, hipStream_t stream);
hipError_t tsa_launch_copy(const uint64_t* src, uint64_t* dst, const int* anc, int nchains, int chain_words,
                           hipStream_t st);
// n zeroed 64-bit words, by a kernel.
hipError_t tsa_launch_zero(unsigned long long* p, int n, hipStream_t st);
// out[k] = the sum of counter k's TSA_STAT_SLOTS slots, k < TSA_NSTAT.
hipError_t tsa_launch_sum_stats(const unsigned long long* slots, unsigned long long* out, hipStream_t st);

// ---------------------------------------------------------------------------------------------------
// Wide path (tsa_wide.hip): par-order sweeps and energies of runtime-width chains, label sets streamed
// from HBM in 16-byte chunks by groups of G lanes per proposal, node arrays in LDS, K workgroups per chain.
// ---------------------------------------------------------------------------------------------------
#define TSA_WIDE_CPL 2        // 16-byte chunks per lane and set with 16 or more lanes (so W <= 2 * 2 * 64 = 256)
// 16-byte chunks per lane of a set in the dense visit and the node-cost pass of G-lane groups: 4 up to 8 lanes,
// 2 from 16 (G * chunks never falls as G grows, so a group at least as wide as the plan's holds the set).  The
// visit's proposal-wide work (Philox, energy, Metropolis) is done once per group, so on an issue-bound kernel
// fewer, fuller lanes per proposal pay: C4's 24 chunks take 8 lanes of 3-4 chunks, not 16 of 1-2.
__host__ __device__ constexpr int tsa_wide_cpl(int G) { return G <= 8 ? 4 : TSA_WIDE_CPL; }
#define TSA_WIDE_MAX_K 16     // workgroups per chain
#define TSA_WIDE_SPIN (1u << 22)  // polls of a chain barrier before the launch gives up (seconds)
#define TSA_WIDE_JOIN (1u << 16)  // default polls of the check-in (milliseconds)

struct TsaWide {
  int on;     // 1: par-order sweeps of this context run k_wide
  int G;      // lanes per proposal (4..64)
  int K;      // workgroups per chain (K > 1: all co-resident, chain barriers between phases)
  int nt;     // threads per workgroup
  int smem;   // dynamic LDS bytes per workgroup
  int eG, eK; // energy: lanes per node, workgroups per chain
  int fold_stage;     // energy fold: 0 reads node costs from HBM, 1 stages them in LDS, 2 also the log2f bitmap
  int fold_smem;      // LDS bytes of stage 1 (0: the costs do not fit)
  int fold_smem_map;  // LDS bytes of stage 2
  int nsw;            // 64-bit words of a chunk summary per label set (0: no summaries; dense streaming)
  int lsum_lds;       // summaries: the input tensors' summaries are staged in LDS too
  int nxcd;           // XCDs of the device (hipDeviceAttributeNumberOfXccs): workgroups are dealt to them in turn
};

// Device state of the wide sweep kernel: the chain barrier words bar[nchains], done[nchains], join[nchains],
// err[1] (all zero between launches); outcome bytes of the visits of the last two phases, out[nchains][2][nint4]
// (K > 1 only); the per-node cost cache ncost / nz [nchains][nint4] (cost and masked size of every internal
// node), which the sweep kernel keeps current on every accepted rotation and the energy kernel folds.
// With chunk summaries (nsw > 0): sum[nchains][nint4][nsw] holds, for every internal node, bit c set iff
// 16-byte chunk c of its label set is nonzero (kept current by the sweep kernel), leafsum[m][nsw] the
// same for the input tensors.
struct TsaWideSync {
  unsigned* bar;
  unsigned* done;
  unsigned* join;  // K > 1: the chain's workgroups check in before they sweep it (see k_wide)
  unsigned* err;
  int nxcd;        // XCDs of the device
  int join_polls;  // polls of the check-in before a workgroup sweeps its chain alone; < 0: at once (tests)
  uint8_t* out;
  float* ncost;
  uint16_t* nz;
  uint64_t* sum;
  const uint64_t* leafsum;
  int nsw;
  int lsum_lds;  // 1: the sweep kernel stages leafsum in LDS (when it fits beside the node arrays)
  // Snapshot of every chain's tree and node-cost cache at the end of the launch (null: none), so that the
  // energy fold and the selection of this level can run beside the next level's sweep:
  // snap_ch[nchains][nint], snap_cost / snap_nz [nchains][nint4] (snap_cost null: the tree alone, for a launch
  // that folds the energies itself).
  uint32_t* snap_ch;
  float* snap_cost;
  uint16_t* snap_nz;
  // Energies of every chain folded by the sweep kernel itself at the end of the launch, from the node-cost
  // cache (null: none; dense plans with one workgroup per chain, and the cache exact when the launch starts):
  // flc / fsc / fns [nchains].
  float* flc;
  int* fsc;
  int* fns;
  // A block of blk_n > 0 levels in one launch (one workgroup per chain, chunk summaries): level i sweeps
  // blk_niters[i] times at blk_beta[i] (the launch's nsweeps is their sum) and, when blk_ch[i] is set, leaves
  // its snapshot (tree and node-cost cache, as snap_ch / snap_cost / snap_nz) there at its end.
  int blk_n;
  float blk_beta[TSA_BLOCK_MAX];
  int blk_niters[TSA_BLOCK_MAX];
  uint32_t* blk_ch[TSA_BLOCK_MAX];
  float* blk_cost[TSA_BLOCK_MAX];
  uint16_t* blk_nz[TSA_BLOCK_MAX];
};

// LDS byte offsets of k_wide (same function on host and device).
// With chunk summaries (nsw > 0) the summaries of the internal sets (sum) are staged too, and those of the
// input tensors (lsum) when mlds = m (0: read from HBM).
struct TsaWideLds {
  int masks, ch, dw, sum, lsum, pri, par, wl, out, bytes;
};
__host__ __device__ static inline TsaWideLds tsa_wide_lds(int nint, int band, int coop, int nsw, int mlds) {
  const int nint4 = (nint + 3) & ~3, ngrp = (nint + 63) / 64;
  TsaWideLds L;
  int b = 0;
  L.masks = b;  b += ngrp * 8;
  L.ch = b;     b += nint4 * 4;
  L.dw = b;     b += band ? nint4 * 4 : 0;
  L.sum = b;    b += nint4 * nsw * 8;
  L.lsum = b;   b += mlds * nsw * 8;
  L.pri = b;    b += nint4 * 2;
  L.par = b;    b += nint4 * 2;
  L.wl = b;     b += nint4 * 2;
  L.out = b;    b += coop ? 0 : nint4;
  L.bytes = (b + 15) & ~15;
  return L;
}

// Plan a wide launch for nchains chains on the current device: chunk summaries (sums: 1 on, -1 off, 0 on
// from 64 words per set), lanes per proposal (want_g, 0 = from W, or 8 with summaries), threads per
// workgroup (want_waves waves, 0 = by chain count), workgroups per chain (want_k, 0 = as many as stay
// co-resident).  Returns hipErrorInvalidValue when the chain does not qualify (W > 2 * TSA_WIDE_CPL * 64,
// a lane count that cannot hold a set, or LDS too small).
hipError_t tsa_wide_plan(const TsaKParams& P, int nchains, int want_waves, int want_k, int want_g, int sums,
                         TsaWide* out);
// Chunk summaries of every internal node of every chain from the label sets (after an upload or a
// population step).
hipError_t tsa_launch_wsum(const TsaWide& X, const TsaKParams& P, const uint64_t* rec, int nchains, uint64_t* sum,
                           hipStream_t st);
hipError_t tsa_launch_wide(const TsaWide& X, int mode, const TsaKParams& P, uint64_t* rec, const uint64_t* leaf,
                           const uint32_t* fix, int nchains, float beta, uint32_t sweep0, int nsweeps,
                           unsigned long long* stats, const TsaWideSync& sy, hipStream_t st,
                           hipEvent_t e0 = nullptr, hipEvent_t e1 = nullptr);
// Chunk summaries of the internal sets (isum[nchains][nint4][nsw]) and of the input tensors (lsum[m][nsw]) that
// match the population; nsw = 0: none.
struct TsaSums {
  const uint64_t* isum;
  const uint64_t* lsum;
  int nsw;
};
// Energies through per-node costs: ncost / nz hold nchains * nint4 node costs and masked sizes, fcnt
// nchains zeroed counters.  nodes = 1: recompute every node cost from the label sets first (with summaries:
// only the chunks in the union of a node's and its children's summaries, where all their nonzero chunks lie);
// nodes = 0: fold the cached costs only.
hipError_t tsa_launch_wide_energy(const TsaWide& X, int mode, const TsaKParams& P, const uint64_t* rec,
                                  const uint64_t* leaf, const uint32_t* fix, int nchains, float* ncost,
                                  uint16_t* nz, unsigned* fcnt, float* lc, int* sc, int* ns, int nodes,
                                  hipStream_t st, TsaSums sums = TsaSums{nullptr, nullptr, 0});
// The folds of F.n levels' cached costs (F.cost / F.z, nchains * nint4 each) into F.lc / F.sc / F.ns in one
// launch (blockIdx.y: the level), as tsa_launch_wide_energy with nodes = 0 does for one.
hipError_t tsa_launch_wide_fold_levels(const TsaWide& X, int mode, const TsaKParams& P, const uint64_t* rec,
                                       const uint64_t* leaf, const uint32_t* fix, int nchains,
                                       const TsaFoldLevels& F, hipStream_t st);
