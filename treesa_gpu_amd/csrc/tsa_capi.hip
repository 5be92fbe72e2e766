// tsa_capi.hip -- host side of libtreesa_hip.so: the C ABI declared in include/treesa_hip.h.
//
// Owns device memory and one HIP stream per context, validates everything a kernel will index with
// before it reaches the GPU (tree structure of uploaded chains, ancestor indices), and prepares the
// host-built tables the kernels read: the lse table (csrc/treesa_gpu.cu:2075) and the log2f correction
// table of tsa_math.h, which is filled by comparing the restated log2f with this process's libm.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "treesa_hip.h"
#include "tsa_kernels.h"

// Snapshot slots of the overlapped selection: an evaluated level's sweep takes the slot that the selection of
// nslots - 1 levels back read, so the host may enqueue that many levels ahead of the device.  Three slots for
// one level per launch, three per level of a block of levels (tsa_anneal), at most TSA_SNAP_MAX.
#define TSA_SNAP_MAX (3 * TSA_BLOCK_MAX)

struct tsa_ctx {
  tsa_layout_t lay;
  tsa_config_t cfg;
  TsaKParams P;
  int mode = 0;
  int nchains = 0;
  int Wt = 0;  // kernel template width (0 = runtime width)
  TsaLaunch L{};
  std::string kname;
  hipStream_t st = nullptr;
  std::vector<hipEvent_t> ev;  // start / stop event pairs of the sweep launches since the last tsa_sweeps_ms
  int npending = 0;            // pairs in use
  TsaSelect sel{};
  int track_levels = 0;
  TsaTrackState* d_track = nullptr;
  TsaTraceRowD* d_trace = nullptr;
  uint64_t* d_best = nullptr;
  unsigned long long* d_ticks0 = nullptr;
  uint64_t* d_rec = nullptr;
  uint64_t* d_rec2 = nullptr;
  uint64_t* d_leaf = nullptr;
  uint32_t* d_fix = nullptr;
  unsigned long long* d_stats = nullptr;
  float* d_lc = nullptr;  // d_lc, d_sc, d_ns: one allocation of 3 * nchains words, copied back at once
  int* d_sc = nullptr;
  int* d_ns = nullptr;
  uint32_t* h_en = nullptr;  // pinned host copy of the three energy arrays
  // pinned staging of tsa_track_end's copies (tracking state, start tick, best tree, trace rows): page-locked
  // copies are enqueued without a wait each, and the call waits once
  char* h_tend = nullptr;
  size_t h_tend_bytes = 0;
  char* d_tend = nullptr;  // the device's address of h_tend (null: not mapped, the results go by copies)
  // tsa_track_begin leaves the session's start (k_track_init) to the next call, which enqueues it before
  // anything else (the same place in the stream's order), or to the level loop's set-up launch, which does it
  bool track_init_pending = false;
  // the last level-loop launch's k_level_best wrote the session's results into h_tend (tsa_track_end then
  // only waits)
  bool tend_staged = false;
  double tick_hz = 0.0;  // the device's wall-clock rate (Hz)
  uint32_t* d_hen = nullptr;  // the device's address of h_en (null: not mapped)
  bool energy_host = false;   // the last sweep launch wrote the energies of the current population into h_en
  int* d_anc = nullptr;
  int* h_anc = nullptr;            // pinned staging of the ancestor list
  int* d_hanc = nullptr;           // the device's address of h_anc (null: not mapped, the list goes by a copy)
  hipEvent_t ev_anc = nullptr;     // recorded after the launch that read h_anc last
  bool anc_pending = false;
  // tsa_resample's copy of the ancestors' records not made yet: the next sweep launch of the LDS kernels reads
  // each chain's record from its ancestor's in d_rec and writes the population into d_rec2 (then the two swap);
  // any other call makes the copy first (flush_resample)
  bool anc_pend = false;
  TsaWide wide{};              // wide path plan (wide.on: par sweeps and energies run tsa_wide.hip)
  TsaWideSync wsync{};         // chain barrier words (one allocation) and visit outcomes
  unsigned* d_wsync = nullptr;
  float* d_ncost = nullptr;    // per-node costs of the wide energy kernel, nchains * nint4
  uint16_t* d_nz = nullptr;    // per-node masked sizes, nchains * nint4
  unsigned* d_fcnt = nullptr;  // per-chain workgroup counters of the wide energy kernel
  int ncu = 0;                 // compute units of the device
  uint64_t* d_sum = nullptr;   // chunk summaries of the internal sets, nchains * nint4 * wide.nsw
  uint64_t* d_leafsum = nullptr;  // chunk summaries of the input tensors, m * wide.nsw
  bool sums_valid = false;     // d_sum matches the population (k_wsum since the last upload or resample,
                               // and every sweep since ran the wide kernel)
  bool costs_valid = false;    // d_ncost / d_nz hold every node's cost (full pass since the last upload,
                               // resample or mode switch, and every sweep since ran the wide kernel)
  bool energy_fresh = false;   // d_lc / d_sc / d_ns hold the energies of the current population (written by
                               // the last sweep launch, cfg.fused_energy)
  bool fold_apart = false;     // cfg.fused_energy on the one-wave kernels with more than twice the chains that
                               // fit on the device at once (or fused_energy 2): the sweep kernel leaves node
                               // costs in d_ncost / d_nz and k_fold folds every chain in one round
  TsaTrackPart* d_tpart = nullptr;  // selection kernel: per-workgroup results and its counter
  unsigned* d_tdone = nullptr;
  // Overlapped tracking (the wide path, and the one-wave kernels with fused energies): each sweep launch
  // leaves a snapshot of every chain's tree and node costs (or energies) in slot `slot` (nslots slots in
  // turn), and tsa_track runs the fold and the selection of that snapshot on the second stream st2
  // while st goes on with the next level's sweep.  ev_sweep[s] marks the sweep that filled slot s,
  // ev_track[s] the selection that read it (the host waits for it before a sweep overwrites the slot).
  bool overlap = false;
  hipStream_t st2 = nullptr;
  // Split sweeps (the one-wave kernels with the overlapped selection and the fold apart, where the population
  // is more than twice what the device holds at once): a level's chains are swept by two launches, the first
  // part on st and the rest on st3, so that each stream's dependent dispatch and the tail of its launch are
  // covered by the other stream's work.  st3's launch waits for what st held before the level's first launch
  // (ev_fork); every other operation first orders st after st3 (join_split).  ev_b[s] follows the second
  // launch of the sweep that filled slot s, when split_slot[s].
  hipStream_t st3 = nullptr;
  hipEvent_t ev_fork = nullptr, ev_join = nullptr;
  hipEvent_t ev_b[TSA_SNAP_MAX] = {};
  bool split_slot[TSA_SNAP_MAX] = {};
  bool split_pending = false;  // st3 holds work st is not yet ordered after
  // st holds work other than the first launches of split levels that st3 is not yet ordered after (every call
  // but tsa_sweeps' split launches and the overlapped tsa_track goes through join_split, which sets it): only
  // then does the next split level's second launch wait for st (ev_fork); otherwise it follows only st3's own
  // previous launch, so that the two halves of the population run their levels independently (the snapshot
  // slots keep them within a few levels of each other)
  bool fork_needed = true;
  long long split_levels = 0;  // sweep calls run as two launches (reported by tsa_describe)
  hipEvent_t ev_sweep[TSA_SNAP_MAX] = {};  // (the stop events of those sweeps' timing pairs)
  hipEvent_t ev_track[TSA_SNAP_MAX] = {};
  // the slot whose ev_track covers slot s (the slots of one block of levels share the event recorded after
  // their one selection launch: every event recorded on a busy stream is a packet the device processes, about
  // 5 us each)
  int track_ev[TSA_SNAP_MAX] = {};
  int last_track = -1;  // the slot whose ev_track was recorded last (st2 runs the selections in order)
  // the session's start was enqueued on st2 (behind the first sweeps) and st has not yet waited for it
  hipEvent_t ev_tinit = nullptr;
  bool tinit_pending = false;
  bool track_pending[TSA_SNAP_MAX] = {};
  int slot = 0, last_slot = -1;  // slot of the next sweep launch / of the last one (-1: none since a reset)
  int nslots = 0;                // slots allocated (their buffers), the ones in turn
  uint32_t* d_snap_ch[TSA_SNAP_MAX] = {};
  float* d_snap_cost[TSA_SNAP_MAX] = {};
  uint16_t* d_snap_nz[TSA_SNAP_MAX] = {};
  uint32_t* d_snap_en[TSA_SNAP_MAX] = {};  // energies folded by the sweep kernel: lc, sc, ns per chain
  int snap_kind[TSA_SNAP_MAX] = {};  // what the sweep that filled a slot left there: a SNAP_* value
  // The level loop on the device (tsa_anneal, TsaLevels): the tracking session's kind (0: nothing tracked
  // yet, TRACK_LEVELS: tsa_track, TRACK_ANNEAL: tsa_anneal), whether the per-chain best still has to be
  // reset, the levels evaluated so far in the session, and the buffers, grown on demand.
  // The host waited for the stream since the last sweep launch (tsa_energy, tsa_download, tsa_wait): the device
  // idles until the next launch, so that launch records its timing events as stream markers around a plain
  // dispatch (about 6 us of host time) rather than in the dispatch itself (about 20 us).
  bool host_waited = false;
  int track_kind = 0;
  bool lv_reset = false;
  int lv_resident[6] = {-1, -1, -1, -1, -1, -1};  // level-loop chains resident per compute unit, per mode and order
  int blocks_k = 0;   // levels per launch of tsa_anneal's last block path (reported by tsa_describe)
  int lv_used = -1;                               // whether the last tsa_anneal ran the level loop (-1: none yet)
  std::vector<char> lv_evaluated;
  int lv_cap_levels = 0, lv_cap_evals = 0;
  bool lv_cnt_fresh = false;  // the arrival counters were (re)allocated and are not yet cleared
  int* d_lv = nullptr;               // per level: beta (as bits), sweeps, evaluated index (-1: not evaluated)
  // pinned staging of d_lv in two halves of lv_cap_levels * 3 words, used in turn: the set-up launch reads
  // one while the host fills the other; ev_lv[h] is recorded after the launches that read half h
  int* h_lv = nullptr;
  int* d_hlv = nullptr;  // the device's address of h_lv (null: not mapped, the table goes by a copy)
  std::vector<int> lv_tab;  // the table d_lv holds (empty: unknown)
  hipEvent_t ev_lv[2] = {nullptr, nullptr};
  bool lv_pending[2] = {false, false};
  int lv_half = 0;
  uint32_t* d_lv_en = nullptr;       // lc | sc | ns per evaluated level and chain
  unsigned* d_lv_cnt = nullptr;      // arrival counters, (ngroups + 1) per evaluated level
  TsaTrackPart* d_lv_part = nullptr; // group results, ngroups per evaluated level
  uint64_t* d_cand = nullptr;        // two candidate trees per chain
  double* d_own = nullptr;           // per chain: best score and the slot of its tree
  int* d_bslot = nullptr;
  std::string err;
};

enum { TRACK_LEVELS = 1, TRACK_ANNEAL = 2 };

static thread_local std::string g_err;

// Contents of a snapshot slot: the wide kernel's node-cost cache, node costs of the one-wave kernel for the
// fold kernel, or energies the one-wave kernel folded itself (with children words in every case).
enum { SNAP_WIDE = 0, SNAP_COSTS = 1, SNAP_ENERGIES = 2 };

static int fail(tsa_ctx* ctx, int code, const std::string& msg) {
  if (ctx) ctx->err = msg;
  else g_err = msg;
  return code;
}

#define TSA_HIP(ctx, call)                                                                          \
  do {                                                                                             \
    hipError_t e_ = (call);                                                                        \
    if (e_ != hipSuccess)                                                                          \
      return fail((ctx), TSA_ERR_HIP, std::string(#call) + ": " + hipGetErrorString(e_));          \
  } while (0)

// ---------------------------------------------------------------------------------------------------
// Host-built tables
// ---------------------------------------------------------------------------------------------------
static std::once_flag g_fix_once;
static std::vector<uint32_t> g_fix;  // TSA_LOG2FIX_WORDS words, then TSA_LOG2MAP_WORDS words of summary bitmap
static long long g_fix_far = 0;      // inputs where the restated log2f is more than 1 ulp from libm

static void build_log2_fix() {
  g_fix.assign(TSA_LOG2FIX_WORDS, 0u);
  unsigned nt = std::thread::hardware_concurrency();
  nt = nt == 0 ? 4 : (nt > 16 ? 16 : nt);
  std::vector<std::thread> th;
  std::vector<long long> far(nt, 0);
  const uint32_t nw = TSA_LOG2FIX_WORDS;
  for (unsigned t = 0; t < nt; t++) {
    th.emplace_back([&, t]() {
      for (uint32_t w = t; w < nw; w += nt) {  // word w covers mantissas 16w .. 16w+15
        uint32_t word = 0;
        for (uint32_t j = 0; j < 16; j++) {
          const uint32_t mant = w * 16 + j;
          const float y = tsa_ffrom(0x3f800000u + mant);
          const int32_t d = (int32_t)(tsa_fbits(log2f(y)) - tsa_fbits(tsa_log2f_core(y)));
          uint32_t code = 0;
          if (d == 1) code = 1;
          else if (d == -1) code = 2;
          else if (d != 0) far[t]++;
          word |= code << (2 * j);
        }
        g_fix[w] = word;
      }
    });
  }
  for (auto& x : th) x.join();
  g_fix.resize(TSA_LOG2FIX_WORDS + TSA_LOG2MAP_WORDS, 0u);
  for (uint32_t w = 0; w < nw; w++)
    if (g_fix[w]) g_fix[nw + (w >> 5)] |= 1u << (w & 31u);
  for (long long f : far) g_fix_far += f;
  if (tsa_fbits(log2f(2.0f)) != tsa_fbits(1.0f)) g_fix_far++;  // tsa_log2f_12 returns 1 at 2
}

// Sampled comparison of the restated expf / exp2f with this process's libm (the exhaustive comparison
// is a test); any disagreement means the host libm is not the one the restatement was checked against.
static long long libm_selftest() {
  long long bad = 0;
  uint32_t s = 0x12345678u;
  for (int i = 0; i < (1 << 18); i++) {
    s = s * 1664525u + 1013904223u;
    const float x = tsa_ffrom(s);
    const float a = expf(x), b = tsa_expf(x), c = exp2f(x), d = tsa_exp2f(x);
    if (tsa_fbits(a) != tsa_fbits(b) && !(std::isnan(a) && std::isnan(b))) bad++;
    if (tsa_fbits(c) != tsa_fbits(d) && !(std::isnan(c) && std::isnan(d))) bad++;
  }
  // the Metropolis range: -beta*dE in [-20, 0] on a fine grid
  for (int i = 0; i < (1 << 18); i++) {
    const float x = -20.0f * (float)i / (float)(1 << 18);
    if (tsa_fbits(expf(x)) != tsa_fbits(tsa_expf(x))) bad++;
  }
  return bad;
}

static void build_lse(float* lse) {
  for (int d = 0; d < 64; d++) lse[d] = (float)std::log2(1.0 + std::exp2(-(double)d));
}

// ---------------------------------------------------------------------------------------------------
// Layout and validation
// ---------------------------------------------------------------------------------------------------
extern "C" int tsa_layout(int32_t m, int32_t nlab, int32_t wide, tsa_layout_t* out) {
  if (!out) return fail(nullptr, TSA_ERR_ARG, "tsa_layout: null output");
  if (m < 3) return fail(nullptr, TSA_ERR_ARG, "need at least 3 tensors");
  if (2 * m - 1 > 65535) return fail(nullptr, TSA_ERR_ARG, "too many tensors (node ids are 16-bit)");
  if (nlab < 1) return fail(nullptr, TSA_ERR_ARG, "need at least one label");
  tsa_layout_t L;
  memset(&L, 0, sizeof L);
  L.m = m;
  L.nint = m - 1;
  L.nlab = nlab;
  const int w64 = (nlab + 63) / 64;
  if (!wide && w64 <= 8) {
    L.W = w64 <= 1 ? 1 : w64 <= 2 ? 2 : w64 <= 4 ? 4 : 8;
    L.runtime_width = 0;
  } else {
    // an even number of words: every label set (and S) is a run of 16-byte chunks, 16-byte aligned
    L.W = (w64 + 1) & ~1;
    L.runtime_width = 1;
  }
  L.ch_off = L.nint * L.W;
  L.s_off = L.ch_off + (L.nint + 1) / 2;
  if (L.runtime_width) L.s_off = (L.s_off + 1) & ~1;
  L.chain_words = (L.s_off + L.W + 1) & ~1;
  *out = L;
  return TSA_OK;
}

// Every chain must be a binary tree over all 2m-1 nodes rooted at 2m-2 (ids < 2m-1, each node reached
// once); the kernels index label sets with these ids.  Reference check: csrc/treesa_gpu.cu:1127-1145.
static bool valid_tree(const uint32_t* ch, int m, std::vector<char>& seen, std::vector<int>& st) {
  const int n = 2 * m - 1;
  seen.assign(n, 0);
  st.clear();
  st.push_back(n - 1);
  int cnt = 0;
  while (!st.empty()) {
    const int v = st.back();
    st.pop_back();
    if (v < 0 || v >= n || seen[v]) return false;
    seen[v] = 1;
    cnt++;
    if (v >= m) {
      st.push_back((int)(ch[v - m] >> 16));
      st.push_back((int)(ch[v - m] & 0xFFFFu));
    }
  }
  return cnt == n;
}

// ---------------------------------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------------------------------
static void free_ctx(tsa_ctx* c) {
  if (!c) return;
  // every stream of the context drained before any of its buffers is released: the split sweep on st3 and the
  // fold and selection on st2 read and write the records, the snapshots and the counters
  for (hipStream_t s : {c->st, c->st3, c->st2})
    if (s) (void)hipStreamSynchronize(s);
  if (c->d_rec) (void)hipFree(c->d_rec);
  if (c->d_rec2) (void)hipFree(c->d_rec2);
  if (c->d_leaf) (void)hipFree(c->d_leaf);
  if (c->d_fix) (void)hipFree(c->d_fix);
  if (c->d_stats) (void)hipFree(c->d_stats);
  if (c->d_lc) (void)hipFree(c->d_lc);
  if (c->h_en) (void)hipHostFree(c->h_en);
  if (c->h_tend) (void)hipHostFree(c->h_tend);
  if (c->d_anc) (void)hipFree(c->d_anc);
  if (c->h_anc) (void)hipHostFree(c->h_anc);
  if (c->ev_anc) (void)hipEventDestroy(c->ev_anc);
  if (c->d_wsync) (void)hipFree(c->d_wsync);
  if (c->wsync.out) (void)hipFree(c->wsync.out);
  if (c->d_ncost) (void)hipFree(c->d_ncost);
  if (c->d_nz) (void)hipFree(c->d_nz);
  if (c->d_fcnt) (void)hipFree(c->d_fcnt);
  if (c->d_sum) (void)hipFree(c->d_sum);
  if (c->d_leafsum) (void)hipFree(c->d_leafsum);
  if (c->d_tpart) (void)hipFree(c->d_tpart);
  if (c->d_tdone) (void)hipFree(c->d_tdone);
  for (hipEvent_t e : c->ev) (void)hipEventDestroy(e);
  if (c->st3) {
    for (hipEvent_t e : {c->ev_fork, c->ev_join})
      if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : c->ev_b)
      if (e) (void)hipEventDestroy(e);
    (void)hipStreamDestroy(c->st3);
  }
  for (int k = 0; k < TSA_SNAP_MAX; k++) {
    if (c->ev_track[k]) (void)hipEventDestroy(c->ev_track[k]);
    if (c->d_snap_ch[k]) (void)hipFree(c->d_snap_ch[k]);
    if (c->d_snap_cost[k]) (void)hipFree(c->d_snap_cost[k]);
    if (c->d_snap_nz[k]) (void)hipFree(c->d_snap_nz[k]);
    if (c->d_snap_en[k]) (void)hipFree(c->d_snap_en[k]);
  }
  if (c->ev_tinit) (void)hipEventDestroy(c->ev_tinit);
  if (c->st2) (void)hipStreamDestroy(c->st2);
  if (c->d_track) (void)hipFree(c->d_track);
  if (c->d_trace) (void)hipFree(c->d_trace);
  if (c->d_best) (void)hipFree(c->d_best);
  if (c->d_ticks0) (void)hipFree(c->d_ticks0);
  if (c->d_lv) (void)hipFree(c->d_lv);
  if (c->h_lv) (void)hipHostFree(c->h_lv);
  for (hipEvent_t e : c->ev_lv)
    if (e) (void)hipEventDestroy(e);
  if (c->d_lv_en) (void)hipFree(c->d_lv_en);
  if (c->d_lv_cnt) (void)hipFree(c->d_lv_cnt);
  if (c->d_lv_part) (void)hipFree(c->d_lv_part);
  if (c->d_cand) (void)hipFree(c->d_cand);
  if (c->d_own) (void)hipFree(c->d_own);
  if (c->d_bslot) (void)hipFree(c->d_bslot);
  if (c->st) (void)hipStreamDestroy(c->st);
  delete c;
}

static void fill_params(const tsa_layout_t& lay, const tsa_config_t& C, int32_t leaf_sc, TsaKParams& P) {
  memset(&P, 0, sizeof P);
  P.m = lay.m;
  P.nint = lay.nint;
  P.W = lay.W;
  P.ch_off = lay.ch_off;
  P.s_off = lay.s_off;
  P.chain_words = lay.chain_words;
  P.leaf_sc = leaf_sc;
  P.slicing = C.slicing ? 1 : 0;
  P.slice_moves = C.slicing ? C.slice_moves : 0;
  P.slice_every = C.slice_every > 0 ? C.slice_every : 1;
  P.max_slices = C.max_slices > 0 ? C.max_slices : lay.nlab;
  P.par_follow = C.par_follow;
  P.par_band = C.par_band;
  P.key0 = C.key0;
  P.key1 = C.key1;
  TsaModel& M = P.model;
  M.sc_target = C.sc_target;
  M.sc_weight = C.sc_weight;
  M.lpeak = C.lpeak;
  M.lbw = C.lbw;
  M.llaunch = C.llaunch;
  M.m0 = C.m0;
  M.n0 = C.n0;
  M.k0 = C.k0;
  M.v2_l3launch = C.v2_l3launch;
  M.v2_lperm2 = C.v2_lperm2;
  M.v2_lcc_bit = C.v2_lcc_bit;
  M.v2_lcc_cell = C.v2_lcc_cell;
  M.v2_ltc_bit = C.v2_ltc_bit;
  M.v2_ltc_pad = C.v2_ltc_pad;
  M.v2_ltc_out = C.v2_ltc_out;
  M.v2_lsmall_cell = C.v2_lsmall_cell;
  M.v2_small_rank = C.v2_small_rank;
  build_lse(P.lse);
}

// Arguments every context-free entry shares with tsa_create: a layout from tsa_layout and a valid config.
static int check_layout_config(const tsa_layout_t* lay, const tsa_config_t* cfg, const char* who) {
  tsa_layout_t chk;
  if (tsa_layout(lay->m, lay->nlab, lay->runtime_width, &chk) != TSA_OK) return TSA_ERR_ARG;
  if (memcmp(&chk, lay, sizeof chk) != 0) return fail(nullptr, TSA_ERR_ARG, std::string(who) + ": layout not from tsa_layout");
  if (cfg->mode < 0 || cfg->mode > 2) return fail(nullptr, TSA_ERR_ARG, std::string(who) + ": mode must be 0, 1 or 2");
  if (cfg->par_band == 1 || cfg->par_band < 0 || cfg->par_band > 16)
    return fail(nullptr, TSA_ERR_ARG, "--par-band L: 0 (off) or 2..16");
  if (cfg->slicing && cfg->slice_moves < 0) return fail(nullptr, TSA_ERR_ARG, std::string(who) + ": slice_moves < 0");
  return TSA_OK;
}

// The host libm must be the one the restated expf / exp2f / log2f were checked against (the log2f correction
// table is built from it); built and checked once per process.
static int check_host_math() {
  std::call_once(g_fix_once, build_log2_fix);
  if (g_fix_far != 0)
    return fail(nullptr, TSA_ERR_LIBM, "host libm log2f is more than 1 ulp from the restated log2f on [1, 2]");
  static long long selftest = -1;
  static std::mutex mu;
  {
    std::lock_guard<std::mutex> g(mu);
    if (selftest < 0) selftest = libm_selftest();
  }
  if (selftest != 0) return fail(nullptr, TSA_ERR_LIBM, "host libm expf/exp2f differ from the restated algorithm");
  return TSA_OK;
}

// The one-wave-per-chain plan: the chain and the leaf table staged in LDS when they fit and the width is a
// register width (or kernel forces it), else the record in HBM with only the node arrays in LDS; up to four
// chains per workgroup, fewer when there are fewer chains than full workgroups on every compute unit (then
// they spread over all units and share each unit's LDS, scalar unit and issue with fewer others).
static int plan_one_wave(const tsa_layout_t* lay, const tsa_config_t* cfg, int nchains, int lds_max, int ncu,
                         TsaLaunch* L, bool* use_lds_out) {
  const int nodew = tsa_node_words(lay->nint) + (cfg->par_band > 0 ? ((lay->nint + 3) & ~3) / 2 : 0);
  const int nodew2 = (nodew + 1) & ~1;
  const int leafw = (lay->m * lay->W + 1) & ~1;
  const int per_wave_lds = lay->chain_words + nodew2;
  const int ldsw = (lds_max - 1024) / 8;  // less room for the kernel's static LDS (under 1 KB)
  const bool lds_fits = !lay->runtime_width && leafw + per_wave_lds <= ldsw;
  bool use_lds;
  if (cfg->kernel == TSA_KERNEL_LDS) {
    if (!lds_fits)
      return fail(nullptr, TSA_ERR_FIT, "chain does not fit in LDS (or the label width is not a register width)");
    use_lds = true;
  } else {
    use_lds = cfg->kernel == TSA_KERNEL_GLOBAL ? false : lds_fits;
  }
  if (use_lds) {
    L->W = lay->W;
    L->lds = 1;
    L->lds_words = per_wave_lds;
    const int wpb = (ldsw - leafw) / per_wave_lds;
    L->wpb = wpb < 1 ? 1 : (wpb > 4 ? 4 : wpb);
  } else {
    if (nodew2 > ldsw) return fail(nullptr, TSA_ERR_FIT, "par: node arrays do not fit in LDS");
    L->W = 0;
    L->lds = 0;
    L->lds_words = nodew2;
    const int wpb = ldsw / nodew2;
    L->wpb = wpb < 1 ? 1 : (wpb > 4 ? 4 : wpb);
  }
  if (ncu > 0 && (long long)nchains < (long long)ncu * L->wpb) {
    const int spread = (nchains + ncu - 1) / ncu;
    L->wpb = spread < 1 ? 1 : spread;
  }
  L->lds_max = ldsw * 8;
  // pre-order sweeps of at most one chain per compute unit are bound by the sweeping wave's chain of
  // dependent steps while three SIMDs idle: there helper waves draw the next sweep's random numbers
  L->draw_waves = cfg->draw_waves > 0 || (cfg->draw_waves == 0 && ncu > 0 && (long long)nchains <= ncu);
  *use_lds_out = use_lds;
  return TSA_OK;
}

extern "C" int tsa_create(const tsa_layout_t* lay, const uint64_t* leaf, int32_t leaf_sc, const tsa_config_t* cfg,
                          int32_t nchains, tsa_ctx** out) {
  if (!lay || !leaf || !cfg || !out) return fail(nullptr, TSA_ERR_ARG, "tsa_create: null argument");
  *out = nullptr;
  if (check_layout_config(lay, cfg, "tsa_create") != TSA_OK) return TSA_ERR_ARG;
  if (nchains < 1 || nchains > (1 << 24)) return fail(nullptr, TSA_ERR_ARG, "tsa_create: nchains out of range");
  for (size_t i = 0; i < (size_t)lay->m * lay->W; i++) {
    const int used = lay->nlab - 64 * (int)(i % lay->W);  // labels that word i may hold
    if (used <= 0 ? leaf[i] != 0 : (used < 64 && (leaf[i] >> used) != 0))
      return fail(nullptr, TSA_ERR_ARG, "tsa_create: leaf label out of range");
  }

  if (check_host_math() != TSA_OK) return TSA_ERR_LIBM;

  tsa_ctx* c = new tsa_ctx();
  c->lay = *lay;
  c->cfg = *cfg;
  c->mode = cfg->mode;
  c->nchains = nchains;
  fill_params(c->lay, c->cfg, leaf_sc, c->P);

  int dev = 0;
  int lds_max = 0, ncu = 0, lds_cu = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess)
    e = hipDeviceGetAttribute(&lds_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev);
  if (e != hipSuccess) {
    free_ctx(c);
    return fail(nullptr, TSA_ERR_HIP, std::string("no HIP device: ") + hipGetErrorString(e));
  }
  c->ncu = ncu;

  bool use_lds = false;
  if (plan_one_wave(lay, cfg, nchains, lds_max, ncu, &c->L, &use_lds) != TSA_OK) {
    free_ctx(c);
    return TSA_ERR_FIT;
  }
  c->Wt = c->L.W;
  const int leafw = (lay->m * lay->W + 1) & ~1;
  if (cfg->fused_energy) {
    // chains resident at once: workgroups of wpb chains, as many per compute unit as its LDS holds
    const long long smem = ((long long)(use_lds ? leafw : 0) + (long long)c->L.wpb * c->L.lds_words) * 8;
    const long long per_cu = smem > 0 ? (long long)(lds_cu > 0 ? lds_cu : lds_max) / smem : 1;
    const long long resident = (long long)ncu * (per_cu < 1 ? 1 : per_cu) * c->L.wpb;
    // the fold kernel costs about as much as two rounds of in-kernel folds (it is bound by the double
    // arithmetic of the lse chain, and adds a launch): worth it from three rounds of resident chains
    c->fold_apart = cfg->fused_energy == 2 || (long long)nchains > 2 * resident;
  }
  // wide path: runtime-width chains without slice moves run par sweeps and energies in tsa_wide.hip
  const bool want_wide = cfg->kernel == TSA_KERNEL_WIDE || (cfg->kernel == TSA_KERNEL_AUTO && !use_lds);
  if (want_wide) {
    hipError_t we = hipErrorInvalidValue;
    if (lay->runtime_width && !cfg->slicing)
      we = tsa_wide_plan(c->P, nchains, cfg->wide_waves, cfg->wide_wgs, cfg->wide_lanes, cfg->sums, &c->wide);
    if (we != hipSuccess) {
      (void)hipGetLastError();  // clear the runtime's last error: the context goes on without the wide path
      c->wide = TsaWide{};
      if (cfg->kernel == TSA_KERNEL_WIDE || cfg->wide_waves > 0 || cfg->wide_wgs > 0 || cfg->wide_lanes > 0) {
        free_ctx(c);
        return fail(nullptr, TSA_ERR_FIT,
                    std::string("wide kernel: no plan (it needs runtime width, no slicing, W <= 256 words, lanes per "
                                "proposal 4/8/16 with summaries or enough for W without, the node arrays in LDS, "
                                "and nchains x workgroups per chain co-resident): ") +
                        hipGetErrorString(we));
      }
    }
  }
  char kb[200];
  if (c->wide.on)
    snprintf(kb, sizeof kb,
             "wide W=%d G=%d sums=%d waves/block=%d blocks/chain=%d lds_bytes/block=%d energy_blocks/chain=%d "
             "fold_stage=%d xcds=%d",
             lay->W, c->wide.G, c->wide.nsw, c->wide.nt / 64, c->wide.K, c->wide.smem, c->wide.eK, c->wide.fold_stage,
             c->wide.nxcd);
  else
    snprintf(kb, sizeof kb, "%s W=%d waves/block=%d lds_bytes/wave=%d%s%s", use_lds ? "lds" : "global",
             use_lds ? c->Wt : lay->W, c->L.wpb, c->L.lds_words * 8,
             cfg->fused_energy && c->fold_apart ? " fold=apart" : "",
             c->L.draw_waves ? " preorder_draw_waves=3" : "");
  c->kname = kb;

  const size_t recb = (size_t)nchains * lay->chain_words * 8;
#define TSA_CREATE_HIP(call)                                                                       \
  do {                                                                                            \
    hipError_t e2 = (call);                                                                       \
    if (e2 != hipSuccess) {                                                                       \
      std::string m_ = std::string(#call) + ": " + hipGetErrorString(e2);                         \
      free_ctx(c);                                                                                \
      return fail(nullptr, TSA_ERR_HIP, m_);                                                      \
    }                                                                                             \
  } while (0)
  TSA_CREATE_HIP(hipStreamCreateWithFlags(&c->st, hipStreamNonBlocking));
  TSA_CREATE_HIP(hipMalloc(&c->d_rec, recb));
  TSA_CREATE_HIP(hipMemsetAsync(c->d_rec, 0, recb, c->st));
  TSA_CREATE_HIP(hipMalloc(&c->d_leaf, (size_t)lay->m * lay->W * 8));
  TSA_CREATE_HIP(hipMemcpyAsync(c->d_leaf, leaf, (size_t)lay->m * lay->W * 8, hipMemcpyHostToDevice, c->st));
  TSA_CREATE_HIP(hipMalloc(&c->d_fix, g_fix.size() * 4));
  TSA_CREATE_HIP(hipMemcpyAsync(c->d_fix, g_fix.data(), g_fix.size() * 4, hipMemcpyHostToDevice, c->st));
  TSA_CREATE_HIP(hipMalloc(&c->d_stats, TSA_NSTAT_ALL * TSA_STAT_SLOTS * sizeof(unsigned long long)));
  TSA_CREATE_HIP(hipMemsetAsync(c->d_stats, 0, TSA_NSTAT_ALL * TSA_STAT_SLOTS * sizeof(unsigned long long), c->st));
  TSA_CREATE_HIP(hipMalloc(&c->d_lc, (size_t)nchains * 12 + 16));  // + the wide path's error word
  TSA_CREATE_HIP(hipMemsetAsync(c->d_lc, 0, (size_t)nchains * 12 + 16, c->st));
  c->d_sc = reinterpret_cast<int*>(c->d_lc) + nchains;
  c->d_ns = reinterpret_cast<int*>(c->d_lc) + 2 * (size_t)nchains;
  TSA_CREATE_HIP(hipHostMalloc(&c->h_en, (size_t)nchains * 12 + 16, hipHostMallocDefault));
  if (hipHostGetDevicePointer(reinterpret_cast<void**>(&c->d_hen), c->h_en, 0) != hipSuccess) {
    (void)hipGetLastError();  // not mapped: energies take the copy path
    c->d_hen = nullptr;
  }
  if (c->wide.on) c->fold_apart = false;
  if (c->fold_apart) {
    const size_t nint4 = (size_t)((lay->nint + 3) & ~3);
    TSA_CREATE_HIP(hipMalloc(&c->d_ncost, (size_t)nchains * nint4 * 4));
    TSA_CREATE_HIP(hipMalloc(&c->d_nz, (size_t)nchains * nint4 * 2));
  }
  if (c->wide.on) {
    const size_t nint4 = (size_t)((lay->nint + 3) & ~3);
    TSA_CREATE_HIP(hipMalloc(&c->d_wsync, (size_t)nchains * 12));
    TSA_CREATE_HIP(hipMemsetAsync(c->d_wsync, 0, (size_t)nchains * 12, c->st));
    c->wsync.bar = c->d_wsync;
    c->wsync.done = c->d_wsync + nchains;
    c->wsync.join = c->d_wsync + 2 * (size_t)nchains;
    c->wsync.nxcd = c->wide.nxcd;
    c->wsync.join_polls = cfg->wide_join;
    c->wsync.err = reinterpret_cast<unsigned*>(c->d_lc) + 3 * (size_t)nchains;
    if (c->wide.K > 1) TSA_CREATE_HIP(hipMalloc(&c->wsync.out, (size_t)nchains * 2 * nint4));
    TSA_CREATE_HIP(hipMalloc(&c->d_ncost, (size_t)nchains * nint4 * 4));
    TSA_CREATE_HIP(hipMalloc(&c->d_nz, (size_t)nchains * nint4 * 2));
    c->wsync.ncost = c->d_ncost;
    c->wsync.nz = c->d_nz;
    TSA_CREATE_HIP(hipMalloc(&c->d_fcnt, (size_t)nchains * 4));
    TSA_CREATE_HIP(hipMemsetAsync(c->d_fcnt, 0, (size_t)nchains * 4, c->st));
    if (c->wide.nsw) {
      const int nsw = c->wide.nsw, nch = lay->W / 2;
      std::vector<uint64_t> ls((size_t)lay->m * nsw, 0ull);
      for (int i = 0; i < lay->m; i++)
        for (int cc = 0; cc < nch; cc++)
          if (leaf[(size_t)i * lay->W + 2 * cc] | leaf[(size_t)i * lay->W + 2 * cc + 1])
            ls[(size_t)i * nsw + cc / 64] |= 1ull << (cc % 64);
      TSA_CREATE_HIP(hipMalloc(&c->d_sum, (size_t)nchains * nint4 * nsw * 8));
      TSA_CREATE_HIP(hipMalloc(&c->d_leafsum, ls.size() * 8));
      TSA_CREATE_HIP(hipMemcpyAsync(c->d_leafsum, ls.data(), ls.size() * 8, hipMemcpyHostToDevice, c->st));
      TSA_CREATE_HIP(hipStreamSynchronize(c->st));  // ls is a local
      c->wsync.sum = c->d_sum;
      c->wsync.leafsum = c->d_leafsum;
      c->wsync.nsw = nsw;
      c->wsync.lsum_lds = c->wide.lsum_lds;
    }
  }
  TSA_CREATE_HIP(hipMalloc(&c->d_anc, (size_t)nchains * 4));
  TSA_CREATE_HIP(hipHostMalloc(&c->h_anc, (size_t)nchains * 4, hipHostMallocDefault));
  if (hipHostGetDevicePointer(reinterpret_cast<void**>(&c->d_hanc), c->h_anc, 0) != hipSuccess) {
    (void)hipGetLastError();  // not mapped: the list goes by a copy
    c->d_hanc = nullptr;
  }
  TSA_CREATE_HIP(hipEventCreateWithFlags(&c->ev_anc, hipEventDisableTiming));
  TSA_CREATE_HIP(hipStreamSynchronize(c->st));
#undef TSA_CREATE_HIP
  *out = c;
  return TSA_OK;
}

// Overlapped tracking: order the main stream after every selection still pending on st2 (they read d_lc /
// d_sc / d_ns and write the tracking state), or wait for st2 on the host and forget the snapshots (before
// the population is replaced).
static void join_track(tsa_ctx* c) {
  // st2 runs the selections in the order they were enqueued, so the last one's event covers every pending one
  // (one wait in the queue: each costs the device a few microseconds even when already satisfied)
  if (c->last_track >= 0 && c->track_pending[c->last_track])
    (void)hipStreamWaitEvent(c->st, c->ev_track[c->last_track], 0);
  else if (c->tinit_pending)
    (void)hipStreamWaitEvent(c->st, c->ev_tinit, 0);
  c->tinit_pending = false;
}

static hipError_t join_split(tsa_ctx* c) {
  c->fork_needed = true;  // the caller enqueues work on st
  if (!c->split_pending) return hipSuccess;
  c->split_pending = false;
  hipError_t e = hipEventRecord(c->ev_join, c->st3);
  if (e == hipSuccess) e = hipStreamWaitEvent(c->st, c->ev_join, 0);
  return e;
}

static hipError_t flush_resample(tsa_ctx* c) {
  if (!c->anc_pend) return hipSuccess;
  c->anc_pend = false;
  hipError_t e = tsa_launch_copy(c->d_rec, c->d_rec2, c->d_hanc ? c->d_hanc : c->d_anc, c->nchains,
                                 c->lay.chain_words, c->st);
  if (e == hipSuccess) e = hipEventRecord(c->ev_anc, c->st);
  c->anc_pending = e == hipSuccess;
  std::swap(c->d_rec, c->d_rec2);
  return e;
}

static hipError_t flush_track_init(tsa_ctx* c, bool on_st2 = false) {
  if (!c->track_init_pending) return hipSuccess;
  c->track_init_pending = false;
  hipError_t e = tsa_launch_track_init(c->d_track, c->d_ticks0, reinterpret_cast<unsigned long long*>(c->d_trace),
                                       (int)((size_t)c->track_levels * sizeof(TsaTraceRowD) / 8),
                                       reinterpret_cast<unsigned long long*>(c->d_best), c->lay.chain_words,
                                       on_st2 ? c->st2 : c->st);
  if (on_st2) {
    if (e == hipSuccess && !c->ev_tinit) e = hipEventCreateWithFlags(&c->ev_tinit, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(c->ev_tinit, c->st2);
    c->tinit_pending = e == hipSuccess;
  }
  return e;
}

// Where tsa_track_end's results sit in the page-locked staging buffer h_tend (byte offsets): the tracking
// state, the start tick, the wide path's error word, the best tree (children words and S: tree bytes) and the
// trace rows (row bytes).
struct TendLayout {
  size_t st, t0, werr, tree, rows, tree_bytes, row_bytes;
};
static TendLayout tend_layout(const tsa_ctx* c) {
  const tsa_layout_t& L = c->lay;
  TendLayout o;
  o.tree_bytes = (size_t)(L.s_off + L.W - L.ch_off) * 8;
  o.row_bytes = (size_t)c->track_levels * sizeof(TsaTraceRowD);
  o.st = 0;
  o.t0 = (sizeof(TsaTrackState) + 15) & ~(size_t)15;
  o.werr = o.t0 + 8;
  o.tree = o.t0 + 16;
  o.rows = o.tree + ((o.tree_bytes + 15) & ~(size_t)15);
  return o;
}

// The wide path's overlapped selection with the fold in the sweep launch: dense plans of one workgroup per chain
// with more chains than compute units (with fewer, the fold of the node-cost snapshot runs beside the next
// sweep as well).
static bool wide_fold_snap(const tsa_ctx* c) {
  return c->wide.on && c->wide.K == 1 && c->wide.nsw == 0 && c->nchains >= c->ncu && !c->cfg.slicing;
}

// Blocks of levels on the wide path (tsa_anneal): one workgroup per chain (no chain barrier between levels)
// with chunk summaries, the overlapped selection with the node-cost snapshots folded apart, the node-cost
// cache of tc mode.
static bool wide_blocks_ok(const tsa_ctx* c, int order) {
  return c->wide.on && c->wide.K == 1 && c->wide.nsw > 0 && c->overlap && !wide_fold_snap(c) && c->mode == 0 &&
         !c->cfg.slicing && order == TSA_ORDER_PAR;
}

static hipError_t quiesce_track(tsa_ctx* c) {
  hipError_t e = hipSuccess;
  if (c->st2) e = hipStreamSynchronize(c->st2);
  for (bool& p : c->track_pending) p = false;
  c->tinit_pending = false;
  c->last_slot = -1;
  return e;
}

// Snapshot slots 0 .. n - 1 allocated (the slots in turn become n; the rotation goes on from where it is).
static int ensure_slots(tsa_ctx* ctx, int n) {
  if (n > TSA_SNAP_MAX) return fail(ctx, TSA_ERR_ARG, "snapshot slots: more than TSA_SNAP_MAX");
  const size_t nint = (size_t)ctx->lay.nint, nint4 = (nint + 3) & ~(size_t)3;
  for (int k = ctx->nslots; k < n; k++) {
    TSA_HIP(ctx, hipMalloc(&ctx->d_snap_ch[k], (size_t)ctx->nchains * nint * 4));
    TSA_HIP(ctx, hipMalloc(&ctx->d_snap_cost[k], (size_t)ctx->nchains * nint4 * 4));
    TSA_HIP(ctx, hipMalloc(&ctx->d_snap_nz[k], (size_t)ctx->nchains * nint4 * 2));
    TSA_HIP(ctx, hipMalloc(&ctx->d_snap_en[k], (size_t)ctx->nchains * 12));
    ctx->nslots = k + 1;
  }
  return TSA_OK;
}

// Before a sweep overwrites snapshot slot s, the selection that last read it must be done.  The host waits
// for it (it ran beside the previous sweep, which is still queued or running, so the device does not idle)
// rather than putting a wait on the stream: a cross-stream wait in the queue costs about 10 us per level
// even when it is already satisfied, and the host is normally many levels ahead of the device.
static hipError_t claim_slot(tsa_ctx* c, int s) {
  hipError_t e = hipSuccess;
  if (c->track_pending[s]) e = hipEventSynchronize(c->ev_track[c->track_ev[s]]);
  c->track_pending[s] = false;
  return e;
}

// The chunk summaries for a full node-cost pass, when they match the population (else none: a dense pass).
static TsaSums wide_sums(const tsa_ctx* c) {
  if (!c->wide.nsw || !c->sums_valid) return TsaSums{nullptr, nullptr, 0};
  return TsaSums{c->d_sum, c->d_leafsum, c->wide.nsw};
}

static hipError_t launch_energy(tsa_ctx* c) {
  join_track(c);
  if (c->energy_fresh) return hipSuccess;  // the last sweep launch left them in d_lc / d_sc / d_ns
  if (c->wide.on) {
    const hipError_t e = tsa_launch_wide_energy(c->wide, c->mode, c->P, c->d_rec, c->d_leaf, c->d_fix, c->nchains,
                                                c->d_ncost, c->d_nz, c->d_fcnt, c->d_lc, c->d_sc, c->d_ns,
                                                c->costs_valid ? 0 : 1, c->st, wide_sums(c));
    c->costs_valid = e == hipSuccess;
    return e;
  }
  return tsa_launch_energy(c->Wt, c->mode, c->P, c->d_rec, c->d_leaf, c->d_fix, c->nchains, c->d_lc, c->d_sc,
                           c->d_ns, c->st);
}

// The wide path's error word (set when a chain barrier gave up, leaving the population undefined):
// reported once by the next synchronizing call, then cleared.  A workgroup the device never started cannot
// cause it (a chain's workgroups check in before its first barrier, and a chain whose check-in times out is
// swept by one workgroup alone); only one of a chain's running workgroups descheduled for seconds could.
static int wide_error(tsa_ctx* c, uint32_t word) {
  if (word == 0) return TSA_OK;
  c->costs_valid = false;
  c->sums_valid = false;
  (void)hipMemsetAsync(c->wsync.err, 0, 4, c->st);
  (void)hipStreamSynchronize(c->st);
  return fail(c, TSA_ERR_HIP,
              "wide sweep kernel: a chain barrier timed out after its workgroups had all started; the population is "
              "undefined");
}

extern "C" int tsa_upload(tsa_ctx* ctx, const uint64_t* population) {
  if (!ctx || !population) return fail(ctx, TSA_ERR_ARG, "tsa_upload: null argument");
  TSA_HIP(ctx, join_split(ctx));
  TSA_HIP(ctx, flush_track_init(ctx));
  const tsa_layout_t& L = ctx->lay;
  std::vector<char> seen;
  std::vector<int> st;
  for (int c = 0; c < ctx->nchains; c++) {
    const uint64_t* rec = population + (size_t)c * L.chain_words;
    if (!valid_tree(reinterpret_cast<const uint32_t*>(rec + L.ch_off), L.m, seen, st))
      return fail(ctx, TSA_ERR_ARG, "tsa_upload: chain " + std::to_string(c) + " is not a valid tree");
  }
  TSA_HIP(ctx, quiesce_track(ctx));
  ctx->anc_pend = false;  // (a resampling not yet made applies to the population this replaces)
  ctx->costs_valid = false;
  ctx->energy_fresh = ctx->energy_host = false;
  ctx->sums_valid = false;
  TSA_HIP(ctx, hipMemcpyAsync(ctx->d_rec, population, (size_t)ctx->nchains * L.chain_words * 8,
                              hipMemcpyHostToDevice, ctx->st));
  // the population's derived data on the wide path, made with it as the reference's start builds the chunk
  // summaries with the labels (csrc/treesa_gpu.cu:1604-1612): the summaries and, in tc mode, the node-cost
  // cache that the visits read (with the energies, which that pass folds)
  if (ctx->wide.on) {
    if (ctx->wide.nsw) {
      TSA_HIP(ctx, tsa_launch_wsum(ctx->wide, ctx->P, ctx->d_rec, ctx->nchains, ctx->d_sum, ctx->st));
      ctx->sums_valid = true;
    }
    if (ctx->mode == 0) {
      TSA_HIP(ctx, tsa_launch_wide_energy(ctx->wide, ctx->mode, ctx->P, ctx->d_rec, ctx->d_leaf, ctx->d_fix,
                                          ctx->nchains, ctx->d_ncost, ctx->d_nz, ctx->d_fcnt, ctx->d_lc, ctx->d_sc,
                                          ctx->d_ns, 1, ctx->st, wide_sums(ctx)));
      ctx->costs_valid = true;
      ctx->energy_fresh = true;
    }
  }
  TSA_HIP(ctx, hipStreamSynchronize(ctx->st));
  ctx->host_waited = true;
  return TSA_OK;
}

extern "C" int tsa_download(tsa_ctx* ctx, int32_t c0, int32_t count, uint64_t* out) {
  if (!ctx || !out) return fail(ctx, TSA_ERR_ARG, "tsa_download: null argument");
  TSA_HIP(ctx, join_split(ctx));
  TSA_HIP(ctx, flush_track_init(ctx));
  TSA_HIP(ctx, flush_resample(ctx));
  if (c0 < 0 || count < 0 || c0 + count > ctx->nchains) return fail(ctx, TSA_ERR_ARG, "tsa_download: range");
  const size_t cw = ctx->lay.chain_words;
  TSA_HIP(ctx, hipMemcpyAsync(out, ctx->d_rec + (size_t)c0 * cw, (size_t)count * cw * 8, hipMemcpyDeviceToHost,
                              ctx->st));
  TSA_HIP(ctx, hipStreamSynchronize(ctx->st));
  ctx->host_waited = true;
  return TSA_OK;
}

extern "C" int tsa_download_async(tsa_ctx* ctx, int32_t c0, int32_t count, uint64_t* out) {
  if (!ctx || !out) return fail(ctx, TSA_ERR_ARG, "tsa_download_async: null argument");
  TSA_HIP(ctx, join_split(ctx));
  TSA_HIP(ctx, flush_track_init(ctx));
  TSA_HIP(ctx, flush_resample(ctx));
  if (c0 < 0 || count < 0 || c0 + count > ctx->nchains) return fail(ctx, TSA_ERR_ARG, "tsa_download_async: range");
  const size_t cw = ctx->lay.chain_words;
  TSA_HIP(ctx, hipMemcpyAsync(out, ctx->d_rec + (size_t)c0 * cw, (size_t)count * cw * 8, hipMemcpyDeviceToHost,
                              ctx->st));
  return TSA_OK;
}

extern "C" int tsa_wait(tsa_ctx* ctx) {
  if (!ctx) return fail(ctx, TSA_ERR_ARG, "tsa_wait: null context");
  TSA_HIP(ctx, join_split(ctx));
  TSA_HIP(ctx, flush_track_init(ctx));
  TSA_HIP(ctx, flush_resample(ctx));
  if (ctx->st2) TSA_HIP(ctx, hipStreamSynchronize(ctx->st2));
  TSA_HIP(ctx, hipStreamSynchronize(ctx->st));
  ctx->host_waited = true;
  return TSA_OK;
}

// The first chain of a split level's second launch: half the chains, in whole workgroups.
static int split_point(const tsa_ctx* ctx) {
  return (ctx->nchains / 2 + ctx->L.wpb - 1) / ctx->L.wpb * ctx->L.wpb;
}

// tsa_sweeps, or with blk set (tsa_anneal; the one-wave kernels with the overlapped selection and the fold
// apart) one launch (one split pair) of a block of levels, nsweeps = blk->total: every level with blk_ev[i] set
// takes a snapshot slot of its own, returned in blk_slots[i] (-1: none), for tsa_track.
static int sweeps_impl(tsa_ctx* ctx, int32_t order, float beta, uint32_t sweep0, int32_t nsweeps, const TsaBlock* blk,
                       const uint8_t* blk_ev, int* blk_slots) {
  if (!ctx) return fail(ctx, TSA_ERR_ARG, "tsa_sweeps: null context");
  if (order != TSA_ORDER_PAR && order != TSA_ORDER_PREORDER) return fail(ctx, TSA_ERR_ARG, "--order par|preorder");
  if (nsweeps < 0) return fail(ctx, TSA_ERR_ARG, "tsa_sweeps: nsweeps < 0");
  if (nsweeps == 0) return TSA_OK;
  // the session's start (tsa_track_begin): with the selection on st2, enqueued there after this call's sweeps,
  // so that the host issues the sweeps first (st2's folds and selections come after it in st2's order, and st
  // waits for it in join_track); otherwise on st before them
  const bool init_on_st2 = ctx->track_init_pending && ctx->overlap && ctx->st2 != nullptr;
  if (!init_on_st2) TSA_HIP(ctx, flush_track_init(ctx));
  while ((int)ctx->ev.size() < 2 * (ctx->npending + 2)) {
    hipEvent_t e;
    TSA_HIP(ctx, hipEventCreate(&e));
    ctx->ev.push_back(e);
  }
  // e0 / e1 take the start and stop times of the sweep kernel alone, recorded by its dispatch (no marker
  // packets between the kernels of a level), or, after a host wait, by markers around it (d0 / d1: the events
  // the dispatch records itself, if any)
  hipEvent_t e0 = ctx->ev[2 * ctx->npending], e1 = ctx->ev[2 * ctx->npending + 1];
  const bool markers = ctx->host_waited;
  ctx->host_waited = false;
  hipEvent_t d0 = markers ? nullptr : e0, d1 = markers ? nullptr : e1;
  ctx->energy_fresh = ctx->energy_host = false;
  if (blk && ctx->wide.on && !wide_blocks_ok(ctx, order))
    return fail(ctx, TSA_ERR_ARG, "block of levels on the wide path: one workgroup per chain, the overlapped "
                                  "selection with the fold apart, tc mode, par order");
  if (ctx->wide.on && order == TSA_ORDER_PAR) {
    TSA_HIP(ctx, join_split(ctx));
    TSA_HIP(ctx, flush_resample(ctx));
    // energies stay a separate fold of the node-cost cache: every chain ends its sweep at about the same
    // time, so folding inside the sweep kernel would only lengthen it
    if (ctx->wide.nsw && !ctx->sums_valid) {
      TSA_HIP(ctx, tsa_launch_wsum(ctx->wide, ctx->P, ctx->d_rec, ctx->nchains, ctx->d_sum, ctx->st));
      ctx->sums_valid = true;
    }
    TsaWideSync sy = ctx->wsync;
    int s = -1;
    // the node-cost cache must be exact before the sweep when the snapshot it leaves is folded as it stands,
    // and when the sweep reads it (tc mode: a visit takes P's old cost and size from it)
    if ((ctx->overlap || ctx->mode == 0) && !ctx->costs_valid) {
      join_track(ctx);
      TSA_HIP(ctx, tsa_launch_wide_energy(ctx->wide, ctx->mode, ctx->P, ctx->d_rec, ctx->d_leaf, ctx->d_fix,
                                          ctx->nchains, ctx->d_ncost, ctx->d_nz, ctx->d_fcnt, ctx->d_lc, ctx->d_sc,
                                          ctx->d_ns, 1, ctx->st, wide_sums(ctx)));
      ctx->costs_valid = true;
    }
    // a dense plan of one workgroup per chain folds the energies at the end of the sweep (the sweep kernel has
    // every chain's cost cache at hand; a fold launch after it would find the device idle but for its one lane
    // group per chain): without the overlap into d_lc / d_sc / d_ns, with it into the snapshot slot, whose tree
    // the selection beside the next sweep reads
    const bool snap_fold = ctx->overlap && wide_fold_snap(ctx) && ctx->costs_valid;
    const bool fold_here = !ctx->overlap && ctx->wide.K == 1 && ctx->wide.nsw == 0 && ctx->costs_valid;
    if (fold_here) {
      join_track(ctx);  // a selection still pending on st2 reads d_lc / d_sc / d_ns
      sy.flc = ctx->d_lc;
      sy.fsc = ctx->d_sc;
      sy.fns = ctx->d_ns;
    }
    if (blk) {
      // the block's evaluated levels leave their snapshots in slots of their own, folded and selected on st2
      sy.blk_n = blk->n;
      for (int i = 0; i < blk->n; i++) {
        sy.blk_beta[i] = blk->beta[i];
        sy.blk_niters[i] = blk->niters[i];
        blk_slots[i] = -1;
        if (!blk_ev[i]) continue;
        const int t = ctx->slot;
        TSA_HIP(ctx, claim_slot(ctx, t));
        ctx->snap_kind[t] = SNAP_WIDE;
        sy.blk_ch[i] = ctx->d_snap_ch[t];
        sy.blk_cost[i] = ctx->d_snap_cost[t];
        sy.blk_nz[i] = ctx->d_snap_nz[t];
        blk_slots[i] = t;
        ctx->slot = (t + 1) % ctx->nslots;
      }
    } else if (ctx->overlap) {
      s = ctx->slot;
      TSA_HIP(ctx, claim_slot(ctx, s));
      sy.snap_ch = ctx->d_snap_ch[s];
      if (snap_fold) {
        sy.flc = reinterpret_cast<float*>(ctx->d_snap_en[s]);
        sy.fsc = reinterpret_cast<int*>(ctx->d_snap_en[s]) + ctx->nchains;
        sy.fns = reinterpret_cast<int*>(ctx->d_snap_en[s]) + 2 * (size_t)ctx->nchains;
        ctx->snap_kind[s] = SNAP_ENERGIES;
      } else {
        sy.snap_cost = ctx->d_snap_cost[s];
        sy.snap_nz = ctx->d_snap_nz[s];
        ctx->snap_kind[s] = SNAP_WIDE;
      }
    }
    if (markers) TSA_HIP(ctx, hipEventRecord(e0, ctx->st));
    TSA_HIP(ctx, tsa_launch_wide(ctx->wide, ctx->mode, ctx->P, ctx->d_rec, ctx->d_leaf, ctx->d_fix, ctx->nchains, beta,
                                 sweep0, nsweeps, ctx->d_stats, sy, ctx->st, d0, d1));
    if (markers) TSA_HIP(ctx, hipEventRecord(e1, ctx->st));
    if (s >= 0) {
      ctx->ev_sweep[s] = e1;  // the selection of this snapshot waits for the sweep's stop event
      ctx->split_slot[s] = false;
      ctx->last_slot = s;
      ctx->slot = (s + 1) % ctx->nslots;
    }
    if (blk)
      for (int i = 0; i < blk->n; i++)
        if (blk_slots[i] >= 0) {
          ctx->ev_sweep[blk_slots[i]] = e1;
          ctx->split_slot[blk_slots[i]] = false;
          ctx->last_slot = blk_slots[i];
        }
    ctx->energy_fresh = fold_here;
  } else {
    ctx->costs_valid = false;
    ctx->sums_valid = false;
    const bool fuse = ctx->cfg.fused_energy != 0;
    const bool apart = fuse && ctx->fold_apart;
    // a split level: chains [0, h) on st, [h, nchains) on st3 (h in whole workgroups)
    const int h = split_point(ctx);
    const bool split = ctx->overlap && apart && h > 0 && h < ctx->nchains;
    if (!split) TSA_HIP(ctx, join_split(ctx));
    // a resampling not yet made: this launch's kernel stages each chain from its ancestor's record (the chain
    // in LDS, one launch), else the copy first
    const bool gather = ctx->anc_pend && ctx->L.lds && !split && !blk;
    if (!gather) TSA_HIP(ctx, flush_resample(ctx));
    TsaEnergyOut eo{fuse && !apart ? ctx->d_lc : nullptr, ctx->d_sc, ctx->d_ns, apart ? ctx->d_ncost : nullptr,
                    apart ? ctx->d_nz : nullptr, nullptr, TsaBlock{}};
    int s = -1;
    if (blk) {
      if (!ctx->overlap || !apart || order != TSA_ORDER_PAR || blk->n < 1 || blk->n > TSA_BLOCK_MAX ||
          blk->total != nsweeps)
        return fail(ctx, TSA_ERR_ARG, "block of levels: needs the overlapped selection with the fold apart, par order");
      // the block's evaluated levels leave their snapshots in slots of their own, folded and selected on st2
      eo.cost = nullptr;
      eo.z = nullptr;
      eo.blk = *blk;
      for (int i = 0; i < blk->n; i++) {
        blk_slots[i] = -1;
        eo.blk.cost[i] = nullptr;
        eo.blk.z[i] = nullptr;
        eo.blk.ch[i] = nullptr;
        if (!blk_ev[i]) continue;
        const int t = ctx->slot;
        TSA_HIP(ctx, claim_slot(ctx, t));
        ctx->snap_kind[t] = SNAP_COSTS;
        eo.blk.cost[i] = ctx->d_snap_cost[t];
        eo.blk.z[i] = ctx->d_snap_nz[t];
        eo.blk.ch[i] = ctx->d_snap_ch[t];
        blk_slots[i] = t;
        ctx->slot = (t + 1) % ctx->nslots;
      }
    } else if (ctx->overlap && fuse) {
      // node costs (or, folded in the kernel, energies) and children words go to snapshot slot s, folded and
      // selected on st2 by tsa_track
      s = ctx->slot;
      TSA_HIP(ctx, claim_slot(ctx, s));
      ctx->snap_kind[s] = apart ? SNAP_COSTS : SNAP_ENERGIES;
      if (apart) {
        eo.cost = ctx->d_snap_cost[s];
        eo.z = ctx->d_snap_nz[s];
      } else {
        eo.lc = reinterpret_cast<float*>(ctx->d_snap_en[s]);
        eo.sc = reinterpret_cast<int*>(ctx->d_snap_en[s]) + ctx->nchains;
        eo.ns = reinterpret_cast<int*>(ctx->d_snap_en[s]) + 2 * (size_t)ctx->nchains;
      }
      eo.ch = ctx->d_snap_ch[s];
    } else {
      ctx->last_slot = -1;  // the snapshots no longer describe the population
      join_track(ctx);      // a pending fold may still read the node-cost snapshot; d_lc is rewritten below
      if (fuse && !apart && ctx->track_levels == 0 && ctx->d_hen) {
        // a host-side level loop reads the energies after every launch: the sweep kernel writes them into
        // the page-locked buffer tsa_energy reads, with no copy after it
        eo.lc = reinterpret_cast<float*>(ctx->d_hen);
        eo.sc = reinterpret_cast<int*>(ctx->d_hen) + ctx->nchains;
        eo.ns = reinterpret_cast<int*>(ctx->d_hen) + 2 * (size_t)ctx->nchains;
        ctx->energy_host = true;
      }
    }
    if (split) {
      if (!ctx->st3) {
        TSA_HIP(ctx, hipStreamCreateWithFlags(&ctx->st3, hipStreamNonBlocking));
        TSA_HIP(ctx, hipEventCreateWithFlags(&ctx->ev_fork, hipEventDisableTiming));
        TSA_HIP(ctx, hipEventCreateWithFlags(&ctx->ev_join, hipEventDisableTiming));
        for (int k = 0; k < TSA_SNAP_MAX; k++)
          TSA_HIP(ctx, hipEventCreateWithFlags(&ctx->ev_b[k], hipEventDisableTiming));
      }
      // the second launch's timing pair follows the first's
      hipEvent_t f0 = ctx->ev[2 * ctx->npending + 2], f1 = ctx->ev[2 * ctx->npending + 3];
      if (ctx->fork_needed) {
        TSA_HIP(ctx, hipEventRecord(ctx->ev_fork, ctx->st));
        TSA_HIP(ctx, hipStreamWaitEvent(ctx->st3, ctx->ev_fork, 0));
        ctx->fork_needed = false;
      }
      if (markers) TSA_HIP(ctx, hipEventRecord(e0, ctx->st));
      TSA_HIP(ctx, tsa_launch_sweeps(ctx->L, ctx->mode, order, ctx->P, ctx->d_rec, ctx->d_leaf, ctx->d_fix, h, beta,
                                     sweep0, nsweeps, ctx->d_stats, eo, ctx->st, d0, d1));
      if (markers) TSA_HIP(ctx, hipEventRecord(e1, ctx->st));
      TsaKParams P2 = ctx->P;
      P2.chain0 = h;
      if (markers) TSA_HIP(ctx, hipEventRecord(f0, ctx->st3));
      TSA_HIP(ctx, tsa_launch_sweeps(ctx->L, ctx->mode, order, P2, ctx->d_rec, ctx->d_leaf, ctx->d_fix,
                                     ctx->nchains, beta, sweep0, nsweeps, ctx->d_stats, eo, ctx->st3,
                                     markers ? nullptr : f0, markers ? nullptr : f1));
      if (markers) TSA_HIP(ctx, hipEventRecord(f1, ctx->st3));
      if (blk) {
        for (int i = 0; i < blk->n; i++)
          if (blk_slots[i] >= 0) {  // (one event for the block: the first evaluated level's, which its
                                    // selection launch waits for)
            TSA_HIP(ctx, hipEventRecord(ctx->ev_b[blk_slots[i]], ctx->st3));
            break;
          }
      } else {
        TSA_HIP(ctx, hipEventRecord(ctx->ev_b[s], ctx->st3));
      }
      ctx->split_pending = true;
      ctx->split_levels++;
      ctx->npending++;  // (the first launch's pair is counted below)
    } else {
      TsaKParams Pg = ctx->P;
      uint64_t* out = ctx->d_rec;
      if (gather) {
        Pg.gsrc = ctx->d_rec;
        Pg.ganc = ctx->d_hanc ? ctx->d_hanc : ctx->d_anc;
        out = ctx->d_rec2;
      }
      if (markers) TSA_HIP(ctx, hipEventRecord(e0, ctx->st));
      TSA_HIP(ctx, tsa_launch_sweeps(ctx->L, ctx->mode, order, Pg, out, ctx->d_leaf, ctx->d_fix, ctx->nchains, beta,
                                     sweep0, nsweeps, ctx->d_stats, eo, ctx->st, d0, d1));
      if (markers) TSA_HIP(ctx, hipEventRecord(e1, ctx->st));
      if (gather) {  // the resampled population, swept, is now in the other buffer
        TSA_HIP(ctx, hipEventRecord(ctx->ev_anc, ctx->st));
        ctx->anc_pending = true;
        ctx->anc_pend = false;
        std::swap(ctx->d_rec, ctx->d_rec2);
      }
    }
    if (blk) {
      for (int i = 0; i < blk->n; i++) {
        const int t = blk_slots[i];
        if (t < 0) continue;
        ctx->split_slot[t] = split;
        ctx->ev_sweep[t] = e1;
        ctx->last_slot = t;
      }
      ctx->energy_fresh = false;
    } else if (s >= 0) {
      ctx->split_slot[s] = split;
      ctx->ev_sweep[s] = e1;
      ctx->last_slot = s;
      ctx->slot = (s + 1) % ctx->nslots;
      ctx->energy_fresh = false;  // the energies of this population exist only once tsa_track folds the slot
    } else {
      if (apart)
        TSA_HIP(ctx, tsa_launch_fold(ctx->P, ctx->d_rec, ctx->d_leaf, ctx->d_fix, ctx->d_ncost, ctx->d_nz,
                                     ctx->nchains, ctx->d_lc, ctx->d_sc, ctx->d_ns, ctx->st));
      ctx->energy_fresh = fuse && !ctx->energy_host;
    }
  }
  ctx->npending++;
  if (init_on_st2) TSA_HIP(ctx, flush_track_init(ctx, true));
  return TSA_OK;
}

extern "C" int tsa_sweeps(tsa_ctx* ctx, int32_t order, float beta, uint32_t sweep0, int32_t nsweeps) {
  return sweeps_impl(ctx, order, beta, sweep0, nsweeps, nullptr, nullptr, nullptr);
}

extern "C" int tsa_sweeps_ms(tsa_ctx* ctx, double* ms) {
  if (!ctx || !ms) return fail(ctx, TSA_ERR_ARG, "tsa_sweeps_ms: null argument");
  TSA_HIP(ctx, join_split(ctx));
  TSA_HIP(ctx, flush_track_init(ctx));
  *ms = 0.0;
  if (ctx->npending == 0) return TSA_OK;
  // the union of the launches' intervals (the two launches of a split level run at the same time), each in ms
  // from the first launch's start
  std::vector<std::pair<double, double>> iv((size_t)ctx->npending);
  for (int k = 0; k < ctx->npending; k++) {
    TSA_HIP(ctx, hipEventSynchronize(ctx->ev[2 * k + 1]));
    float a = 0.f, b = 0.f;
    if (k > 0) TSA_HIP(ctx, hipEventElapsedTime(&a, ctx->ev[0], ctx->ev[2 * k]));
    TSA_HIP(ctx, hipEventElapsedTime(&b, ctx->ev[0], ctx->ev[2 * k + 1]));
    iv[(size_t)k] = {(double)a, (double)b};
  }
  std::sort(iv.begin(), iv.end());
  double sum = 0.0, lo = 0.0, hi = 0.0;
  for (size_t k = 0; k < iv.size(); k++) {
    if (k == 0 || iv[k].first > hi) {
      sum += hi - lo;
      lo = iv[k].first;
      hi = iv[k].second;
    } else if (iv[k].second > hi) {
      hi = iv[k].second;
    }
  }
  sum += hi - lo;
  ctx->npending = 0;
  *ms = sum;
  return TSA_OK;
}

extern "C" int tsa_track_begin(tsa_ctx* ctx, const tsa_select_t* sel, int32_t max_levels) {
  if (!ctx || !sel) return fail(ctx, TSA_ERR_ARG, "tsa_track_begin: null argument");
  TSA_HIP(ctx, join_split(ctx));
  if (max_levels < 1) return fail(ctx, TSA_ERR_ARG, "tsa_track_begin: max_levels < 1");
  ctx->sel.mode = sel->mode;
  ctx->sel.slicing = sel->slicing;
  ctx->sel.select_sc = sel->select_sc;
  ctx->sel.sc_target = sel->sc_target;
  ctx->sel.sc_weight = sel->sc_weight;
  if (!ctx->d_track) TSA_HIP(ctx, hipMalloc(&ctx->d_track, sizeof(TsaTrackState)));
  if (!ctx->d_ticks0) TSA_HIP(ctx, hipMalloc(&ctx->d_ticks0, sizeof(unsigned long long)));
  if (!ctx->d_best) TSA_HIP(ctx, hipMalloc(&ctx->d_best, (size_t)ctx->lay.chain_words * 8));
  if (!ctx->d_tpart) {
    // (room for a selection launch of TSA_BLOCK_MAX levels: per level its groups' results and counter, then
    // each level's best and the launch's counter)
    TSA_HIP(ctx, hipMalloc(&ctx->d_tpart,
                           (size_t)(TSA_BLOCK_MAX + 1) * ((ctx->nchains + 255) / 256) * sizeof(TsaTrackPart)));
    TSA_HIP(ctx, hipMalloc(&ctx->d_tdone, (TSA_BLOCK_MAX + 1) * sizeof(unsigned)));
    TSA_HIP(ctx, hipMemsetAsync(ctx->d_tdone, 0, (TSA_BLOCK_MAX + 1) * sizeof(unsigned), ctx->st));
  }
  if (max_levels > ctx->track_levels) {
    if (ctx->d_trace) TSA_HIP(ctx, hipFree(ctx->d_trace));
    ctx->d_trace = nullptr;
    TSA_HIP(ctx, hipMalloc(&ctx->d_trace, (size_t)max_levels * sizeof(TsaTraceRowD)));
  }
  ctx->track_levels = max_levels;
  {
    const tsa_layout_t& L = ctx->lay;
    const size_t need = sizeof(TsaTrackState) + 16 + (size_t)(L.s_off + L.W - L.ch_off) * 8 +
                        (size_t)max_levels * sizeof(TsaTraceRowD) + 64;
    if (need > ctx->h_tend_bytes) {
      // (a level-loop launch of an unfinished session may still write its results there)
      if (ctx->h_tend) TSA_HIP(ctx, hipStreamSynchronize(ctx->st));
      if (ctx->h_tend) TSA_HIP(ctx, hipHostFree(ctx->h_tend));
      ctx->h_tend = nullptr;
      ctx->h_tend_bytes = 0;
      TSA_HIP(ctx, hipHostMalloc(reinterpret_cast<void**>(&ctx->h_tend), need, hipHostMallocDefault));
      ctx->h_tend_bytes = need;
      if (hipHostGetDevicePointer(reinterpret_cast<void**>(&ctx->d_tend), ctx->h_tend, 0) != hipSuccess) {
        (void)hipGetLastError();  // not mapped: the copies
        ctx->d_tend = nullptr;
      }
    }
    if (ctx->tick_hz == 0.0) {
      int dev = 0, khz = 0;
      TSA_HIP(ctx, hipGetDevice(&dev));
      TSA_HIP(ctx, hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev));
      ctx->tick_hz = (double)khz * 1e3;
    }
  }
  // timing events for the sweep launches of every level (two for a split level), created here rather than
  // inside the level loop, where their creation would hold up the host's enqueueing of short levels
  while ((int)ctx->ev.size() < 2 * (ctx->npending + 2 * max_levels)) {
    hipEvent_t e;
    TSA_HIP(ctx, hipEventCreate(&e));
    ctx->ev.push_back(e);
  }
  TSA_HIP(ctx, quiesce_track(ctx));
  // The fold and the selection of a level run beside the next level's sweep, on the snapshot the sweep
  // left: on the wide path with one workgroup per chain (a chain barrier, K > 1, needs all of the sweep's
  // workgroups resident at once, so nothing may take their place) and fewer chains than compute units (with
  // more, the fold's workgroups, which stage 64 KB of tables in LDS, take the places of sweep workgroups:
  // C4's sweep 265 -> 353 us; there a dense plan folds in the sweep launch itself and only the selection, one
  // wave per 256 chains, runs beside the next sweep), and on the one-wave kernels with fused energies.  The
  // fold and the selection are serial chains of dependent operations: beside a sweep they fill issue slots and
  // compute units the sweep leaves idle (its last round of workgroups, its waves' memory or LDS waits) instead
  // of adding their latency to every level.  Slice moves rewrite S, which the fold and the selection read from
  // the records, so they keep the serial order.
  const bool want_overlap =
      ctx->cfg.track_overlap >= 0 &&
      ((ctx->wide.on && ctx->wide.K == 1 && ctx->nchains < ctx->ncu) || wide_fold_snap(ctx) ||
       (!ctx->wide.on && ctx->cfg.fused_energy != 0 && !ctx->cfg.slicing));
  if (want_overlap && !ctx->st2) {
    TSA_HIP(ctx, hipStreamCreateWithFlags(&ctx->st2, hipStreamNonBlocking));
    for (int k = 0; k < TSA_SNAP_MAX; k++)
      TSA_HIP(ctx, hipEventCreateWithFlags(&ctx->ev_track[k], hipEventDisableTiming));
  }
  if (want_overlap && ensure_slots(ctx, 3) != TSA_OK) return TSA_ERR_HIP;
  ctx->overlap = want_overlap;
  ctx->slot = 0;
  ctx->track_kind = 0;
  ctx->lv_reset = true;
  ctx->lv_evaluated.assign((size_t)max_levels, 0);
  static_assert(sizeof(TsaTraceRowD) % 8 == 0, "trace rows are whole words");
  ctx->track_init_pending = true;
  ctx->tend_staged = false;
  return TSA_OK;
}

// The fold and the selection of the evaluated levels of one block of levels (tsa_anneal), on st2 beside the next
// block's sweeps: one fold launch for all of their snapshots (each level's energies into its own slot; with the
// block split over two launches, one fold per part, each after its own part, so that only the second part's fold
// follows the block's last sweep) and one selection launch that writes their trace rows and keeps the best in
// level order.
static int track_block(tsa_ctx* ctx, const int* slots, const int* levels, int n) {
  if (n == 0) return TSA_OK;
  ctx->track_kind = TRACK_LEVELS;
  ctx->tend_staged = false;
  TsaSelect S = ctx->sel;
  S.mode = ctx->mode;
  const tsa_layout_t& L = ctx->lay;
  TsaFoldLevels F{};
  TsaTrackLevels T{};
  F.n = T.n = n;
  for (int i = 0; i < n; i++) {
    const int s = slots[i];
    float* lc = reinterpret_cast<float*>(ctx->d_snap_en[s]);
    int* sc = reinterpret_cast<int*>(ctx->d_snap_en[s]) + ctx->nchains;
    int* ns = reinterpret_cast<int*>(ctx->d_snap_en[s]) + 2 * (size_t)ctx->nchains;
    F.cost[i] = ctx->d_snap_cost[s];
    F.z[i] = ctx->d_snap_nz[s];
    F.lc[i] = lc;
    F.sc[i] = sc;
    F.ns[i] = ns;
    T.lev[i] = levels[i];
    T.lc[i] = lc;
    T.sc[i] = sc;
    T.ns[i] = ns;
    T.ch[i] = ctx->d_snap_ch[s];
  }
  // (every slot of the block has the same sweep events)
  const int s0 = slots[0];
  TSA_HIP(ctx, hipStreamWaitEvent(ctx->st2, ctx->ev_sweep[s0], 0));
  if (ctx->split_slot[s0]) {
    const int h = split_point(ctx);
    TSA_HIP(ctx, tsa_launch_fold_levels(ctx->P, ctx->d_rec, ctx->d_leaf, ctx->d_fix, F, 0, h, ctx->st2));
    TSA_HIP(ctx, hipStreamWaitEvent(ctx->st2, ctx->ev_b[s0], 0));
    TSA_HIP(ctx, tsa_launch_fold_levels(ctx->P, ctx->d_rec, ctx->d_leaf, ctx->d_fix, F, h, ctx->nchains, ctx->st2));
  } else {
    TSA_HIP(ctx, tsa_launch_fold_levels(ctx->P, ctx->d_rec, ctx->d_leaf, ctx->d_fix, F, 0, ctx->nchains, ctx->st2));
  }
  TSA_HIP(ctx, tsa_launch_track_levels(T, ctx->nchains, S, ctx->d_rec, L.chain_words, L.ch_off, L.s_off, L.W, L.nint,
                                       ctx->d_track, ctx->d_trace, ctx->d_best, ctx->d_tpart, ctx->d_tdone, ctx->st2,
                                       false));
  const int sl = slots[n - 1];
  TSA_HIP(ctx, hipEventRecord(ctx->ev_track[sl], ctx->st2));
  for (int i = 0; i < n; i++) {
    ctx->track_pending[slots[i]] = true;
    ctx->track_ev[slots[i]] = sl;
  }
  ctx->last_track = sl;
  ctx->energy_fresh = false;
  return TSA_OK;
}

// The same for a block of levels on the wide path: one launch folds every evaluated level's node-cost
// snapshot into the slot's energies (the folds of the levels side by side: one level's is a serial lse chain
// of some 50 us on C5's trees), then one selection launch for them all.
static int track_wide_block(tsa_ctx* ctx, const int* slots, const int* levels, int n) {
  if (n == 0) return TSA_OK;
  ctx->track_kind = TRACK_LEVELS;
  ctx->tend_staged = false;
  TsaSelect S = ctx->sel;
  S.mode = ctx->mode;
  const tsa_layout_t& L = ctx->lay;
  TsaTrackLevels T{};
  TsaFoldLevels F{};
  T.n = F.n = n;
  TSA_HIP(ctx, hipStreamWaitEvent(ctx->st2, ctx->ev_sweep[slots[0]], 0));  // (one sweep launch for the block)
  for (int i = 0; i < n; i++) {
    const int s = slots[i];
    float* lc = reinterpret_cast<float*>(ctx->d_snap_en[s]);
    int* sc = reinterpret_cast<int*>(ctx->d_snap_en[s]) + ctx->nchains;
    int* ns = reinterpret_cast<int*>(ctx->d_snap_en[s]) + 2 * (size_t)ctx->nchains;
    F.cost[i] = ctx->d_snap_cost[s];
    F.z[i] = ctx->d_snap_nz[s];
    F.lc[i] = lc;
    F.sc[i] = sc;
    F.ns[i] = ns;
    T.lev[i] = levels[i];
    T.lc[i] = lc;
    T.sc[i] = sc;
    T.ns[i] = ns;
    T.ch[i] = ctx->d_snap_ch[s];
  }
  TSA_HIP(ctx, tsa_launch_wide_fold_levels(ctx->wide, ctx->mode, ctx->P, ctx->d_rec, ctx->d_leaf, ctx->d_fix,
                                           ctx->nchains, F, ctx->st2));
  TSA_HIP(ctx, tsa_launch_track_levels(T, ctx->nchains, S, ctx->d_rec, L.chain_words, L.ch_off, L.s_off, L.W, L.nint,
                                       ctx->d_track, ctx->d_trace, ctx->d_best, ctx->d_tpart, ctx->d_tdone, ctx->st2,
                                       false));
  const int sl = slots[n - 1];
  TSA_HIP(ctx, hipEventRecord(ctx->ev_track[sl], ctx->st2));
  for (int i = 0; i < n; i++) {
    ctx->track_pending[slots[i]] = true;
    ctx->track_ev[slots[i]] = sl;
  }
  ctx->last_track = sl;
  ctx->energy_fresh = false;
  return TSA_OK;
}

extern "C" int tsa_track(tsa_ctx* ctx, int32_t level) {
  if (!ctx) return fail(ctx, TSA_ERR_ARG, "tsa_track: null context");
  if (ctx->track_levels == 0) return fail(ctx, TSA_ERR_ARG, "tsa_track: no tsa_track_begin");
  TSA_HIP(ctx, flush_track_init(ctx));
  TSA_HIP(ctx, flush_resample(ctx));
  if (level < 0 || level >= ctx->track_levels) return fail(ctx, TSA_ERR_ARG, "tsa_track: level out of range");
  if (ctx->track_kind == TRACK_ANNEAL)
    return fail(ctx, TSA_ERR_ARG, "tsa_track: this tracking session runs its levels with tsa_anneal");
  ctx->track_kind = TRACK_LEVELS;
  ctx->tend_staged = false;
  TsaSelect S = ctx->sel;
  S.mode = ctx->mode;
  const tsa_layout_t& L = ctx->lay;
  if (ctx->overlap && ctx->last_slot >= 0) {
    // the last sweep's snapshot: fold its node costs and select on st2, beside the next sweep on st
    const int s = ctx->last_slot;
    TSA_HIP(ctx, hipStreamWaitEvent(ctx->st2, ctx->ev_sweep[s], 0));
    if (ctx->split_slot[s]) TSA_HIP(ctx, hipStreamWaitEvent(ctx->st2, ctx->ev_b[s], 0));
    const int kind = ctx->snap_kind[s];
    if (kind == SNAP_WIDE)
      TSA_HIP(ctx, tsa_launch_wide_energy(ctx->wide, ctx->mode, ctx->P, ctx->d_rec, ctx->d_leaf, ctx->d_fix,
                                          ctx->nchains, ctx->d_snap_cost[s], ctx->d_snap_nz[s], ctx->d_fcnt,
                                          ctx->d_lc, ctx->d_sc, ctx->d_ns, 0, ctx->st2));
    else if (kind == SNAP_COSTS)
      TSA_HIP(ctx, tsa_launch_fold(ctx->P, ctx->d_rec, ctx->d_leaf, ctx->d_fix, ctx->d_snap_cost[s],
                                   ctx->d_snap_nz[s], ctx->nchains, ctx->d_lc, ctx->d_sc, ctx->d_ns, ctx->st2));
    const bool folded = kind == SNAP_ENERGIES;  // the sweep kernel left the energies in the slot
    const float* lc = folded ? reinterpret_cast<const float*>(ctx->d_snap_en[s]) : ctx->d_lc;
    const int* sc = folded ? reinterpret_cast<const int*>(ctx->d_snap_en[s]) + ctx->nchains : ctx->d_sc;
    const int* ns = folded ? reinterpret_cast<const int*>(ctx->d_snap_en[s]) + 2 * (size_t)ctx->nchains : ctx->d_ns;
    TSA_HIP(ctx, tsa_launch_track(lc, sc, ns, ctx->nchains, S, level, ctx->d_rec,
                                  L.chain_words, L.ch_off, L.s_off, L.W, L.nint, ctx->d_snap_ch[s], ctx->d_track,
                                  ctx->d_trace, ctx->d_best, ctx->d_tpart, ctx->d_tdone, ctx->st2, false));
    TSA_HIP(ctx, hipEventRecord(ctx->ev_track[s], ctx->st2));
    ctx->track_ev[s] = s;
    ctx->track_pending[s] = true;
    ctx->last_track = s;
    ctx->energy_fresh = false;  // d_lc / d_sc / d_ns now hold the snapshot's energies
    return TSA_OK;
  }
  TSA_HIP(ctx, join_split(ctx));
  TSA_HIP(ctx, launch_energy(ctx));  // (orders st after any selection pending on st2)
  TSA_HIP(ctx, tsa_launch_track(ctx->d_lc, ctx->d_sc, ctx->d_ns, ctx->nchains, S, level, ctx->d_rec, L.chain_words,
                                L.ch_off, L.s_off, L.W, L.nint, nullptr, ctx->d_track, ctx->d_trace, ctx->d_best,
                                ctx->d_tpart, ctx->d_tdone, ctx->st, true));
  return TSA_OK;
}

extern "C" int tsa_track_end(tsa_ctx* ctx, int32_t* best_chain, int32_t* best_level, double* best_score,
                             uint64_t* best_record, tsa_trace_row_t* rows, uint64_t* ticks0, double* tick_hz) {
  if (!ctx || !best_chain || !best_level || !best_score || !best_record || !rows || !ticks0 || !tick_hz)
    return fail(ctx, TSA_ERR_ARG, "tsa_track_end: null argument");
  TSA_HIP(ctx, join_split(ctx));
  TSA_HIP(ctx, flush_track_init(ctx));
  TSA_HIP(ctx, flush_resample(ctx));
  if (ctx->track_levels == 0) return fail(ctx, TSA_ERR_ARG, "tsa_track_end: no tsa_track_begin");
  static_assert(sizeof(TsaTraceRowD) == sizeof(tsa_trace_row_t), "trace row layout");
  TsaTrackState h;
  unsigned long long t0 = 0;
  // The results are written by the selections on st2 when they run there (the wide path's error word, which
  // its sweeps write, aside): then the results' launch follows them on st2 and the host waits for both
  // streams, instead of a wait of st for st2 in the queue (about 10 us on the device)
  const bool on2 = ctx->st2 && !ctx->wide.on && ctx->d_tend &&
                   ((ctx->last_track >= 0 && ctx->track_pending[ctx->last_track]) || ctx->tinit_pending);
  hipStream_t so = on2 ? ctx->st2 : ctx->st;
  if (!on2) join_track(ctx);
  // every copy into the pinned staging buffer, one wait, then the caller's buffers from there
  const tsa_layout_t& L = ctx->lay;
  const TendLayout tl = tend_layout(ctx);
  const size_t cwb = tl.tree_bytes, rowb = tl.row_bytes;
  char* const hs = ctx->h_tend;
  char* const h_state = hs + tl.st;
  char* const h_t0 = hs + tl.t0;
  char* const h_werr = hs + tl.werr;
  char* const h_tree = hs + tl.tree;
  char* const h_rows = hs + tl.rows;
  // the best chain's tree: children words and S (the label words of best_record are not written)
  static_assert(sizeof(TsaTrackState) % 8 == 0, "the tracking state is whole words");
  uint32_t werr = 0;
  if (ctx->tend_staged && ctx->d_tend) {
    // the last level-loop launch's selection of the best wrote them (behind it on st)
  } else if (ctx->d_tend) {
    // one launch writes them all into the mapped staging buffer (four or five copies cost about 5 us each)
    char* const d = ctx->d_tend;
    TSA_HIP(ctx, tsa_launch_track_out(
                     reinterpret_cast<const unsigned long long*>(ctx->d_track), (int)(sizeof h / 8), ctx->d_ticks0,
                     reinterpret_cast<const unsigned long long*>(ctx->d_best + L.ch_off), (int)(cwb / 8),
                     reinterpret_cast<const unsigned long long*>(ctx->d_trace), (int)(rowb / 8),
                     ctx->wide.on ? ctx->wsync.err : nullptr, reinterpret_cast<unsigned long long*>(d + (h_state - hs)),
                     reinterpret_cast<unsigned long long*>(d + (h_t0 - hs)),
                     reinterpret_cast<unsigned long long*>(d + (h_tree - hs)),
                     reinterpret_cast<unsigned long long*>(d + (h_rows - hs)),
                     reinterpret_cast<unsigned*>(d + (h_werr - hs)), so));
  } else {
    TSA_HIP(ctx, hipMemcpyAsync(h_state, ctx->d_track, sizeof h, hipMemcpyDeviceToHost, ctx->st));
    TSA_HIP(ctx, hipMemcpyAsync(h_t0, ctx->d_ticks0, sizeof t0, hipMemcpyDeviceToHost, ctx->st));
    TSA_HIP(ctx, hipMemcpyAsync(h_tree, ctx->d_best + L.ch_off, cwb, hipMemcpyDeviceToHost, ctx->st));
    TSA_HIP(ctx, hipMemcpyAsync(h_rows, ctx->d_trace, rowb, hipMemcpyDeviceToHost, ctx->st));
    if (ctx->wide.on) TSA_HIP(ctx, hipMemcpyAsync(h_werr, ctx->wsync.err, 4, hipMemcpyDeviceToHost, ctx->st));
  }
  // (st first: its sweeps ended before the selections on st2 that follow them, so its wait -- the wait for
  // the join of the third stream included -- passes while st2 still runs, instead of after it)
  TSA_HIP(ctx, hipStreamSynchronize(ctx->st));
  if (on2) TSA_HIP(ctx, hipStreamSynchronize(ctx->st2));
  ctx->host_waited = true;
  ctx->tend_staged = false;
  std::memcpy(&h, h_state, sizeof h);
  std::memcpy(&t0, h_t0, sizeof t0);
  std::memcpy(best_record + L.ch_off, h_tree, cwb);
  std::memcpy(rows, h_rows, rowb);
  if (ctx->wide.on) std::memcpy(&werr, h_werr, 4);
  TSA_HIP(ctx, quiesce_track(ctx));
  if (wide_error(ctx, werr) != TSA_OK) return TSA_ERR_HIP;
  if (ctx->track_kind == TRACK_ANNEAL) {
    // the device kept the best after each level-loop launch (the lowest score over the evaluated levels' rows,
    // the first level on ties) and copied that chain's kept tree; the rows must agree
    double s = INFINITY;
    int bc = -1, bl = -1;
    for (int l = 0; l < ctx->track_levels; l++)
      if (ctx->lv_evaluated[l] && rows[l].chain >= 0 && rows[l].score < s) {
        s = rows[l].score;
        bc = rows[l].chain;
        bl = l;
      }
    if (bc != h.best_chain || bl != h.best_level || (bc >= 0 && s != h.best_score))
      return fail(ctx, TSA_ERR_HIP, "tsa_track_end: the level loop's best disagrees with its trace rows");
  }
  *best_chain = h.best_chain;
  *best_level = h.best_level;
  *best_score = h.best_score;
  *ticks0 = t0;
  *tick_hz = ctx->tick_hz;
  return TSA_OK;
}

// Grow the level loop's buffers to nlev levels with nev evaluated ones (the sizes only grow).
static int levels_alloc(tsa_ctx* ctx, int nlev, int nev) {
  const int n = ctx->nchains, ng = (n + 255) / 256;
  const tsa_layout_t& L = ctx->lay;
  if (!ctx->d_cand) {
    const size_t cw = (size_t)(L.s_off + L.W - L.ch_off);
    TSA_HIP(ctx, hipMalloc(&ctx->d_cand, 2 * (size_t)n * cw * 8));
    TSA_HIP(ctx, hipMalloc(&ctx->d_own, (size_t)n * 8));
    TSA_HIP(ctx, hipMalloc(&ctx->d_bslot, (size_t)n * 4));
    for (hipEvent_t& e : ctx->ev_lv) TSA_HIP(ctx, hipEventCreateWithFlags(&e, hipEventDisableTiming));
  }
  if (nlev > ctx->lv_cap_levels) {
    for (int k = 0; k < 2; k++) {
      if (ctx->lv_pending[k]) TSA_HIP(ctx, hipEventSynchronize(ctx->ev_lv[k]));
      ctx->lv_pending[k] = false;
    }
    if (ctx->d_lv) TSA_HIP(ctx, hipFree(ctx->d_lv));
    if (ctx->h_lv) TSA_HIP(ctx, hipHostFree(ctx->h_lv));
    ctx->d_lv = nullptr;
    ctx->h_lv = nullptr;
    ctx->d_hlv = nullptr;
    TSA_HIP(ctx, hipMalloc(&ctx->d_lv, (size_t)nlev * 3 * 4));
    ctx->lv_tab.clear();
    TSA_HIP(ctx, hipHostMalloc(&ctx->h_lv, 2 * (size_t)nlev * 3 * 4, hipHostMallocDefault));
    if (hipHostGetDevicePointer(reinterpret_cast<void**>(&ctx->d_hlv), ctx->h_lv, 0) != hipSuccess) {
      (void)hipGetLastError();  // not mapped: the table goes by a copy
      ctx->d_hlv = nullptr;
    }
    ctx->lv_cap_levels = nlev;
  }
  if (nev > ctx->lv_cap_evals) {
    TSA_HIP(ctx, hipStreamSynchronize(ctx->st));  // a running level loop may still use the old buffers
    if (ctx->d_lv_en) TSA_HIP(ctx, hipFree(ctx->d_lv_en));
    if (ctx->d_lv_cnt) TSA_HIP(ctx, hipFree(ctx->d_lv_cnt));
    if (ctx->d_lv_part) TSA_HIP(ctx, hipFree(ctx->d_lv_part));
    ctx->d_lv_en = nullptr;
    ctx->d_lv_cnt = nullptr;
    ctx->d_lv_part = nullptr;
    TSA_HIP(ctx, hipMalloc(&ctx->d_lv_en, (size_t)nev * n * 3 * 4));
    TSA_HIP(ctx, hipMalloc(&ctx->d_lv_cnt, ((size_t)nev * (ng + 1) + 1) / 2 * 8));  // cleared as 64-bit words
    ctx->lv_cnt_fresh = true;
    TSA_HIP(ctx, hipMalloc(&ctx->d_lv_part, (size_t)nev * ng * sizeof(TsaTrackPart)));
    ctx->lv_cap_evals = nev;
  }
  return TSA_OK;
}

extern "C" int tsa_anneal(tsa_ctx* ctx, int32_t order, int32_t level0, int32_t nlevels, const float* betas,
                          const int32_t* niters, const uint8_t* evaluated, uint32_t sweep0) {
  if (!ctx) return fail(ctx, TSA_ERR_ARG, "tsa_anneal: null context");
  TSA_HIP(ctx, join_split(ctx));
  TSA_HIP(ctx, flush_resample(ctx));
  if (order != TSA_ORDER_PAR && order != TSA_ORDER_PREORDER) return fail(ctx, TSA_ERR_ARG, "--order par|preorder");
  if (!betas || !niters || !evaluated || nlevels < 1) return fail(ctx, TSA_ERR_ARG, "tsa_anneal: no levels");
  if (ctx->track_levels == 0) return fail(ctx, TSA_ERR_ARG, "tsa_anneal: no tsa_track_begin");
  if (level0 < 0 || nlevels > ctx->track_levels - level0)
    return fail(ctx, TSA_ERR_ARG, "tsa_anneal: levels beyond tsa_track_begin's max_levels");
  long long total = 0;
  int nev = 0;
  for (int l = 0; l < nlevels; l++) {
    if (niters[l] < 1) return fail(ctx, TSA_ERR_ARG, "tsa_anneal: a level with no sweep");
    total += niters[l];
    nev += evaluated[l] != 0;
  }
  if (total > INT32_MAX) return fail(ctx, TSA_ERR_ARG, "tsa_anneal: more than 2^31 - 1 sweeps in one call");
  // One launch for the whole call when the context's kernels run the level loop (the LDS kernels), it is not
  // turned off, and either it is asked for or every chain of it is resident at once: with more chains than
  // that, a chain resident only after others have run all their levels would leave the per-level launches'
  // fold of every chain in one round and their occupancy for nothing.  A session that began with one kind
  // stays with it (the best is tracked per chain by the level loop, per level by tsa_track).
  bool loop = ctx->track_kind == TRACK_ANNEAL;
  if (ctx->track_kind == 0 && !ctx->wide.on && ctx->L.lds && ctx->cfg.level_loop >= 0) {
    loop = ctx->cfg.level_loop > 0;
    if (!loop) {
      int& r = ctx->lv_resident[ctx->mode * 2 + order];
      if (r < 0) {
        TsaLevels q{};
        const TsaEnergyOut eo{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
        TSA_HIP(ctx, tsa_launch_sweeps(ctx->L, ctx->mode, order, ctx->P, ctx->d_rec, ctx->d_leaf, ctx->d_fix,
                                       ctx->nchains, 0.0f, 0u, 0, ctx->d_stats, eo, ctx->st, nullptr, nullptr, &q, &r));
      }
      loop = (long long)r * ctx->ncu >= ctx->nchains;
    }
  }
  ctx->lv_used = loop ? 1 : 0;
  // (a pending session start: the first sweeps enqueue it, or the level loop's set-up launch does it)
  // Several levels per sweep launch (the one-wave LDS kernels with the overlapped selection and the fold apart,
  // where the population is more than twice what the device holds at once): a launch ends with a tail in which
  // fewer and fewer chains are left to run, and a level of one sweep per chain is short next to it; a block of
  // levels has one tail for all of them.  Each evaluated level of a block leaves its snapshot in a slot of its
  // own, whose fold and selection tsa_track runs as for one level.
  if (ctx->cfg.level_blocks < 0 || ctx->cfg.level_blocks > TSA_BLOCK_MAX)
    return fail(ctx, TSA_ERR_ARG, "tsa_config_t.level_blocks: 0 (automatic) or 1..8");
  const int K = ctx->cfg.level_blocks > 0 ? ctx->cfg.level_blocks : TSA_BLOCK_MAX;
  const bool wide_blocks = !loop && K > 1 && wide_blocks_ok(ctx, order);
  if (wide_blocks || (!loop && K > 1 && ctx->overlap && !ctx->wide.on && ctx->L.lds && ctx->cfg.fused_energy != 0 &&
                      ctx->fold_apart && !ctx->cfg.slicing && order == TSA_ORDER_PAR)) {
    ctx->lv_used = 2;
    ctx->blocks_k = K;
    if (ensure_slots(ctx, 3 * K) != TSA_OK) return TSA_ERR_HIP;
    uint32_t sw = sweep0;
    for (int l = 0; l < nlevels; l += K) {
      TsaBlock blk{};
      uint8_t bev[TSA_BLOCK_MAX];
      int slots[TSA_BLOCK_MAX];
      blk.n = nlevels - l < K ? nlevels - l : K;
      for (int i = 0; i < blk.n; i++) {
        blk.beta[i] = betas[l + i];
        blk.niters[i] = niters[l + i];
        blk.total += niters[l + i];
        bev[i] = evaluated[l + i] != 0;
      }
      int rc = sweeps_impl(ctx, order, blk.beta[0], sw, blk.total, &blk, bev, slots);
      if (rc != TSA_OK) return rc;
      sw += (uint32_t)blk.total;
      int es[TSA_BLOCK_MAX], el[TSA_BLOCK_MAX], ne = 0;
      for (int i = 0; i < blk.n; i++) {
        if (slots[i] < 0) continue;
        es[ne] = slots[i];
        el[ne++] = level0 + l + i;
      }
      rc = wide_blocks ? track_wide_block(ctx, es, el, ne) : track_block(ctx, es, el, ne);
      if (rc != TSA_OK) return rc;
    }
    return TSA_OK;
  }
  if (!loop) {  // one sweep launch per level, a selection at each evaluated one
    uint32_t sw = sweep0;
    for (int l = 0; l < nlevels; l++) {
      int rc = tsa_sweeps(ctx, order, betas[l], sw, niters[l]);
      sw += (uint32_t)niters[l];
      if (rc == TSA_OK && evaluated[l]) rc = tsa_track(ctx, level0 + l);
      if (rc != TSA_OK) return rc;
    }
    return TSA_OK;
  }
  if (levels_alloc(ctx, nlevels, nev > 0 ? nev : 1) != TSA_OK) return TSA_ERR_HIP;
  ctx->track_kind = TRACK_ANNEAL;
  const int n = ctx->nchains, ng = (n + 255) / 256;
  // the schedule, through the half of the pinned staging that the call before the previous one read
  const int half = ctx->lv_half;
  ctx->lv_half ^= 1;
  if (ctx->lv_pending[half]) TSA_HIP(ctx, hipEventSynchronize(ctx->ev_lv[half]));
  ctx->lv_pending[half] = false;
  const size_t hoff = (size_t)half * 3 * ctx->lv_cap_levels;
  int* h = ctx->h_lv + hoff;
  for (int l = 0, e = 0; l < nlevels; l++) {
    memcpy(&h[l], &betas[l], 4);
    h[nlevels + l] = niters[l];
    h[2 * nlevels + l] = evaluated[l] ? e++ : -1;
    if (evaluated[l]) ctx->lv_evaluated[level0 + l] = 1;
  }
  join_track(ctx);
  ctx->last_slot = -1;
  ctx->energy_fresh = ctx->energy_host = false;
  ctx->costs_valid = ctx->sums_valid = false;
  // The session's start (when this is its first call) and the chains' best reset are made by the level-loop
  // kernel itself; a set-up launch copies the table from the pinned staging when d_lv does not hold it already
  // (the previous call's table) and zeroes freshly allocated arrival counters (every launch leaves them at zero)
  const bool tinit = ctx->track_init_pending, reset = ctx->lv_reset;
  ctx->track_init_pending = false;
  ctx->lv_reset = false;
  TsaAnnealInit A{};
  const bool same_tab = ctx->lv_tab.size() == (size_t)3 * nlevels &&
                        std::memcmp(ctx->lv_tab.data(), h, (size_t)3 * nlevels * 4) == 0;
  if (!same_tab) {
    if (ctx->d_hlv) {
      A.tab_src = ctx->d_hlv + hoff;
      A.tab_dst = ctx->d_lv;
      A.tab_words = 3 * nlevels;
    } else {
      TSA_HIP(ctx, hipMemcpyAsync(ctx->d_lv, h, (size_t)nlevels * 3 * 4, hipMemcpyHostToDevice, ctx->st));
    }
    ctx->lv_tab.assign(h, h + 3 * (size_t)nlevels);
  }
  if (ctx->lv_cnt_fresh) {
    const size_t cnt_words = (size_t)ctx->lv_cap_evals * (ng + 1);
    A.cnt = reinterpret_cast<unsigned long long*>(ctx->d_lv_cnt);
    A.cnt_words = (int)((cnt_words + 1) / 2);
    ctx->lv_cnt_fresh = false;
  }
  if (A.tab_src || A.cnt) TSA_HIP(ctx, tsa_launch_anneal_init(A, ctx->st));
  while ((int)ctx->ev.size() < 2 * (ctx->npending + 1)) {
    hipEvent_t e;
    TSA_HIP(ctx, hipEventCreate(&e));
    ctx->ev.push_back(e);
  }
  hipEvent_t e0 = ctx->ev[2 * ctx->npending], e1 = ctx->ev[2 * ctx->npending + 1];
  // the timing events as markers around a plain dispatch, which costs the host less time before the kernel
  // starts than events recorded by the dispatch (about 6 against 20 us); a launch of whole levels is long
  // next to the gap a marker may leave before the kernel
  const bool markers = true;
  ctx->host_waited = false;
  TsaLevels lv{};
  lv.beta = reinterpret_cast<const float*>(ctx->d_lv);
  lv.niters = ctx->d_lv + nlevels;
  lv.eval = ctx->d_lv + 2 * nlevels;
  lv.nlev = nlevels;
  lv.total = (int)total;
  lv.level0 = level0;
  lv.en_lc = reinterpret_cast<float*>(ctx->d_lv_en);
  lv.en_sc = reinterpret_cast<int*>(ctx->d_lv_en) + (size_t)ctx->lv_cap_evals * n;
  lv.en_ns = reinterpret_cast<int*>(ctx->d_lv_en) + 2 * (size_t)ctx->lv_cap_evals * n;
  lv.cnt = ctx->d_lv_cnt;
  lv.part = ctx->d_lv_part;
  lv.cand = ctx->d_cand;
  lv.cand_words = ctx->lay.s_off + ctx->lay.W - ctx->lay.ch_off;
  lv.own = ctx->d_own;
  lv.bslot = ctx->d_bslot;
  lv.trace = ctx->d_trace;
  lv.S = ctx->sel;
  lv.S.mode = ctx->mode;
  lv.reset = reset ? 1 : 0;
  if (tinit) {
    lv.tinit = ctx->d_track;
    lv.ticks0 = ctx->d_ticks0;
    lv.trace_words = (int)((size_t)ctx->track_levels * sizeof(TsaTraceRowD) / 8);
    lv.best = ctx->d_best;
    lv.best_words = ctx->lay.chain_words;
  }
  const TsaEnergyOut eo{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
  if (markers) TSA_HIP(ctx, hipEventRecord(e0, ctx->st));
  TSA_HIP(ctx, tsa_launch_sweeps(ctx->L, ctx->mode, order, ctx->P, ctx->d_rec, ctx->d_leaf, ctx->d_fix, n, 0.0f,
                                 sweep0, 0, ctx->d_stats, eo, ctx->st, markers ? nullptr : e0,
                                 markers ? nullptr : e1, &lv));
  if (markers) TSA_HIP(ctx, hipEventRecord(e1, ctx->st));
  ctx->npending++;
  // the session's best over the launch's levels and its tree, on the device (tsa_track_end then copies it with
  // the trace rows instead of asking for the chain's kept tree after reading them)
  if (nev > 0) {
    // (and the session's results into the staging buffer, so that tsa_track_end only waits)
    TsaTrackOut O{};
    if (ctx->d_tend) {
      const TendLayout tl = tend_layout(ctx);
      O.h_st = reinterpret_cast<unsigned long long*>(ctx->d_tend + tl.st);
      O.h_t0 = reinterpret_cast<unsigned long long*>(ctx->d_tend + tl.t0);
      O.h_tree = reinterpret_cast<unsigned long long*>(ctx->d_tend + tl.tree);
      O.h_rows = reinterpret_cast<unsigned long long*>(ctx->d_tend + tl.rows);
      O.ticks0 = ctx->d_ticks0;
      O.row_words = (int)(tl.row_bytes / 8);
    }
    TSA_HIP(ctx, tsa_launch_level_best(lv, n, ctx->d_track, ctx->d_best, ctx->lay.ch_off, O, ctx->st));
    ctx->tend_staged = ctx->d_tend != nullptr;
  }
  TSA_HIP(ctx, hipEventRecord(ctx->ev_lv[half], ctx->st));
  ctx->lv_pending[half] = true;
  return TSA_OK;
}

extern "C" int tsa_energy(tsa_ctx* ctx, float* lc, int32_t* sc, int32_t* ns) {
  if (!ctx || !lc || !sc || !ns) return fail(ctx, TSA_ERR_ARG, "tsa_energy: null argument");
  TSA_HIP(ctx, join_split(ctx));
  TSA_HIP(ctx, flush_track_init(ctx));
  TSA_HIP(ctx, flush_resample(ctx));
  const size_t b = (size_t)ctx->nchains * 4;
  if (ctx->energy_host) {  // the last sweep launch wrote them into h_en
    TSA_HIP(ctx, hipStreamSynchronize(ctx->st));
  } else {
    TSA_HIP(ctx, launch_energy(ctx));
    TSA_HIP(ctx, hipMemcpyAsync(ctx->h_en, ctx->d_lc, 3 * b + 4, hipMemcpyDeviceToHost, ctx->st));
    TSA_HIP(ctx, hipStreamSynchronize(ctx->st));
  }
  if (ctx->wide.on && wide_error(ctx, ctx->h_en[3 * (size_t)ctx->nchains]) != TSA_OK) return TSA_ERR_HIP;
  memcpy(lc, ctx->h_en, b);
  memcpy(sc, ctx->h_en + ctx->nchains, b);
  memcpy(ns, ctx->h_en + 2 * (size_t)ctx->nchains, b);
  ctx->host_waited = true;
  return TSA_OK;
}

extern "C" int tsa_resample(tsa_ctx* ctx, const int32_t* anc) {
  if (!ctx || !anc) return fail(ctx, TSA_ERR_ARG, "tsa_resample: null argument");
  TSA_HIP(ctx, join_split(ctx));
  TSA_HIP(ctx, flush_track_init(ctx));
  TSA_HIP(ctx, flush_resample(ctx));  // (the previous one, if not made yet)
  for (int c = 0; c < ctx->nchains; c++)
    if (anc[c] < 0 || anc[c] >= ctx->nchains) return fail(ctx, TSA_ERR_ARG, "tsa_resample: ancestor out of range");
  if (!ctx->d_rec2) TSA_HIP(ctx, hipMalloc(&ctx->d_rec2, (size_t)ctx->nchains * ctx->lay.chain_words * 8));
  TSA_HIP(ctx, quiesce_track(ctx));
  // the ancestors go through the pinned staging buffer, which the kernels read where it is mapped (else an
  // asynchronous copy to d_anc); the last launch that read it must be done before it is overwritten
  if (ctx->anc_pending) TSA_HIP(ctx, hipEventSynchronize(ctx->ev_anc));
  ctx->anc_pending = false;
  memcpy(ctx->h_anc, anc, (size_t)ctx->nchains * 4);
  if (!ctx->d_hanc)
    TSA_HIP(ctx, hipMemcpyAsync(ctx->d_anc, ctx->h_anc, (size_t)ctx->nchains * 4, hipMemcpyHostToDevice, ctx->st));
  ctx->costs_valid = false;
  ctx->energy_fresh = ctx->energy_host = false;
  ctx->sums_valid = false;
  // the copy itself is left to the next sweep launch (its kernel stages each chain from its ancestor's record)
  // or to the next other call (flush_resample), in stream order: no wait here
  ctx->anc_pend = true;
  return TSA_OK;
}

extern "C" int tsa_set_mode(tsa_ctx* ctx, int32_t mode) {
  if (!ctx) return fail(ctx, TSA_ERR_ARG, "tsa_set_mode: null context");
  TSA_HIP(ctx, join_split(ctx));
  TSA_HIP(ctx, flush_track_init(ctx));
  TSA_HIP(ctx, flush_resample(ctx));
  if (mode < 0 || mode > 2) return fail(ctx, TSA_ERR_ARG, "tsa_set_mode: mode must be 0, 1 or 2");
  if (mode != ctx->mode) {
    TSA_HIP(ctx, quiesce_track(ctx));
    ctx->costs_valid = ctx->energy_fresh = ctx->energy_host = false;
  }
  ctx->mode = mode;
  return TSA_OK;
}

extern "C" int tsa_stats(tsa_ctx* ctx, uint64_t out[7]) {
  if (!ctx || !out) return fail(ctx, TSA_ERR_ARG, "tsa_stats: null argument");
  TSA_HIP(ctx, join_split(ctx));
  TSA_HIP(ctx, flush_track_init(ctx));
  unsigned long long s[TSA_NSTAT * TSA_STAT_SLOTS];
  TSA_HIP(ctx, hipMemcpyAsync(s, ctx->d_stats, sizeof s, hipMemcpyDeviceToHost, ctx->st));
  TSA_HIP(ctx, hipStreamSynchronize(ctx->st));
  for (int i = 0; i < TSA_NSTAT; i++) {
    out[i] = 0;
    for (int k = 0; k < TSA_STAT_SLOTS; k++) out[i] += s[i * TSA_STAT_SLOTS + k];
  }
  return TSA_OK;
}

extern "C" int tsa_chunk_stats(tsa_ctx* ctx, uint64_t out[2]) {
  if (!ctx || !out) return fail(ctx, TSA_ERR_ARG, "tsa_chunk_stats: null argument");
  TSA_HIP(ctx, join_split(ctx));
  TSA_HIP(ctx, flush_track_init(ctx));
  unsigned long long s[2 * TSA_STAT_SLOTS];
  TSA_HIP(ctx, hipMemcpyAsync(s, ctx->d_stats + TSA_ST_CHUNKS * TSA_STAT_SLOTS, sizeof s, hipMemcpyDeviceToHost,
                              ctx->st));
  TSA_HIP(ctx, hipStreamSynchronize(ctx->st));
  for (int i = 0; i < 2; i++) {
    out[i] = 0;
    for (int k = 0; k < TSA_STAT_SLOTS; k++) out[i] += s[i * TSA_STAT_SLOTS + k];
  }
  return TSA_OK;
}

extern "C" int tsa_describe(tsa_ctx* ctx, char* buf, int32_t len) {
  if (!ctx || !buf || len < 1) return fail(ctx, TSA_ERR_ARG, "tsa_describe: null argument");
  char sp[48] = "";
  if (ctx->split_levels > 0) snprintf(sp, sizeof sp, " split_levels=%lld", ctx->split_levels);
  char an[40] = "";
  if (ctx->lv_used == 2) snprintf(an, sizeof an, " anneal=level_blocks%d", ctx->blocks_k);
  else if (ctx->lv_used >= 0) snprintf(an, sizeof an, "%s", ctx->lv_used ? " anneal=level_loop" : " anneal=level_launches");
  snprintf(buf, (size_t)len, "%s%s%s", ctx->kname.c_str(), sp, an);
  return TSA_OK;
}

extern "C" int tsa_destroy(tsa_ctx* ctx) {
  if (!ctx) return TSA_OK;
  free_ctx(ctx);  // (waits for every stream of the context first)
  return TSA_OK;
}

extern "C" const char* tsa_last_error(const tsa_ctx* ctx) { return ctx ? ctx->err.c_str() : g_err.c_str(); }

extern "C" void* tsa_host_alloc(size_t bytes) {
  void* p = nullptr;
  if (hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocDefault) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  return p;
}

extern "C" void tsa_host_free(void* p) {
  if (p) (void)hipHostFree(p);
}

extern "C" float tsa_host_math(int32_t which, float x) {
  if (which == 0) return tsa_expf(x);
  if (which == 1) return tsa_exp2f(x);
  std::call_once(g_fix_once, build_log2_fix);
  const TsaMathTabs T{tsa_exp2_tab_h, g_fix.data(), g_fix.data() + TSA_LOG2FIX_WORDS, tsa_log2_tab_h};
  return tsa_log2f_12(x, T);
}

// ---------------------------------------------------------------------------------------------------
// The allocation-free entry point: sweeps (and energies) of a population the caller holds in device memory
// ---------------------------------------------------------------------------------------------------
// Scratch of tsa_sweeps_noalloc: the statistic counters (TSA_NSTAT_ALL x TSA_STAT_SLOTS words), then the node
// costs (float) and masked sizes (uint16) the sweep kernel leaves for the fold kernel, nint4 per chain each.
// Every GPU the library runs on holds its own copy until the process ends; every call on a GPU shares it.
#define TSA_SCRATCH_BYTES (32u << 20)
static __device__ __align__(256) unsigned char scratch[TSA_SCRATCH_BYTES];
// The log2f correction table and its summary bitmap (what tsa_create copies into every context), filled once
// per device by the first call there.
static __device__ __align__(256) uint32_t log2_fix_table[TSA_LOG2FIX_WORDS + TSA_LOG2MAP_WORDS];

namespace {
struct StaticDevice {
  bool ready = false;
  unsigned char* scratch = nullptr;  // device address of `scratch` on this device
  uint32_t* fix = nullptr;           // device address of `log2_fix_table` on this device
  int lds_max = 0, ncu = 0;
};
constexpr int kMaxDevices = 64;
StaticDevice g_static[kMaxDevices];
std::mutex g_static_mu;
constexpr size_t kCounterBytes = ((size_t)TSA_NSTAT_ALL * TSA_STAT_SLOTS * 8 + 255) & ~(size_t)255;
}  // namespace

// First call on the current device: the device addresses of the two static arrays (the arrays' names are
// host-side stand-ins, never passed to a kernel), the correction table copied in, the device's LDS and
// compute-unit counts.
static int static_device(StaticDevice** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(nullptr, TSA_ERR_HIP, std::string("no HIP device: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(nullptr, TSA_ERR_ARG, "tsa_sweeps_noalloc: device index too large");
  std::lock_guard<std::mutex> g(g_static_mu);
  StaticDevice& d = g_static[dev];
  if (!d.ready) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return fail(nullptr, TSA_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    void* f = nullptr;
    e = hipGetSymbolAddress(&f, HIP_SYMBOL(log2_fix_table));
    if (e != hipSuccess)
      return fail(nullptr, TSA_ERR_HIP, std::string("hipGetSymbolAddress(log2_fix_table): ") + hipGetErrorString(e));
    static_assert(sizeof(log2_fix_table) == (TSA_LOG2FIX_WORDS + TSA_LOG2MAP_WORDS) * 4, "table size");
    if (g_fix.size() * 4 != sizeof(log2_fix_table)) return fail(nullptr, TSA_ERR_ARG, "log2f table size");
    e = hipMemcpy(f, g_fix.data(), g_fix.size() * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&d.lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&d.ncu, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return fail(nullptr, TSA_ERR_HIP, std::string("tsa_sweeps_noalloc set-up: ") + hipGetErrorString(e));
    d.scratch = static_cast<unsigned char*>(p);
    d.fix = static_cast<uint32_t*>(f);
    d.ready = true;
  }
  *out = &d;
  return TSA_OK;
}

extern "C" int tsa_sweeps_noalloc(const tsa_layout_t* lay, const tsa_config_t* cfg, int32_t leaf_sc,
                                  const uint64_t* leaf_dev, uint64_t* population_dev, int32_t nchains, int32_t order,
                                  float beta, uint32_t sweep0, int32_t nsweeps, float* lc_dev, int32_t* sc_dev,
                                  int32_t* ns_dev, uint64_t* stats_dev, void* stream) {
  if (!lay || !cfg || !leaf_dev || !population_dev)
    return fail(nullptr, TSA_ERR_ARG, "tsa_sweeps_noalloc: null argument");
  if ((lc_dev == nullptr) != (sc_dev == nullptr) || (lc_dev == nullptr) != (ns_dev == nullptr))
    return fail(nullptr, TSA_ERR_ARG, "tsa_sweeps_noalloc: lc, sc and ns are all given or all null");
  if (check_layout_config(lay, cfg, "tsa_sweeps_noalloc") != TSA_OK) return TSA_ERR_ARG;
  if (lay->runtime_width)
    return fail(nullptr, TSA_ERR_ARG, "tsa_sweeps_noalloc: register-width layouts only (at most 512 labels, not wide)");
  if (order != TSA_ORDER_PAR && order != TSA_ORDER_PREORDER) return fail(nullptr, TSA_ERR_ARG, "--order par|preorder");
  if (nsweeps < 0) return fail(nullptr, TSA_ERR_ARG, "tsa_sweeps_noalloc: nsweeps < 0");
  if (nchains < 1 || nchains > (1 << 24)) return fail(nullptr, TSA_ERR_ARG, "tsa_sweeps_noalloc: nchains out of range");
  const size_t nint4 = (size_t)((lay->nint + 3) & ~3);
  const size_t need = kCounterBytes + (lc_dev ? (size_t)nchains * nint4 * 6 : 0);
  if (need > TSA_SCRATCH_BYTES)
    return fail(nullptr, TSA_ERR_ARG,
                "tsa_sweeps_noalloc: " + std::to_string(nchains) + " chains x " + std::to_string(lay->nint) +
                    " nodes need " + std::to_string(need) + " bytes of scratch, more than its " +
                    std::to_string(TSA_SCRATCH_BYTES) + " (fewer chains per call, or no energies)");
  if (check_host_math() != TSA_OK) return TSA_ERR_LIBM;
  StaticDevice* d = nullptr;
  if (static_device(&d) != TSA_OK) return TSA_ERR_HIP;
  TsaLaunch L{};
  bool in_lds = false;
  if (plan_one_wave(lay, cfg, nchains, d->lds_max, d->ncu, &L, &in_lds) != TSA_OK) return TSA_ERR_FIT;
  TsaKParams P;
  fill_params(*lay, *cfg, leaf_sc, P);
  hipStream_t st = static_cast<hipStream_t>(stream);
  unsigned long long* counters = reinterpret_cast<unsigned long long*>(d->scratch);
  float* cost = reinterpret_cast<float*>(d->scratch + kCounterBytes);
  uint16_t* z = reinterpret_cast<uint16_t*>(d->scratch + kCounterBytes + (size_t)nchains * nint4 * 4);
  // the counters start at zero on every call (the scratch keeps the last call's contents)
  hipError_t e = tsa_launch_zero(counters, TSA_NSTAT_ALL * TSA_STAT_SLOTS, st);
  if (e == hipSuccess && nsweeps > 0) {
    const TsaEnergyOut eo{nullptr, nullptr, nullptr, lc_dev ? cost : nullptr, lc_dev ? z : nullptr, nullptr};
    e = tsa_launch_sweeps(L, cfg->mode, order, P, population_dev, leaf_dev, d->fix, nchains, beta, sweep0, nsweeps,
                          counters, eo, st);
    if (e == hipSuccess && lc_dev)
      e = tsa_launch_fold(P, population_dev, leaf_dev, d->fix, cost, z, nchains, lc_dev, sc_dev, ns_dev, st);
  } else if (e == hipSuccess && lc_dev) {
    // no sweeps: the energies of the population as it stands
    e = tsa_launch_energy(L.W, cfg->mode, P, population_dev, leaf_dev, d->fix, nchains, lc_dev, sc_dev, ns_dev, st);
  }
  if (e == hipSuccess && stats_dev) e = tsa_launch_sum_stats(counters, reinterpret_cast<unsigned long long*>(stats_dev), st);
  if (e != hipSuccess) return fail(nullptr, TSA_ERR_HIP, std::string("tsa_sweeps_noalloc launch: ") + hipGetErrorString(e));
  return TSA_OK;
}
