// tsa_kernels.hip -- TreeSA kernels for gfx950 (MI355X): the unmasked variants of the sweep kernel k_sweep
// (tsa_sweep.h), the fold, energy, copy and selection kernels, and their launchers.
#include "tsa_sweep.h"

// Per-chain energy from node costs a sweep launch left (TsaEnergyOut.cost / z), one 32-lane half-wave per
// chain: the reference's fold (csrc/treesa_gpu.cu:386-434) of every chain at once, instead of at the end of
// each chain's sweep, where the serial lse chain is paid once per round of resident chains.  blockIdx.y: the
// level (several levels' snapshots fold in one launch).
__global__ void __launch_bounds__(256) k_fold(TsaKParams P, const uint64_t* __restrict__ rec,
                                              const uint64_t* __restrict__ leaf, const uint32_t* __restrict__ fix,
                                              TsaFoldLevels F, int chain0, int nchains) {
  const int li = (int)blockIdx.y;
  const float* __restrict__ cost = F.cost[li];
  const uint16_t* __restrict__ z = F.z[li];
  float* __restrict__ lc = F.lc[li];
  int* __restrict__ sc = F.sc[li];
  int* __restrict__ ns = F.ns[li];
  __shared__ uint64_t s_exp2[32];
  if (threadIdx.x < 32) s_exp2[threadIdx.x] = tsa_exp2_tab_d[threadIdx.x];
  __syncthreads();
  const TsaMathTabs T{s_exp2, fix, fix + TSA_LOG2FIX_WORDS, tsa_log2_tab_d};
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  const int c = chain0 + (t >> 5), l32 = threadIdx.x & 31;
  const int cc = c < nchains ? c : nchains - 1;  // a half-wave past the end duplicates the last chain
  const size_t nint4 = (size_t)((P.nint + 3) & ~3);
  const uint64_t* S = P.slicing ? rec + (size_t)cc * P.chain_words + P.s_off : nullptr;
  const TsaEvalOut e = tsa_fold32(P, cost + (size_t)cc * nint4, z + (size_t)cc * nint4, S, leaf, P.W, T, l32);
  if (l32 == 0 && c < nchains) {
    lc[c] = e.lcost;
    sc[c] = e.sc;
    ns[c] = e.ns;
  }
}

hipError_t tsa_launch_fold(const TsaKParams& P, const uint64_t* rec, const uint64_t* leaf, const uint32_t* fix,
                           const float* cost, const uint16_t* z, int nchains, float* lc, int* sc, int* ns,
                           hipStream_t st) {
  TsaFoldLevels F{};
  F.n = 1;
  F.cost[0] = cost;
  F.z[0] = z;
  F.lc[0] = lc;
  F.sc[0] = sc;
  F.ns[0] = ns;
  return tsa_launch_fold_levels(P, rec, leaf, fix, F, 0, nchains, st);
}

hipError_t tsa_launch_fold_levels(const TsaKParams& P, const uint64_t* rec, const uint64_t* leaf, const uint32_t* fix,
                                  const TsaFoldLevels& F, int chain0, int nchains, hipStream_t st) {
  if (F.n < 1 || F.n > TSA_BLOCK_MAX || chain0 < 0 || chain0 >= nchains) return hipErrorInvalidValue;
  const int threads = 256, grid = ((nchains - chain0) * 32 + threads - 1) / threads;
  hipLaunchKernelGGL(k_fold, dim3(grid, F.n), dim3(threads), 0, st, P, rec, leaf, fix, F, chain0, nchains);
  return hipGetLastError();
}

// Per-chain energy, one 32-lane half-wave per chain (csrc/treesa_gpu.cu:999-1014).
template <int W, int MODE>
__global__ void __launch_bounds__(256) k_energy(TsaKParams P, const uint64_t* __restrict__ rec,
                                                const uint64_t* __restrict__ leaf, const uint32_t* __restrict__ fix,
                                                int nchains, float* __restrict__ lc, int* __restrict__ sc,
                                                int* __restrict__ ns) {
  __shared__ uint64_t s_exp2[32];
  if (threadIdx.x < 32) s_exp2[threadIdx.x] = tsa_exp2_tab_d[threadIdx.x];
  __syncthreads();
  const TsaMathTabs T{s_exp2, fix, fix + TSA_LOG2FIX_WORDS, tsa_log2_tab_d};
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  const int c = t >> 5, l32 = threadIdx.x & 31;
  const int cc = c < nchains ? c : nchains - 1;  // a half-wave past the end duplicates the last chain
  const uint64_t* lab = rec + (size_t)cc * P.chain_words;
  const uint32_t* ch = reinterpret_cast<const uint32_t*>(lab + P.ch_off);
  const uint64_t* S = P.slicing ? lab + P.s_off : nullptr;
  const TsaEvalOut e = tsa_eval32<W, MODE>(P, lab, ch, S, leaf, T, l32);
  if (l32 == 0 && c < nchains) {
    lc[c] = e.lcost;
    sc[c] = e.sc;
    ns[c] = e.ns;
  }
}

// Population resampling: dst chain c <- src chain anc[c] (csrc/treesa_gpu.cu:1016-1022).
__global__ void __launch_bounds__(256) k_copy(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                              const int* __restrict__ anc, int n4) {
  const uint4* s = src + (size_t)anc[blockIdx.x] * n4;
  uint4* d = dst + (size_t)blockIdx.x * n4;
  tsa_copy_inflight<uint4, 4>(d, s, n4, (int)threadIdx.x, (int)blockDim.x);
}

// One entry of the selection's reduction: best score and its chain, sums of E and |S|.
struct TsaTrackAcc {
  double s, e, n;
  int i;
};

// a (lower position) combined with b: the lower score, the lower chain on ties; the sums added.
__device__ __forceinline__ void tsa_track_comb(TsaTrackAcc& a, const TsaTrackAcc& b) {
  if (b.s < a.s || (b.s == a.s && b.i < a.i)) {
    a.s = b.s;
    a.i = b.i;
  }
  a.e += b.e;
  a.n += b.n;
}

// 256 entries (entry t = lane + 64 j in v[j]) reduced in the order of a halving tree over 256 positions
// (position t takes t + 128, then t + 64, then 32, 16, ..., 1) by one wave: lane 0 returns the result.
__device__ __forceinline__ TsaTrackAcc tsa_track_tree(TsaTrackAcc (&v)[4], int lane) {
  tsa_track_comb(v[0], v[2]);
  tsa_track_comb(v[1], v[3]);
  tsa_track_comb(v[0], v[1]);
  for (int o = 32; o > 0; o >>= 1) {
    TsaTrackAcc b;
    b.s = __shfl_down(v[0].s, o);
    b.e = __shfl_down(v[0].e, o);
    b.n = __shfl_down(v[0].n, o);
    b.i = __shfl_down(v[0].i, o);
    if (lane < o) tsa_track_comb(v[0], b);
  }
  return v[0];
}

// Best tracking of L.n levels (csrc/treesa_gpu.cu:1810-1832), one wave per group of 256 chains and level
// (blockIdx.y): every chain scored, argmin with the lowest index on ties and the population sums reduced per
// group in a fixed tree order; the last group of a level to finish reduces the groups' results in index order
// and writes the level's trace row; the last level to finish keeps the best over the launch's levels in level
// order (the lowest score; the first level on ties, as one launch per level would) and copies the new best
// chain's tree.  Sums are deterministic.  WAVES = 1: no LDS, so that the selection's waves fit beside sweep
// workgroups that fill a compute unit's LDS (each lane scores four chains in turn); WAVES = 4, for a selection
// that runs alone between sweeps: the four waves score a chain per lane at once and hand the entries to wave 0
// through LDS, which reduces them in the same order.
__device__ __forceinline__ TsaTrackAcc tsa_track_entry(int c, int n, const float* __restrict__ lc,
                                                       const int* __restrict__ sc, const int* __restrict__ ns,
                                                       const TsaSelect& S) {
  TsaTrackAcc v{INFINITY, 0.0, 0.0, n};
  if (c < n) {
    const double s = tsa_score(lc[c], sc[c], ns[c], S);
    v.s = s;
    v.i = s < INFINITY ? c : n;
    v.e = tsa_energyE(lc[c], sc[c], ns[c], S);
    v.n = (double)ns[c];
  }
  return v;
}

template <int WAVES>
__global__ void __launch_bounds__(64 * WAVES) k_track(TsaTrackLevels L, int n, TsaSelect S,
                                                      const uint64_t* __restrict__ rec, int chain_words, int ch_off,
                                                      int s_off, int W, int nint, TsaTrackState* __restrict__ st,
                                                      TsaTraceRowD* __restrict__ trace, uint64_t* __restrict__ best_rec,
                                                      TsaTrackPart* __restrict__ part, unsigned* __restrict__ done) {
  const int lane = (int)threadIdx.x & 63, g = (int)blockIdx.x, li = (int)blockIdx.y, G = (int)gridDim.x;
  const float* __restrict__ lc = L.lc[li];
  const int* __restrict__ sc = L.sc[li];
  const int* __restrict__ ns = L.ns[li];
  TsaTrackAcc v[4];
  if constexpr (WAVES == 1) {
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = tsa_track_entry(g * 256 + lane + 64 * j, n, lc, sc, ns, S);
  } else {
    static_assert(WAVES == 4, "one wave, or four waves of 64 chains each");
    __shared__ TsaTrackAcc sh[256];
    const int w = (int)threadIdx.x >> 6;
    sh[threadIdx.x] = tsa_track_entry(g * 256 + lane + 64 * w, n, lc, sc, ns, S);
    __syncthreads();
    if (w != 0) return;
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = sh[lane + 64 * j];
  }
  const TsaTrackAcc r = tsa_track_tree(v, lane);
  int last = 0;
  if (lane == 0) {
    part[li * G + g] = TsaTrackPart{r.s, r.e, r.n, r.i};
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const unsigned old = __hip_atomic_fetch_add(done + li, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old == (unsigned)G - 1u;
    if (last) __hip_atomic_store(done + li, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!__shfl(last, 0)) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  // the level's group results, in group order: position t (= lane + 64 j) folds groups t, t + 256, ... then the
  // same tree
  TsaTrackAcc w[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    w[j] = TsaTrackAcc{INFINITY, 0.0, 0.0, n};
    for (int k = lane + 64 * j; k < G; k += 256) {
      const TsaTrackPart q = part[li * G + k];
      tsa_track_comb(w[j], TsaTrackAcc{q.score, q.sumE, q.sumNs, q.idx});
    }
  }
  const TsaTrackAcc a = tsa_track_tree(w, lane);
  int blast = 0;
  if (lane == 0) {
    const int b = a.i;
    TsaTraceRowD row;
    row.chain = b < n ? b : -1;
    row.lc = b < n ? lc[b] : 0.0f;
    row.sc = b < n ? sc[b] : 0;
    row.ns = b < n ? ns[b] : 0;
    row.score = a.s;
    row.meanE = a.e / n;
    row.meanNs = a.n / n;
    row.ticks = wall_clock64();
    trace[L.lev[li]] = row;
    part[L.n * G + li] = TsaTrackPart{a.s, 0.0, 0.0, b};  // the level's best, for the launch's last level
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const unsigned old = __hip_atomic_fetch_add(done + L.n, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    blast = old == (unsigned)L.n - 1u;
    if (blast) __hip_atomic_store(done + L.n, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!__shfl(blast, 0)) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  int win = -1, wc = 0;
  if (lane == 0) {
    for (int i = 0; i < L.n; i++) {
      const TsaTrackPart q = part[L.n * G + i];
      const bool better = q.idx < n && q.score < st->best_score;
      if (better) {
        st->best_score = q.score;
        st->best_chain = q.idx;
        st->best_level = L.lev[i];
        win = i;
        wc = q.idx;
      }
      st->snap = better ? q.idx : -1;
    }
  }
  win = __shfl(win, 0);
  wc = __shfl(wc, 0);
  if (win >= 0) {  // the new best chain's tree: children words and S (label words follow from the tree)
    const uint64_t* src = rec + (size_t)wc * chain_words;
    const uint32_t* chs = L.ch[win] ? L.ch[win] + (size_t)wc * nint : reinterpret_cast<const uint32_t*>(src + ch_off);
    uint32_t* chd = reinterpret_cast<uint32_t*>(best_rec + ch_off);
    // (eight loads in flight per lane: a copy that stores each word before loading the next waits a cache
    // latency per 64 words, about 20 us for a tree of 4 095 nodes)
    tsa_copy_inflight<uint32_t, 8>(chd, chs, nint, lane, 64);
    tsa_copy_inflight<uint64_t, 8>(best_rec + s_off, src + s_off, W, lane, 64);
  }
}

// A tracking session's start: the tracking state, the start tick, and the trace rows and best record cleared
// (one launch instead of two memsets and a launch).
__global__ void __launch_bounds__(256) k_track_init(TsaTrackState* st, unsigned long long* ticks0,
                                                    unsigned long long* trace, int trace_words,
                                                    unsigned long long* best, int best_words) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x, nt = gridDim.x * blockDim.x;
  for (int i = t; i < trace_words; i += nt) trace[i] = 0ull;
  for (int i = t; i < best_words; i += nt) best[i] = 0ull;
  if (t == 0) {
    st->best_score = INFINITY;
    st->best_chain = -1;
    st->best_level = -1;
    st->snap = -1;
    *ticks0 = wall_clock64();
  }
}

// ---------------------------------------------------------------------------------------------------
// Host-side launchers
// ---------------------------------------------------------------------------------------------------
// The kernels without slice code (sets never masked) are instantiated here, the slicing ones in
// tsa_sweep_sliced.hip.
hipError_t tsa_launch_sweeps(const TsaLaunch& L, int mode, int order, const TsaKParams& P, uint64_t* rec,
                             const uint64_t* leaf, const uint32_t* fix, int nchains, float beta, uint32_t sweep0,
                             int nsweeps, unsigned long long* stats, const TsaEnergyOut& eo, hipStream_t st,
                             hipEvent_t e0, hipEvent_t e1, const TsaLevels* lv, int* res) {
  if (P.slicing)
    return tsa_launch_sweeps_sliced(L, mode, order, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, eo, st,
                                    e0, e1, lv, res);
  return tsa_launch_sweeps_t<false>(L, mode, order, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, eo, st, e0,
                                    e1, lv, res);
}

template <int W, int MODE>
static hipError_t launch_energy_t(const TsaKParams& P, const uint64_t* rec, const uint64_t* leaf, const uint32_t* fix,
                                  int nchains, float* lc, int* sc, int* ns, hipStream_t st) {
  const int threads = 256, grid = (nchains * 32 + threads - 1) / threads;
  hipLaunchKernelGGL((k_energy<W, MODE>), dim3(grid), dim3(threads), 0, st, P, rec, leaf, fix, nchains, lc, sc, ns);
  return hipGetLastError();
}

template <int W>
static hipError_t launch_energy_w(int mode, const TsaKParams& P, const uint64_t* rec, const uint64_t* leaf,
                                  const uint32_t* fix, int nchains, float* lc, int* sc, int* ns, hipStream_t st) {
  if (mode == 0) return launch_energy_t<W, 0>(P, rec, leaf, fix, nchains, lc, sc, ns, st);
  if (mode == 1) return launch_energy_t<W, 1>(P, rec, leaf, fix, nchains, lc, sc, ns, st);
  return launch_energy_t<W, 2>(P, rec, leaf, fix, nchains, lc, sc, ns, st);
}

hipError_t tsa_launch_energy(int Wt, int mode, const TsaKParams& P, const uint64_t* rec, const uint64_t* leaf,
                             const uint32_t* fix, int nchains, float* lc, int* sc, int* ns, hipStream_t st) {
  switch (Wt) {
    case 1: return launch_energy_w<1>(mode, P, rec, leaf, fix, nchains, lc, sc, ns, st);
    case 2: return launch_energy_w<2>(mode, P, rec, leaf, fix, nchains, lc, sc, ns, st);
    case 4: return launch_energy_w<4>(mode, P, rec, leaf, fix, nchains, lc, sc, ns, st);
    case 8: return launch_energy_w<8>(mode, P, rec, leaf, fix, nchains, lc, sc, ns, st);
    case 0: return launch_energy_w<0>(mode, P, rec, leaf, fix, nchains, lc, sc, ns, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t tsa_launch_track_levels(const TsaTrackLevels& L, int nchains, const TsaSelect& S, const uint64_t* rec,
                                   int chain_words, int ch_off, int s_off, int W, int nint, TsaTrackState* stt,
                                   TsaTraceRowD* trace, uint64_t* best_rec, TsaTrackPart* part, unsigned* done,
                                   hipStream_t stream, bool alone) {
  if (L.n < 1 || L.n > TSA_BLOCK_MAX || nchains < 1) return hipErrorInvalidValue;
  const dim3 grid((nchains + 255) / 256, L.n);
  if (alone)
    hipLaunchKernelGGL(k_track<4>, grid, dim3(256), 0, stream, L, nchains, S, rec, chain_words, ch_off, s_off, W, nint,
                       stt, trace, best_rec, part, done);
  else
    hipLaunchKernelGGL(k_track<1>, grid, dim3(64), 0, stream, L, nchains, S, rec, chain_words, ch_off, s_off, W, nint,
                       stt, trace, best_rec, part, done);
  return hipGetLastError();
}

hipError_t tsa_launch_track(const float* lc, const int* sc, const int* ns, int nchains, const TsaSelect& S, int level,
                            const uint64_t* rec, int chain_words, int ch_off, int s_off, int W, int nint,
                            const uint32_t* ch_snap, TsaTrackState* stt, TsaTraceRowD* trace, uint64_t* best_rec,
                            TsaTrackPart* part, unsigned* done, hipStream_t stream, bool alone) {
  TsaTrackLevels L{};
  L.n = 1;
  L.lev[0] = level;
  L.lc[0] = lc;
  L.sc[0] = sc;
  L.ns[0] = ns;
  L.ch[0] = ch_snap;
  return tsa_launch_track_levels(L, nchains, S, rec, chain_words, ch_off, s_off, W, nint, stt, trace, best_rec, part,
                                 done, stream, alone);
}

// The session's best after a level-loop launch (tsa_launch_level_best): lane l takes the launch's levels l,
// l + 64, ... (all trace rows read at once), the wave reduces their lowest (score, level), and lane 0 keeps it
// when it beats st's; the wave then copies that chain's kept tree.  The chains' bslot are the launch's final
// values (the launch has ended).
__global__ void __launch_bounds__(64) k_level_best(TsaLevels Lv, int n, TsaTrackState* __restrict__ st,
                                                   uint64_t* __restrict__ best_rec, int ch_off, TsaTrackOut O) {
  const int lane = (int)threadIdx.x;
  double bs = INFINITY;
  int bl = -1, bc = -1;
  for (int l = lane; l < Lv.nlev; l += 64) {
    if (Lv.eval[l] < 0) continue;
    const TsaTraceRowD q = Lv.trace[Lv.level0 + l];
    if (q.chain >= 0 && q.score < bs) {  // (a lane's levels rise, so the first of equal scores stays)
      bs = q.score;
      bc = q.chain;
      bl = Lv.level0 + l;
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const double s2 = __shfl_down(bs, o, 64);
    const int l2 = __shfl_down(bl, o, 64), c2 = __shfl_down(bc, o, 64);
    if (lane + o < 64 && l2 >= 0 && (s2 < bs || (s2 == bs && (bl < 0 || l2 < bl)))) {
      bs = s2;
      bl = l2;
      bc = c2;
    }
  }
  int slot = -1;
  if (lane == 0) {
    if (bc >= 0 && bs < st->best_score) {
      slot = Lv.bslot[bc];
      if (slot == 0 || slot == 1) {  // (a chain with a finite score has kept a tree)
        st->best_score = bs;
        st->best_chain = bc;
        st->best_level = bl;
        st->snap = bc;
      }
    }
  }
  slot = __shfl(slot, 0, 64);
  bc = __shfl(bc, 0, 64);
  const bool kept = slot == 0 || slot == 1;
  const uint64_t* const src = kept ? Lv.cand + ((size_t)slot * n + bc) * Lv.cand_words : nullptr;
  if (kept) tsa_copy_inflight<uint64_t, 8>(best_rec + ch_off, src, Lv.cand_words, lane, 64);
  if (!O.h_st) return;
  // the session's results: the best tree from the words just copied (their source) or, unchanged by this launch,
  // from best_rec; the state as lane 0 left it; every trace row (the earlier launches' too)
  tsa_copy_inflight<unsigned long long, 8>(O.h_tree, reinterpret_cast<const unsigned long long*>(kept ? src : best_rec + ch_off),
                                           Lv.cand_words, lane, 64);
  tsa_copy_inflight<unsigned long long, 8>(O.h_rows, reinterpret_cast<const unsigned long long*>(Lv.trace),
                                           O.row_words, lane, 64);
  if (lane == 0) {
    const unsigned long long* const sw = reinterpret_cast<const unsigned long long*>(st);
    for (int i = 0; i < (int)(sizeof(TsaTrackState) / 8); i++) O.h_st[i] = sw[i];
    *O.h_t0 = *O.ticks0;
  }
}

hipError_t tsa_launch_level_best(const TsaLevels& Lv, int nchains, TsaTrackState* stt, uint64_t* best_rec, int ch_off,
                                 const TsaTrackOut& O, hipStream_t stream) {
  hipLaunchKernelGGL(k_level_best, dim3(1), dim3(64), 0, stream, Lv, nchains, stt, best_rec, ch_off, O);
  return hipGetLastError();
}

hipError_t tsa_launch_track_init(TsaTrackState* stt, unsigned long long* ticks0, unsigned long long* trace,
                                 int trace_words, unsigned long long* best, int best_words, hipStream_t stream) {
  const int n = trace_words > best_words ? trace_words : best_words;
  int grid = (n + 255) / 256;
  if (grid < 1) grid = 1;
  if (grid > 64) grid = 64;
  hipLaunchKernelGGL(k_track_init, dim3(grid), dim3(256), 0, stream, stt, ticks0, trace, trace_words, best, best_words);
  return hipGetLastError();
}

__global__ void __launch_bounds__(256) k_anneal_init(TsaAnnealInit A) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x, nt = gridDim.x * blockDim.x;
  if (A.tab_src)
    for (int i = t; i < A.tab_words; i += nt) A.tab_dst[i] = A.tab_src[i];
  if (A.cnt)
    for (int i = t; i < A.cnt_words; i += nt) A.cnt[i] = 0ull;
}

hipError_t tsa_launch_anneal_init(const TsaAnnealInit& A, hipStream_t stream) {
  int n = 1;
  if (A.tab_src && A.tab_words > n) n = A.tab_words;
  if (A.cnt && A.cnt_words > n) n = A.cnt_words;
  int grid = (n + 255) / 256;
  if (grid > 64) grid = 64;
  hipLaunchKernelGGL(k_anneal_init, dim3(grid), dim3(256), 0, stream, A);
  return hipGetLastError();
}

__global__ void __launch_bounds__(256) k_track_out(const unsigned long long* __restrict__ st, int st_words,
                                                   const unsigned long long* __restrict__ ticks0,
                                                   const unsigned long long* __restrict__ tree, int tree_words,
                                                   const unsigned long long* __restrict__ rows, int row_words,
                                                   const unsigned* __restrict__ werr, unsigned long long* h_st,
                                                   unsigned long long* h_t0, unsigned long long* h_tree,
                                                   unsigned long long* h_rows, unsigned* h_werr) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x, nt = gridDim.x * blockDim.x;
  tsa_copy_inflight<unsigned long long, 4>(h_rows, rows, row_words, t, nt);
  tsa_copy_inflight<unsigned long long, 4>(h_tree, tree, tree_words, t, nt);
  if (t < st_words) h_st[t] = st[t];
  if (t == 0) *h_t0 = *ticks0;
  if (t == 0 && werr) *h_werr = *werr;
}

hipError_t tsa_launch_track_out(const unsigned long long* st, int st_words, const unsigned long long* ticks0,
                                const unsigned long long* tree, int tree_words, const unsigned long long* rows,
                                int row_words, const unsigned* werr, unsigned long long* h_st,
                                unsigned long long* h_t0, unsigned long long* h_tree, unsigned long long* h_rows,
                                unsigned* h_werr, hipStream_t stream) {
  int n = row_words > tree_words ? row_words : tree_words;
  if (st_words > n) n = st_words;
  int grid = (n + 255) / 256;
  if (grid < 1) grid = 1;
  if (grid > 16) grid = 16;
  hipLaunchKernelGGL(k_track_out, dim3(grid), dim3(256), 0, stream, st, st_words, ticks0, tree, tree_words, rows,
                     row_words, werr, h_st, h_t0, h_tree, h_rows, h_werr);
  return hipGetLastError();
}

// Clears n 64-bit words (a kernel rather than hipMemsetAsync, so that the call can sit in a captured graph).
__global__ void k_zero_u64(unsigned long long* __restrict__ p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0ull;
}

// out[k] = sum of the TSA_STAT_SLOTS slots of counter k, k < TSA_NSTAT (one wave).
__global__ void k_sum_stats(const unsigned long long* __restrict__ slots, unsigned long long* __restrict__ out) {
  const int k = threadIdx.x;
  if (k >= TSA_NSTAT) return;
  unsigned long long s = 0;
  for (int j = 0; j < TSA_STAT_SLOTS; j++) s += slots[k * TSA_STAT_SLOTS + j];
  out[k] = s;
}

hipError_t tsa_launch_zero(unsigned long long* p, int n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_zero_u64, dim3((n + 255) / 256), dim3(256), 0, st, p, n);
  return hipGetLastError();
}

hipError_t tsa_launch_sum_stats(const unsigned long long* slots, unsigned long long* out, hipStream_t st) {
  hipLaunchKernelGGL(k_sum_stats, dim3(1), dim3(64), 0, st, slots, out);
  return hipGetLastError();
}

hipError_t tsa_launch_copy(const uint64_t* src, uint64_t* dst, const int* anc, int nchains, int chain_words,
                           hipStream_t st) {
  hipLaunchKernelGGL(k_copy, dim3(nchains), dim3(256), 0, st, reinterpret_cast<const uint4*>(src),
                     reinterpret_cast<uint4*>(dst), anc, chain_words / 2);
  return hipGetLastError();
}
