// tsa_kernels.hip -- TreeSA kernels for gfx950 (MI355X): the unmasked variants of the sweep kernel k_sweep
// (tsa_sweep.h), the fold, energy, copy and selection kernels, and their launchers.
#include "tsa_sweep.h"

// Per-chain energy from node costs a sweep launch left (TsaEnergyOut.cost / z), one 32-lane half-wave per
// chain: the reference's fold (csrc/treesa_gpu.cu:386-434) of every chain at once, instead of at the end of
// each chain's sweep, where the serial lse chain is paid once per round of resident chains.
__global__ void __launch_bounds__(256) k_fold(TsaKParams P, const uint64_t* __restrict__ rec,
                                              const uint64_t* __restrict__ leaf, const uint32_t* __restrict__ fix,
                                              const float* __restrict__ cost, const uint16_t* __restrict__ z,
                                              int nchains, float* __restrict__ lc, int* __restrict__ sc,
                                              int* __restrict__ ns) {
  __shared__ uint64_t s_exp2[32];
  if (threadIdx.x < 32) s_exp2[threadIdx.x] = tsa_exp2_tab_d[threadIdx.x];
  __syncthreads();
  const TsaMathTabs T{s_exp2, fix, fix + TSA_LOG2FIX_WORDS, tsa_log2_tab_d};
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  const int c = t >> 5, l32 = threadIdx.x & 31;
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
  const int threads = 256, grid = (nchains * 32 + threads - 1) / threads;
  hipLaunchKernelGGL(k_fold, dim3(grid), dim3(threads), 0, st, P, rec, leaf, fix, cost, z, nchains, lc, sc, ns);
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
  for (int i = threadIdx.x; i < n4; i += blockDim.x) d[i] = s[i];
}

// Best tracking of one level (csrc/treesa_gpu.cu:1810-1832): every chain scored by its own thread, argmin
// with the lowest index on ties and the population sums reduced per workgroup of 256 in a fixed tree order,
// then the last workgroup to finish reduces the per-workgroup results in index order, writes the trace
// row, keeps the best so far and snapshots it when it improves.  Sums are therefore deterministic.
__global__ void __launch_bounds__(256) k_track(const float* __restrict__ lc, const int* __restrict__ sc,
                                               const int* __restrict__ ns, int n, TsaSelect S, int level,
                                               const uint64_t* __restrict__ rec, int chain_words, int ch_off,
                                               int s_off, int W, int nint, const uint32_t* __restrict__ ch_snap,
                                               TsaTrackState* __restrict__ st, TsaTraceRowD* __restrict__ trace,
                                               uint64_t* __restrict__ best_rec, TsaTrackPart* __restrict__ part,
                                               unsigned* __restrict__ done) {
  __shared__ double s_s[256], s_e[256], s_n[256];
  __shared__ int s_i[256];
  __shared__ int s_last, s_copy, s_bi;
  const int t = threadIdx.x, c = blockIdx.x * 256 + t;
  double bs = INFINITY, se = 0.0, sn = 0.0;
  int bi = n;
  if (c < n) {
    bs = tsa_score(lc[c], sc[c], ns[c], S);
    bi = bs < INFINITY ? c : n;
    se = tsa_energyE(lc[c], sc[c], ns[c], S);
    sn = (double)ns[c];
  }
  s_s[t] = bs;
  s_i[t] = bi;
  s_e[t] = se;
  s_n[t] = sn;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (t < o) {
      const double a = s_s[t], b = s_s[t + o];
      const int ia = s_i[t], ib = s_i[t + o];
      if (b < a || (b == a && ib < ia)) {
        s_s[t] = b;
        s_i[t] = ib;
      }
      s_e[t] += s_e[t + o];
      s_n[t] += s_n[t + o];
    }
    __syncthreads();
  }
  if (t == 0) {
    part[blockIdx.x] = TsaTrackPart{s_s[0], s_e[0], s_n[0], s_i[0]};
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const unsigned old = __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = old == gridDim.x - 1;
    if (last) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      __hip_atomic_store(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;
  // the per-workgroup results, in workgroup order: thread t folds workgroups t, t+256, ... then a tree
  bs = INFINITY;
  bi = n;
  se = 0.0;
  sn = 0.0;
  for (int k = t; k < (int)gridDim.x; k += 256) {
    const TsaTrackPart q = part[k];
    if (q.score < bs || (q.score == bs && q.idx < bi)) {
      bs = q.score;
      bi = q.idx;
    }
    se += q.sumE;
    sn += q.sumNs;
  }
  s_s[t] = bs;
  s_i[t] = bi;
  s_e[t] = se;
  s_n[t] = sn;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (t < o) {
      const double a = s_s[t], b = s_s[t + o];
      const int ia = s_i[t], ib = s_i[t + o];
      if (b < a || (b == a && ib < ia)) {
        s_s[t] = b;
        s_i[t] = ib;
      }
      s_e[t] += s_e[t + o];
      s_n[t] += s_n[t + o];
    }
    __syncthreads();
  }
  if (t == 0) {
    const int b = s_i[0];
    TsaTraceRowD row;
    row.chain = b < n ? b : -1;
    row.lc = b < n ? lc[b] : 0.0f;
    row.sc = b < n ? sc[b] : 0;
    row.ns = b < n ? ns[b] : 0;
    row.score = s_s[0];
    row.meanE = s_e[0] / n;
    row.meanNs = s_n[0] / n;
    row.ticks = wall_clock64();
    trace[level] = row;
    const bool better = b < n && s_s[0] < st->best_score;
    if (better) {
      st->best_score = s_s[0];
      st->best_chain = b;
      st->best_level = level;
    }
    st->snap = better ? b : -1;
    s_copy = better ? 1 : 0;
    s_bi = b;
  }
  __syncthreads();
  if (s_copy) {  // the new best chain's tree: children words and S (label words follow from the tree)
    const uint64_t* src = rec + (size_t)s_bi * chain_words;
    const uint32_t* chs = ch_snap ? ch_snap + (size_t)s_bi * nint : reinterpret_cast<const uint32_t*>(src + ch_off);
    uint32_t* chd = reinterpret_cast<uint32_t*>(best_rec + ch_off);
    for (int i = t; i < nint; i += 256) chd[i] = chs[i];
    for (int w = t; w < W; w += 256) best_rec[s_off + w] = src[s_off + w];
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

hipError_t tsa_launch_track(const float* lc, const int* sc, const int* ns, int nchains, const TsaSelect& S, int level,
                            const uint64_t* rec, int chain_words, int ch_off, int s_off, int W, int nint,
                            const uint32_t* ch_snap, TsaTrackState* stt, TsaTraceRowD* trace, uint64_t* best_rec,
                            TsaTrackPart* part, unsigned* done, hipStream_t stream) {
  hipLaunchKernelGGL(k_track, dim3((nchains + 255) / 256), dim3(256), 0, stream, lc, sc, ns, nchains, S, level, rec,
                     chain_words, ch_off, s_off, W, nint, ch_snap, stt, trace, best_rec, part, done);
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

// The level loop's per-chain best: score +inf, no candidate slot.
__global__ void k_levels_init(double* __restrict__ own, int* __restrict__ bslot, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    own[i] = INFINITY;
    bslot[i] = -1;
  }
}

hipError_t tsa_launch_levels_init(double* own, int* bslot, int n, hipStream_t stream) {
  hipLaunchKernelGGL(k_levels_init, dim3((n + 255) / 256), dim3(256), 0, stream, own, bslot, n);
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
