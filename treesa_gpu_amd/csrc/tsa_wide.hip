// tsa_wide.hip -- par-order sweeps and chain energies for wide label sets (runtime width W, an even number
// of 64-bit words, so every label set is a run of W/2 16-byte chunks, 16-byte aligned in HBM).
//
// Sweep kernel k_wide (the reference's k_par with cooperative visits, csrc/treesa_gpu.cu:829-997 and
// 237-373, re-planned for gfx950).  K workgroups own one chain.  Every workgroup keeps a private copy of the
// chain's node arrays in LDS (children words, priorities, parents, work list) and works the label sets in
// HBM.  A phase:
//   1. scan (every workgroup, redundantly): the independent set of the phase -- unvisited nodes whose
//      (priority, id) key beats their unvisited parent and internal children -- compacted in node order
//      into the work list with wave ballots and a prefix over the 64-node groups;
//   2. visits: workgroup k takes the k-th of K contiguous shares of the work list, and its waves take
//      entries from that share 64/G at a time through an LDS counter (one entry per lane group), so
//      that faster waves take more; the G lanes of a
//      group load the label sets D, O, K, M (and P, except in tc mode, where the costs of P and v before the
//      move and P's size come from the node-cost cache) in 16-byte chunks (chunk t, t+G, ...), count with
//      popcounts, sum the counters (packed two per 32-bit word) with xor shuffles inside the group, all
//      lanes evaluate the same dE and Metropolis test, and on accept each lane stores its chunks of
//      X = (K|O)&(M|D) into P's set.  The group leader publishes one outcome byte (accepted, pivot slot,
//      moved-grandchild slot);
//   3. chain barrier (K > 1) or workgroup barrier (K = 1);
//   4. replay (every workgroup): apply every published outcome to the LDS copies -- the two children
//      words of an accepted rotation, the parents of the two moved subtrees, priority 0 for the visited
//      node and the follow-up priority of a re-armed pivot.
// Visits of one phase touch disjoint words (a visit at v writes P's set and the words of v, P, O and M;
// an active node is never the parent, child or grandchild of another active node's pivot), so the visits,
// and the replays, of one phase commute.  Every proposal draws Philox((v, sweep, chain)), so the result is
// the CPU phase-by-phase sweep bit for bit, whatever K and G.
//
// Check-in (K > 1): before it changes anything of its chain, each workgroup adds 1 to the chain's join word
// and waits, with a bounded number of polls, until all K have arrived.  All K arrived means all K are
// resident, and they stay resident until they leave, so the chain barriers below cannot wait on a workgroup
// that the device has not started.  A workgroup that runs out of polls first (another one is not resident:
// the device is shared with other work, or the plan's occupancy was wrong) claims the chain by setting the
// join word's top bit with a compare-and-swap that fails if anyone arrived meanwhile; it then sweeps the
// chain alone (K = 1 within the same kernel: the result is the same bit for bit), and every workgroup of the
// chain that arrives later sees the bit and leaves at once.
//
// Chain barrier: thread 0 of each workgroup releases at agent scope, adds 1 to the chain's counter and polls
// it until K * (barriers so far) with a bounded number of polls (seconds: only a workgroup descheduled for
// that long could make a checked-in barrier wait); a workgroup that runs out of polls sets the error word, and
// every workgroup that sees the error word stops, so every wave reaches the end of the kernel.  The last
// workgroup of a chain to leave (all K of them leave, including those that only checked in) resets the
// chain's words to zero for the next launch.
#include "tsa_kernels.h"
#include "tsa_fold.h"

namespace {

struct alignas(16) TsaW2 {
  uint64_t a, b;
};

__device__ __forceinline__ uint64_t wide_lt_mask(int lane) { return (1ull << lane) - 1ull; }

// Counters of one proposal as a flat list: |d|, |P|, |X|, then K0..K3 (mode 0) or B0..3, M0..3, N0..3,
// K0..3 (modes 1, 2).
template <int MODE>
struct TsaFlat {
  static constexpr int N = MODE == 0 ? 7 : 19;
  static constexpr int NP = (N + 1) / 2;
};

template <int MODE>
__device__ __forceinline__ void counts_pack(const TsaCounts& c, uint32_t (&a)[TsaFlat<MODE>::NP]) {
  int f[TsaFlat<MODE>::NP * 2];
  f[0] = c.sd;
  f[1] = c.sp;
  f[2] = c.sx;
  if (MODE == 0) {
#pragma unroll
    for (int q = 0; q < 4; q++) f[3 + q] = c.K[q];
    f[7] = 0;
  } else {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      f[3 + q] = c.B[q];
      f[7 + q] = c.M[q];
      f[11 + q] = c.N[q];
      f[15 + q] = c.K[q];
    }
    f[19] = 0;
  }
#pragma unroll
  for (int i = 0; i < TsaFlat<MODE>::NP; i++) a[i] = (uint32_t)f[2 * i] | ((uint32_t)f[2 * i + 1] << 16);
}

template <int MODE>
__device__ __forceinline__ void counts_unpack(const uint32_t (&a)[TsaFlat<MODE>::NP], TsaCounts& c) {
  int f[TsaFlat<MODE>::NP * 2];
#pragma unroll
  for (int i = 0; i < TsaFlat<MODE>::NP; i++) {
    f[2 * i] = (int)(a[i] & 0xFFFFu);
    f[2 * i + 1] = (int)(a[i] >> 16);
  }
  c.sd = f[0];
  c.sp = f[1];
  c.sx = f[2];
  if (MODE == 0) {
#pragma unroll
    for (int q = 0; q < 4; q++) c.K[q] = f[3 + q];
  } else {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      c.B[q] = f[3 + q];
      c.M[q] = f[7 + q];
      c.N[q] = f[11 + q];
      c.K[q] = f[15 + q];
    }
  }
}

// Sum over the G lanes of a group (xor butterfly: every lane ends with the total).  Each packed half
// stays below 2^16: a label set has at most 2 * TSA_WIDE_CPL * 64 * 64 = 16384 labels.
template <int G, int N>
__device__ __forceinline__ void group_sum(uint32_t (&a)[N]) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) {
#pragma unroll
    for (int i = 0; i < N; i++) a[i] += (uint32_t)__shfl_xor((int)a[i], o, G);
  }
}

// Check-in of thread 0 (see the file comment): 0 sweep with the other K - 1, 1 sweep the chain alone, 2 leave.
#define TSA_JOIN_CLAIMED 0x80000000u
__device__ int chain_join(const TsaWideSync& sy, int c, int K) {
  const unsigned old = __hip_atomic_fetch_add(sy.join + c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (old & TSA_JOIN_CLAIMED) return 2;
  const unsigned limit = sy.join_polls > 0 ? (unsigned)sy.join_polls : TSA_WIDE_JOIN;
  unsigned polls = 0;
  for (;;) {
    unsigned v = __hip_atomic_load(sy.join + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (v & TSA_JOIN_CLAIMED) return 2;
    if (v >= (unsigned)K) return 0;
    if (sy.join_polls < 0 || ++polls >= limit) {
      if (__hip_atomic_compare_exchange_strong(sy.join + c, &v, v | TSA_JOIN_CLAIMED, __ATOMIC_RELAXED,
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
        return 1;
      continue;  // someone arrived (or claimed) meanwhile: look again
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

// The last of the chain's K workgroups to leave resets its words for the next launch (thread 0).
__device__ void chain_leave(const TsaWideSync& sy, int c, int K) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  const unsigned old = __hip_atomic_fetch_add(sy.done + c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (old == (unsigned)(K - 1)) {  // every workgroup of the chain has left
    __hip_atomic_store(sy.bar + c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(sy.join + c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(sy.done + c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Chain barrier (see the file comment).  Block-uniform result: false when the launch gave up.
__device__ bool chain_barrier(const TsaWideSync& sy, int c, unsigned target, int* s_ok) {
  __syncthreads();
  if (threadIdx.x == 0) {
    int ok = 1;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __hip_atomic_fetch_add(sy.bar + c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned polls = 0;
    for (;;) {
      if (__hip_atomic_load(sy.bar + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target) break;
      if (__hip_atomic_load(sy.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) {
        ok = 0;
        break;
      }
      if (++polls >= TSA_WIDE_SPIN) {
        __hip_atomic_store(sy.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    *s_ok = ok;
  }
  __syncthreads();
  return *s_ok != 0;
}

__device__ __forceinline__ long long wide_wave_sum(long long x) {
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

// Chunk summaries: the chunks of a proposal are the set bits of the union u = u0 | u1 << 64 of the
// summaries of D, O, K and M; lane t of a group of G takes the bits of rank t, t + G, t + 2G, ... so that the
// loads spread evenly over the group whatever the positions, SC of them per round.  sum_pick returns the
// positions of ranks r, r + G, ..., r + (SC - 1) G (-1 where u has fewer set bits).
template <int G>
struct TsaSumRound {
  static constexpr int SC = G <= 2 ? 4 : 2;  // chunks per lane and round
};

template <int G, int SC>
__device__ __forceinline__ void sum_pick(uint64_t u0, uint64_t u1, int r, int (&ii)[SC]) {
#pragma unroll
  for (int q = 0; q < SC; q++) ii[q] = -1;
  int k = 0;
  for (uint64_t u = u0; u; u &= u - 1ull, k++) {
    const int d = k - r;
#pragma unroll
    for (int q = 0; q < SC; q++)
      if (d == q * G) ii[q] = __builtin_ctzll(u);
  }
  for (uint64_t u = u1; u; u &= u - 1ull, k++) {
    const int d = k - r;
#pragma unroll
    for (int q = 0; q < SC; q++)
      if (d == q * G) ii[q] = 64 + __builtin_ctzll(u);
  }
}

// The fold of one chain's cached node costs by the calling workgroup: with stage >= 1 the costs (and with
// stage 2 the log2f summary bitmap) are first copied into the workgroup's LDS at lds (vector copies, all
// loads in flight at once: the fold reads them in a serial chain per lane); lanes 0..31 then fold in the
// reference's order and lane 0 writes lc / sc / ns of chain c.  Every thread of the workgroup calls it.
__device__ __forceinline__ void wide_fold(const TsaKParams& P, int c, const float* cst, const uint16_t* zz,
                                          const uint64_t* S, const uint64_t* leaf, const uint32_t* fix,
                                          const uint64_t* s_mt, int stage, unsigned char* lds, float* lc, int* sc,
                                          int* ns) {
  const int nint4 = (P.nint + 3) & ~3;
  const uint32_t* const gmap = fix + TSA_LOG2FIX_WORDS;
  const uint32_t* map = gmap;
  if (stage) {
    float* const scst = reinterpret_cast<float*>(lds);
    uint16_t* const szz = reinterpret_cast<uint16_t*>(lds + (size_t)nint4 * 4);
    const int n4 = nint4 / 4;
#pragma unroll 4
    for (int i = threadIdx.x; i < n4; i += blockDim.x) {
      const float4 cv = reinterpret_cast<const float4*>(cst)[i];
      const uint2 zv = reinterpret_cast<const uint2*>(zz)[i];
      reinterpret_cast<float4*>(scst)[i] = cv;
      reinterpret_cast<uint2*>(szz)[i] = zv;
    }
    if (stage == 2) {
      uint4* const smap = reinterpret_cast<uint4*>(lds + (((size_t)nint4 * 6 + 15) & ~(size_t)15));
      const uint4* src = reinterpret_cast<const uint4*>(gmap);
#pragma unroll 16
      for (int i = threadIdx.x; i < (int)(TSA_LOG2MAP_WORDS / 4); i += blockDim.x) smap[i] = src[i];
      map = reinterpret_cast<const uint32_t*>(smap);
    }
    __syncthreads();
  }
  if (threadIdx.x < 32) {
    const TsaMathTabs T{s_mt, fix, map, s_mt + 32};
    // two call sites, so that each inlined fold knows whether it reads LDS or global memory
    const TsaEvalOut e = stage ? tsa_fold32(P, reinterpret_cast<const float*>(lds),
                                            reinterpret_cast<const uint16_t*>(lds + (size_t)nint4 * 4), S, leaf, P.W,
                                            T, (int)threadIdx.x)
                               : tsa_fold32(P, cst, zz, S, leaf, P.W, T, (int)threadIdx.x);
    if (threadIdx.x == 0) {
      lc[c] = e.lcost;
      sc[c] = e.sc;
      ns[c] = e.ns;
    }
  }
}

// (SUMS: at most 512 threads, so that the summary visit has 256 registers and does not spill)
template <int G, int MODE, bool COOP, bool SUMS>
__global__ void __launch_bounds__(SUMS ? 512 : 1024) k_wide(TsaKParams P, uint64_t* __restrict__ rec,
                                               const uint64_t* __restrict__ leaf, const uint32_t* __restrict__ fix,
                                               int nchains, int K, float beta0, uint32_t sweep0, int nsweeps,
                                               unsigned long long* __restrict__ stats, TsaWideSync sy) {
  extern __shared__ __align__(16) unsigned char tsa_wsm[];
  __shared__ float s_lse[64];
  __shared__ uint64_t s_mt[TSA_MT_WORDS];
  __shared__ int s_cnt, s_ok, s_next, s_role;
  const int NT = blockDim.x, nwv = NT >> 6, lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int m = P.m, nint = P.nint, nint4 = (nint + 3) & ~3, ngrp = (nint + 63) >> 6;
  const int NW = P.W, nch = NW >> 1;
  // Workgroups are dealt to the X = sy.nxcd XCDs of the device in turn (workgroup b to XCD b % X), each XCD
  // with its own L2.  With K > 1 the K workgroups of a chain are taken from one XCD -- b = X (K (c / X) + k) +
  // c % X -- so that they share that L2 for the chain's label sets; the grid is K * nchains rounded up to a
  // multiple of X chains, and workgroups past the last chain leave at once.
  int c, k;
  if constexpr (COOP) {
    const int X = sy.nxcd;
    const int x = (int)(blockIdx.x % (unsigned)X), sl = (int)(blockIdx.x / (unsigned)X);
    c = (sl / K) * X + x;
    k = sl - (sl / K) * K;
  } else {
    c = (int)blockIdx.x;
    k = 0;
  }
  if (c >= nchains) return;  // whole workgroups
  const int nsw = SUMS ? sy.nsw : 0;
  const bool lsum_in_lds = SUMS && sy.lsum_lds;
  const TsaWideLds Lo = tsa_wide_lds(nint, P.par_band > 0, COOP ? 1 : 0, nsw, lsum_in_lds ? m : 0);
  uint64_t* const masks = reinterpret_cast<uint64_t*>(tsa_wsm + Lo.masks);
  uint32_t* const ch = reinterpret_cast<uint32_t*>(tsa_wsm + Lo.ch);
  uint32_t* const dw = reinterpret_cast<uint32_t*>(tsa_wsm + Lo.dw);
  uint16_t* const pri = reinterpret_cast<uint16_t*>(tsa_wsm + Lo.pri);
  uint16_t* const par = reinterpret_cast<uint16_t*>(tsa_wsm + Lo.par);
  uint16_t* const wl = reinterpret_cast<uint16_t*>(tsa_wsm + Lo.wl);
  uint8_t* const outl = tsa_wsm + Lo.out;
  uint64_t* const ssum = reinterpret_cast<uint64_t*>(tsa_wsm + Lo.sum);  // SUMS: summaries of the internal sets
  uint64_t* const lsum = reinterpret_cast<uint64_t*>(tsa_wsm + Lo.lsum);  // and of the input tensors
  if (threadIdx.x < 64) s_lse[threadIdx.x] = P.lse[threadIdx.x];
  tsa_math_stage(s_mt);
  const TsaMathTabs T{s_mt, fix, fix + TSA_LOG2FIX_WORDS, s_mt + 32};
  uint64_t* const lab = rec + (size_t)c * P.chain_words;
  uint32_t* const gch = reinterpret_cast<uint32_t*>(lab + P.ch_off);
  tsa_copy_inflight<uint32_t, 8>(ch, gch, nint, threadIdx.x, NT);
  uint64_t* const gsum = SUMS ? sy.sum + (size_t)c * nint4 * nsw : nullptr;
  if constexpr (SUMS) {
    tsa_copy_inflight<uint64_t, 8>(ssum, gsum, nint * nsw, threadIdx.x, NT);
    if (lsum_in_lds) tsa_copy_inflight<uint64_t, 8>(lsum, sy.leafsum, m * nsw, threadIdx.x, NT);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nint; i += NT) {
    const uint32_t cw = ch[i];
    const int l = (int)(cw & 0xFFFFu), r = (int)(cw >> 16);
    if (l >= m) par[l - m] = (uint16_t)(m + i);
    if (r >= m) par[r - m] = (uint16_t)(m + i);
  }
  if (threadIdx.x == 0) par[nint - 1] = 0xFFFFu;
  __syncthreads();

  // K > 1: check in (see the file comment); a chain claimed by one workgroup is swept by it alone (Ke = 1)
  int Ke = K, ke = k;
  if constexpr (COOP) {
    if (threadIdx.x == 0) s_role = chain_join(sy, c, K);
    __syncthreads();
    const int role = s_role;
    if (role == 2) {
      if (threadIdx.x == 0) chain_leave(sy, c, K);
      return;
    }
    if (role == 1) {
      Ke = 1;
      ke = 0;
    }
  }

  constexpr int gpw = 64 / G;
  constexpr bool CACHED = MODE == 0;  // tc-mode visits take P's old cost and size from the node-cost cache
  const int ngr = nwv * gpw;
  const int t = lane & (G - 1);
  const int gsub = lane / G;  // lane group within the wave
  int np = 0, na = 0, nv = 0, nst = 0, nck = 0, nxk = 0;
  unsigned nb = 0;
  bool ok = true;
  // a block of levels (one workgroup per chain, chunk summaries): the current level, its beta and its sweeps
  // left
  const bool blocked = SUMS && !COOP && sy.blk_n > 0;
  int lv = 0, left = blocked ? sy.blk_niters[0] : nsweeps;
  float beta = blocked ? sy.blk_beta[0] : beta0;

  for (int s = 0; s < nsweeps && ok; s++) {
    const uint32_t sw = sweep0 + (uint32_t)s;
    const uint32_t hs = tsa_sweep_hash(sw, (uint32_t)c, P.key0);
    for (int i = threadIdx.x; i < nint; i += NT) pri[i] = (uint16_t)tsa_par_pri((uint32_t)(m + i), hs);
    if (P.par_band > 0) {
      // depth at sweep start by pointer jumping on (depth << 16 | ancestor) words; an update that reads an
      // already advanced ancestor word still keeps depth(v) = d + depth(ancestor)
      for (int i = threadIdx.x; i < nint; i += NT) dw[i] = par[i] == 0xFFFFu ? 0xFFFFu : (0x10000u | par[i]);
      __syncthreads();
      for (;;) {
        int any = 0;
        for (int i = threadIdx.x; i < nint; i += NT) {
          const uint32_t w = dw[i], a = w & 0xFFFFu;
          if (a != 0xFFFFu) {
            const uint32_t w2 = dw[a - m];
            dw[i] = ((w & 0xFFFF0000u) + (w2 & 0xFFFF0000u)) | (w2 & 0xFFFFu);
            any = 1;
          }
        }
        if (!__syncthreads_or(any)) break;
      }
      const int L = P.par_band;
      for (int i = threadIdx.x; i < nint; i += NT)
        pri[i] = (uint16_t)((((uint32_t)((L - 1 - (int)(dw[i] >> 16) % L) & 15)) << 12) | (pri[i] & 0x0FFEu) | 1u);
    }
    if (threadIdx.x == 0) {  // the counters of the work list and of the visits (reset again after each replay)
      s_cnt = 0;
      s_next = 0;
    }
    __syncthreads();
    // nodes not yet visited (without par_follow, which re-arms visited pivots): when none is left the next
    // scan would find no active node, and it is skipped (while any is left, the one with the largest key is
    // active)
    int unvisited = nint;
    for (;;) {
      if (!P.par_follow && unvisited == 0) break;  // uniform across the workgroup
      // 1. scan: a wave takes 64-node groups; each lane reads its node's priority, parent and children
      // words, then the three neighbour priorities, in two rounds of independent LDS reads (indices are
      // clamped instead of branched on, so that every read of a round is in flight at once)
      // a wave takes its groups eight at a time: eight ballots, then (one workgroup per chain) one append
      for (int g0 = wv; g0 < ngrp; g0 += 8 * nwv) {
        uint64_t bb[8];
#pragma unroll
        for (int q = 0; q < 8; q++) {
          const int gi = g0 + q * nwv;
          const int i = gi * 64 + lane;
          const int ic = i < nint ? i : nint - 1;
          const uint32_t pv = pri[ic], p = par[ic], cw = ch[ic];
          const uint32_t l = cw & 0xFFFFu, r = cw >> 16;
          const bool hp = p != 0xFFFFu, hl = l >= (uint32_t)m, hr = r >= (uint32_t)m;
          const uint32_t pp = pri[hp ? (int)p - m : ic], pl = pri[hl ? (int)l - m : ic], pr = pri[hr ? (int)r - m : ic];
          const uint32_t key = (pv << 16) | (uint32_t)(m + i);
          const bool act = gi < ngrp && i < nint && pv != 0u && !(hp && pp && ((pp << 16) | p) > key) &&
                           !(hl && pl && ((pl << 16) | l) > key) && !(hr && pr && ((pr << 16) | r) > key);
          bb[q] = __ballot(act);
          if (COOP && lane == 0 && gi < ngrp) masks[gi] = bb[q];
        }
        if constexpr (!COOP) {
          // one workgroup per chain: append the active nodes (any order will do: the visits of a phase
          // commute and every entry carries its own node id)
          int tot = 0;
#pragma unroll
          for (int q = 0; q < 8; q++) tot += __popcll(bb[q]);
          int base = 0;
          if (lane == 0 && tot) base = atomicAdd(&s_cnt, tot);
          base = __builtin_amdgcn_readfirstlane(base);
#pragma unroll
          for (int q = 0; q < 8; q++) {
            const uint64_t b = bb[q];
            if ((b >> lane) & 1ull) wl[base + __popcll(b & wide_lt_mask(lane))] = (uint16_t)(m + (g0 + q * nwv) * 64 + lane);
            base += __popcll(b);
          }
        }
      }
      __syncthreads();
      if constexpr (COOP) {
        // every workgroup of the chain builds the same list: each wave forms the prefix over the group counts
        // itself and compacts its own groups, in node order
        int base = 0;
        for (int g0 = 0; g0 < ngrp; g0 += 64) {
          const int gl = g0 + lane;
          const uint64_t b = gl < ngrp ? masks[gl] : 0ull;
          const int x = __popcll(b);
          int y = x;
#pragma unroll
          for (int o = 1; o < 64; o <<= 1) {
            const int u = __shfl_up(y, o, 64);
            if (lane >= o) y += u;
          }
          const int excl = base + y - x;
          const int gend = g0 + 64 < ngrp ? g0 + 64 : ngrp;
          for (int gi = g0 + (wv - g0 % nwv + nwv) % nwv; gi < gend; gi += nwv) {
            const uint32_t blo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, gi - g0);
            const uint32_t bhi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), gi - g0);
            const uint64_t bm = ((uint64_t)bhi << 32) | blo;
            const int off = __builtin_amdgcn_readlane(excl, gi - g0);
            if ((bm >> lane) & 1ull) wl[off + __popcll(bm & wide_lt_mask(lane))] = (uint16_t)(m + gi * 64 + lane);
          }
          base += __builtin_amdgcn_readlane(y, 63);
        }
        if (threadIdx.x == 0) s_cnt = base;
        __syncthreads();
      }
      const int cnt = s_cnt;
      if (cnt == 0) break;
      nst++;
      unvisited -= cnt;
      uint8_t* const out = COOP ? sy.out + ((size_t)c * 2 + (nb & 1u)) * (size_t)nint4 : outl;

      // 2. visits: this workgroup's share of the work list -- entries k, k + K, k + 2K, ... (interleaved, so
      // that neighbouring entries, which cost alike, spread over the workgroups) -- handed out gpw at a time
      // to whichever wave asks next (an LDS counter), so that waves that run ahead take more
      const int nk = (cnt - ke + Ke - 1) / Ke;
      for (;;) {
        int i0 = 0;
        if (lane == 0) i0 = atomicAdd(&s_next, gpw);
        i0 = __shfl(i0, 0, 64);
        if (i0 >= nk) break;  // uniform within the wave
        const int j = ke + Ke * (i0 + gsub);
        if (i0 + gsub < nk) {  // uniform within a lane group
          const int v = wl[j];
          const uint32_t chv = ch[v - m];
          const int l = (int)(chv & 0xFFFFu), r = (int)(chv >> 16);
          const bool li = l >= m, ri = r >= m;
          uint32_t o = 0;
          if (li || ri) {
            const bool rev = (pri[v - m] & 1u) == 0;  // a follow-up visit draws its own numbers
            const uint32_t swv = sw | (rev ? 0x80000000u : 0u);
            const TsaU4 rnd = tsa_philox(TsaU4{(uint32_t)v, swv, (uint32_t)c, 0u}, P.key0, P.key1);
            const int rule = tsa_pick_rule(li, ri, rnd.x);
            const int slotP = tsa_slot_p(rule), slotM = tsa_slot_m(rule);
            const int Pn = slotP ? r : l, On = slotP ? l : r;
            const uint32_t chp = ch[Pn - m];
            const int Mn = slotM ? (int)(chp >> 16) : (int)(chp & 0xFFFFu);
            const int Kn = slotM ? (int)(chp & 0xFFFFu) : (int)(chp >> 16);
            const TsaW2* qD = reinterpret_cast<const TsaW2*>(lab + (size_t)(v - m) * NW);
            TsaW2* qP = reinterpret_cast<TsaW2*>(lab + (size_t)(Pn - m) * NW);
            const TsaW2* qO = reinterpret_cast<const TsaW2*>(On >= m ? lab + (size_t)(On - m) * NW : leaf + (size_t)On * NW);
            const TsaW2* qK = reinterpret_cast<const TsaW2*>(Kn >= m ? lab + (size_t)(Kn - m) * NW : leaf + (size_t)Kn * NW);
            const TsaW2* qM = reinterpret_cast<const TsaW2*>(Mn >= m ? lab + (size_t)(Mn - m) * NW : leaf + (size_t)Mn * NW);
            TsaCounts cn;
            tsa_counts_zero(cn);
            // tc mode: the costs of P and v before the move and P's size come from the node-cost cache
            // (exact: every accept rewrites both costs and P's size, and a sweep starts from a full pass), so
            // P's set is never read
            int costP = 0, costV = 0, szP = 0;
            if constexpr (CACHED) {
              const size_t cb = (size_t)c * nint4;
              costP = (int)sy.ncost[cb + (Pn - m)];
              costV = (int)sy.ncost[cb + (v - m)];
              szP = (int)sy.nz[cb + (Pn - m)];
            }
            constexpr int SC = TsaSumRound<G>::SC;
            constexpr int XN = SUMS ? SC : tsa_wide_cpl(G);
            TsaW2 xx[XN];  // only X stays live across the energy evaluation
            // SUMS: the population count of the union (uniform in the group) and the chunk positions of this
            // lane's first round
            int pc = 0, ix[SC];
            if constexpr (SUMS) {
              // summary word q of node n: LDS, or HBM for an input tensor whose table is not staged
              auto sumw = [&](int n, int q) -> uint64_t {
                if (n >= m) return ssum[(size_t)(n - m) * nsw + q];
                return lsum_in_lds ? lsum[(size_t)n * nsw + q] : sy.leafsum[(size_t)n * nsw + q];
              };
              const uint64_t u0 = sumw(v, 0) | sumw(On, 0) | sumw(Kn, 0) | sumw(Mn, 0);
              const uint64_t u1 = nsw > 1 ? (sumw(v, 1) | sumw(On, 1) | sumw(Kn, 1) | sumw(Mn, 1)) : 0ull;
              pc = __popcll(u0) + __popcll(u1);
#pragma unroll
              for (int q = 0; q < SC; q++) {
                xx[q] = TsaW2{0ull, 0ull};
                ix[q] = -1;
              }
              // a chunk outside the union is zero in D, O, K and M, hence in P (a subset of K | M) and in X:
              // it adds nothing to any count, and P's and X's values there are both zero
              for (int r0 = 0; r0 < pc; r0 += SC * G) {  // one round unless the union has more than SC * G chunks
                int ii[SC];
                sum_pick<G, SC>(u0, u1, r0 + t, ii);
                TsaW2 dd[SC], pp[SC], oo[SC], kk[SC], mm[SC];
#pragma unroll
                for (int q = 0; q < SC; q++) {
                  if (ii[q] >= 0) {
                    dd[q] = qD[ii[q]];
                    if constexpr (!CACHED) pp[q] = qP[ii[q]];
                    oo[q] = qO[ii[q]];
                    kk[q] = qK[ii[q]];
                    mm[q] = qM[ii[q]];
                  } else {
                    dd[q] = pp[q] = oo[q] = kk[q] = mm[q] = TsaW2{0ull, 0ull};
                  }
                }
#pragma unroll
                for (int q = 0; q < SC; q++) {
                  TsaW2 x;
                  x.a = tsa_xset(kk[q].a, oo[q].a, mm[q].a, dd[q].a);
                  x.b = tsa_xset(kk[q].b, oo[q].b, mm[q].b, dd[q].b);
                  if constexpr (CACHED) {
                    tsa_acc_after_tc(cn, kk[q].a, mm[q].a, oo[q].a, dd[q].a, x.a);
                    tsa_acc_after_tc(cn, kk[q].b, mm[q].b, oo[q].b, dd[q].b, x.b);
                  } else {
                    tsa_acc<MODE>(cn, kk[q].a, mm[q].a, pp[q].a, oo[q].a, dd[q].a, x.a);
                    tsa_acc<MODE>(cn, kk[q].b, mm[q].b, pp[q].b, oo[q].b, dd[q].b, x.b);
                  }
                  if (r0 == 0) {
                    xx[q] = x;
                    ix[q] = ii[q];
                  }
                }
              }
            } else {
              constexpr int CPL = tsa_wide_cpl(G);
              TsaW2 dd[CPL], pp[CPL], oo[CPL], kk[CPL], mm[CPL];
#pragma unroll
              for (int q = 0; q < tsa_wide_cpl(G); q++) {
                const int cc = t + q * G;
                if (cc < nch) {
                  dd[q] = qD[cc];
                  if constexpr (!CACHED) pp[q] = qP[cc];
                  oo[q] = qO[cc];
                  kk[q] = qK[cc];
                  mm[q] = qM[cc];
                } else {
                  dd[q] = pp[q] = oo[q] = kk[q] = mm[q] = TsaW2{0ull, 0ull};
                }
              }
#pragma unroll
              for (int q = 0; q < tsa_wide_cpl(G); q++) {
                xx[q].a = tsa_xset(kk[q].a, oo[q].a, mm[q].a, dd[q].a);
                xx[q].b = tsa_xset(kk[q].b, oo[q].b, mm[q].b, dd[q].b);
                if constexpr (CACHED) {
                  tsa_acc_after_tc(cn, kk[q].a, mm[q].a, oo[q].a, dd[q].a, xx[q].a);
                  tsa_acc_after_tc(cn, kk[q].b, mm[q].b, oo[q].b, dd[q].b, xx[q].b);
                } else {
                  tsa_acc<MODE>(cn, kk[q].a, mm[q].a, pp[q].a, oo[q].a, dd[q].a, xx[q].a);
                  tsa_acc<MODE>(cn, kk[q].b, mm[q].b, pp[q].b, oo[q].b, dd[q].b, xx[q].b);
                }
              }
            }
            float dE;
            if constexpr (CACHED) {
              uint32_t pk[2] = {(uint32_t)cn.sd | ((uint32_t)cn.sx << 16), (uint32_t)cn.K[2] | ((uint32_t)cn.K[3] << 16)};
              group_sum<G, 2>(pk);
              cn.sd = (int)(pk[0] & 0xFFFFu);
              cn.sx = (int)(pk[0] >> 16);
              cn.K[2] = (int)(pk[1] & 0xFFFFu);
              cn.K[3] = (int)(pk[1] >> 16);
              dE = tsa_energy_tc_cached(costP, costV, szP, cn.sd, cn.sx, cn.K[2], cn.K[3], P.model, s_lse);
            } else {
              uint32_t pk[TsaFlat<MODE>::NP];
              counts_pack<MODE>(cn, pk);
              group_sum<G, TsaFlat<MODE>::NP>(pk);
              counts_unpack<MODE>(pk, cn);
              dE = tsa_energy_from_counts<MODE>(cn, P.model, s_lse, T);
            }
            const bool acc = tsa_metropolis(rnd.y, beta, dE, T.exp2);
            if (acc) {
              if constexpr (SUMS) {
                // X's chunks inside the union, and P's new summary (OR over the group).  The first round's
                // chunks are still in registers; later rounds (more than SC * G chunks, rare) rebuild the union
                // and the set pointers from LDS, so that neither stays live across the energy evaluation
                uint64_t xs0 = 0, xs1 = 0;
#pragma unroll
                for (int q = 0; q < SC; q++) {
                  if (ix[q] >= 0) {
                    qP[ix[q]] = xx[q];
                    if (xx[q].a | xx[q].b) {
                      if (ix[q] < 64) xs0 |= 1ull << ix[q];
                      else xs1 |= 1ull << (ix[q] - 64);
                    }
                  }
                }
                if (pc > SC * G) {  // uniform within the group
                  const uint32_t cv2 = ch[v - m];
                  const int l2 = (int)(cv2 & 0xFFFFu), r2 = (int)(cv2 >> 16);
                  const int O2 = slotP ? l2 : r2;
                  const uint32_t cp2 = ch[Pn - m];
                  const int M2 = slotM ? (int)(cp2 >> 16) : (int)(cp2 & 0xFFFFu);
                  const int K2 = slotM ? (int)(cp2 & 0xFFFFu) : (int)(cp2 >> 16);
                  const TsaW2* rD = reinterpret_cast<const TsaW2*>(lab + (size_t)(v - m) * NW);
                  const TsaW2* rO = reinterpret_cast<const TsaW2*>(O2 >= m ? lab + (size_t)(O2 - m) * NW : leaf + (size_t)O2 * NW);
                  const TsaW2* rK = reinterpret_cast<const TsaW2*>(K2 >= m ? lab + (size_t)(K2 - m) * NW : leaf + (size_t)K2 * NW);
                  const TsaW2* rM = reinterpret_cast<const TsaW2*>(M2 >= m ? lab + (size_t)(M2 - m) * NW : leaf + (size_t)M2 * NW);
                  auto sumw = [&](int n, int q) -> uint64_t {
                    if (n >= m) return ssum[(size_t)(n - m) * nsw + q];
                    return lsum_in_lds ? lsum[(size_t)n * nsw + q] : sy.leafsum[(size_t)n * nsw + q];
                  };
                  const uint64_t w0 = sumw(v, 0) | sumw(O2, 0) | sumw(K2, 0) | sumw(M2, 0);
                  const uint64_t w1 = nsw > 1 ? (sumw(v, 1) | sumw(O2, 1) | sumw(K2, 1) | sumw(M2, 1)) : 0ull;
                  for (int r0 = SC * G; r0 < pc; r0 += SC * G) {
                    int ii[SC];
                    sum_pick<G, SC>(w0, w1, r0 + t, ii);
#pragma unroll
                    for (int q = 0; q < SC; q++) {
                      if (ii[q] >= 0) {
                        const TsaW2 d = rD[ii[q]], o2 = rO[ii[q]], k2 = rK[ii[q]], m2 = rM[ii[q]];
                        TsaW2 x;
                        x.a = (k2.a | o2.a) & (m2.a | d.a);
                        x.b = (k2.b | o2.b) & (m2.b | d.b);
                        qP[ii[q]] = x;
                        if (x.a | x.b) {
                          if (ii[q] < 64) xs0 |= 1ull << ii[q];
                          else xs1 |= 1ull << (ii[q] - 64);
                        }
                      }
                    }
                  }
                }
#pragma unroll
                for (int o2 = G / 2; o2 > 0; o2 >>= 1) {
                  xs0 |= (uint64_t)__shfl_xor((unsigned long long)xs0, o2, G);
                  xs1 |= (uint64_t)__shfl_xor((unsigned long long)xs1, o2, G);
                }
                if (t == 0) {
                  // this workgroup's copy now (no other visit of the phase reads P's summary), the other
                  // workgroups' copies from HBM in their replay
                  ssum[(size_t)(Pn - m) * nsw] = xs0;
                  gsum[(size_t)(Pn - m) * nsw] = xs0;
                  if (nsw > 1) {
                    ssum[(size_t)(Pn - m) * nsw + 1] = xs1;
                    gsum[(size_t)(Pn - m) * nsw + 1] = xs1;
                  }
                }
              } else {
#pragma unroll
                for (int q = 0; q < tsa_wide_cpl(G); q++) {
                  const int cc = t + q * G;
                  if (cc < nch) qP[cc] = xx[q];
                }
              }
            }
            if (SUMS && t == 0) {
              nck += pc;
              nxk += acc ? pc : 0;
            }
            o = 8u | (acc ? 1u : 0u) | ((uint32_t)slotP << 1) | ((uint32_t)slotM << 2);
            if (t == 0) {
              np++;
              na += acc ? 1 : 0;
              if (acc) {
                // the two node costs the rotation changes: P with children K and O (O in M's slot) and v with
                // children P and M (M in O's slot); count3 order is (left child, right child, node)
                const size_t cb = (size_t)c * nint4;
                sy.ncost[cb + (Pn - m)] = tsa_node_cost<MODE>(cn.B[2], slotM ? cn.M[2] : cn.N[2],
                                                              slotM ? cn.N[2] : cn.M[2], cn.K[2], cn.sx, P.model, T);
                sy.nz[cb + (Pn - m)] = (uint16_t)cn.sx;
                sy.ncost[cb + (v - m)] = tsa_node_cost<MODE>(cn.B[3], slotP ? cn.N[3] : cn.M[3],
                                                             slotP ? cn.M[3] : cn.N[3], cn.K[3], cn.sd, P.model, T);
              }
            }
          }
          if (t == 0) {
            out[j] = (uint8_t)o;
            nv++;
          }
        }
      }

      // 3. barrier
      if constexpr (COOP) {
        nb++;
        if (!chain_barrier(sy, c, nb * (unsigned)Ke, &s_ok)) {
          ok = false;
          break;
        }
      } else {
        __syncthreads();
      }

      // 4. replay
      if (threadIdx.x == 0) {  // every thread read cnt before the visits; the next scan appends from 0
        s_cnt = 0;
        s_next = 0;
      }
      for (int j = threadIdx.x; j < cnt; j += NT) {
        const int v = wl[j];
        const uint32_t o = out[j];
        const uint32_t pv = pri[v - m];
        if (o & 1u) {
          const uint32_t chv = ch[v - m];
          const int slotP = (int)((o >> 1) & 1u), slotM = (int)((o >> 2) & 1u);
          const int l = (int)(chv & 0xFFFFu), r = (int)(chv >> 16);
          const int Pn = slotP ? r : l, On = slotP ? l : r;
          const uint32_t chp = ch[Pn - m];
          const int Mn = slotM ? (int)(chp >> 16) : (int)(chp & 0xFFFFu);
          ch[Pn - m] = slotM ? ((chp & 0xFFFFu) | ((uint32_t)On << 16)) : ((chp & 0xFFFF0000u) | (uint32_t)On);
          ch[v - m] = slotP ? ((chv & 0xFFFF0000u) | (uint32_t)Mn) : ((chv & 0xFFFFu) | ((uint32_t)Mn << 16));
          if (On >= m) par[On - m] = (uint16_t)Pn;
          if (Mn >= m) par[Mn - m] = (uint16_t)v;
          if (P.par_follow && (pv & 1u) && pri[Pn - m] == 0) pri[Pn - m] = (uint16_t)tsa_follow_pri((uint32_t)Pn, hs);
          if (SUMS && j % Ke != ke)  // P's new summary, written by another workgroup's visit
            for (int q = 0; q < nsw; q++) ssum[(size_t)(Pn - m) * nsw + q] = gsum[(size_t)(Pn - m) * nsw + q];
        }
        pri[v - m] = 0;
      }
      __syncthreads();
    }
    if (blocked && --left == 0) {
      // the level's end: its snapshot, the tree from LDS and the node-cost cache (final after the sweep's last
      // barrier), read by all before the next level's first accept rewrites the cache
      if (sy.blk_ch[lv]) {
        uint32_t* const sch = sy.blk_ch[lv] + (size_t)c * nint;
        for (int i = threadIdx.x; i < nint; i += NT) sch[i] = ch[i];
        const size_t cb = (size_t)c * nint4;
        tsa_copy_inflight<float, 8>(sy.blk_cost[lv] + cb, sy.ncost + cb, nint, threadIdx.x, NT);
        tsa_copy_inflight<uint16_t, 8>(sy.blk_nz[lv] + cb, sy.nz + cb, nint, threadIdx.x, NT);
        __syncthreads();
      }
      if (++lv < sy.blk_n) {
        left = sy.blk_niters[lv];
        beta = sy.blk_beta[lv];
      }
    }
  }

  if (ok && ke == 0) {
    for (int i = threadIdx.x; i < nint; i += NT) gch[i] = ch[i];
    if (sy.snap_ch) {  // the level's snapshot: tree from LDS, node costs (final after the last barrier)
      uint32_t* const sch = sy.snap_ch + (size_t)c * nint;
      for (int i = threadIdx.x; i < nint; i += NT) sch[i] = ch[i];
      if (sy.snap_cost) {
        const size_t cb = (size_t)c * nint4;
        tsa_copy_inflight<float, 8>(sy.snap_cost + cb, sy.ncost + cb, nint, threadIdx.x, NT);
        tsa_copy_inflight<uint16_t, 8>(sy.snap_nz + cb, sy.nz + cb, nint, threadIdx.x, NT);
      }
    }
  }
  if constexpr (!COOP && !SUMS) {
    // the launch's energies, folded by this workgroup rather than by a launch of their own: every accept
    // rewrote its entries of the node-cost cache before the loop's last barrier, so the cache is the final
    // tree's; the costs are staged in the sweep's LDS, whose last reads (the tree, above) end at the barrier
    if (sy.flc) {
      __syncthreads();
      const size_t cb = (size_t)c * nint4;
      wide_fold(P, c, sy.ncost + cb, sy.nz + cb, P.slicing ? lab + P.s_off : nullptr, leaf, fix, s_mt,
                nint4 * 6 <= Lo.bytes ? 1 : 0, tsa_wsm, sy.flc, sy.fsc, sy.fns);
    }
  }
  const long long sp_ = wide_wave_sum(np), sa_ = wide_wave_sum(na), sv_ = wide_wave_sum(nv);
  const long long sk_ = SUMS ? wide_wave_sum(nck) : 0, sx_ = SUMS ? wide_wave_sum(nxk) : 0;
  if (lane == 0) {  // counters spread over TSA_STAT_SLOTS addresses each, summed by the host
    unsigned long long* st = stats + ((c * 16 + wv) & (TSA_STAT_SLOTS - 1));
    atomicAdd(&st[TSA_ST_PROP * TSA_STAT_SLOTS], (unsigned long long)sp_);
    atomicAdd(&st[TSA_ST_ACC * TSA_STAT_SLOTS], (unsigned long long)sa_);
    atomicAdd(&st[TSA_ST_VISITS * TSA_STAT_SLOTS], (unsigned long long)sv_);
    atomicAdd(&st[TSA_ST_BUSY * TSA_STAT_SLOTS], (unsigned long long)sv_);
    if (ke == 0 && wv == 0) atomicAdd(&st[TSA_ST_STEPS * TSA_STAT_SLOTS], (unsigned long long)nst);
    if (SUMS) {
      atomicAdd(&st[TSA_ST_CHUNKS * TSA_STAT_SLOTS], (unsigned long long)sk_);
      atomicAdd(&st[TSA_ST_XCHUNKS * TSA_STAT_SLOTS], (unsigned long long)sx_);
    }
  }
  if constexpr (COOP) {
    __syncthreads();
    if (threadIdx.x == 0) chain_leave(sy, c, K);
  }
}

// Chain energies in two steps (csrc/treesa_gpu.cu:999-1014 computes both in one 32-lane loop):
// node costs -- G lanes per internal node count B, M, N, K, Z of (left, right) -> node with label sets
// masked by ~S, and the group leader stores tsa_node_cost and Z -- by eK workgroups per chain (skipped when
// nodes = 0: the sweep kernel has kept the cached costs current); then the last workgroup of the chain to
// finish folds them in the reference's 32-lane order (lane t folds nodes t, t+32, ... from -inf with
// lse_f, then an xor butterfly 16, 8, 4, 2, 1), so lcost is bit-identical to the one-loop evaluation.
template <int G, int MODE>
__global__ void __launch_bounds__(256) k_wcost(TsaKParams P, const uint64_t* __restrict__ rec,
                                               const uint64_t* __restrict__ leaf, const uint32_t* __restrict__ fix,
                                               int nchains, int K2, int nodes, int stage, float* __restrict__ ncost,
                                               uint16_t* __restrict__ nz, unsigned* __restrict__ fcnt,
                                               float* __restrict__ lc, int* __restrict__ sc, int* __restrict__ ns,
                                               TsaSums sums, TsaFoldLevels FL) {
  // LDS (stage != 0): the chain's node costs f32[nint4] and sizes u16[nint4], then (stage == 2) the log2f
  // summary bitmap at the next 16-byte boundary
  extern __shared__ __align__(16) unsigned char s_dyn[];
  __shared__ uint64_t s_mt[TSA_MT_WORDS];
  __shared__ int s_last;
  tsa_math_stage(s_mt);
  __syncthreads();
  const uint32_t* const gmap = fix + TSA_LOG2FIX_WORDS;
  const int c = blockIdx.x / K2, k = blockIdx.x - c * K2;
  if (c >= nchains) return;
  const int m = P.m, nint = P.nint, nint4 = (nint + 3) & ~3, NW = P.W, nch = NW >> 1;
  const uint64_t* const lab = rec + (size_t)c * P.chain_words;
  const uint64_t* const S = P.slicing ? lab + P.s_off : nullptr;
  if (FL.n > 0) {  // several levels' folds (nodes = 0): this workgroup's level is blockIdx.y
    const int li = (int)blockIdx.y;
    wide_fold(P, c, FL.cost[li] + (size_t)c * nint4, FL.z[li] + (size_t)c * nint4, S, leaf, fix, s_mt, stage, s_dyn,
              FL.lc[li], FL.sc[li], FL.ns[li]);
    return;
  }
  float* const cst = ncost + (size_t)c * nint4;
  uint16_t* const zz = nz + (size_t)c * nint4;

  if (nodes) {
    const TsaMathTabs T{s_mt, fix, gmap, s_mt + 32};
    const uint32_t* const ch = reinterpret_cast<const uint32_t*>(lab + P.ch_off);
    const int gpb = (int)blockDim.x / G, grp = (int)threadIdx.x / G, t = (int)threadIdx.x & (G - 1);
    const int npb = (nint + K2 - 1) / K2, i0 = k * npb, i1 = (i0 + npb < nint) ? i0 + npb : nint;
    constexpr int CPL = tsa_wide_cpl(G);
    TsaW2 sm[CPL];
#pragma unroll
    for (int q = 0; q < CPL; q++) {
      const int cc = t + q * G;
      if (S && cc < nch) {
        const TsaW2 sv = reinterpret_cast<const TsaW2*>(S)[cc];
        sm[q] = TsaW2{~sv.a, ~sv.b};
      } else {
        sm[q] = TsaW2{~0ull, ~0ull};
      }
    }
    for (int b = i0; b < i1; b += gpb) {
      const int i = b + grp;
      if (i < i1) {  // uniform within a lane group
        const uint32_t cw = ch[i];
        const int l = (int)(cw & 0xFFFFu), r = (int)(cw >> 16);
        const TsaW2* qx = reinterpret_cast<const TsaW2*>(l >= m ? lab + (size_t)(l - m) * NW : leaf + (size_t)l * NW);
        const TsaW2* qy = reinterpret_cast<const TsaW2*>(r >= m ? lab + (size_t)(r - m) * NW : leaf + (size_t)r * NW);
        const TsaW2* qz = reinterpret_cast<const TsaW2*>(lab + (size_t)i * NW);
        // with summaries only the chunks in the union of the three sets' summaries are read (a chunk outside it
        // is zero in all three and adds nothing to any count)
        uint64_t u0 = ~0ull, u1 = ~0ull;
        if (sums.nsw) {
          const int nsw = sums.nsw;
          const uint64_t* const is = sums.isum + (size_t)c * nint4 * nsw;
          auto sw = [&](int n, int q) -> uint64_t {
            return n >= m ? is[(size_t)(n - m) * nsw + q] : sums.lsum[(size_t)n * nsw + q];
          };
          u0 = sw(l, 0) | sw(r, 0) | is[(size_t)i * nsw];
          u1 = nsw > 1 ? (sw(l, 1) | sw(r, 1) | is[(size_t)i * nsw + 1]) : 0ull;
        }
        TsaW2 xx[CPL], yy[CPL], zv[CPL];
#pragma unroll
        for (int q = 0; q < CPL; q++) {
          const int cc = t + q * G;
          if (cc < nch && (((cc < 64 ? u0 >> cc : u1 >> (cc - 64)) & 1ull) != 0ull)) {
            xx[q] = qx[cc];
            yy[q] = qy[cc];
            zv[q] = qz[cc];
          } else {
            xx[q] = yy[q] = zv[q] = TsaW2{0ull, 0ull};
          }
        }
        int B = 0, M = 0, N = 0, Kc = 0, Z = 0;
#pragma unroll
        for (int q = 0; q < CPL; q++) {
          const uint64_t za = zv[q].a & sm[q].a, zb = zv[q].b & sm[q].b;
          tsa_count3(xx[q].a & sm[q].a, yy[q].a & sm[q].a, za, B, M, N, Kc);
          tsa_count3(xx[q].b & sm[q].b, yy[q].b & sm[q].b, zb, B, M, N, Kc);
          Z += __popcll(za) + __popcll(zb);
        }
        uint32_t a[3] = {(uint32_t)B | ((uint32_t)M << 16), (uint32_t)N | ((uint32_t)Kc << 16), (uint32_t)Z};
        group_sum<G, 3>(a);
        if (t == 0) {
          B = (int)(a[0] & 0xFFFFu);
          M = (int)(a[0] >> 16);
          N = (int)(a[1] & 0xFFFFu);
          Kc = (int)(a[1] >> 16);
          Z = (int)a[2];
          cst[i] = tsa_node_cost<MODE>(B, M, N, Kc, Z, P.model, T);
          zz[i] = (uint16_t)Z;
        }
      }
    }
    // the last workgroup of the chain to finish folds
    __syncthreads();
    if (threadIdx.x == 0) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      const unsigned old = __hip_atomic_fetch_add(fcnt + c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int last = old == (unsigned)(K2 - 1);
      if (last) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        __hip_atomic_store(fcnt + c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      s_last = last;
    }
    __syncthreads();
    if (!s_last) return;
  }

  wide_fold(P, c, cst, zz, S, leaf, fix, s_mt, stage, s_dyn, lc, sc, ns);
}

template <int G, int MODE, bool SUMS>
hipError_t launch_wide_gms(const TsaWide& X, const TsaKParams& P, uint64_t* rec, const uint64_t* leaf,
                           const uint32_t* fix, int nchains, float beta, uint32_t sweep0, int nsweeps,
                           unsigned long long* stats, const TsaWideSync& sy, hipStream_t st, hipEvent_t e0,
                           hipEvent_t e1) {
  // e0 / e1 (null: none) take the kernel's start and stop times in the dispatch itself
  if (X.K > 1) {
    // an ordinary launch: the plan admits K > 1 only when all nchains * K workgroups fit on the device at
    // once, so on an idle device they are all resident together (the cooperative launch API gives the same
    // guarantee but costs tens of microseconds per launch on the host side); if they ever are not, a chain
    // barrier runs out of polls, sets the error word and every workgroup leaves
    const int nchainsx = (nchains + X.nxcd - 1) / X.nxcd * X.nxcd;  // (chains grouped by XCD, see k_wide)
    hipExtLaunchKernelGGL((k_wide<G, MODE, true, SUMS>), dim3(nchainsx * X.K), dim3(X.nt), (uint32_t)X.smem, st, e0,
                          e1, 0u, P, rec, leaf, fix, nchains, X.K, beta, sweep0, nsweeps, stats, sy);
    return hipGetLastError();
  }
  hipExtLaunchKernelGGL((k_wide<G, MODE, false, SUMS>), dim3(nchains), dim3(X.nt), (uint32_t)X.smem, st, e0, e1, 0u,
                        P, rec, leaf, fix, nchains, 1, beta, sweep0, nsweeps, stats, sy);
  return hipGetLastError();
}

template <int G, bool SUMS>
hipError_t launch_wide_g(const TsaWide& X, int mode, const TsaKParams& P, uint64_t* rec, const uint64_t* leaf,
                         const uint32_t* fix, int nchains, float beta, uint32_t sweep0, int nsweeps,
                         unsigned long long* stats, const TsaWideSync& sy, hipStream_t st, hipEvent_t e0,
                         hipEvent_t e1) {
  if (mode == 0)
    return launch_wide_gms<G, 0, SUMS>(X, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, sy, st, e0, e1);
  if (mode == 1)
    return launch_wide_gms<G, 1, SUMS>(X, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, sy, st, e0, e1);
  return launch_wide_gms<G, 2, SUMS>(X, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, sy, st, e0, e1);
}

template <int G, int MODE>
hipError_t launch_wcost_gm(const TsaWide& X, const TsaKParams& P, const uint64_t* rec, const uint64_t* leaf,
                           const uint32_t* fix, int nchains, float* ncost, uint16_t* nz, unsigned* fcnt, float* lc,
                           int* sc, int* ns, int nodes, hipStream_t st, TsaSums sums) {
  const int K2 = nodes ? X.eK : 1;
  const int stage = nodes ? (X.fold_smem > 0 ? 1 : 0) : X.fold_stage;
  const size_t smem = stage == 2 ? (size_t)X.fold_smem_map : stage == 1 ? (size_t)X.fold_smem : 0;
  hipLaunchKernelGGL((k_wcost<G, MODE>), dim3(nchains * K2), dim3(256), smem, st, P, rec, leaf, fix, nchains, K2, nodes,
                     stage, ncost, nz, fcnt, lc, sc, ns, sums, TsaFoldLevels{});
  return hipGetLastError();
}

template <int G, int MODE>
hipError_t launch_wfold_levels_gm(const TsaWide& X, const TsaKParams& P, const uint64_t* rec, const uint64_t* leaf,
                                  const uint32_t* fix, int nchains, const TsaFoldLevels& F, hipStream_t st) {
  const int stage = X.fold_stage;
  const size_t smem = stage == 2 ? (size_t)X.fold_smem_map : stage == 1 ? (size_t)X.fold_smem : 0;
  hipLaunchKernelGGL((k_wcost<G, MODE>), dim3(nchains, F.n), dim3(256), smem, st, P, rec, leaf, fix, nchains, 1, 0,
                     stage, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, TsaSums{nullptr, nullptr, 0}, F);
  return hipGetLastError();
}

template <int G>
hipError_t launch_wcost_g(const TsaWide& X, int mode, const TsaKParams& P, const uint64_t* rec, const uint64_t* leaf,
                          const uint32_t* fix, int nchains, float* ncost, uint16_t* nz, unsigned* fcnt, float* lc,
                          int* sc, int* ns, int nodes, hipStream_t st, TsaSums sums) {
  if (mode == 0) return launch_wcost_gm<G, 0>(X, P, rec, leaf, fix, nchains, ncost, nz, fcnt, lc, sc, ns, nodes, st, sums);
  if (mode == 1) return launch_wcost_gm<G, 1>(X, P, rec, leaf, fix, nchains, ncost, nz, fcnt, lc, sc, ns, nodes, st, sums);
  return launch_wcost_gm<G, 2>(X, P, rec, leaf, fix, nchains, ncost, nz, fcnt, lc, sc, ns, nodes, st, sums);
}

// Largest number of co-resident workgroups per CU of the multi-workgroup sweep kernel over the three modes,
// at smem bytes of dynamic LDS.  Raises the dynamic-LDS cap of every sweep instantiation of this G to
// lds_cap first (the largest any context asks for).
template <int G, bool SUMS>
hipError_t wide_occupancy(int nt, int smem, int lds_cap, int* per_cu) {
  const void* coop[3] = {reinterpret_cast<const void*>(&k_wide<G, 0, true, SUMS>),
                         reinterpret_cast<const void*>(&k_wide<G, 1, true, SUMS>),
                         reinterpret_cast<const void*>(&k_wide<G, 2, true, SUMS>)};
  const void* one[3] = {reinterpret_cast<const void*>(&k_wide<G, 0, false, SUMS>),
                        reinterpret_cast<const void*>(&k_wide<G, 1, false, SUMS>),
                        reinterpret_cast<const void*>(&k_wide<G, 2, false, SUMS>)};
  for (int i = 0; i < 6; i++) {
    const hipError_t e =
        hipFuncSetAttribute(i < 3 ? coop[i] : one[i - 3], hipFuncAttributeMaxDynamicSharedMemorySize, lds_cap);
    if (e != hipSuccess) return e;
  }
  int best = 1 << 30;
  for (int i = 0; i < 3; i++) {
    int nb = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, coop[i], nt, (size_t)smem);
    if (e != hipSuccess) return e;
    best = nb < best ? nb : best;
  }
  *per_cu = best;
  return hipSuccess;
}

template <int G>
hipError_t wcost_lds_cap(int lds_cap) {
  const void* fns[3] = {reinterpret_cast<const void*>(&k_wcost<G, 0>), reinterpret_cast<const void*>(&k_wcost<G, 1>),
                        reinterpret_cast<const void*>(&k_wcost<G, 2>)};
  for (int i = 0; i < 3; i++) {
    const hipError_t e = hipFuncSetAttribute(fns[i], hipFuncAttributeMaxDynamicSharedMemorySize, lds_cap);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t wide_occupancy_g(int G, bool sums, int nt, int smem, int lds_cap, int* per_cu) {
  if (sums) {
    switch (G) {
      case 1: return wide_occupancy<1, true>(nt, smem, lds_cap, per_cu);
      case 2: return wide_occupancy<2, true>(nt, smem, lds_cap, per_cu);
      case 4: return wide_occupancy<4, true>(nt, smem, lds_cap, per_cu);
      case 8: return wide_occupancy<8, true>(nt, smem, lds_cap, per_cu);
      case 16: return wide_occupancy<16, true>(nt, smem, lds_cap, per_cu);
      default: return hipErrorInvalidValue;
    }
  }
  switch (G) {
    case 4: return wide_occupancy<4, false>(nt, smem, lds_cap, per_cu);
    case 8: return wide_occupancy<8, false>(nt, smem, lds_cap, per_cu);
    case 16: return wide_occupancy<16, false>(nt, smem, lds_cap, per_cu);
    case 32: return wide_occupancy<32, false>(nt, smem, lds_cap, per_cu);
    case 64: return wide_occupancy<64, false>(nt, smem, lds_cap, per_cu);
    default: return hipErrorInvalidValue;
  }
}

hipError_t wcost_lds_cap_g(int G, int lds_cap) {
  switch (G) {
    case 4: return wcost_lds_cap<4>(lds_cap);
    case 8: return wcost_lds_cap<8>(lds_cap);
    case 16: return wcost_lds_cap<16>(lds_cap);
    case 32: return wcost_lds_cap<32>(lds_cap);
    case 64: return wcost_lds_cap<64>(lds_cap);
    default: return hipErrorInvalidValue;
  }
}

// Summaries of every internal set of every chain: one wave per set, lane l tests chunks l and l + 64.
__global__ void __launch_bounds__(256) k_wsum(TsaKParams P, const uint64_t* __restrict__ rec, int nchains, int nsw,
                                              uint64_t* __restrict__ sum) {
  const int lane = threadIdx.x & 63, nint = P.nint, nint4 = (nint + 3) & ~3, nch = P.W >> 1;
  const long long nsets = (long long)nchains * nint;
  const long long step = (long long)gridDim.x * (blockDim.x >> 6);
  for (long long s = (long long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); s < nsets; s += step) {
    const int c = (int)(s / nint), i = (int)(s - (long long)c * nint);
    const TsaW2* q = reinterpret_cast<const TsaW2*>(rec + (size_t)c * P.chain_words + (size_t)i * P.W);
    for (int h = 0; h < nsw; h++) {
      const int cc = h * 64 + lane;
      bool nz = false;
      if (cc < nch) {
        const TsaW2 x = q[cc];
        nz = (x.a | x.b) != 0ull;
      }
      const uint64_t b = __ballot(nz);
      if (lane == 0) sum[((size_t)c * nint4 + i) * nsw + h] = b;
    }
  }
}

}  // namespace

hipError_t tsa_wide_plan(const TsaKParams& P, int nchains, int want_waves, int want_k, int want_g, int sums,
                         TsaWide* out) {
  TsaWide X{};
  const int nch = P.W / 2;
  if ((P.W & 1) || nch < 1 || nch > tsa_wide_cpl(64) * 64) return hipErrorInvalidValue;
  // dense streaming needs G * tsa_wide_cpl(G) >= chunks per set; the energy kernel always streams densely
  int Gd = 4;
  while (Gd < 64 && (nch + Gd - 1) / Gd > tsa_wide_cpl(Gd)) Gd *= 2;
  X.nsw = (sums > 0 || (sums == 0 && P.W >= 64)) ? (nch + 63) / 64 : 0;
  // summaries: one lane per proposal (the union of a visit is a few chunks: whole-wave SIMD efficiency
  // matters more than spreading loads) and one workgroup per chain (no chain barriers)
  int G = want_g > 0 ? want_g : (X.nsw ? 1 : Gd);
  if (X.nsw ? (G < 1 || G > 16 || (G & (G - 1))) : (G < Gd || G > 64 || (G & (G - 1)))) return hipErrorInvalidValue;
  X.G = G;
  int dev = 0, ncu = 0, lds_max = 0, nxcd = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
  if (e != hipSuccess) return e;
  // XCDs of the device (8 on MI355X in its single-partition mode, 1 per partition otherwise)
  if (hipDeviceGetAttribute(&nxcd, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || nxcd < 1 || nxcd > ncu) {
    (void)hipGetLastError();
    nxcd = 1;
  }
  X.nxcd = nxcd;
  // measured on MI355X: with at least one chain per CU, one 8-wave workgroup per chain streams best; with
  // fewer chains, 16-wave workgroups, as many per chain as stay co-resident
  // (the summary path is compiled for at most 8 waves per workgroup: its visit needs more registers)
  const int max_waves = X.nsw ? 8 : 16;
  int waves = want_waves > 0 ? want_waves : (nchains >= ncu ? 8 : max_waves);
  waves = waves < 1 ? 1 : (waves > max_waves ? max_waves : waves);
  X.nt = 64 * waves;
  const int band = P.par_band > 0 ? 1 : 0;
  // dynamic LDS cap: the device maximum less room for the kernels' static LDS (under 1 KB today)
  const int nint4 = (P.nint + 3) & ~3, lds_cap = lds_max - 4096;
  if (X.nsw) {  // the input tensors' summaries go to LDS too when they fit
    X.lsum_lds = tsa_wide_lds(P.nint, band, 0, X.nsw, P.m).bytes <= lds_cap ? 1 : 0;
    if (!X.lsum_lds && tsa_wide_lds(P.nint, band, 0, X.nsw, 0).bytes > lds_cap) {
      if (sums > 0 || want_g > 0) return hipErrorInvalidValue;
      X.nsw = 0;  // automatic summaries: the summary table does not fit beside the node arrays
      G = Gd;
      X.G = G;
      waves = want_waves > 0 ? want_waves : (nchains >= ncu ? 8 : 16);
      waves = waves < 1 ? 1 : (waves > 16 ? 16 : waves);
      X.nt = 64 * waves;
    }
  }
  const int mlds = X.lsum_lds ? P.m : 0;
  const TsaWideLds L1 = tsa_wide_lds(P.nint, band, 0, X.nsw, mlds), Lc = tsa_wide_lds(P.nint, band, 1, X.nsw, mlds);
  if (L1.bytes > lds_cap) return hipErrorInvalidValue;
  // the fold stages a chain's node costs (6 B per node) and, when it also fits, the log2f summary bitmap
  X.fold_smem = nint4 * 6 <= lds_cap ? nint4 * 6 : 0;
  X.fold_smem_map = ((nint4 * 6 + 15) & ~15) + (int)TSA_LOG2MAP_WORDS * 4;
  X.fold_stage = X.fold_smem == 0 ? 0 : (X.fold_smem_map <= lds_cap ? 2 : 1);
  int per_cu = 0;
  e = wide_occupancy_g(G, X.nsw > 0, X.nt, L1.bytes, lds_cap, &per_cu);
  if (e == hipSuccess) e = wcost_lds_cap_g(Gd, lds_cap);
  if (e != hipSuccess) return e;
  if (per_cu < 1) return hipErrorInvalidValue;
  // with K > 1 a chain's workgroups share one XCD (see k_wide): the chains of the fullest XCD times K must
  // be resident on its ncu / nxcd compute units at once (when they are not -- the device is shared with other
  // work -- a chain's check-in times out and one of its workgroups sweeps it alone)
  const int kmax = per_cu * (ncu / nxcd) / ((nchains + nxcd - 1) / nxcd);
  int K = want_k > 0 ? want_k : (X.nsw ? 1 : kmax);
  K = K < 1 ? 1 : (K > TSA_WIDE_MAX_K ? TSA_WIDE_MAX_K : K);
  if (K > 1 && K > kmax) return hipErrorCooperativeLaunchTooLarge;
  X.K = K;
  X.smem = K > 1 ? Lc.bytes : L1.bytes;
  X.eG = Gd;
  const int gpb = 256 / Gd, maxk = (P.nint + gpb - 1) / gpb;
  int eK = (4 * ncu + nchains - 1) / nchains;
  X.eK = eK < 1 ? 1 : (eK > maxk ? maxk : eK);
  X.on = 1;
  *out = X;
  return hipSuccess;
}

hipError_t tsa_launch_wide(const TsaWide& X, int mode, const TsaKParams& P, uint64_t* rec, const uint64_t* leaf,
                           const uint32_t* fix, int nchains, float beta, uint32_t sweep0, int nsweeps,
                           unsigned long long* stats, const TsaWideSync& sy, hipStream_t st, hipEvent_t e0,
                           hipEvent_t e1) {
  if (X.nsw) {
    switch (X.G) {
      case 1: return launch_wide_g<1, true>(X, mode, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, sy, st, e0, e1);
      case 2: return launch_wide_g<2, true>(X, mode, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, sy, st, e0, e1);
      case 4: return launch_wide_g<4, true>(X, mode, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, sy, st, e0, e1);
      case 8: return launch_wide_g<8, true>(X, mode, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, sy, st, e0, e1);
      case 16: return launch_wide_g<16, true>(X, mode, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, sy, st, e0, e1);
      default: return hipErrorInvalidValue;
    }
  }
  switch (X.G) {
    case 4: return launch_wide_g<4, false>(X, mode, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, sy, st, e0, e1);
    case 8: return launch_wide_g<8, false>(X, mode, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, sy, st, e0, e1);
    case 16: return launch_wide_g<16, false>(X, mode, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, sy, st, e0, e1);
    case 32: return launch_wide_g<32, false>(X, mode, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, sy, st, e0, e1);
    case 64: return launch_wide_g<64, false>(X, mode, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, sy, st, e0, e1);
    default: return hipErrorInvalidValue;
  }
}

hipError_t tsa_launch_wsum(const TsaWide& X, const TsaKParams& P, const uint64_t* rec, int nchains, uint64_t* sum,
                           hipStream_t st) {
  if (!X.nsw) return hipSuccess;
  const long long nsets = (long long)nchains * P.nint;
  const long long nb = (nsets + 3) / 4;
  const int grid = (int)(nb < 8192 ? nb : 8192);
  hipLaunchKernelGGL(k_wsum, dim3(grid), dim3(256), 0, st, P, rec, nchains, X.nsw, sum);
  return hipGetLastError();
}

hipError_t tsa_launch_wide_energy(const TsaWide& X, int mode, const TsaKParams& P, const uint64_t* rec,
                                  const uint64_t* leaf, const uint32_t* fix, int nchains, float* ncost,
                                  uint16_t* nz, unsigned* fcnt, float* lc, int* sc, int* ns, int nodes,
                                  hipStream_t st, TsaSums sums) {
  if (!nodes || !sums.isum || !sums.lsum) sums.nsw = 0;
  switch (X.eG) {
    case 4: return launch_wcost_g<4>(X, mode, P, rec, leaf, fix, nchains, ncost, nz, fcnt, lc, sc, ns, nodes, st, sums);
    case 8: return launch_wcost_g<8>(X, mode, P, rec, leaf, fix, nchains, ncost, nz, fcnt, lc, sc, ns, nodes, st, sums);
    case 16: return launch_wcost_g<16>(X, mode, P, rec, leaf, fix, nchains, ncost, nz, fcnt, lc, sc, ns, nodes, st, sums);
    case 32: return launch_wcost_g<32>(X, mode, P, rec, leaf, fix, nchains, ncost, nz, fcnt, lc, sc, ns, nodes, st, sums);
    case 64: return launch_wcost_g<64>(X, mode, P, rec, leaf, fix, nchains, ncost, nz, fcnt, lc, sc, ns, nodes, st, sums);
    default: return hipErrorInvalidValue;
  }
}

hipError_t tsa_launch_wide_fold_levels(const TsaWide& X, int mode, const TsaKParams& P, const uint64_t* rec,
                                       const uint64_t* leaf, const uint32_t* fix, int nchains,
                                       const TsaFoldLevels& F, hipStream_t st) {
  if (F.n < 1 || F.n > TSA_BLOCK_MAX) return hipErrorInvalidValue;
#define TSA_WFL(G)                                                                             \
  return mode == 0 ? launch_wfold_levels_gm<G, 0>(X, P, rec, leaf, fix, nchains, F, st)        \
         : mode == 1 ? launch_wfold_levels_gm<G, 1>(X, P, rec, leaf, fix, nchains, F, st)      \
                     : launch_wfold_levels_gm<G, 2>(X, P, rec, leaf, fix, nchains, F, st)
  switch (X.eG) {
    case 4: TSA_WFL(4);
    case 8: TSA_WFL(8);
    case 16: TSA_WFL(16);
    case 32: TSA_WFL(32);
    case 64: TSA_WFL(64);
    default: return hipErrorInvalidValue;
  }
#undef TSA_WFL
}
