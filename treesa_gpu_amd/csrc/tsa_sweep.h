// tsa_sweep.h -- the sweep kernel k_sweep for gfx950 (MI355X), its device functions and the launchers of its
// variants.
//
// One wave64 owns one chain.  A workgroup holds several waves (chains) that never wait on each other
// after the prologue.  When the chain record fits, it is staged in LDS together with the shared leaf
// table (LDS variant: every label-set access is a ds_read); otherwise the record stays in HBM and only
// the per-node arrays live in LDS (global variant, runtime label width).
//
// A sweep gives every internal node exactly one proposal.  Par order (the reference's k_par,
// csrc/treesa_gpu.cu:829-997): random 16-bit priorities per node and sweep; each phase scans the
// internal nodes not yet visited (all of them on chains of more than 512 nodes or with par_follow),
// compacts the independent set (unvisited nodes whose (priority, id) key beats their unvisited parent and
// internal children) into a work list with a 64-lane ballot, and visits it 64 nodes at a time, one node
// per lane; the sweep ends when no node is left unvisited.  Pre-order (the reference's k_warp, csrc/treesa_gpu.cu:585-722):
// a work list of ready nodes (parent already visited), up to 64 visited per step, children pushed by
// ballot prefix.  Every visit draws Philox((node, sweep, chain)), so both mappings reproduce the CPU
// recursion and the CPU phase-by-phase sweep bit for bit.
//
// Wave-local ordering: lanes of one wave exchange data only through LDS/global words that a later
// instruction of the same wave reads; tsa_wave_sync() (wavefront-scope release/acquire fences around
// a wave barrier) keeps the compiler from moving those accesses across the exchange points.
//
// Included by two translation units that instantiate the kernel's two SLICE variants, so that they compile
// in parallel: tsa_kernels.hip (SLICE = false: label sets never masked, no slice step) and tsa_sweep_sliced.hip
// (SLICE = true: masked sets and the slice step).  tsa_launch_sweeps picks the variant by P.slicing.
#pragma once
#include "tsa_kernels.h"
#include "tsa_fold.h"

__device__ __forceinline__ void tsa_wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint64_t tsa_lt_mask(int lane) { return (1ull << lane) - 1ull; }

// position of the n-th (0-based) set bit of x, n < popc(x)
__device__ __forceinline__ int tsa_nth_bit(uint64_t x, int n) {
  for (int k = 0; k < n; k++) x &= x - 1;
  return __ffsll((unsigned long long)x) - 1;
}

// n-th label (set bit) of A & ~S over NW words; S may be null (csrc/treesa_gpu.cu:125-133)
__device__ __forceinline__ int tsa_nth_label(const uint64_t* A, const uint64_t* S, int NW, int n) {
  for (int w = 0; w < NW; w++) {
    const uint64_t a = A[w] & (S ? ~S[w] : ~0ull);
    const int c = __popcll(a);
    if (n < c) return w * 64 + tsa_nth_bit(a, n);
    n -= c;
  }
  return -1;
}

// Metropolis of a visit: with draws made ahead (PRE), x = -beta * dE against the node's threshold T(u), the
// least float whose expf exceeds u (a number for every u the kernels draw, u = 0 included); else u < expf(x).
template <bool PRE>
__device__ __forceinline__ bool tsa_visit_accept(uint32_t ry, float thr, float beta, float dE, const TsaMathTabs& T) {
  if constexpr (PRE) return -beta * dE >= thr;
  else return tsa_metropolis(ry, beta, dE, T.exp2);
}

// Draws of one sweep made ahead: internal node i's first Philox word and Metropolis threshold, threads
// t0, t0 + ts, ... of the workgroup.
__device__ __forceinline__ void tsa_draw_ahead(const TsaKParams& P, uint32_t* dx, float* dt, uint32_t sw,
                                               uint32_t chain, int t0, int ts, const uint64_t* exp2tab) {
  for (int i = t0; i < P.nint; i += ts) {
    const TsaU4 r = tsa_philox(TsaU4{(uint32_t)(P.m + i), sw, chain, 0u}, P.key0, P.key1);
    dx[i] = r.x;
    dt[i] = tsa_accept_threshold(r.y, exp2tab);
  }
}

struct TsaVisit {
  uint32_t cw;  // the visited node's children word after the visit
  int Pn, On, Mn;
  bool prop, acc;
};

// One proposal at internal node v by one lane (csrc/treesa_gpu.cu:156-235; CPU twin
// csrc/cpu_ref.h:87-126).  lf: leaf sets (m*NW words), lab: internal sets, ch: children words, Sm: slice
// set (SL: slicing on; else unused and no masking).  UNI: the leaf sets sit right below the internal ones
// (lab == lf + m*NW), so that any node's set is at lf + node*NW without a select.  With P the pivot child,
// O the other child, M the grandchild under P that moves up and K the one that stays, every rule swaps M and
// O, and P gets X = (K|O)&(M|d).  PRE: pre_x / pre_t hold every internal node's first Philox word and
// Metropolis threshold for this sweep, drawn ahead; they are read beside the children word, so that the rule
// is known when that word arrives.  Else the visit draws its own.  CC (tc mode, no slicing, register width):
// cc_cost / cc_size hold every internal node's cost and size, exact on entry; the costs of P and v before the
// move and P's size come from there instead of from P's set (the same dE: tsa_energy_tc_cached), and an accept
// rewrites the two costs and P's size.
template <int W, int MODE, bool SL, bool UNI, bool PRE, bool CC = false>
__device__ __forceinline__ TsaVisit tsa_visit(const TsaKParams& P, uint64_t* lab, uint32_t* ch, const uint64_t* Sm,
                                              const uint64_t* lf, const float* lse, const TsaMathTabs& T, int v,
                                              float beta, uint32_t sw, uint32_t chain,
                                              const uint32_t* pre_x = nullptr, const float* pre_t = nullptr,
                                              float* cc_cost = nullptr, uint16_t* cc_size = nullptr) {
  static_assert(!CC || (MODE == 0 && !SL && W > 0), "the cost cache serves tc-mode register-width visits");
  const int m = P.m;
  const int NW = W > 0 ? W : P.W;
  TsaVisit o;
  o.prop = false;
  o.acc = false;
  o.Pn = o.On = o.Mn = 0;
  const uint32_t chv = ch[v - m];
  uint32_t rx = 0u, ry = 0u;
  float thr = 0.0f;
  if constexpr (PRE) {
    rx = pre_x[v - m];
    thr = pre_t[v - m];
  }
  o.cw = chv;
  const int l = (int)(chv & 0xFFFFu), r = (int)(chv >> 16);
  const bool li = l >= m, ri = r >= m;
  if (!li && !ri) return o;
  if constexpr (!PRE) {
    const TsaU4 rnd = tsa_philox(TsaU4{(uint32_t)v, sw, chain, 0u}, P.key0, P.key1);
    rx = rnd.x;
    ry = rnd.y;
  }
  const int rule = tsa_pick_rule(li, ri, rx);
  const int slotP = tsa_slot_p(rule), slotM = tsa_slot_m(rule);
  const int Pn = slotP ? r : l, On = slotP ? l : r;
  const uint32_t chp = ch[Pn - m];
  const int Mn = slotM ? (int)(chp >> 16) : (int)(chp & 0xFFFFu);
  const int Kn = slotM ? (int)(chp & 0xFFFFu) : (int)(chp >> 16);
  const uint64_t* const U = lab - (size_t)m * NW;  // UNI: every node's set at U + node * NW
  uint64_t* pP = lab + (size_t)(Pn - m) * NW;
  const uint64_t* pD = lab + (size_t)(v - m) * NW;
  const uint64_t* pO = UNI ? U + (size_t)On * NW : (On >= m ? lab + (size_t)(On - m) * NW : lf + (size_t)On * NW);
  const uint64_t* pK = UNI ? U + (size_t)Kn * NW : (Kn >= m ? lab + (size_t)(Kn - m) * NW : lf + (size_t)Kn * NW);
  const uint64_t* pM = UNI ? U + (size_t)Mn * NW : (Mn >= m ? lab + (size_t)(Mn - m) * NW : lf + (size_t)Mn * NW);
  TsaCounts cnt;
  tsa_counts_zero(cnt);
  bool acc;
  if constexpr (CC) {
    const int costP = (int)cc_cost[Pn - m], costV = (int)cc_cost[v - m], szP = (int)cc_size[Pn - m];
    uint64_t X[W];
#pragma unroll
    for (int i = 0; i < W; i++) {
      const uint64_t d = pD[i], oo = pO[i], k = pK[i], mm = pM[i];
      const uint64_t x = tsa_xset(k, oo, mm, d);
      X[i] = x;
      tsa_acc_after_tc(cnt, k, mm, oo, d, x);
    }
    const float dE = tsa_energy_tc_cached(costP, costV, szP, cnt.sd, cnt.sx, cnt.K[2], cnt.K[3], P.model, lse);
    acc = tsa_visit_accept<PRE>(ry, thr, beta, dE, T);
    if (acc) {
#pragma unroll
      for (int i = 0; i < W; i++) pP[i] = X[i];
      cc_cost[Pn - m] = (float)(cnt.sx + cnt.K[2]);  // tsa_node_cost<0> of (K, O) -> P and (P, M) -> v
      cc_cost[v - m] = (float)(cnt.sd + cnt.K[3]);
      cc_size[Pn - m] = (uint16_t)cnt.sx;
    }
  } else if constexpr (W > 0) {
    uint64_t X[W];
#pragma unroll
    for (int i = 0; i < W; i++) {
      const uint64_t d = pD[i], p = pP[i], oo = pO[i], k = pK[i], mm = pM[i];
      const uint64_t x = tsa_xset(k, oo, mm, d);
      X[i] = x;
      if constexpr (SL) {
        const uint64_t nm = ~Sm[i];
        tsa_acc<MODE>(cnt, k & nm, mm & nm, p & nm, oo & nm, d & nm, x & nm);
      } else {
        tsa_acc<MODE>(cnt, k, mm, p, oo, d, x);
      }
    }
    const float dE = tsa_energy_from_counts<MODE>(cnt, P.model, lse, T);
    acc = tsa_visit_accept<PRE>(ry, thr, beta, dE, T);
    if (acc) {
#pragma unroll
      for (int i = 0; i < W; i++) pP[i] = X[i];
    }
  } else {
    for (int i = 0; i < NW; i++) {
      const uint64_t d = pD[i], p = pP[i], oo = pO[i], k = pK[i], mm = pM[i];
      const uint64_t x = tsa_xset(k, oo, mm, d);
      if constexpr (SL) {
        const uint64_t nm = ~Sm[i];
        tsa_acc<MODE>(cnt, k & nm, mm & nm, p & nm, oo & nm, d & nm, x & nm);
      } else {
        tsa_acc<MODE>(cnt, k, mm, p, oo, d, x);
      }
    }
    const float dE = tsa_energy_from_counts<MODE>(cnt, P.model, lse, T);
    acc = tsa_visit_accept<PRE>(ry, thr, beta, dE, T);
    if (acc)
      for (int i = 0; i < NW; i++) pP[i] = (pK[i] | pO[i]) & (pM[i] | pD[i]);
  }
  o.prop = true;
  if (acc) {
    const uint32_t nchp = slotM ? ((chp & 0xFFFFu) | ((uint32_t)On << 16)) : ((chp & 0xFFFF0000u) | (uint32_t)On);
    const uint32_t nchv = slotP ? ((chv & 0xFFFF0000u) | (uint32_t)Mn) : ((chv & 0xFFFFu) | ((uint32_t)Mn << 16));
    ch[Pn - m] = nchp;
    ch[v - m] = nchv;
    o.cw = nchv;
  }
  o.acc = acc;
  o.Pn = Pn;
  o.On = On;
  o.Mn = Mn;
  return o;
}

// Whole-chain evaluation by a 32-lane group (l32 = lane within the group), in the reference's fold
// order (csrc/treesa_gpu.cu:386-434): lane t folds nodes t, t+32, ... with lse_f starting from -inf,
// then an xor butterfly 16, 8, 4, 2, 1 combines the lanes; sc, the number of internal nodes of maximal
// masked size and |S| are integer reductions.  Costs use label sets masked by ~S (S may be null).
template <int W, int MODE>
__device__ TsaEvalOut tsa_eval32(const TsaKParams& P, const uint64_t* lab, const uint32_t* ch, const uint64_t* S,
                                 const uint64_t* lf, const TsaMathTabs& T, int l32) {
  const int NW = W > 0 ? W : P.W, m = P.m;
  float acc = -INFINITY;
  int scl = 0, cntl = 0;
  for (int i = l32; i < P.nint; i += 32) {
    const uint32_t cw = ch[i];
    const int l = (int)(cw & 0xFFFFu), r = (int)(cw >> 16);
    const uint64_t* x = l >= m ? lab + (size_t)(l - m) * NW : lf + (size_t)l * NW;
    const uint64_t* y = r >= m ? lab + (size_t)(r - m) * NW : lf + (size_t)r * NW;
    const uint64_t* z = lab + (size_t)i * NW;
    int B = 0, M = 0, N = 0, K = 0, Z = 0;
    for (int w = 0; w < NW; w++) {
      const uint64_t nm = S ? ~S[w] : ~0ull;
      const uint64_t zz = z[w] & nm;
      tsa_count3(x[w] & nm, y[w] & nm, zz, B, M, N, K);
      Z += __popcll(zz);
    }
    acc = tsa_lse_f(acc, tsa_node_cost<MODE>(B, M, N, K, Z, P.model, T), T);
    if (Z > scl) {
      scl = Z;
      cntl = 1;
    } else if (Z == scl) {
      cntl++;
    }
  }
  int scmax = scl;
  for (int o = 16; o > 0; o >>= 1) {
    acc = tsa_lse_f(acc, __shfl_xor(acc, o, 32), T);
    const int t = __shfl_xor(scmax, o, 32);
    scmax = scmax > t ? scmax : t;
  }
  int cnt = (scl == scmax) ? cntl : 0, ns = 0;
  if (S)
    for (int w = l32; w < NW; w += 32) ns += __popcll(S[w]);
  for (int o = 16; o > 0; o >>= 1) {
    cnt += __shfl_xor(cnt, o, 32);
    ns += __shfl_xor(ns, o, 32);
  }
  int sc = scmax > P.leaf_sc ? scmax : P.leaf_sc;
  if (S && P.leaf_sc > scmax) {  // a leaf may be the largest tensor: masked leaf sizes
    int ll = 0;
    for (int i = l32; i < m; i += 32) {
      int Z = 0;
      for (int w = 0; w < NW; w++) Z += __popcll(lf[(size_t)i * NW + w] & ~S[w]);
      ll = ll > Z ? ll : Z;
    }
    for (int o = 16; o > 0; o >>= 1) {
      const int t = __shfl_xor(ll, o, 32);
      ll = ll > t ? ll : t;
    }
    sc = scmax > ll ? scmax : ll;
  }
  TsaEvalOut e;
  e.lcost = acc;
  e.sc = sc;
  e.sc_int = scmax;
  e.ncand = cnt;
  e.ns = ns;
  return e;
}

// E = |S| + log2(per-slice cost) + sc_weight * max(0, sc - sc_target), in float
// (csrc/treesa_gpu.cu:436-439).
__device__ __forceinline__ float tsa_slice_energy(const TsaEvalOut& e, const TsaKParams& P) {
  const float pen = (float)e.sc > P.model.sc_target ? P.model.sc_weight * ((float)e.sc - P.model.sc_target) : 0.0f;
  return (float)e.ns + e.lcost + pen;
}

// Whole-chain evaluation by the whole wave, tc mode: every lane computes the costs (integers, |z| + |x & y & ~z|
// outside S) and masked sizes of internal nodes lane, lane + 64, ... into ncost / nz (node arrays the sweep has
// finished with), then the 32-lane fold of tsa_fold32 in the reference's order: the same floats as tsa_eval32,
// with half the node passes.
template <int W>
__device__ TsaEvalOut tsa_eval64_tc(const TsaKParams& P, const uint64_t* lab, const uint32_t* ch, const uint64_t* S,
                                    const uint64_t* lf, const TsaMathTabs& T, int lane, uint16_t* ncost,
                                    uint16_t* nz) {
  const int NW = W > 0 ? W : P.W;
  tsa_wave_sync();  // a previous fold's reads of ncost / nz come first
  for (int i = lane; i < P.nint; i += 64) {
    int Z;
    ncost[i] = (uint16_t)tsa_node_eval<W, 0>(P, lab, ch, S, lf, T, i, Z);
    nz[i] = (uint16_t)Z;
  }
  tsa_wave_sync();
  return tsa_fold32(P, ncost, nz, S, lf, NW, T, lane & 31);
}

// Slice moves of one chain by one wave (csrc/treesa_gpu.cu:445-502); lane 0 alone writes S.  Returns the
// evaluation of the chain as the step leaves it.  In tc mode with ncost / nz given (nint 16-bit words each, free
// for the step) the evaluations use the whole wave (tsa_eval64_tc) and the candidate scan reads the sizes they
// leave; otherwise both 32-lane halves run the reference's 32-lane algorithm on the same data.
template <int W, int MODE>
__device__ TsaEvalOut tsa_slice_step(const TsaKParams& P, const uint64_t* lab, const uint32_t* ch, uint64_t* S,
                                     const uint64_t* lf, const TsaMathTabs& T, float beta, uint32_t sw, uint32_t chain,
                                     int lane, int& nsp, int& nsa, uint16_t* ncost = nullptr, uint16_t* nz = nullptr) {
  const int NW = W > 0 ? W : P.W;
  const int l32 = lane & 31;
  constexpr bool TC = MODE == 0;
  const bool wide = TC && ncost != nullptr;
  auto evaluate = [&]() {
    if constexpr (TC) {
      if (wide) return tsa_eval64_tc<W>(P, lab, ch, S, lf, T, lane, ncost, nz);
    }
    return tsa_eval32<W, MODE>(P, lab, ch, S, lf, T, l32);
  };
  TsaEvalOut cur = evaluate();
  bool zcur = wide;  // nz holds the sizes of the current slice set
  float Ecur = tsa_slice_energy(cur, P);
  for (int j = 0; j < P.slice_moves; j++) {
    const TsaU4 r1 = tsa_philox(TsaU4{0x10000u + 2u * (uint32_t)j, sw, chain, 0u}, P.key0, P.key1);
    const TsaU4 r2 = tsa_philox(TsaU4{0x10001u + 2u * (uint32_t)j, sw, chain, 0u}, P.key0, P.key1);
    int type;  // 0 add, 1 remove, 2 swap
    if (cur.ns == 0) type = 0;
    else if (cur.ns >= P.max_slices) type = (r1.x >> 31) ? 1 : 2;
    else type = r1.x < 0x80000000u ? 0 : (r1.x < 0xC0000000u ? 1 : 2);
    int ladd = -1, lrem = -1;
    if (type != 1 && cur.ncand > 0 && cur.sc_int > 0) {
      // the (r1.y % ncand)-th internal node of maximal masked size, in node-id order
      int rr = (int)(r1.y % (uint32_t)cur.ncand), node = -1;
      if (wide) {
        for (int base = 0; base < P.nint && node < 0; base += 64) {
          const int i = base + lane;
          int Z = -1;
          if (i < P.nint) {
            if (zcur) {
              Z = nz[i];
            } else {
              Z = 0;
              const uint64_t* z = lab + (size_t)i * NW;
              for (int w = 0; w < NW; w++) Z += __popcll(z[w] & ~S[w]);
            }
          }
          const uint64_t b = __ballot(Z == cur.sc_int);
          const int c = __popcll(b);
          if (rr < c) node = base + tsa_nth_bit(b, rr);
          else rr -= c;
        }
      } else {
        for (int base = 0; base < P.nint && node < 0; base += 32) {
          const int i = base + l32;
          int Z = -1;
          if (i < P.nint) {
            Z = 0;
            const uint64_t* z = lab + (size_t)i * NW;
            for (int w = 0; w < NW; w++) Z += __popcll(z[w] & ~S[w]);
          }
          const uint32_t b = (uint32_t)(__ballot(Z == cur.sc_int) >> (lane & 32));
          const int c = __popc(b);
          if (rr < c) node = base + tsa_nth_bit(b, rr);
          else rr -= c;
        }
      }
      if (node >= 0) ladd = tsa_nth_label(lab + (size_t)node * NW, S, NW, (int)(r1.z % (uint32_t)cur.sc_int));
    }
    if (type != 0) lrem = tsa_nth_label(S, nullptr, NW, (int)(r1.w % (uint32_t)cur.ns));
    if (type == 2 && ladd < 0) type = 1;
    if (type == 0 && ladd < 0) continue;
    tsa_wave_sync();
    if (lane == 0) {
      if (type != 1) S[ladd >> 6] |= 1ull << (ladd & 63);
      if (type != 0) S[lrem >> 6] &= ~(1ull << (lrem & 63));
    }
    tsa_wave_sync();
    const TsaEvalOut nxt = evaluate();
    const float Enew = tsa_slice_energy(nxt, P);
    nsp++;
    if (tsa_metropolis(r2.x, beta, Enew - Ecur, T.exp2)) {
      nsa++;
      cur = nxt;
      Ecur = Enew;
      zcur = wide;
    } else {
      zcur = false;  // nz holds the rejected set's sizes
      tsa_wave_sync();
      if (lane == 0) {
        if (type != 1) S[ladd >> 6] &= ~(1ull << (ladd & 63));
        if (type != 0) S[lrem >> 6] |= 1ull << (lrem & 63);
      }
      tsa_wave_sync();
    }
  }
  return cur;
}

__device__ __forceinline__ long long tsa_wave_sum(long long x) {
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

// 64-node groups per batch of the par scan.
#define TSA_SCAN_GROUPS 8

// ---------------------------------------------------------------------------------------------------
// The level loop on the device (TsaLevels): the selection of an evaluated level, by the last chain to
// arrive, in the order k_track reduces (csrc/treesa_gpu.cu:1810-1832 is the loop it replaces).
// ---------------------------------------------------------------------------------------------------

// One entry of the selection's reduction: best score and its chain, sums of E and |S|.
struct TsaRed {
  double s, e, n;
  int i;
};

// k_track's combination of entries a (lower position) and b: the lower score, the lower chain on ties.
__device__ __forceinline__ void tsa_red_merge(TsaRed& a, const TsaRed& b) {
  if (b.s < a.s || (b.s == a.s && b.i < a.i)) {
    a.s = b.s;
    a.i = b.i;
  }
  a.e += b.e;
  a.n += b.n;
}

// k_track's 256-entry tree (strides 128, 64, ..., 1, entry t combined with t + stride) by one wave: entry
// t = lane + 64 j sits in v[j]; the result is lane 0's.
__device__ __forceinline__ TsaRed tsa_red_tree256(TsaRed* v) {
  tsa_red_merge(v[0], v[2]);
  tsa_red_merge(v[1], v[3]);
  tsa_red_merge(v[0], v[1]);
  TsaRed a = v[0];
  for (int o = 32; o > 0; o >>= 1) {
    TsaRed b;
    b.s = __shfl_down(a.s, o, 64);
    b.e = __shfl_down(a.e, o, 64);
    b.n = __shfl_down(a.n, o, 64);
    b.i = __shfl_down(a.i, o, 64);
    tsa_red_merge(a, b);
  }
  return a;
}

// A chain's best score over the levels evaluated so far and the candidate slot holding that tree (-1: none).
struct TsaOwn {
  double s;
  int slot;
};

// Chain c's arrival at evaluated level (ev, its index among the launch's evaluated levels; level, its trace
// row), by one whole wave; lc / sc / ns (lane 0's count) are the chain's energies, o its best so far, cslot
// the slot this level's tree was just written to; returns the chain's best (uniform over the wave).  The
// last chain of the group of 256 reduces the group as a k_track workgroup does; the last group reduces the
// groups as k_track's last workgroup does and writes the trace row.  Inlined into the chain's own wave (a call
// there saves some 160 registers to scratch per lane at every evaluated level of every chain); with helper
// waves, wave 1 calls it through tsa_level_fold_arrive, whose registers then stay out of the sweeping wave's.
__device__ __forceinline__ TsaOwn tsa_level_arrive(const TsaLevels& Lv, int n, int c, int ev, int level, float lc, int sc,
                                                int ns, TsaOwn o, int cslot, int lane) {
  double own = o.s;
  int bslot = o.slot;
  const int ng = (n + 255) >> 8, g = c >> 8;
  unsigned* const cnt = Lv.cnt + (size_t)ev * (ng + 1);
  const size_t e0 = (size_t)ev * n;
  int last = 0;
  if (lane == 0) {
    Lv.en_lc[e0 + c] = lc;
    Lv.en_sc[e0 + c] = sc;
    Lv.en_ns[e0 + c] = ns;
    const double s = tsa_score(lc, sc, ns, Lv.S);
    if (s < own) {
      own = s;
      bslot = cslot;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const int gsize = n - (g << 8) < 256 ? n - (g << 8) : 256;
    const unsigned old = __hip_atomic_fetch_add(cnt + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old == (unsigned)gsize - 1u;
  }
  own = __shfl(own, 0, 64);
  bslot = __shfl(bslot, 0, 64);
  const TsaOwn res{own, bslot};
  if (!__shfl(last, 0, 64)) return res;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  TsaRed v[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int cc = (g << 8) + lane + 64 * j;
    v[j] = TsaRed{INFINITY, 0.0, 0.0, n};
    if (cc < n) {
      const float l = Lv.en_lc[e0 + cc];
      const int s = Lv.en_sc[e0 + cc], z = Lv.en_ns[e0 + cc];
      v[j].s = tsa_score(l, s, z, Lv.S);
      v[j].i = v[j].s < INFINITY ? cc : n;
      v[j].e = tsa_energyE(l, s, z, Lv.S);
      v[j].n = (double)z;
    }
  }
  TsaRed r = tsa_red_tree256(v);
  int top = 0;
  if (lane == 0) {
    __hip_atomic_store(cnt + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    Lv.part[(size_t)ev * ng + g] = TsaTrackPart{r.s, r.e, r.n, r.i};
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const unsigned old = __hip_atomic_fetch_add(cnt + ng, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    top = old == (unsigned)ng - 1u;
  }
  if (!__shfl(top, 0, 64)) return res;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  // the groups' results, in group order: entry t folds groups t, t + 256, ... then the tree
#pragma unroll
  for (int j = 0; j < 4; j++) {
    v[j] = TsaRed{INFINITY, 0.0, 0.0, n};
    for (int k = lane + 64 * j; k < ng; k += 256) {
      const TsaTrackPart q = Lv.part[(size_t)ev * ng + k];
      tsa_red_merge(v[j], TsaRed{q.score, q.sumE, q.sumNs, q.idx});
    }
  }
  r = tsa_red_tree256(v);
  if (lane == 0) {
    __hip_atomic_store(cnt + ng, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int b = r.i;
    TsaTraceRowD row;
    row.chain = b < n ? b : -1;
    row.lc = b < n ? Lv.en_lc[e0 + b] : 0.0f;
    row.sc = b < n ? Lv.en_sc[e0 + b] : 0;
    row.ns = b < n ? Lv.en_ns[e0 + b] : 0;
    row.score = r.s;
    row.meanE = r.e / n;
    row.meanNs = r.n / n;
    row.ticks = wall_clock64();
    Lv.trace[Lv.level0 + level] = row;
  }
  return res;
}

// The record words [ch_off, s_off + W) (children words and S) of the chain at base into its candidate slot
// cslot, by nthr threads (this one tid).
__device__ __forceinline__ void tsa_level_keep(const TsaLevels& Lv, const TsaKParams& P, const uint64_t* base, int n,
                                               int c, int cslot, int tid, int nthr) {
  uint64_t* const d = Lv.cand + ((size_t)cslot * n + c) * Lv.cand_words;
  const uint64_t* const s = base + P.ch_off;
  for (int i = tid; i < Lv.cand_words; i += nthr) d[i] = s[i];
}

// Parent of every internal node from the children words (the root's is 0xFFFF), by one wave.
__device__ __forceinline__ void tsa_par_from_children(const uint32_t* ch, uint16_t* par, int nint, int m, int lane) {
  for (int i = lane; i < nint; i += 64) {
    const uint32_t cw = ch[i];
    const int l = (int)(cw & 0xFFFFu), r = (int)(cw >> 16);
    if (l >= m) par[l - m] = (uint16_t)(m + i);
    if (r >= m) par[r - m] = (uint16_t)(m + i);
  }
  if (lane == 0) par[nint - 1] = 0xFFFFu;
}

// An evaluated level's end for a chain swept by one wave: node costs into the node arrays (pri and par hold
// nint4 floats, wl nint4 sizes; their sweep contents are rebuilt by the next sweep, par by the caller), the
// 32-lane fold as k_energy's, the tree into a candidate slot, then the chain's arrival.
template <int W, int MODE>
__device__ __forceinline__ TsaOwn tsa_level_wave(const TsaKParams& P, const TsaLevels& Lv, const uint64_t* base,
                                              const uint64_t* lab, const uint32_t* ch, const uint64_t* Sm,
                                              const uint64_t* lf, TsaMathTabs T, uint16_t* pri, uint16_t* wl, int n,
                                              int c, int ev, int level, TsaOwn o, int lane) {
  const int NW = W > 0 ? W : P.W;
  tsa_wave_sync();
  float* const ncost = reinterpret_cast<float*>(pri);
  for (int i = lane; i < P.nint; i += 64) {
    int Z;
    ncost[i] = tsa_node_eval<W, MODE>(P, lab, ch, Sm, lf, T, i, Z);
    wl[i] = (uint16_t)Z;
  }
  tsa_wave_sync();
  const TsaEvalOut e = tsa_fold32(P, ncost, wl, Sm, lf, NW, T, lane & 31);
  const int cslot = o.slot < 0 ? 0 : o.slot ^ 1;
  tsa_level_keep(Lv, P, base, n, c, cslot, lane, 64);
  o = tsa_level_arrive(Lv, n, c, ev, level, e.lcost, e.sc, e.ns, o, cslot, lane);
  tsa_wave_sync();
  return o;
}

// The rest of an evaluated level's end for a chain swept by wave 0 of a workgroup with helper waves, by wave 1
// while wave 0 sweeps on: the fold of the node costs and sizes the workgroup left in cost / z (S: a copy of
// the slice set as it was then), then the chain's arrival.  Returns the chain's best.
template <int W>
__device__ __forceinline__ TsaOwn tsa_level_fold_arrive(const TsaKParams& P, const TsaLevels& Lv, const float* cost,
                                                     const uint16_t* z, const uint64_t* S, const uint64_t* lf,
                                                     TsaMathTabs T, int n, int c, int ev, int level, TsaOwn o,
                                                     int cslot, int lane) {
  const int NW = W > 0 ? W : P.W;
  const TsaEvalOut e = tsa_fold32(P, cost, z, S, lf, NW, T, lane & 31);
  return tsa_level_arrive(Lv, n, c, ev, level, e.lcost, e.sc, e.ns, o, cslot, lane);
}

// Sweep kernel.  ORDER 0: par, 1: pre-order.  LDS: chain and leaf table staged in LDS.  LVL: the level loop
// (TsaLevels) of independent chains in one launch, the chain staying staged from its first level to its last.
// LDS layout (words): [leaf table (LDS variant only), rounded to even] then per wave lds_words:
// [chain record (LDS variant only)][pri u16 x nint4][par u16 x nint4][work list u16 x nint4]
// [band words u32 x nint4 when par_band > 0].
// (The par level loop in tc mode keeps three waves per SIMD, as many as the chains' LDS allows: its level
// functions' registers would otherwise take one of them; the float modes need more registers than that.)
template <int W, int MODE, int ORDER, bool LDS, bool LVL, bool SLICE>
__global__ void __launch_bounds__(256, (LVL && ORDER == 0 && MODE == 0) ? 3 : 1) k_sweep(TsaKParams P, uint64_t* __restrict__ rec,
                                               const uint64_t* __restrict__ leaf, const uint32_t* __restrict__ fix,
                                               int nchains, int lds_words, float beta1, uint32_t sweep0, int nsweeps,
                                               unsigned long long* __restrict__ stats, TsaEnergyOut eo, TsaLevels Lv) {
  extern __shared__ uint64_t tsa_smem[];
  __shared__ float s_lse[64];
  __shared__ uint64_t s_exp2[32];
  __shared__ uint64_t s_S[8];  // helper mode, level loop: the slice set at a level's end, for wave 1's fold
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, wpb = blockDim.x >> 6;
  const int NW = W > 0 ? W : P.W;
  const int m = P.m, nint = P.nint, nint4 = (nint + 3) & ~3;
  // the small tables every proposal indexes per lane live in LDS
  if (threadIdx.x < 64) s_lse[threadIdx.x] = P.lse[threadIdx.x];
  if (threadIdx.x < 32) s_exp2[threadIdx.x] = tsa_exp2_tab_d[threadIdx.x];
  // the log2 tables only serve energies here; the correction table's summary bitmap follows its words
  const TsaMathTabs T{s_exp2, fix, fix + TSA_LOG2FIX_WORDS, tsa_log2_tab_d};
  const uint64_t* lf = leaf;
  int leafw = 0;
  if constexpr (LDS) {
    // the leaf sets end where the first wave's chain begins (their rounding gap below them)
    leafw = (m * NW + 1) & ~1;
    uint64_t* const sl = tsa_smem + (leafw - m * NW);
    for (int i = threadIdx.x; i < m * NW; i += blockDim.x) sl[i] = leaf[i];
    lf = sl;
  }
  __syncthreads();
  // with helper waves the workgroup holds one chain, swept by wave 0; else wave wv holds chain wpb*block + wv
  // (both counted from P.chain0)
  const bool helped = ORDER == 1 && P.helpers > 0;
  const int c = P.chain0 + (helped ? (int)blockIdx.x : (int)blockIdx.x * wpb + wv);
  if (c >= nchains) return;  // whole waves (whole workgroups with helpers); every barrier below is the
                             // helper mode's, reached by all of its waves
  uint64_t* const g = rec + (size_t)c * P.chain_words;
  uint64_t* const wbase = tsa_smem + leafw + (size_t)(helped ? 0 : wv) * lds_words;
  uint64_t* base;
  uint16_t* nodes;
  if constexpr (LDS) {
    base = wbase;
    if (!helped || wv == 0) {  // with helpers wave 0 copies while the others draw the first sweep's numbers
      const uint4* src = reinterpret_cast<const uint4*>(P.ganc ? P.gsrc + (size_t)P.ganc[c] * P.chain_words : g);
      uint4* dst = reinterpret_cast<uint4*>(base);
      const int n16 = P.chain_words / 2;
      int i = lane;
      for (; i + 192 < n16; i += 256) {  // four loads in flight per lane
        const uint4 a = src[i], b = src[i + 64], d = src[i + 128], e = src[i + 192];
        dst[i] = a;
        dst[i + 64] = b;
        dst[i + 128] = d;
        dst[i + 192] = e;
      }
      for (; i < n16; i += 64) dst[i] = src[i];
    }
    nodes = reinterpret_cast<uint16_t*>(base + P.chain_words);
  } else {
    base = g;
    nodes = reinterpret_cast<uint16_t*>(wbase);
  }
  uint64_t* const lab = base;
  uint32_t* const ch = reinterpret_cast<uint32_t*>(base + P.ch_off);
  uint64_t* const S = base + P.s_off;
  const bool slicing = SLICE && P.slicing;  // (launched with SLICE only when P.slicing is set)
  const uint64_t* const Sm = slicing ? S : nullptr;
  uint16_t* const pri = nodes;
  uint16_t* const par = nodes + nint4;
  uint16_t* const wl = par + nint4;
  uint32_t* const dw = reinterpret_cast<uint32_t*>(wl + nint4);
  int np = 0, na = 0, nst = 0, nv = 0, nsp = 0, nsa = 0, nbusy = 0;
  // the evaluation a slice step left of the chain as it stands (valid until the next sweep changes the tree)
  TsaEvalOut last_e{};
  bool have_e = false;
  // the level loop (Lv.nlev > 0) or the launch's one level: sweeps in all, the current level, its sweeps left
  // and beta; the chain's best score and the candidate slot of its tree, kept by the wave that tracks the chain
  // (wave 1 with helpers, else the chain's wave)
  // (or a block of levels, eo.blk: their sweeps in all, the current level, its sweeps left and its beta)
  const bool blocked = !LVL && ORDER == 0 && eo.blk.n > 0;
  const int nsw = LVL ? Lv.total : (blocked ? eo.blk.total : nsweeps);
  int lv = 0, left = LVL ? Lv.niters[0] : (blocked ? eo.blk.niters[0] : nsweeps);
  float beta = LVL ? Lv.beta[0] : (blocked ? eo.blk.beta[0] : beta1);
  const bool tracker = LVL && (!helped || wv == 1);
  TsaOwn own{INFINITY, -1};
  if (tracker && !Lv.reset) own = TsaOwn{Lv.own[c], Lv.bslot[c]};
  if (tracker && Lv.tinit && c == 0) {
    // the session's start: its stores precede this chain's first arrival (release), which every trace row's
    // writer waits for (acquire)
    unsigned long long* const tr = reinterpret_cast<unsigned long long*>(Lv.trace);
    for (int i = lane; i < Lv.trace_words; i += 64) tr[i] = 0ull;
    for (int i = lane; i < Lv.best_words; i += 64) Lv.best[i] = 0ull;
    if (lane == 0) {
      Lv.tinit->best_score = INFINITY;
      Lv.tinit->best_chain = -1;
      Lv.tinit->best_level = -1;
      Lv.tinit->snap = -1;
      *Lv.ticks0 = wall_clock64();
    }
  }
  tsa_wave_sync();

  if constexpr (ORDER == 0) {
    tsa_par_from_children(ch, par, nint, m, lane);
    tsa_wave_sync();
    for (int s = 0; s < nsw; s++) {
      const uint32_t sw = sweep0 + (uint32_t)s;
      const uint32_t hs = tsa_sweep_hash(sw, (uint32_t)c, P.key0);
      for (int i = lane; i < nint; i += 64) pri[i] = (uint16_t)tsa_par_pri((uint32_t)(m + i), hs);
      if (P.par_band > 0) {
        // depth at sweep start by pointer jumping on (depth << 16 | ancestor) words; an update that reads
        // an already advanced ancestor word still keeps depth(v) = d + depth(ancestor)
        for (int i = lane; i < nint; i += 64) dw[i] = par[i] == 0xFFFFu ? 0xFFFFu : (0x10000u | par[i]);
        tsa_wave_sync();
        for (;;) {
          bool any = false;
          for (int i = lane; i < nint; i += 64) {
            const uint32_t w = dw[i], a = w & 0xFFFFu;
            if (a != 0xFFFFu) {
              const uint32_t w2 = dw[a - m];
              dw[i] = ((w & 0xFFFF0000u) + (w2 & 0xFFFF0000u)) | (w2 & 0xFFFFu);
              any = true;
            }
          }
          tsa_wave_sync();
          if (__ballot(any) == 0ull) break;
        }
        const int L = P.par_band;
        for (int i = lane; i < nint; i += 64)
          pri[i] = (uint16_t)((((uint32_t)((L - 1 - (int)(dw[i] >> 16) % L) & 15)) << 12) | (pri[i] & 0x0FFEu) | 1u);
      }
      tsa_wave_sync();
      // nodes with a nonzero priority: while any is left, the one with the largest key beats its unvisited
      // neighbours, so the next scan finds a nonempty phase; when none is left that scan would find nothing
      // and is skipped
      int unvisited = nint;
      // Scan list: with at most 64 * TSA_SCAN_GROUPS internal nodes (one batch: every list entry is read
      // before the scan writes any) and without par_follow (which re-arms visited pivots), a scan reads only
      // the nodes not yet visited, kept in any order at the top of the work-list array, wl[nint4 - unvisited,
      // nint4); the scan writes the phase's active nodes at the bottom, wl[0, cnt), and the others back at the
      // top.  Otherwise every scan reads all nodes.  The visits of a phase commute, so the order of the
      // work list changes no result.
      const bool shrink = nint <= 64 * TSA_SCAN_GROUPS && !P.par_follow;
      if (shrink) {
        for (int i = lane; i < nint; i += 64) wl[nint4 - nint + i] = (uint16_t)(m + i);
        tsa_wave_sync();
      }
      for (;;) {
        if (unvisited == 0) break;
        // scan: the phase's independent set into the work list.  Node v is active when its priority is
        // nonzero and its (priority, id) key beats those of its unvisited parent and internal children.
        // TSA_SCAN_GROUPS 64-entry groups at a time, branch-free: every lane reads its node (from the list),
        // the node's priority, parent and children words, then the three neighbour priorities (index 0
        // where there is no such neighbour), so a batch costs two (three with the list) dependent LDS round
        // trips.
        const int total = shrink ? unvisited : nint;  // entries to scan
        const int ubase = nint4 - unvisited;          // the list's first entry
        int cnt = 0, kept = 0;
        for (int i0 = 0; i0 < total; i0 += 64 * TSA_SCAN_GROUPS) {
          const int ng = (total - i0 + 63) >> 6;  // groups present in this batch (wave-uniform)
          int ni[TSA_SCAN_GROUPS];
          uint32_t pv[TSA_SCAN_GROUPS], pw[TSA_SCAN_GROUPS], cw[TSA_SCAN_GROUPS];
#pragma unroll
          for (int q = 0; q < TSA_SCAN_GROUPS; q++) {
            ni[q] = 0;
            pv[q] = 0u;
            pw[q] = 0xFFFFu;
            cw[q] = 0u;
            if (q < ng) {
              const int j = i0 + 64 * q + lane;
              const int jj = j < total ? j : 0;
              const int ii = shrink ? (int)wl[ubase + jj] - m : jj;
              ni[q] = ii;
              pv[q] = pri[ii];
              pw[q] = par[ii];
              cw[q] = ch[ii];
            }
          }
          uint32_t np_[TSA_SCAN_GROUPS], nl[TSA_SCAN_GROUPS], nr[TSA_SCAN_GROUPS];
#pragma unroll
          for (int q = 0; q < TSA_SCAN_GROUPS; q++) {
            np_[q] = nl[q] = nr[q] = 0u;
            if (q < ng) {
              const uint32_t p = pw[q], l = cw[q] & 0xFFFFu, r = cw[q] >> 16;
              np_[q] = pri[p != 0xFFFFu ? p - (uint32_t)m : 0u];
              nl[q] = pri[l >= (uint32_t)m ? l - (uint32_t)m : 0u];
              nr[q] = pri[r >= (uint32_t)m ? r - (uint32_t)m : 0u];
            }
          }
#pragma unroll
          for (int q = 0; q < TSA_SCAN_GROUPS; q++) {
            if (q >= ng) break;
            const bool valid = i0 + 64 * q + lane < total;
            const uint32_t v = (uint32_t)(m + ni[q]);
            const uint32_t key = (pv[q] << 16) | v;
            const uint32_t p = pw[q], l = cw[q] & 0xFFFFu, r = cw[q] >> 16;
            const bool beat_p = p != 0xFFFFu && np_[q] != 0u && ((np_[q] << 16) | p) > key;
            const bool beat_l = l >= (uint32_t)m && nl[q] != 0u && ((nl[q] << 16) | l) > key;
            const bool beat_r = r >= (uint32_t)m && nr[q] != 0u && ((nr[q] << 16) | r) > key;
            const bool act = valid && pv[q] != 0u && !beat_p && !beat_l && !beat_r;
            const uint64_t b = __ballot(act);
            if (act) wl[cnt + __popcll(b & tsa_lt_mask(lane))] = (uint16_t)v;
            cnt += __popcll(b);
            if (shrink) {
              const bool keep = valid && !act;
              const uint64_t bk = __ballot(keep);
              if (keep) wl[nint4 - 1 - (kept + __popcll(bk & tsa_lt_mask(lane)))] = (uint16_t)v;
              kept += __popcll(bk);
            }
          }
        }
        if (cnt == 0) break;
        nst++;
        unvisited -= cnt;
        tsa_wave_sync();
        for (int b0 = 0; b0 < cnt; b0 += 64) {
          const int j = b0 + lane;
          bool rearm = false;
          if (j < cnt) {
            const int v = wl[j];
            const bool rev = (pri[v - m] & 1u) == 0;  // a follow-up visit draws its own numbers
            const uint32_t swv = sw | (rev ? 0x80000000u : 0u);
            const TsaVisit o = slicing
                                   ? tsa_visit<W, MODE, true, false, false>(P, lab, ch, Sm, lf, s_lse, T, v, beta, swv, (uint32_t)c)
                                   : tsa_visit<W, MODE, false, false, false>(P, lab, ch, Sm, lf, s_lse, T, v, beta, swv, (uint32_t)c);
            nv++;
            nbusy++;
            np += o.prop;
            if (o.acc) {
              na++;
              if (o.On >= m) par[o.On - m] = (uint16_t)o.Pn;
              if (o.Mn >= m) par[o.Mn - m] = (uint16_t)v;
              if (P.par_follow && !rev && pri[o.Pn - m] == 0) {
                pri[o.Pn - m] = (uint16_t)tsa_follow_pri((uint32_t)o.Pn, hs);
                rearm = true;  // the pivots of one phase are distinct nodes
              }
            }
            pri[v - m] = 0;
          }
          if (P.par_follow) unvisited += __popcll(__ballot(rearm));
        }
        tsa_wave_sync();
      }
      if constexpr (SLICE) {
        have_e = false;
        if (P.slice_moves > 0 && (sw + 1u) % (uint32_t)P.slice_every == 0u) {
          // (pri and the work list are free until the next sweep)
          last_e = tsa_slice_step<W, MODE>(P, lab, ch, S, lf, T, beta, sw, (uint32_t)c, lane, nsp, nsa, pri, wl);
          have_e = true;
          tsa_wave_sync();
        }
      }
      if constexpr (LVL) {
        if (--left == 0) {  // the level's last sweep
          const int ev = Lv.eval[lv];
          if (ev >= 0) {
            own = tsa_level_wave<W, MODE>(P, Lv, base, lab, ch, Sm, lf, T, pri, wl, nchains, c, ev, lv, own, lane);
            tsa_par_from_children(ch, par, nint, m, lane);  // the evaluation overwrote par
            tsa_wave_sync();
          }
          if (++lv < Lv.nlev) {
            beta = Lv.beta[lv];
            left = Lv.niters[lv];
          }
        }
      } else {
        if (blocked && --left == 0) {  // a block's level ends: its snapshot (node costs, sizes, children words)
          if (eo.blk.cost[lv]) {
            float* const gc = eo.blk.cost[lv] + (size_t)c * nint4;
            uint16_t* const gz = eo.blk.z[lv] + (size_t)c * nint4;
            uint32_t* const gch = eo.blk.ch[lv] + (size_t)c * nint;
            for (int i = lane; i < nint; i += 64) {
              int Z;
              gc[i] = tsa_node_eval<W, MODE>(P, lab, ch, Sm, lf, T, i, Z);
              gz[i] = (uint16_t)Z;
              gch[i] = ch[i];
            }
          }
          if (++lv < eo.blk.n) {
            beta = eo.blk.beta[lv];
            left = eo.blk.niters[lv];
          }
        }
      }
    }
  } else {
    const int root = 2 * m - 2;
    // helper waves: every internal node's Philox word x and Metropolis threshold of sweep s sit in buffer s & 1
    // (after the wave's node arrays) before sweep s starts, so that no visit of a sweep's dependent chain of
    // steps waits on Philox or expf.  The helpers draw sweep 0 while wave 0 copies the record, and sweep s + 1
    // during sweep s; a workgroup barrier closes each of these.
    uint32_t* const dbuf = helped ? reinterpret_cast<uint32_t*>(wbase + lds_words) : nullptr;
    // level loop with helpers: the node sizes of an evaluated level, after the draw buffers
    uint16_t* const lz = LVL && helped ? reinterpret_cast<uint16_t*>(dbuf + 4 * nint4) : nullptr;
    // tc mode with helpers, no slicing: every internal node's cost and size (the visits' cost cache), after lz
    const bool cc = MODE == 0 && W > 0 && helped && !slicing;
    float* const cc_cost = cc ? reinterpret_cast<float*>(dbuf + 4 * nint4 + (LVL ? nint4 / 2 : 0)) : nullptr;
    uint16_t* const cc_size = cc ? reinterpret_cast<uint16_t*>(cc_cost + nint4) : nullptr;
    if (helped) {
      if (wv > 0)
        tsa_draw_ahead(P, dbuf, reinterpret_cast<float*>(dbuf + nint4), sweep0, (uint32_t)c, (int)threadIdx.x - 64,
                       (int)blockDim.x - 64, T.exp2);
      __syncthreads();
      if (cc) {  // the cache from the record just staged
        for (int i = threadIdx.x; i < nint; i += blockDim.x) {
          int Z;
          cc_cost[i] = tsa_node_eval<W, MODE>(P, lab, ch, Sm, lf, T, i, Z);
          cc_size[i] = (uint16_t)Z;
        }
        __syncthreads();
      }
    }
    // an evaluated level's end with helpers: the whole workgroup evaluates the node costs into pri / par (free in
    // pre-order sweeps) and the sizes into lz (with the cost cache: a copy of it, which the visits of the next
    // sweep leave alone); then wave 0 returns to its sweeps at once and wave 1 folds, arrives (and selects when it
    // is the last chain) beside them
    float* const ncost = reinterpret_cast<float*>(pri);
    auto level_costs = [&]() {
      for (int i = threadIdx.x; i < nint; i += blockDim.x) {
        if (cc) {
          ncost[i] = cc_cost[i];
          lz[i] = cc_size[i];
        } else {
          int Z;
          ncost[i] = tsa_node_eval<W, MODE>(P, lab, ch, Sm, lf, T, i, Z);
          lz[i] = (uint16_t)Z;
        }
      }
    };
    // The sweeping wave and the helper waves run loops of their own, which meet at the same workgroup barriers
    // (one per sweep, one more at an evaluated level's end): wave 1's fold is a call, and in a loop of its own
    // only the helpers' few values are live across it (in a loop shared with the sweep, every value the sweep
    // keeps would be saved to scratch around the call at every level)
    if (helped && wv > 0) {
      for (int s = 0; s < nsw; s++) {
        if (s + 1 < nsw) {
          uint32_t* const nx = dbuf + (size_t)((s + 1) & 1) * 2 * nint4;
          tsa_draw_ahead(P, nx, reinterpret_cast<float*>(nx + nint4), sweep0 + (uint32_t)s + 1u, (uint32_t)c,
                         (int)threadIdx.x - 64, (int)blockDim.x - 64, T.exp2);
        }
        __syncthreads();
        if constexpr (LVL) {
          if (--left == 0) {  // the level's last sweep
            const int ev = Lv.eval[lv];
            if (ev >= 0) {
              level_costs();
              const int cslot = own.slot < 0 ? 0 : own.slot ^ 1;
              if (wv == 1) {
                tsa_level_keep(Lv, P, base, nchains, c, cslot, lane, 64);
                if (slicing && lane < NW) s_S[lane] = S[lane];
              }
              __syncthreads();
              if (wv == 1)
                own = tsa_level_fold_arrive<W>(P, Lv, ncost, lz, slicing ? s_S : nullptr, lf, T, nchains, c, ev,
                                               lv, own, cslot, lane);
            }
            if (++lv < Lv.nlev) left = Lv.niters[lv];
          }
        }
      }
    } else {
      for (int s = 0; s < nsw; s++) {
        const uint32_t sw = sweep0 + (uint32_t)s;
        const uint32_t* const pre_x = helped ? dbuf + (size_t)(s & 1) * 2 * nint4 : nullptr;
        const float* const pre_t = helped ? reinterpret_cast<const float*>(pre_x + nint4) : nullptr;
        if (lane == 0) wl[0] = (uint16_t)root;
        int sp = 1;
        tsa_wave_sync();
        while (sp > 0) {
          const int k = sp < 64 ? sp : 64, b0 = sp - k;
          const int v = lane < k ? (int)wl[b0 + lane] : 0;
          tsa_wave_sync();  // every lane has read its node before pushes overwrite the list
          uint32_t cw = 0;
          if (lane < k) {
            // with helpers (one chain per workgroup) the staged leaf sets end where the chain's internal sets begin
            // (LDS records) and the draws are made ahead
            const TsaVisit o =
                slicing ? (helped ? tsa_visit<W, MODE, true, LDS, true>(P, lab, ch, Sm, lf, s_lse, T, v, beta, sw, (uint32_t)c, pre_x, pre_t)
                                    : tsa_visit<W, MODE, true, false, false>(P, lab, ch, Sm, lf, s_lse, T, v, beta, sw, (uint32_t)c))
                          : (helped ? tsa_visit<W, MODE, false, LDS, true, MODE == 0 && (W > 0)>(P, lab, ch, Sm, lf, s_lse, T, v, beta, sw, (uint32_t)c, pre_x, pre_t,
                                                                             cc_cost, cc_size)
                                    : tsa_visit<W, MODE, false, false, false>(P, lab, ch, Sm, lf, s_lse, T, v, beta, sw, (uint32_t)c));
            cw = o.cw;
            nv++;
            nbusy++;
            np += o.prop;
            na += o.acc;
          }
          nst++;
          const bool c1 = lane < k && (int)(cw & 0xFFFFu) >= m;
          const bool c2 = lane < k && (int)(cw >> 16) >= m;
          const uint64_t b1 = __ballot(c1), b2 = __ballot(c2);
          int pos = b0 + __popcll(b1 & tsa_lt_mask(lane)) + __popcll(b2 & tsa_lt_mask(lane));
          if (c2) wl[pos++] = (uint16_t)(cw >> 16);
          if (c1) wl[pos] = (uint16_t)(cw & 0xFFFFu);
          sp = b0 + __popcll(b1) + __popcll(b2);
          tsa_wave_sync();
        }
        if constexpr (SLICE) {
          have_e = false;
          if (P.slice_moves > 0 && (sw + 1u) % (uint32_t)P.slice_every == 0u) {
            // (pri and the work list are free in pre-order after the sweep)
            last_e = tsa_slice_step<W, MODE>(P, lab, ch, S, lf, T, beta, sw, (uint32_t)c, lane, nsp, nsa, pri, wl);
            have_e = true;
            tsa_wave_sync();
          }
        }
        if (helped) __syncthreads();
        if constexpr (LVL) {
          if (--left == 0) {  // the level's last sweep
            const int ev = Lv.eval[lv];
            if (ev >= 0) {
              if (helped) {
                level_costs();
                __syncthreads();
              } else {
                own = tsa_level_wave<W, MODE>(P, Lv, base, lab, ch, Sm, lf, T, pri, wl, nchains, c, ev, lv, own, lane);
              }
            }
            if (++lv < Lv.nlev) {
              beta = Lv.beta[lv];
              left = Lv.niters[lv];
            }
          }
        }
      }
    }
  }
  if constexpr (LVL) {
    if (tracker && lane == 0) {
      Lv.own[c] = own.s;
      Lv.bslot[c] = own.slot;
    }
  }


  // with helper waves the whole workgroup evaluates the node costs, then the helpers write the snapshot and
  // the record back while wave 0 folds the energy
  const int e0 = helped ? (int)threadIdx.x : lane, es = helped ? (int)blockDim.x : 64;
  if (eo.cost) {
    // node costs and masked sizes, for k_fold
    float* const gc = eo.cost + (size_t)c * nint4;
    uint16_t* const gz = eo.z + (size_t)c * nint4;
    for (int i = e0; i < nint; i += es) {
      int Z;
      gc[i] = tsa_node_eval<W, MODE>(P, lab, ch, Sm, lf, T, i, Z);
      gz[i] = (uint16_t)Z;
    }
  } else if (eo.lc && !helped && have_e) {
    // the last sweep's slice step evaluated the chain as it stands: the same energy k_energy would compute
    if (lane == 0) {
      eo.lc[c] = last_e.lcost;
      eo.sc[c] = last_e.sc;
      eo.ns[c] = last_e.ns;
    }
  } else if (eo.lc) {
    // the chain's energy, as k_energy computes it: node costs into the node arrays (free after the sweeps:
    // pri and par hold nint4 floats, wl nint4 sizes), then the 32-lane fold
    tsa_wave_sync();
    float* const ncost = reinterpret_cast<float*>(pri);
    for (int i = e0; i < nint; i += es) {
      int Z;
      ncost[i] = tsa_node_eval<W, MODE>(P, lab, ch, Sm, lf, T, i, Z);
      wl[i] = (uint16_t)Z;
    }
    if (helped) __syncthreads();
    else tsa_wave_sync();
    if (!helped || wv == 0) {
      const TsaEvalOut e = tsa_fold32(P, ncost, wl, Sm, lf, NW, T, lane & 31);
      if (lane == 0) {
        eo.lc[c] = e.lcost;
        eo.sc[c] = e.sc;
        eo.ns[c] = e.ns;
      }
    }
  }
  if (!helped || wv > 0) {
    const int u0 = helped ? (int)threadIdx.x - 64 : lane, us = helped ? (int)blockDim.x - 64 : 64;
    if (eo.ch) {
      uint32_t* const gch = eo.ch + (size_t)c * nint;
      for (int i = u0; i < nint; i += us) gch[i] = ch[i];
    }
    if constexpr (LDS) {
      tsa_wave_sync();
      const uint4* src = reinterpret_cast<const uint4*>(base);
      uint4* dst = reinterpret_cast<uint4*>(g);
      for (int i = u0; i < P.chain_words / 2; i += us) dst[i] = src[i];
    }
  }
  if (helped && wv > 0) return;
  const long long sp_ = tsa_wave_sum(np), sa_ = tsa_wave_sum(na), sv_ = tsa_wave_sum(nv), sb_ = tsa_wave_sum(nbusy);
  if (lane == 0) {  // counters spread over TSA_STAT_SLOTS addresses each, summed by the host
    unsigned long long* st = stats + (c & (TSA_STAT_SLOTS - 1));
    atomicAdd(&st[TSA_ST_PROP * TSA_STAT_SLOTS], (unsigned long long)sp_);
    atomicAdd(&st[TSA_ST_ACC * TSA_STAT_SLOTS], (unsigned long long)sa_);
    atomicAdd(&st[TSA_ST_STEPS * TSA_STAT_SLOTS], (unsigned long long)nst);
    atomicAdd(&st[TSA_ST_VISITS * TSA_STAT_SLOTS], (unsigned long long)sv_);
    atomicAdd(&st[TSA_ST_SPROP * TSA_STAT_SLOTS], (unsigned long long)nsp);
    atomicAdd(&st[TSA_ST_SACC * TSA_STAT_SLOTS], (unsigned long long)nsa);
    atomicAdd(&st[TSA_ST_BUSY * TSA_STAT_SLOTS], (unsigned long long)sb_);
  }
}

template <int W, int MODE, int ORDER, bool LDS, bool LVL, bool SLICE>
static hipError_t launch_sweep_t(const TsaLaunch& L, const TsaKParams& P, uint64_t* rec, const uint64_t* leaf,
                                 const uint32_t* fix, int nchains, float beta, uint32_t sweep0, int nsweeps,
                                 unsigned long long* stats, const TsaEnergyOut& eo, hipStream_t st, hipEvent_t e0,
                                 hipEvent_t e1, const TsaLevels* lv, int* res) {
  const int NW = W > 0 ? W : P.W;
  const size_t leafw = LDS ? (size_t)((P.m * NW + 1) & ~1) : 0;
  // pre-order sweeps with helper waves: one chain per workgroup of 1 + TSA_DRAW_HELPERS waves, with two draw
  // buffers after the chain's words, when they fit
  TsaKParams P2 = P;
  P2.helpers = 0;
  int wpb = L.wpb, threads = 64 * L.wpb;
  size_t smem = (leafw + (size_t)L.wpb * L.lds_words) * 8;
  if (ORDER == 1 && L.draw_waves) {
    // (the level loop adds a node-size array after the draw buffers; tc mode then a node-cost cache, 4 + 2 B
    // per node)
    const size_t nint4 = (size_t)((P.nint + 3) & ~3);
    const size_t zw = LVL ? (nint4 * 2 + 7) / 8 : 0, cw = MODE == 0 && W > 0 ? (nint4 * 6 + 7) / 8 : 0;
    const size_t hs = (leafw + (size_t)L.lds_words + tsa_draw_words(P.nint) + zw + cw) * 8;
    if (hs <= (size_t)L.lds_max) {
      P2.helpers = TSA_DRAW_HELPERS;
      wpb = 1;
      threads = 64 * (1 + TSA_DRAW_HELPERS);
      smem = hs;
    }
  }
  static size_t attr_set = 0;
  if (smem > 65536 && smem > attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_sweep<W, MODE, ORDER, LDS, LVL, SLICE>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) return e;
    attr_set = smem;
  }
  if (res) {  // a query: chains resident per compute unit, no launch
    int nb = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &nb, reinterpret_cast<const void*>(&k_sweep<W, MODE, ORDER, LDS, LVL, SLICE>), threads, smem);
    *res = nb * wpb;
    return e;
  }
  if (P.chain0 < 0 || P.chain0 >= nchains) return hipErrorInvalidValue;
  const int grid = (nchains - P.chain0 + wpb - 1) / wpb;
  if (eo.blk.n > 0 && (ORDER != 0 || LVL || eo.blk.n > TSA_BLOCK_MAX || eo.blk.total != nsweeps))
    return hipErrorInvalidValue;  // a block of levels: par sweeps of one launch's total sweeps
  // e0 / e1 (null: none) take the kernel's start and stop times in the dispatch itself
  hipExtLaunchKernelGGL((k_sweep<W, MODE, ORDER, LDS, LVL, SLICE>), dim3(grid), dim3(threads), (uint32_t)smem, st, e0, e1, 0u,
                        P2, rec, leaf, fix, nchains, L.lds_words, beta, sweep0, nsweeps, stats, eo,
                        lv ? *lv : TsaLevels{});
  return hipGetLastError();
}

template <int W, int MODE, bool SLICE>
static hipError_t launch_sweep_wm(const TsaLaunch& L, int order, const TsaKParams& P, uint64_t* rec,
                                  const uint64_t* leaf, const uint32_t* fix, int nchains, float beta, uint32_t sweep0,
                                  int nsweeps, unsigned long long* stats, const TsaEnergyOut& eo, hipStream_t st,
                                  hipEvent_t e0, hipEvent_t e1, const TsaLevels* lv, int* res) {
  if constexpr (W > 0) {
    if (L.lds) {
      // the level loop (lv set) is a kernel of its own: its level functions are calls the plain sweep kernel
      // does not carry
      if (lv) {
        if (order == 0) return launch_sweep_t<W, MODE, 0, true, true, SLICE>(L, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, eo, st, e0, e1, lv, res);
        return launch_sweep_t<W, MODE, 1, true, true, SLICE>(L, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, eo, st, e0, e1, lv, res);
      }
      if (order == 0) return launch_sweep_t<W, MODE, 0, true, false, SLICE>(L, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, eo, st, e0, e1, lv, res);
      return launch_sweep_t<W, MODE, 1, true, false, SLICE>(L, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, eo, st, e0, e1, lv, res);
    }
    return hipErrorInvalidValue;  // the register-width kernels exist only in the LDS variant
  } else {
    if (L.lds || lv) return hipErrorInvalidValue;  // the level loop runs on the register-width kernels only
    if (order == 0) return launch_sweep_t<0, MODE, 0, false, false, SLICE>(L, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, eo, st, e0, e1, nullptr, res);
    return launch_sweep_t<0, MODE, 1, false, false, SLICE>(L, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, eo, st, e0, e1, nullptr, res);
  }
}

template <int W, bool SLICE>
static hipError_t launch_sweep_w(const TsaLaunch& L, int mode, int order, const TsaKParams& P, uint64_t* rec,
                                 const uint64_t* leaf, const uint32_t* fix, int nchains, float beta, uint32_t sweep0,
                                 int nsweeps, unsigned long long* stats, const TsaEnergyOut& eo, hipStream_t st,
                                 hipEvent_t e0, hipEvent_t e1, const TsaLevels* lv, int* res) {
  if (mode == 0) return launch_sweep_wm<W, 0, SLICE>(L, order, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, eo, st, e0, e1, lv, res);
  if (mode == 1) return launch_sweep_wm<W, 1, SLICE>(L, order, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, eo, st, e0, e1, lv, res);
  return launch_sweep_wm<W, 2, SLICE>(L, order, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, eo, st, e0, e1, lv, res);
}

// Every sweep kernel of one SLICE variant, by label width, energy mode, order and level loop.
template <bool SLICE>
hipError_t tsa_launch_sweeps_t(const TsaLaunch& L, int mode, int order, const TsaKParams& P, uint64_t* rec,
                               const uint64_t* leaf, const uint32_t* fix, int nchains, float beta, uint32_t sweep0,
                               int nsweeps, unsigned long long* stats, const TsaEnergyOut& eo, hipStream_t st,
                               hipEvent_t e0, hipEvent_t e1, const TsaLevels* lv, int* res) {
  switch (L.W) {
    case 1: return launch_sweep_w<1, SLICE>(L, mode, order, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, eo, st, e0, e1, lv, res);
    case 2: return launch_sweep_w<2, SLICE>(L, mode, order, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, eo, st, e0, e1, lv, res);
    case 4: return launch_sweep_w<4, SLICE>(L, mode, order, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, eo, st, e0, e1, lv, res);
    case 8: return launch_sweep_w<8, SLICE>(L, mode, order, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, eo, st, e0, e1, lv, res);
    case 0: return launch_sweep_w<0, SLICE>(L, mode, order, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, eo, st, e0, e1, lv, res);
    default: return hipErrorInvalidValue;
  }
}

