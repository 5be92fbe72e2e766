// tsa_arith.h -- arithmetic of one TreeSA proposal, shared by the HIP kernels and the host side of the
// library (both compiled by hipcc with -ffp-contract=off).
//
// Semantics follow the reference's shared header csrc/common.h: Philox4x32-10 keyed by
// (node, sweep, chain) (common.h:36-47), the rotation rule choice (common.h:231-238), the popcount
// counters of a move (common.h:165-196), dE from the counters (common.h:198-222), the Metropolis test
// (common.h:224-229) and the par-order priorities (common.h:250-272).  Label sets here are dense
// 64-bit words (the reference uses 32-bit words); popcounts are additive over words, so every counter
// is the same integer.
#pragma once
#include <stdint.h>
#include "tsa_math.h"

#if defined(__HIPCC__)
#define TSA_HD __host__ __device__ static inline
#else
#define TSA_HD static inline
#endif

struct TsaU4 {
  uint32_t x, y, z, w;
};

// Philox4x32-10 (Salmon et al., SC'11), counter c, key (k0, k1).  csrc/common.h:36-47.
TSA_HD TsaU4 tsa_philox(TsaU4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int i = 0; i < 10; i++) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c.x;
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c.z;
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    c = TsaU4{hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0};
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c;
}

TSA_HD int tsa_popc64(uint64_t x) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __popcll(x);
#else
  return __builtin_popcountll(x);
#endif
}

// 32-bit finalizer of MurmurHash3 (csrc/common.h:250-257).
TSA_HD uint32_t tsa_mix32(uint32_t h) {
  h ^= h >> 16;
  h *= 0x85EBCA6Bu;
  h ^= h >> 13;
  h *= 0xC2B2AE35u;
  h ^= h >> 16;
  return h;
}

// Per-sweep hash of chain c (common.h:261): hs = mix32(s * 0x85EBCA77 + mix32(c ^ key0)).
TSA_HD uint32_t tsa_sweep_hash(uint32_t s, uint32_t c, uint32_t key0) {
  return tsa_mix32(s * 0x85EBCA77u + tsa_mix32(c ^ key0));
}
// Par-order priority of internal node v, odd and nonzero (0 marks "visited"): common.h:260-263.
TSA_HD uint32_t tsa_par_pri(uint32_t v, uint32_t hs) { return (tsa_mix32(v * 0x9E3779B1u + hs) >> 16) | 1u; }
// par_band priority from the depth d at sweep start (common.h:266-268).
TSA_HD uint32_t tsa_band_pri(uint32_t v, uint32_t hs, int d, int L) {
  return ((uint32_t)((L - 1 - d % L) & 15) << 12) | (tsa_par_pri(v, hs) & 0x0FFEu) | 1u;
}
// par_follow priority of a follow-up visit, even and nonzero (common.h:270-272).
TSA_HD uint32_t tsa_follow_pri(uint32_t v, uint32_t hs) {
  return ((tsa_mix32((v * 0x9E3779B1u + hs) ^ 0x5BD1E995u) >> 16) & 0xFFFEu) | 2u;
}

// Rule 0..3 (Julia rules 1..4) from the top bits of r given which children are internal, -1 if none
// applies.  common.h:233-238.
TSA_HD int tsa_pick_rule(bool li, bool ri, uint32_t r) {
  if (li && ri) return (int)(r >> 30);
  if (li) return (int)(r >> 31);
  if (ri) return 2 + (int)(r >> 31);
  return -1;
}

// Energy-model parameters (the reference's Params fields that the arithmetic reads, common.h:60-94).
struct TsaModel {
  float sc_target, sc_weight;
  float lpeak, lbw, llaunch;
  int m0, n0, k0;
  float v2_l3launch, v2_lperm2, v2_lcc_bit, v2_lcc_cell, v2_ltc_bit, v2_ltc_pad, v2_ltc_out, v2_lsmall_cell;
  int v2_small_rank;
};

// log2(2^a + 2^b) for integers with the float table lse[d] = (float)log2(1 + 2^-d) (0 for d >= 53).
// common.h:104-118.
TSA_HD float tsa_lse_i(int a, int b, const float* lse) {
  const int mx = a > b ? a : b;
  int d = a > b ? a - b : b - a;
  d = d < 63 ? d : 63;
  return (float)mx + lse[d];
}

// log2 of the modeled time of one contraction, GPU roofline model (common.h:129-135).
TSA_HD float tsa_gpu_lt(int B, int M, int N, int K, const TsaModel& P, const TsaMathTabs& T) {
  const int Me = M > P.m0 ? M : P.m0, Ne = N > P.n0 ? N : P.n0, Ke = K > P.k0 ? K : P.k0;
  const float lops = (float)(1 + B + Me + Ne + Ke) - P.lpeak;
  const float lbits = tsa_lse_f(tsa_lse_f((float)(B + M + K), (float)(B + N + K), T), (float)(B + M + N), T) - P.lbw;
  const float lt = lops > lbits ? lops : lbits;
  return tsa_lse_f(lt, P.llaunch, T);
}

// log2 of the modeled time of one contraction, measured H100 model (common.h:138-151).
TSA_HD float tsa_h100_lt(int B, int M, int N, int K, const TsaModel& P, const TsaMathTabs& T) {
  if (B + M + N <= P.v2_small_rank) return P.v2_lsmall_cell + (float)(B + M + N + K);
  const float la = (float)(B + M + K), lb = (float)(B + N + K), lc = (float)(B + M + N);
  const float lab = tsa_lse_f(la, lb, T), lmoved = tsa_lse_f(lab, lc, T);
  const float perm = P.v2_lperm2 + lab;
  float best = tsa_lse_f(P.v2_lcc_bit + lmoved, P.v2_lcc_cell + (float)(B + M + N + K), T);
  const int MN = M > N ? M : N;
  if (K >= 7 && MN >= 5) {
    const int Me = M > 6 ? M : 6, Ne = N > 6 ? N : 6, Ke = K > 8 ? K : 8;
    const float tc =
        tsa_lse_f(tsa_lse_f(P.v2_ltc_bit + lmoved, P.v2_ltc_pad + (float)(B + Me + Ne + Ke), T), P.v2_ltc_out + lc, T);
    best = tc < best ? tc : best;
  }
  return tsa_lse_f(tsa_lse_f(P.v2_l3launch, perm, T), best, T);
}

// Cost (log2) of contraction (x, y) -> z with counts B=|xyz|, M=|x~yz|, N=|~xyz|, K=|xy~z|, Z=|z|.
// Mode 0 is tc = |z| + |x & y & ~z| (common.h:159-163).
template <int MODE>
TSA_HD float tsa_node_cost(int B, int M, int N, int K, int Z, const TsaModel& P, const TsaMathTabs& T) {
  if (MODE == 0) return (float)(Z + K);
  return MODE == 1 ? tsa_gpu_lt(B, M, N, K, P, T) : tsa_h100_lt(B, M, N, K, P, T);
}

// Counters of one proposal: sizes of d (the visited node), P (pivot child) and X (P's new label set),
// and per contraction q (0: (K,M)->P, 1: (P,O)->d before; 2: (K,O)->X, 3: (X,M)->d after) the counts.
// csrc/common.h:165-170.
struct TsaCounts {
  int sd, sp, sx;
  int B[4], M[4], N[4], K[4];
};

TSA_HD void tsa_counts_zero(TsaCounts& c) {
  c.sd = c.sp = c.sx = 0;
  for (int q = 0; q < 4; q++) c.B[q] = c.M[q] = c.N[q] = c.K[q] = 0;
}

// Three-input bitwise functions by truth table: bit i of f is the result for the operand bits
// (a, b, c) = (i >> 2 & 1, i >> 1 & 1, i & 1), i.e. f = g(0xF0, 0xCC, 0xAA) for the function g.  On the device
// one v_bitop3_b32 per 32-bit half; on the host the same table bit by bit.
#define TSA_F_AB_NC 0x40u   // a & b & ~c
#define TSA_F_ABC 0x80u     // a & b & c
#define TSA_F_A_NB_C 0x20u  // a & ~b & c
#define TSA_F_NA_BC 0x08u   // ~a & b & c
#define TSA_F_A_BORC 0xE0u  // a & (b | c)
template <uint32_t F>
TSA_HD uint32_t tsa_bitop3(uint32_t a, uint32_t b, uint32_t c) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_bitop3_b32(a, b, c, F);
#else
  uint32_t r = 0;
  for (int i = 0; i < 8; i++)
    if ((F >> i) & 1u) r |= ((i & 4) ? a : ~a) & ((i & 2) ? b : ~b) & ((i & 1) ? c : ~c);
  return r;
#endif
}

// popcount of g(a, b, c) over a 64-bit word, as two 32-bit halves
template <uint32_t F>
TSA_HD int tsa_popc3(uint64_t a, uint64_t b, uint64_t c) {
  const uint32_t lo = tsa_bitop3<F>((uint32_t)a, (uint32_t)b, (uint32_t)c);
  const uint32_t hi = tsa_bitop3<F>((uint32_t)(a >> 32), (uint32_t)(b >> 32), (uint32_t)(c >> 32));
  return tsa_popc64(((uint64_t)hi << 32) | lo);
}

// x = (k|o)&(m|d), P's label set after a move
TSA_HD uint64_t tsa_xset(uint64_t k, uint64_t o, uint64_t m, uint64_t d) {
  const uint64_t t = k | o;
  const uint32_t lo = tsa_bitop3<TSA_F_A_BORC>((uint32_t)t, (uint32_t)m, (uint32_t)d);
  const uint32_t hi = tsa_bitop3<TSA_F_A_BORC>((uint32_t)(t >> 32), (uint32_t)(m >> 32), (uint32_t)(d >> 32));
  return ((uint64_t)hi << 32) | lo;
}

TSA_HD void tsa_count3(uint64_t x, uint64_t y, uint64_t z, int& B, int& M, int& N, int& K) {
  B += tsa_popc3<TSA_F_ABC>(x, y, z);
  M += tsa_popc3<TSA_F_A_NB_C>(x, y, z);
  N += tsa_popc3<TSA_F_NA_BC>(x, y, z);
  K += tsa_popc3<TSA_F_AB_NC>(x, y, z);
}

// One 64-bit word of the masked sets k, m, p, o, d and x = (k|o)&(m|d).  common.h:180-196.
template <int MODE>
TSA_HD void tsa_acc(TsaCounts& c, uint64_t k, uint64_t m, uint64_t p, uint64_t o, uint64_t d, uint64_t x) {
  c.sd += tsa_popc64(d);
  c.sp += tsa_popc64(p);
  c.sx += tsa_popc64(x);
  if (MODE == 0) {
    c.K[0] += tsa_popc3<TSA_F_AB_NC>(k, m, p);
    c.K[1] += tsa_popc3<TSA_F_AB_NC>(p, o, d);
    c.K[2] += tsa_popc3<TSA_F_AB_NC>(k, o, x);
    c.K[3] += tsa_popc3<TSA_F_AB_NC>(x, m, d);
  } else {
    tsa_count3(k, m, p, c.B[0], c.M[0], c.N[0], c.K[0]);
    tsa_count3(p, o, d, c.B[1], c.M[1], c.N[1], c.K[1]);
    tsa_count3(k, o, x, c.B[2], c.M[2], c.N[2], c.K[2]);
    tsa_count3(x, m, d, c.B[3], c.M[3], c.N[3], c.K[3]);
  }
}

// The tc-mode counts of the configuration after the move only (sd, sx, K2, K3), for callers that take the
// configuration before it from cached node costs (tsa_energy_tc_cached).
TSA_HD void tsa_acc_after_tc(TsaCounts& c, uint64_t k, uint64_t m, uint64_t o, uint64_t d, uint64_t x) {
  c.sd += tsa_popc64(d);
  c.sx += tsa_popc64(x);
  c.K[2] += tsa_popc3<TSA_F_AB_NC>(k, o, x);
  c.K[3] += tsa_popc3<TSA_F_AB_NC>(x, m, d);
}

// dE of the move (common.h:202-222):
//   dtc = log2(2^c2 + 2^c3) - log2(2^c0 + 2^c1); dE = w*(sc1 - sc0) + dtc with sc0 = max(|P|,|d|),
//   sc1 = max(|X|,|d|) and w = sc_weight if max(sc0, sc1) > sc_target else 0.
// The tc-mode form from the two node costs before the move, costP = |P| + |K & M & ~P| and costV =
// |d| + |P & O & ~d| (the costs of contractions (K, M) -> P and (P, O) -> d, symmetric in the two inputs),
// the counts after it and sp = |P|: a caller that keeps every node's cost and size current gets the float
// tsa_energy_from_counts<0> gets from the counted sets, without reading P's set.
TSA_HD float tsa_energy_tc_cached(int costP, int costV, int sp, int sd, int sx, int K2, int K3, const TsaModel& P,
                                  const float* lse) {
  const float dtc = tsa_lse_i(sx + K2, sd + K3, lse) - tsa_lse_i(costP, costV, lse);
  const int sc0 = sp > sd ? sp : sd;
  const int sc1 = sx > sd ? sx : sd;
  const int scmax = sc0 > sc1 ? sc0 : sc1;
  const float w = ((float)scmax > P.sc_target) ? P.sc_weight : 0.0f;
  return w * (float)(sc1 - sc0) + dtc;
}

template <int MODE>
TSA_HD float tsa_energy_from_counts(const TsaCounts& c, const TsaModel& P, const float* lse, const TsaMathTabs& T) {
  if (MODE == 0) return tsa_energy_tc_cached(c.sp + c.K[0], c.sd + c.K[1], c.sp, c.sd, c.sx, c.K[2], c.K[3], P, lse);
  const float t0 = tsa_lse_f(tsa_node_cost<MODE>(c.B[0], c.M[0], c.N[0], c.K[0], c.sp, P, T),
                             tsa_node_cost<MODE>(c.B[1], c.M[1], c.N[1], c.K[1], c.sd, P, T), T);
  const float t1 = tsa_lse_f(tsa_node_cost<MODE>(c.B[2], c.M[2], c.N[2], c.K[2], c.sx, P, T),
                             tsa_node_cost<MODE>(c.B[3], c.M[3], c.N[3], c.K[3], c.sd, P, T), T);
  const float dtc = t1 - t0;
  const int sc0 = c.sp > c.sd ? c.sp : c.sd;
  const int sc1 = c.sx > c.sd ? c.sx : c.sd;
  const int scmax = sc0 > sc1 ? sc0 : sc1;
  const float w = ((float)scmax > P.sc_target) ? P.sc_weight : 0.0f;
  return w * (float)(sc1 - sc0) + dtc;
}

// Metropolis: u = (r >> 8) * 2^-24 < expf(-beta * dE).  common.h:226-229.
TSA_HD bool tsa_metropolis(uint32_t r, float beta, float dE, const uint64_t* exp2tab) {
  const float u = (float)(r >> 8) * (1.0f / 16777216.0f);
  return u < tsa_expf_t(-beta * dE, exp2tab);
}

// The Metropolis test as a threshold on x = -beta * dE: tsa_expf is non-decreasing over the floats (checked on
// every float), so {x : expf(x) > u} is every float from its least element T(u) up and u < expf(x) exactly when
// x >= T(u).  For u = (r >> 8) * 2^-24 > 0 the set's least element lies below zero, where a float's bit pattern
// grows as the float falls.  The search starts at the float nearest log(u + ulp(u) / 2) (where a correctly
// rounded expf would first exceed u), doubles its step in bit patterns until it brackets the boundary, then
// halves the bracket: one or two expf evaluations for most u, about 2 log2 of the distance in ulps near u = 1
// (where t is much finer than expf's output).  u = 0 takes the same search (its boundary lies where expf
// stops underflowing to zero).  NaN for a search that does not settle within its bound, which no u of the
// 2^24 the kernels draw reaches (checked for every one of them, on the host and on the device).
TSA_HD float tsa_accept_threshold(uint32_t r, const uint64_t* exp2tab) {
  const float nan = tsa_ffrom(0x7fc00000u);
  const uint32_t k = r >> 8;
  const float u = (float)k * (1.0f / 16777216.0f);
  const double half = 0.5 * ((double)tsa_ffrom(tsa_fbits(u) + 1u) - (double)u);
  const float t0 = (float)log((double)u + half);
  if (!(t0 < 0.0f)) return nan;
  // in(b): the float with bit pattern b (below zero) has expf above u
  const uint32_t neg_zero = 0x80000000u, neg_inf = 0xff800000u;
  uint32_t b = tsa_fbits(t0);
  int evals = 0;
  auto in = [&](uint32_t bits) { evals++; return tsa_expf_t(tsa_ffrom(bits), exp2tab) > u; };
  uint32_t inside, outside;  // a pattern in the set and one below it (larger pattern) outside it
  if (in(b)) {
    inside = b;
    uint32_t step = 1u;
    for (;;) {
      const uint32_t probe = inside + step < neg_inf && inside + step > inside ? inside + step : neg_inf;
      if (!in(probe)) {
        outside = probe;
        break;
      }
      if (probe == neg_inf || evals > 40) return nan;
      inside = probe;
      step <<= 1;
    }
  } else {
    outside = b;
    uint32_t step = 1u;
    for (;;) {
      const uint32_t probe = outside - step > neg_zero && outside - step < outside ? outside - step : neg_zero + 1u;
      if (in(probe)) {
        inside = probe;
        break;
      }
      if (probe == neg_zero + 1u || evals > 40) return nan;
      outside = probe;
      step <<= 1;
    }
  }
  while (outside - inside > 1u) {  // inside < outside as patterns; the least float in the set is the largest
    const uint32_t mid = inside + (outside - inside) / 2u;  // pattern inside it
    if (in(mid)) inside = mid;
    else outside = mid;
    if (evals > 80) return nan;
  }
  return tsa_ffrom(inside);
}

// Slots of rule r (reference comment csrc/treesa_gpu.cu:137-144): the pivot P is the left child
// (slotP 0) for rules 0, 1 and the right child for rules 2, 3; M, the grandchild under P that moves
// up, is P's left child (slotM 0) for rules 1, 2 and its right child for rules 0, 3.  Every rule swaps
// M with the other child O, keeping slots, and gives P the labels X = (K|O)&(M|d).
TSA_HD int tsa_slot_p(int rule) { return rule >> 1; }
TSA_HD int tsa_slot_m(int rule) { return ((rule ^ (rule >> 1)) & 1) ^ 1; }
