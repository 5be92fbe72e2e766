// tsa_fold.h -- whole-chain evaluation from per-node costs (device code shared by tsa_kernels.hip and
// tsa_wide.hip).
//
// The reference evaluates a chain with 32 lanes (csrc/treesa_gpu.cu:386-434): lane t computes the cost of
// internal nodes t, t+32, ... and folds them with lse_f from -inf, then an xor butterfly 16, 8, 4, 2, 1
// combines the lanes; sc, the number of internal nodes of maximal size and |S| are integer reductions.
// Node costs do not depend on the fold, so they may be computed by any lanes in any order and held in
// memory; tsa_fold32 then runs the fold in the reference's order and is bit-identical to the one-loop form.
#pragma once
#include "tsa_kernels.h"

struct TsaEvalOut {
  float lcost;
  int sc, sc_int, ncand, ns;
};

// Cost (log2) and masked size Z of internal node i: (left child, right child) -> i, every label set masked
// by ~S (S may be null).  NW = words per label set (W, or P.W when W = 0).
template <int W, int MODE>
__device__ __forceinline__ float tsa_node_eval(const TsaKParams& P, const uint64_t* lab, const uint32_t* ch,
                                               const uint64_t* S, const uint64_t* lf, const TsaMathTabs& T, int i,
                                               int& Zout) {
  const int NW = W > 0 ? W : P.W, m = P.m;
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
  Zout = Z;
  return tsa_node_cost<MODE>(B, M, N, K, Z, P.model, T);
}

// The 32-lane fold of cost[0..nint) / z[0..nint) (l32 = lane within a 32-lane group; every lane of the
// group returns the result).  lf / S / NW serve the masked leaf sizes when S is set.  The lse chain of a
// lane is serial; its operands are read TSA_FOLD_BATCH at a time ahead of it, so that no step waits on a
// load, and the size statistics run in a loop of their own.
// Costs are floats, or (tc mode, whose node costs are integers) 16-bit integers converted exactly.
#define TSA_FOLD_BATCH 8
template <typename CT>
__device__ __forceinline__ TsaEvalOut tsa_fold32(const TsaKParams& P, const CT* cost, const uint16_t* z,
                                                 const uint64_t* S, const uint64_t* lf, int NW, const TsaMathTabs& T,
                                                 int l32) {
  const int nint = P.nint, m = P.m;
  float acc = -INFINITY;
  for (int i0 = l32; i0 < nint; i0 += 32 * TSA_FOLD_BATCH) {
    float cb[TSA_FOLD_BATCH];
#pragma unroll
    for (int q = 0; q < TSA_FOLD_BATCH; q++) {
      const int i = i0 + 32 * q;
      cb[q] = i < nint ? (float)cost[i] : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < TSA_FOLD_BATCH; q++)
      if (i0 + 32 * q < nint) acc = tsa_lse_f(acc, cb[q], T);
  }
  int scl = 0, cntl = 0;
  for (int i0 = l32; i0 < nint; i0 += 32 * TSA_FOLD_BATCH) {  // (the sizes read ahead too)
    int zb[TSA_FOLD_BATCH];
#pragma unroll
    for (int q = 0; q < TSA_FOLD_BATCH; q++) {
      const int i = i0 + 32 * q;
      zb[q] = i < nint ? (int)z[i] : -1;
    }
#pragma unroll
    for (int q = 0; q < TSA_FOLD_BATCH; q++) {
      const int Z = zb[q];
      if (Z > scl) {
        scl = Z;
        cntl = 1;
      } else if (Z == scl) {
        cntl++;
      }
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
