// tsa_math.h -- float exp/exp2/log2 that return exactly what the host C library returns.
//
// Every Metropolis test of the annealer compares a 24-bit uniform against expf(-beta*dE), and the
// whole-chain energy folds node costs with log2(2^a + 2^b) = mx + log2f(1 + exp2f(mn - mx)).  The
// accept decisions (and therefore whole trajectories) are only reproducible across host and device if
// these three functions return bit-identical floats on both sides, so they are restated here:
//
//  * expf / exp2f: the table method of Szabolcs Nagy's "optimized-routines" (Arm Ltd., published in
//    glibc >= 2.28 as sysdeps/ieee754/flt-32/e_expf.c / e_exp2f.c): x*N/ln2 = k + r with N = 32,
//    2^(k/N) from a 32-entry table of 2^(i/32) (correctly rounded doubles, entry i stored as
//    bits(2^(i/32)) - (i << 47) so that adding k << 47 scales by 2^(k div 32)), and a degree-3
//    polynomial for 2^(r/N) evaluated in double, rounded once to float.  The expf table carries entry
//    31 raised by 30 ulp: with it the restatement agrees with glibc 2.35's expf on all 2^32 inputs
//    (any raise in [12, 47] does; the unraised entry disagrees on exactly two inputs, both in
//    bucket 31).  exp2f agrees with the unraised table on all 2^32 inputs.  Both claims are checked
//    exhaustively by tests/test_math_exhaustive.py against the host libm.
//  * log2f is only ever called on 1 + exp2f(d) with d <= 0, i.e. on [1, 2].  It is evaluated in double
//    (a 128-entry table of reciprocals and their logarithms, then a degree-6 series), rounded to float,
//    and then corrected by a 2-bit table over the 2^23 floats of [1, 2) that the library's host side
//    fills by comparing this same function with its libm log2f (build_log2_fix in tsa_capi.hip).  The
//    correction is a pure function of the input float, so host and device agree bit for bit wherever the
//    table came from the host libm that the oracle uses.
//
// All arithmetic is IEEE double (+, -, *, / and explicit fma), which is correctly rounded on both
// gfx950 and x86-64; the file must be compiled with -ffp-contract=off so that no further fusing happens.
#pragma once
#include <stdint.h>
#include <string.h>
#include <math.h>

#if defined(__HIPCC__)
#define TSA_MATH_FN __host__ __device__ static inline
#else
#define TSA_MATH_FN static inline
#endif

TSA_MATH_FN uint64_t tsa_dbits(double x) { uint64_t u; memcpy(&u, &x, 8); return u; }
TSA_MATH_FN double tsa_dfrom(uint64_t u) { double x; memcpy(&x, &u, 8); return x; }
TSA_MATH_FN uint32_t tsa_fbits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
TSA_MATH_FN float tsa_ffrom(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

// bits(2^(i/32)) - (i << 47), i = 0..31: 2^(i/32) correctly rounded to double
#define TSA_EXP2_TAB                                                                                  \
  {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,       \
   0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,       \
   0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,       \
   0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,       \
   0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,       \
   0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,       \
   0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,       \
   0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

#if defined(__HIPCC__)
__constant__ static const uint64_t tsa_exp2_tab_d[32] = TSA_EXP2_TAB;
#endif
static const uint64_t tsa_exp2_tab_h[32] = TSA_EXP2_TAB;  // host copy (host code of .hip files too)
#if defined(__HIP_DEVICE_COMPILE__)
#define TSA_EXP2_TABLE tsa_exp2_tab_d
#else
#define TSA_EXP2_TABLE tsa_exp2_tab_h
#endif

// 2^(r/N) polynomial, N = 32 (exp2f form: r in units of 1, scaled for expf below)
#define TSA_EXP2_C0 0x1.c6af84b912394p-5
#define TSA_EXP2_C1 0x1.ebfce50fac4f3p-3
#define TSA_EXP2_C2 0x1.62e42ff0c52d6p-1
#define TSA_EXP_SHIFT 0x1.8p+52
#define TSA_EXP_INVLN2N (0x1.71547652b82fep+0 * 32)
#define TSA_EXPF_RAISE31 30ull

// expf with the 2^(i/32) table passed in (kernels pass a copy staged in LDS: a per-lane index into a
// constant or kernel-argument array would be a vector memory load on every call).
TSA_MATH_FN float tsa_expf_t(float x, const uint64_t* tab) {
  const uint32_t abstop = (tsa_fbits(x) >> 20) & 0x7ff;
  if (abstop >= 0x42b) {  // |x| >= 88: infinities, NaN, overflow and underflow
    if (tsa_fbits(x) == 0xff800000u) return 0.0f;
    if (abstop >= 0x7f8) return x + x;
    if (x > 0x1.62e42ep6f) return INFINITY;
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  const double xd = (double)x;
  const double z = TSA_EXP_INVLN2N * xd;
  double kd = z + TSA_EXP_SHIFT;
  const uint64_t ki = tsa_dbits(kd);
  kd -= TSA_EXP_SHIFT;
  const double r = z - kd;
  const uint32_t i = (uint32_t)(ki & 31u);
  const uint64_t t = tab[i] + (i == 31u ? TSA_EXPF_RAISE31 : 0ull) + (ki << 47);
  const double s = tsa_dfrom(t);
  const double c0 = TSA_EXP2_C0 / 32 / 32 / 32, c1 = TSA_EXP2_C1 / 32 / 32, c2 = TSA_EXP2_C2 / 32;
  const double zz = fma(c0, r, c1);
  const double r2 = r * r;
  double y = fma(c2, r, 1.0);
  y = fma(zz, r2, y);
  return (float)(y * s);
}

TSA_MATH_FN float tsa_exp2f_t(float x, const uint64_t* tab) {
  const uint32_t abstop = (tsa_fbits(x) >> 20) & 0x7ff;
  if (abstop >= 0x430) {  // |x| >= 128
    if (tsa_fbits(x) == 0xff800000u) return 0.0f;
    if (abstop >= 0x7f8) return x + x;
    if (x > 0.0f) return INFINITY;
    if (x <= -150.0f) return 0.0f;
  }
  const double xd = (double)x;
  double kd = xd + TSA_EXP_SHIFT / 32;
  const uint64_t ki = tsa_dbits(kd);
  kd -= TSA_EXP_SHIFT / 32;
  const double r = xd - kd;
  const uint64_t t = tab[ki & 31u] + (ki << 47);
  const double s = tsa_dfrom(t);
  const double zz = fma(TSA_EXP2_C0, r, TSA_EXP2_C1);
  const double r2 = r * r;
  double y = fma(TSA_EXP2_C2, r, 1.0);
  y = fma(zz, r2, y);
  return (float)(y * s);
}

// exp2f's main path alone, for |x| < 128 (where tsa_exp2f_t takes it): no branches.
TSA_MATH_FN float tsa_exp2f_core(float x, const uint64_t* tab) {
  const double xd = (double)x;
  double kd = xd + TSA_EXP_SHIFT / 32;
  const uint64_t ki = tsa_dbits(kd);
  kd -= TSA_EXP_SHIFT / 32;
  const double r = xd - kd;
  const uint64_t t = tab[ki & 31u] + (ki << 47);
  const double s = tsa_dfrom(t);
  const double zz = fma(TSA_EXP2_C0, r, TSA_EXP2_C1);
  const double r2 = r * r;
  double y = fma(TSA_EXP2_C2, r, 1.0);
  y = fma(zz, r2, y);
  return (float)(y * s);
}

TSA_MATH_FN float tsa_expf(float x) { return tsa_expf_t(x, TSA_EXP2_TABLE); }
TSA_MATH_FN float tsa_exp2f(float x) { return tsa_exp2f_t(x, TSA_EXP2_TABLE); }

// log2 on [1, 2) in double, for float inputs: y = c_j * (1 + z) with c_j = 1 + j/128 and j the top 7 bits
// of y's mantissa, z = y * inv_j - 1 in one fused multiply-add (|z| < 2^-7), and
// log2(y) = t_j + log2(1 + z) with t_j = -log2(inv_j) from the table and log2(1 + z) by its Taylor series
// to z^6 (truncation below 2^-42 relative).  The table (inv_j, t_j as IEEE-754 bit patterns) and the
// coefficients A_k = (-1)^(k+1) / (k ln 2), all rounded to double, are printed by gen_log2_table.py.
#define TSA_LOG2_TAB \
  {0x3ff0000000000000ull, 0x0000000000000000ull, 0x3fefc07f01fc07f0ull, 0x3f86fe50b6ef085dull, \
   0x3fef81f81f81f820ull, 0x3f96e79685c2d212ull, 0x3fef44659e4a4271ull, 0x3fa11cd1d513341bull, \
   0x3fef07c1f07c1f08ull, 0x3fa6bad3758efd81ull, 0x3feecc07b301ecc0ull, 0x3fac4dfab90aab6aull, \
   0x3fee9131abf0b767ull, 0x3fb0eb389fa29f9dull, 0x3fee573ac901e574ull, 0x3fb3aa2fdd27f1bfull, \
   0x3fee1e1e1e1e1e1eull, 0x3fb663f6fac91318ull, 0x3fede5d6e3f8868aull, 0x3fb918a16e46335eull, \
   0x3fedae6076b981dbull, 0x3fbbc84240adabb9ull, 0x3fed77b654b82c34ull, 0x3fbe72ec117fa5adull, \
   0x3fed41d41d41d41dull, 0x3fc08c588cda79e5ull, 0x3fed0cb58f6ec074ull, 0x3fc1dcd197552b7dull, \
   0x3fecd85689039b0bull, 0x3fc32ae9e278ae19ull, 0x3feca4b3055ee191ull, 0x3fc476a9f983f74dull, \
   0x3fec71c71c71c71cull, 0x3fc5c01a39fbd68bull, 0x3fec3f8f01c3f8f0ull, 0x3fc70742d4ef0280ull, \
   0x3fec0e070381c0e0ull, 0x3fc84c2bd02f03b6ull, 0x3febdd2b899406f7ull, 0x3fc98edd077e70e1ull, \
   0x3febacf914c1bad0ull, 0x3fcacf5e2db4ec91ull, 0x3feb7d6c3dda338bull, 0x3fcc0db6cdd94defull, \
   0x3feb4e81b4e81b4full, 0x3fcd49ee4c32596cull, 0x3feb2036406c80d9ull, 0x3fce840be74e6a4dull, \
   0x3feaf286bca1af28ull, 0x3fcfbc16b902680dull, 0x3feac5701ac5701bull, 0x3fd0790adbb03009ull, \
   0x3fea98ef606a63beull, 0x3fd11307dad30b74ull, 0x3fea6d01a6d01a6dull, 0x3fd1ac05b291f070ull, \
   0x3fea41a41a41a41aull, 0x3fd24407ab0e073aull, 0x3fea16d3f97a4b02ull, 0x3fd2db10fc4d9aaeull, \
   0x3fe9ec8e951033d9ull, 0x3fd37124cea4cdedull, 0x3fe9c2d14ee4a102ull, 0x3fd406463b1b0448ull, \
   0x3fe999999999999aull, 0x3fd49a784bcd1b8aull, 0x3fe970e4f80cb872ull, 0x3fd52dbdfc4c96b5ull, \
   0x3fe948b0fcd6e9e0ull, 0x3fd5c01a39fbd689ull, 0x3fe920fb49d0e229ull, 0x3fd6518fe4677ba6ull, \
   0x3fe8f9c18f9c18faull, 0x3fd6e221cd9d0cddull, 0x3fe8d3018d3018d3ull, 0x3fd771d2ba7efb3cull, \
   0x3fe8acb90f6bf3aaull, 0x3fd800a563161c53ull, 0x3fe886e5f0abb04aull, 0x3fd88e9c72e0b224ull, \
   0x3fe8618618618618ull, 0x3fd91bba891f170aull, 0x3fe83c977ab2beddull, 0x3fd9a802391e2330ull, \
   0x3fe8181818181818ull, 0x3fda33760a7f6051ull, 0x3fe7f405fd017f40ull, 0x3fdabe18797f1f4aull, \
   0x3fe7d05f417d05f4ull, 0x3fdb47ebf73882a1ull, 0x3fe7ad2208e0ecc3ull, 0x3fdbd0f2e9e79032ull, \
   0x3fe78a4c8178a4c8ull, 0x3fdc592fad295b57ull, 0x3fe767dce434a9b1ull, 0x3fdce0a4923a587dull, \
   0x3fe745d1745d1746ull, 0x3fdd6753e032ea0eull, 0x3fe724287f46debcull, 0x3fdded3fd442364cull, \
   0x3fe702e05c0b8170ull, 0x3fde726aa1e754d3ull, 0x3fe6e1f76b4337c7ull, 0x3fdef6d67328e220ull, \
   0x3fe6c16c16c16c17ull, 0x3fdf7a8568cb06ceull, 0x3fe6a13cd1537290ull, 0x3fdffd799a83ff9cull, \
   0x3fe6816816816817ull, 0x3fe03fda8b97997eull, 0x3fe661ec6a5122f9ull, 0x3fe0809cf27f703dull, \
   0x3fe642c8590b2164ull, 0x3fe0c10500d63aa7ull, 0x3fe623fa77016240ull, 0x3fe10113b153c8eaull, \
   0x3fe6058160581606ull, 0x3fe140c9faa1e543ull, 0x3fe5e75bb8d015e7ull, 0x3fe18028cf72976bull, \
   0x3fe5c9882b931057ull, 0x3fe1bf311e95d00eull, 0x3fe5ac056b015ac0ull, 0x3fe1fde3d30e8127ull, \
   0x3fe58ed2308158edull, 0x3fe23c41d42727c8ull, 0x3fe571ed3c506b3aull, 0x3fe27a4c0585cbf7ull, \
   0x3fe5555555555555ull, 0x3fe2b803473f7ad2ull, 0x3fe5390948f40febull, 0x3fe2f56875eb3f26ull, \
   0x3fe51d07eae2f815ull, 0x3fe3327c6ab49ca7ull, 0x3fe5015015015015ull, 0x3fe36f3ffb6d9162ull, \
   0x3fe4e5e0a72f0539ull, 0x3fe3abb3faa02168ull, 0x3fe4cab88725af6eull, 0x3fe3e7d9379f7017ull, \
   0x3fe4afd6a052bf5bull, 0x3fe423b07e986aa8ull, 0x3fe49539e3b2d067ull, 0x3fe45f3a98a20738ull, \
   0x3fe47ae147ae147bull, 0x3fe49a784bcd1b8bull, 0x3fe460cbc7f5cf9aull, 0x3fe4d56a5b33cec5ull, \
   0x3fe446f86562d9fbull, 0x3fe510118708a8f9ull, 0x3fe42d6625d51f87ull, 0x3fe54a6e8ca5438eull, \
   0x3fe4141414141414ull, 0x3fe5848226989d34ull, 0x3fe3fb013fb013fbull, 0x3fe5be4d0cb51435ull, \
   0x3fe3e22cbce4a902ull, 0x3fe5f7cff41e09b0ull, 0x3fe3c995a47babe7ull, 0x3fe6310b8f553049ull, \
   0x3fe3b13b13b13b14ull, 0x3fe66a008e4788cbull, 0x3fe3991c2c187f63ull, 0x3fe6a2af9e5a0f0bull, \
   0x3fe3813813813814ull, 0x3fe6db196a761949ull, 0x3fe3698df3de0748ull, 0x3fe7133e9b156c7bull, \
   0x3fe3521cfb2b78c1ull, 0x3fe74b1fd64e0754ull, 0x3fe33ae45b57bcb2ull, 0x3fe782bdbfdda657ull, \
   0x3fe323e34a2b10bfull, 0x3fe7ba18f93502e5ull, 0x3fe30d190130d190ull, 0x3fe7f1322182cf16ull, \
   0x3fe2f684bda12f68ull, 0x3fe82809d5be7074ull, 0x3fe2e025c04b8097ull, 0x3fe85ea0b0b27b26ull, \
   0x3fe2c9fb4d812ca0ull, 0x3fe894f74b06ef8bull, 0x3fe2b404ad012b40ull, 0x3fe8cb0e3b4b3bbeull, \
   0x3fe29e4129e4129eull, 0x3fe900e6160002ceull, 0x3fe288b01288b013ull, 0x3fe9367f6da0ab2dull, \
   0x3fe27350b8812735ull, 0x3fe96bdad2acb5f6ull, 0x3fe25e22708092f1ull, 0x3fe9a0f8d3b0e050ull, \
   0x3fe2492492492492ull, 0x3fe9d5d9fd5010b4ull, 0x3fe23456789abcdfull, 0x3fea0a7eda4c112dull, \
   0x3fe21fb78121fb78ull, 0x3fea3ee7f38e181full, 0x3fe20b470c67c0d9ull, 0x3fea7315d02f20c7ull, \
   0x3fe1f7047dc11f70ull, 0x3feaa708f58014d4ull, 0x3fe1e2ef3b3fb874ull, 0x3feadac1e711c833ull, \
   0x3fe1cf06ada2811dull, 0x3feb0e4126bcc86cull, 0x3fe1bb4a4046ed29ull, 0x3feb418734a9008cull, \
   0x3fe1a7b9611a7b96ull, 0x3feb74948f5532daull, 0x3fe19453808ca29cull, 0x3feba769b39e4964ull, \
   0x3fe1811811811812ull, 0x3febda071cc67e6cull, 0x3fe16e0689427379ull, 0x3fec0c6d447c5dd3ull, \
   0x3fe15b1e5f75270dull, 0x3fec3e9ca2e1a055ull, 0x3fe1485f0e0acd3bull, 0x3fec7095ae91e1c8ull, \
   0x3fe135c81135c811ull, 0x3feca258dca93317ull, 0x3fe12358e75d3033ull, 0x3fecd3e6a0ca8908ull, \
   0x3fe1111111111111ull, 0x3fed053f6d260897ull, 0x3fe0fef010fef011ull, 0x3fed3663b27f31d5ull, \
   0x3fe0ecf56be69c90ull, 0x3fed6753e032ea0full, 0x3fe0db20a88f4696ull, 0x3fed9810643d6614ull, \
   0x3fe0c9714fbcda3bull, 0x3fedc899ab3ff56cull, 0x3fe0b7e6ec259dc8ull, 0x3fedf8f02086af2bull, \
   0x3fe0a6810a6810a7ull, 0x3fee29142e0e013full, 0x3fe0953f39010954ull, 0x3fee59063c8822ceull, \
   0x3fe0842108421084ull, 0x3fee88c6b3626a73ull, 0x3fe073260a47f7c6ull, 0x3feeb855f8ca88fcull, \
   0x3fe0624dd2f1a9fcull, 0x3feee7b471b3a950ull, 0x3fe05197f7d73404ull, 0x3fef16e281db7630ull, \
   0x3fe0410410410410ull, 0x3fef45e08bcf0656ull, 0x3fe03091b51f5e1aull, 0x3fef74aef0efafafull, \
   0x3fe0204081020408ull, 0x3fefa34e1177c234ull, 0x3fe0101010101010ull, 0x3fefd1be4c7f2af9ull}
#define TSA_LOG2_A1 0x1.71547652b82fep+0
#define TSA_LOG2_A2 -0x1.71547652b82fep-1
#define TSA_LOG2_A3 0x1.ec709dc3a03fdp-2
#define TSA_LOG2_A4 -0x1.71547652b82fep-2
#define TSA_LOG2_A5 0x1.2776c50ef9bfep-2
#define TSA_LOG2_A6 -0x1.ec709dc3a03fdp-3

#if defined(__HIPCC__)
__constant__ static const uint64_t tsa_log2_tab_d[256] = TSA_LOG2_TAB;
#endif
static const uint64_t tsa_log2_tab_h[256] = TSA_LOG2_TAB;

// Words of the tables a kernel stages in LDS for the float math: the 32-entry 2^(i/32) table, then the
// 256-word log2 core table.
#define TSA_MT_WORDS 288
#if defined(__HIPCC__)
// Every thread of the workgroup calls it; a workgroup barrier must follow before the first use.
__device__ __forceinline__ void tsa_math_stage(uint64_t* s) {
  for (int i = (int)threadIdx.x; i < TSA_MT_WORDS; i += (int)blockDim.x)
    s[i] = i < 32 ? tsa_exp2_tab_d[i] : tsa_log2_tab_d[i - 32];
}
#endif

// lg: the table (kernels pass a copy staged in LDS).  y must lie in [1, 2).
TSA_MATH_FN float tsa_log2f_core_t(float y, const uint64_t* lg) {
  const uint32_t j = (tsa_fbits(y) >> 16) & 127u;
  const double inv = tsa_dfrom(lg[2 * j]), t = tsa_dfrom(lg[2 * j + 1]);
  const double z = fma((double)y, inv, -1.0);
  double q = TSA_LOG2_A6;
  q = fma(q, z, TSA_LOG2_A5);
  q = fma(q, z, TSA_LOG2_A4);
  q = fma(q, z, TSA_LOG2_A3);
  q = fma(q, z, TSA_LOG2_A2);
  q = fma(q, z, TSA_LOG2_A1);
  return (float)fma(q, z, t);
}

// host code only
static inline float tsa_log2f_core(float y) { return tsa_log2f_core_t(y, tsa_log2_tab_h); }

// Number of 32-bit words of the log2f correction table: 2 bits for each of the 2^23 floats of [1, 2),
// 16 per word, so word mant >> 4 holds mantissa mant.
#define TSA_LOG2FIX_WORDS (1u << 19)

// Words of the summary bitmap of the correction table: bit w is set iff fix word w is nonzero (about one
// word in ten is), so a reader holding the 64 KB bitmap close by skips most reads of the 2 MB table.
#define TSA_LOG2MAP_WORDS (TSA_LOG2FIX_WORDS / 32u)

// The correction step of log2f on [1, 2): r = tsa_log2f_core(y), fix the host-libm correction table
// (2 bits per input: 0 keep, 1 +1 ulp, 2 -1 ulp) and, when map is not null, its summary bitmap.
TSA_MATH_FN float tsa_log2f_corr(float y, float r, const uint32_t* fix, const uint32_t* map) {
  const uint32_t mant = tsa_fbits(y) & 0x7fffffu;
  const uint32_t w = mant >> 4;
  if (map && ((map[w >> 5] >> (w & 31u)) & 1u) == 0u) return r;
  const uint32_t code = (fix[w] >> ((mant & 15u) * 2u)) & 3u;
  if (code == 0u) return r;
  return tsa_ffrom(tsa_fbits(r) + (code == 1u ? 1u : 0xffffffffu));
}

// Tables the float math reads: the 2^(i/32) table, the log2 core table, the log2f correction table and
// optionally its summary bitmap.
struct TsaMathTabs {
  const uint64_t* exp2;
  const uint32_t* fix;
  const uint32_t* map;
  const uint64_t* lg;
};

// log2f on [1, 2] with the host-libm correction table.  Inputs outside [1, 2] only arise from NaN
// operands and return NaN.
TSA_MATH_FN float tsa_log2f_12(float y, const TsaMathTabs& T) {
  if (!(y >= 1.0f && y <= 2.0f)) return y - y + NAN;
  if (y == 2.0f) return 1.0f;
  return tsa_log2f_corr(y, tsa_log2f_core_t(y, T.lg), T.fix, T.map);
}

// log2(2^a + 2^b) for floats (a or b may be -inf), the fold of modeled node costs:
// mx + log2f(1 + exp2f(mn - mx)) with mx = max(a, b), mn = min(a, b).  Cases, each as the reference's
// formula evaluates it:
//  * mx = -inf: -inf;
//  * d = mn - mx <= -24: exp2f gives at most 2^-24, 1 + that rounds to 1.0f (2^-24 is half an ulp of 1:
//    ties to even) and log2f(1) = +0, so the result is mx + 0.0f;
//  * d NaN (a NaN operand, or mx = mn = +inf): NaN;
//  * d = 0: 1 + exp2f(0) = 2 and log2f(2) = 1;
//  * otherwise y = 1 + exp2f(d) lies in [1, 2) and log2f(y) is the core value r corrected by the table.
//    The correction moves r by at most one ulp, to r- or r+, and float addition rounds monotonically, so
//    when mx + r- and mx + r+ round to the same float the corrected sum is that float too and the table is
//    not read (for mx of a few units and more that holds for all but a few per cent of the inputs).
// The arithmetic runs unconditionally on a clamped d (the branch-free form is faster on a GPU than the
// early returns, which diverge between lanes); only the rare table read is a branch.
TSA_MATH_FN float tsa_lse_f(float a, float b, const TsaMathTabs& T) {
  const float mx = a > b ? a : b;
  const float mn = a > b ? b : a;
  const float d = mn - mx;
  const bool full = d > -24.0f;  // false for NaN
  const float y = 1.0f + tsa_exp2f_core(full ? d : -24.0f, T.exp2);
  const bool two = y == 2.0f;
  const float r = two ? 1.0f : tsa_log2f_core_t(y, T.lg);
  float res = mx + r;
  const uint32_t rb = tsa_fbits(r);  // r >= +0: y >= 1
  if (full && !two && (rb == 0u || mx + tsa_ffrom(rb - 1u) != mx + tsa_ffrom(rb + 1u)))
    res = mx + tsa_log2f_corr(y, r, T.fix, T.map);
  res = full ? res : (d != d ? d : mx + 0.0f);
  return mx == -INFINITY ? mx : res;
}
