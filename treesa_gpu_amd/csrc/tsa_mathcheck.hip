// tsa_mathcheck.hip -- bin/tsa_mathcheck: the float math the sweep kernels restate (tsa_math.h, tsa_arith.h),
// evaluated on this GPU and compared bit for bit with this host's C library, exhaustively:
//   expf, exp2f        every one of the 2^32 floats (tsa_expf_t / tsa_exp2f_t, table staged in LDS as the
//                      kernels stage it) against libm expf / exp2f; NaN results compare as NaN
//   log2f on [1, 2]    every float of [1, 2] (tsa_log2f_12 with the correction table, built here from libm
//                      log2f the way the library builds it) against libm log2f
//   lse                log2(2^a + 2^b) = mx + log2f(1 + exp2f(mn - mx)) (the reference's fold, csrc/common.h:
//                      119-125) for every float difference d in [-24, 0] at six values of mx, tsa_lse_f against
//                      the formula with libm
//   thresholds         the Metropolis threshold T(u) (tsa_accept_threshold) for every uniform u = k * 2^-24 the
//                      kernels draw, device against host; the host's are checked against expf by the tests
// Prints one JSON line of mismatch counts (and the evaluation count of each check); exit status 0 iff every
// count is zero.  Chunks of 2^27 results are computed on the device, copied to page-locked host memory and
// compared by all host threads.
#include <hip/hip_runtime.h>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "tsa_arith.h"

#define CHUNK (1u << 27)

#define CK(call)                                                              \
  do {                                                                        \
    hipError_t e_ = (call);                                                   \
    if (e_ != hipSuccess) {                                                   \
      fprintf(stderr, "%s: %s\n", #call, hipGetErrorString(e_));              \
      exit(1);                                                                \
    }                                                                         \
  } while (0)

// out1[i] = expf(x), out2[i] = exp2f(x) for the float with bit pattern base + i, i < n
__global__ void __launch_bounds__(256) k_exp(uint32_t base, uint32_t n, float* __restrict__ out1,
                                             float* __restrict__ out2) {
  __shared__ uint64_t tab[32];
  if (threadIdx.x < 32) tab[threadIdx.x] = tsa_exp2_tab_d[threadIdx.x];
  __syncthreads();
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const float x = tsa_ffrom(base + i);
    out1[i] = tsa_expf_t(x, tab);
    out2[i] = tsa_exp2f_t(x, tab);
  }
}

// out[i] = log2f(y), y = 1 + i * 2^-23, i <= 2^23
__global__ void __launch_bounds__(256) k_log2(uint32_t n, const uint32_t* __restrict__ fix, float* __restrict__ out) {
  __shared__ uint64_t tab[TSA_MT_WORDS];
  tsa_math_stage(tab);
  __syncthreads();
  const TsaMathTabs T{tab, fix, fix + TSA_LOG2FIX_WORDS, tab + 32};
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    out[i] = tsa_log2f_12(tsa_ffrom(0x3f800000u + i), T);
}

// out[i] = lse(mx, d) for the float d with bit pattern base + i (negative floats: -0 up to -24)
__global__ void __launch_bounds__(256) k_lse(float mx, uint32_t base, uint32_t n, const uint32_t* __restrict__ fix,
                                             float* __restrict__ out) {
  __shared__ uint64_t tab[TSA_MT_WORDS];
  tsa_math_stage(tab);
  __syncthreads();
  const TsaMathTabs T{tab, fix, fix + TSA_LOG2FIX_WORDS, tab + 32};
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    out[i] = tsa_lse_f(mx, mx + tsa_ffrom(base + i), T);
}

// out[k] = T(u) for u = k * 2^-24
__global__ void __launch_bounds__(256) k_thr(uint32_t n, float* __restrict__ out) {
  __shared__ uint64_t tab[32];
  if (threadIdx.x < 32) tab[threadIdx.x] = tsa_exp2_tab_d[threadIdx.x];
  __syncthreads();
  for (uint32_t k = blockIdx.x * blockDim.x + threadIdx.x; k < n; k += gridDim.x * blockDim.x)
    out[k] = tsa_accept_threshold(k << 8, tab);
}

static unsigned host_threads() {
  const unsigned n = std::thread::hardware_concurrency();
  return n == 0 ? 4 : (n > 16 ? 16 : n);
}

// runs f(i) for i in [0, n) on all host threads, returns the sum of its results
template <class F>
static long long parallel_count(uint32_t n, F f) {
  const unsigned nt = host_threads();
  std::vector<long long> part(nt, 0);
  std::vector<std::thread> th;
  for (unsigned t = 0; t < nt; t++)
    th.emplace_back([&, t]() {
      long long c = 0;
      for (uint32_t i = t; i < n; i += nt) c += f(i);
      part[t] = c;
    });
  for (auto& x : th) x.join();
  long long s = 0;
  for (long long c : part) s += c;
  return s;
}

static bool same(float a, float b) { return (a != a && b != b) || tsa_fbits(a) == tsa_fbits(b); }

// the correction table of tsa_log2f_12, from this host's log2f (2 bits per float of [1, 2), then the summary
// bitmap of its nonzero words)
static std::vector<uint32_t> log2_fix() {
  std::vector<uint32_t> fix(TSA_LOG2FIX_WORDS + TSA_LOG2MAP_WORDS, 0u);
  parallel_count(TSA_LOG2FIX_WORDS, [&](uint32_t w) {
    uint32_t word = 0;
    for (uint32_t j = 0; j < 16; j++) {
      const float y = tsa_ffrom(0x3f800000u + w * 16 + j);
      const int32_t d = (int32_t)(tsa_fbits(log2f(y)) - tsa_fbits(tsa_log2f_core(y)));
      word |= (d == 1 ? 1u : d == -1 ? 2u : 0u) << (2 * j);
    }
    fix[w] = word;
    return 0LL;
  });
  for (uint32_t w = 0; w < TSA_LOG2FIX_WORDS; w++)
    if (fix[w]) fix[TSA_LOG2FIX_WORDS + (w >> 5)] |= 1u << (w & 31u);
  return fix;
}

int main() {
  float *d1 = nullptr, *d2 = nullptr, *h1 = nullptr, *h2 = nullptr;
  uint32_t* dfix = nullptr;
  CK(hipMalloc(&d1, (size_t)CHUNK * 4));
  CK(hipMalloc(&d2, (size_t)CHUNK * 4));
  CK(hipHostMalloc(&h1, (size_t)CHUNK * 4, hipHostMallocDefault));
  CK(hipHostMalloc(&h2, (size_t)CHUNK * 4, hipHostMallocDefault));
  const dim3 grid(4096), block(256);

  // expf / exp2f over all 2^32 floats
  long long bad_exp = 0, bad_exp2 = 0;
  for (uint64_t base = 0; base < (1ull << 32); base += CHUNK) {
    hipLaunchKernelGGL(k_exp, grid, block, 0, 0, (uint32_t)base, CHUNK, d1, d2);
    CK(hipGetLastError());
    CK(hipMemcpy(h1, d1, (size_t)CHUNK * 4, hipMemcpyDeviceToHost));
    CK(hipMemcpy(h2, d2, (size_t)CHUNK * 4, hipMemcpyDeviceToHost));
    bad_exp += parallel_count(CHUNK, [&](uint32_t i) { return (long long)!same(h1[i], expf(tsa_ffrom((uint32_t)base + i))); });
    bad_exp2 += parallel_count(CHUNK, [&](uint32_t i) { return (long long)!same(h2[i], exp2f(tsa_ffrom((uint32_t)base + i))); });
  }

  // log2f on [1, 2]
  const std::vector<uint32_t> fix = log2_fix();
  CK(hipMalloc(&dfix, fix.size() * 4));
  CK(hipMemcpy(dfix, fix.data(), fix.size() * 4, hipMemcpyHostToDevice));
  const uint32_t nlog = (1u << 23) + 1;
  hipLaunchKernelGGL(k_log2, grid, block, 0, 0, nlog, dfix, d1);
  CK(hipGetLastError());
  CK(hipMemcpy(h1, d1, (size_t)nlog * 4, hipMemcpyDeviceToHost));
  const long long bad_log2 =
      parallel_count(nlog, [&](uint32_t i) { return (long long)!same(h1[i], log2f(tsa_ffrom(0x3f800000u + i))); });

  // lse at six magnitudes, every difference d in [-24, 0] (bit patterns 0x80000000 .. 0xC1C00000)
  const float mxs[6] = {0.0f, 1.0f, 3.5f, 17.25f, 100.125f, 1234.5f};
  const uint64_t dlo = 0x80000000ull, dhi = 0xC1C00000ull;
  long long bad_lse = 0, n_lse = 0;
  for (float mx : mxs) {
    for (uint64_t base = dlo; base <= dhi; base += CHUNK) {
      const uint32_t n = (uint32_t)((dhi + 1 - base) < CHUNK ? (dhi + 1 - base) : CHUNK);
      hipLaunchKernelGGL(k_lse, grid, block, 0, 0, mx, (uint32_t)base, n, dfix, d1);
      CK(hipGetLastError());
      CK(hipMemcpy(h1, d1, (size_t)n * 4, hipMemcpyDeviceToHost));
      bad_lse += parallel_count(n, [&](uint32_t i) {
        // the reference's formula on the same operands (b = mx + d rounded as the kernel rounds it)
        const float a = mx, b = mx + tsa_ffrom((uint32_t)base + i);
        const float hi = a > b ? a : b, lo = a > b ? b : a;
        const float want = hi == -INFINITY ? hi : hi + log2f(1.0f + exp2f(lo - hi));
        return (long long)!same(h1[i], want);
      });
      n_lse += n;
    }
  }

  // Metropolis thresholds, device against host
  const uint32_t nthr = 1u << 24;
  hipLaunchKernelGGL(k_thr, grid, block, 0, 0, nthr, d1);
  CK(hipGetLastError());
  CK(hipMemcpy(h1, d1, (size_t)nthr * 4, hipMemcpyDeviceToHost));
  const long long bad_thr = parallel_count(nthr, [&](uint32_t k) {
    const float want = tsa_accept_threshold(k << 8, tsa_exp2_tab_h);
    return (long long)(!same(h1[k], want) || h1[k] != h1[k]);
  });

  printf("{\"expf_mismatch\": %lld, \"exp2f_mismatch\": %lld, \"exp_inputs\": %llu, \"log2f_mismatch\": %lld, "
         "\"log2f_inputs\": %u, \"lse_mismatch\": %lld, \"lse_inputs\": %lld, \"threshold_mismatch\": %lld, "
         "\"threshold_inputs\": %u, \"host_threads\": %u}\n",
         bad_exp, bad_exp2, 1ull << 32, bad_log2, nlog, bad_lse, n_lse, bad_thr, nthr, host_threads());
  CK(hipFree(d1));
  CK(hipFree(d2));
  CK(hipFree(dfix));
  CK(hipHostFree(h1));
  CK(hipHostFree(h2));
  return bad_exp || bad_exp2 || bad_log2 || bad_lse || bad_thr ? 1 : 0;
}
