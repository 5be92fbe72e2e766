// lds_peak.hip -- bin/lds_peak: the LDS read bandwidth of the current GPU, the peak of the roofline of the sweep
// kernels whose chains sit in LDS (their label sets are read from LDS, not from HBM).
//
// Every compute unit runs two workgroups of 16 waves, each with 64 KiB of LDS filled once; every lane then
// reads 16 bytes per access (ds_read_b128), consecutive lanes consecutive addresses, with a stride that changes
// every access, and folds the values with xor so that no read is dead.  Bytes read / kernel time, best of
// several launches, printed as one JSON line.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>

#define LDS_WORDS 4096  // uint4 = 64 KiB
#define READS 8         // reads per loop trip

__global__ void __launch_bounds__(1024) k_lds_read(uint4* __restrict__ out, int trips, unsigned salt) {
  extern __shared__ uint4 buf[];
  const unsigned t = threadIdx.x;
  for (unsigned i = t; i < LDS_WORDS; i += blockDim.x) buf[i] = make_uint4(i ^ salt, i * 3u, i * 5u + salt, i * 7u);
  __syncthreads();
  uint4 acc = make_uint4(0u, 0u, 0u, 0u);
  unsigned base = t;
  for (int k = 0; k < trips; k++) {
#pragma unroll
    for (int r = 0; r < READS; r++) {
      const uint4 v = buf[(base + (unsigned)r * 512u) & (LDS_WORDS - 1)];
      acc.x ^= v.x;
      acc.y ^= v.y;
      acc.z ^= v.z;
      acc.w ^= v.w;
    }
    base += 64u * 9u;  // a new offset every trip, still 64 consecutive 16-byte words per wave
  }
  // never true for the values written above, but the compiler cannot know: every read stays live
  if ((acc.x & acc.y & acc.z & acc.w) == 0xFFFFFFFFu) out[blockIdx.x * blockDim.x + t] = acc;
}

#define CK(call)                                                                  \
  do {                                                                            \
    hipError_t e_ = (call);                                                       \
    if (e_ != hipSuccess) {                                                       \
      fprintf(stderr, "%s: %s\n", #call, hipGetErrorString(e_));                  \
      return 1;                                                                   \
    }                                                                             \
  } while (0)

int main(int argc, char** argv) {
  const int trips = argc > 1 ? atoi(argv[1]) : 4096;
  int dev = 0, ncu = 0, clk = 0;
  CK(hipGetDevice(&dev));
  CK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
  CK(hipDeviceGetAttribute(&clk, hipDeviceAttributeClockRate, dev));
  const int threads = 1024, blocks = 2 * ncu;
  const size_t smem = LDS_WORDS * sizeof(uint4);
  CK(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_lds_read), hipFuncAttributeMaxDynamicSharedMemorySize,
                         (int)smem));
  uint4* out = nullptr;
  CK(hipMalloc(&out, (size_t)blocks * threads * sizeof(uint4)));
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  float best = 1e30f;
  for (int rep = 0; rep < 6; rep++) {
    CK(hipEventRecord(e0));
    hipLaunchKernelGGL(k_lds_read, dim3(blocks), dim3(threads), smem, 0, out, trips, (unsigned)rep);
    CK(hipGetLastError());
    CK(hipEventRecord(e1));
    CK(hipEventSynchronize(e1));
    float ms = 0;
    CK(hipEventElapsedTime(&ms, e0, e1));
    if (rep > 0 && ms < best) best = ms;  // the first launch loads the code object
  }
  const double bytes = (double)blocks * threads * trips * READS * 16.0;
  const double gbs = bytes / (best * 1e-3) / 1e9;
  printf("{\"lds_read_GBps\": %.1f, \"compute_units\": %d, \"clock_mhz\": %d, \"bytes\": %.0f, \"ms\": %.4f, "
         "\"bytes_per_clock_per_cu\": %.1f}\n",
         gbs, ncu, clk / 1000, bytes, (double)best, gbs * 1e9 / ((double)clk * 1e3) / ncu);
  CK(hipFree(out));
  return 0;
}
