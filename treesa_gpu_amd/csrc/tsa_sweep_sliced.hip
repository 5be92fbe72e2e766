// tsa_sweep_sliced.hip -- the sweep kernels with slice code (label sets masked by the slice set, the slice
// step after each sweep when slice moves are on), instantiated apart from tsa_kernels.hip so that the two
// halves of the kernel variants compile in parallel.
#include "tsa_sweep.h"

hipError_t tsa_launch_sweeps_sliced(const TsaLaunch& L, int mode, int order, const TsaKParams& P, uint64_t* rec,
                                    const uint64_t* leaf, const uint32_t* fix, int nchains, float beta, uint32_t sweep0,
                                    int nsweeps, unsigned long long* stats, const TsaEnergyOut& eo, hipStream_t st,
                                    hipEvent_t e0, hipEvent_t e1, const TsaLevels* lv, int* res) {
  return tsa_launch_sweeps_t<true>(L, mode, order, P, rec, leaf, fix, nchains, beta, sweep0, nsweeps, stats, eo, st, e0,
                                   e1, lv, res);
}
