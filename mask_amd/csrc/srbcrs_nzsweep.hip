// spmm_nzsweep instantiations and their launcher.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "srbcrs_kernels.h"
#include "srbcrs_nzsweep.hpp"

namespace srbcrs {

// W 4 or 8 windows per group (tile rows and the padding row fit the entry's
// top byte); U entries per sub-batch and D sub-batches in
// the gather ring: (16, 2), (16, 4), (32, 2), (32, 4) or (64, 2).
bool nz_setting_ok(int W, int U, int D) {
  if (W != 4 && W != 8) return false;
  return (U == 16 && (D == 2 || D == 4)) || (U == 32 && (D == 2 || D == 4)) || (U == 64 && D == 2);
}

template <int W, int U, int D>
static hipError_t launch_nz_t(const NzArgs& z, const StreamArgs& a, hipStream_t st) {
  const int n_chunks = a.N / 64;
  const int64_t n_groups = ((int64_t)z.Mo + W - 1) / W;
  const int64_t nwg = merged_grid(n_groups, n_chunks);
  if (nwg == 0) return hipSuccess;
  if (nwg > INT32_MAX) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((spmm_nzsweep<W, U, D>), dim3((unsigned)nwg), dim3(64), 0, st, z.eoff, z.pairs, a.B, a.C,
                     a.rowmap, a.M, a.N, a.ldb, a.ldc, n_chunks, n_groups, a.relu);
  return hipGetLastError();
}

template <int W>
static hipError_t launch_nz_w(const NzArgs& z, const StreamArgs& a, int U, int D, hipStream_t st) {
  if (U == 64) return launch_nz_t<W, 64, 2>(z, a, st);
  if (U == 32) return D == 4 ? launch_nz_t<W, 32, 4>(z, a, st) : launch_nz_t<W, 32, 2>(z, a, st);
  return D == 4 ? launch_nz_t<W, 16, 4>(z, a, st) : launch_nz_t<W, 16, 2>(z, a, st);
}

hipError_t launch_nzsweep(const NzArgs& z, const StreamArgs& a, int U, int D, hipStream_t st) {
  if (!nz_setting_ok(z.W, U, D) || a.N % 64 != 0) return hipErrorInvalidValue;
  return z.W == 8 ? launch_nz_w<8>(z, a, U, D, st) : launch_nz_w<4>(z, a, U, D, st);
}

}  // namespace srbcrs
