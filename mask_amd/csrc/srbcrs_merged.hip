// spmm_merged instantiations (compact A, vector width 4) and their launcher.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "srbcrs_kernels.h"
#include "srbcrs_merged.hpp"

namespace srbcrs {

// Grid of spmm_merged: rounds of 8 workgroups, one per XCD (see xcd_chunk),
// or one workgroup per (group, chunk) for chunk counts xcd_chunk does not pin.
int64_t merged_grid(int64_t n_groups, int n_chunks) {
  if (!merged_chunks_ok(n_chunks)) return n_groups * n_chunks;
  if (n_chunks <= kNumXcd) {
    const int per = kNumXcd / n_chunks;
    return (n_groups + per - 1) / per * kNumXcd;
  }
  return n_groups * n_chunks;
}

bool merged_chunks_ok(int n_chunks) {
  return n_chunks >= 1 && (n_chunks <= kNumXcd ? kNumXcd % n_chunks == 0 : n_chunks % kNumXcd == 0);
}

template <int G, int W, int DEPTH>
static hipError_t launch_merged_t(const MergedArgs& m, const StreamArgs& a, hipStream_t st) {
  constexpr int WCOLS = 64 * G;
  const int n_chunks = a.N / WCOLS;
  const int64_t n_groups = ((int64_t)m.Mo + W - 1) / W;
  const int64_t nwg = merged_grid(n_groups, n_chunks);
  if (nwg == 0) return hipSuccess;
  if (nwg > INT32_MAX) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((spmm_merged<4, G, W, DEPTH, CompactA>), dim3((unsigned)nwg), dim3(64), 0, st, m.moff, m.Mo,
                     m.sidx, CompactA{m.words, a.a_packed}, a.B, a.C, a.rowmap, a.M, a.N, a.ldb, a.ldc, n_chunks,
                     n_groups, a.relu);
  return hipGetLastError();
}

// cols 64 or 128 columns per wave, W 4 or 8 windows, depth 2 or 4, with 8
// windows only at 64 columns and depth 2: 8 windows of 128 columns (256
// accumulator registers) or a 4-deep ring beside 8 windows' tiles spill
// to scratch.
bool merged_setting_ok(int cols, int W, int depth) {
  if (cols != 64 && cols != 128) return false;
  if (depth != 2 && depth != 4) return false;
  if (W == 4) return true;
  return W == 8 && cols == 64 && depth == 2;
}

hipError_t launch_merged(const MergedArgs& m, const StreamArgs& a, int cols, int depth, hipStream_t st) {
  if (!merged_setting_ok(cols, m.W, depth)) return hipErrorInvalidValue;
  if (m.W == 8) return launch_merged_t<1, 8, 2>(m, a, st);
  if (cols == 64) return depth == 4 ? launch_merged_t<1, 4, 4>(m, a, st) : launch_merged_t<1, 4, 2>(m, a, st);
  return depth == 4 ? launch_merged_t<2, 4, 4>(m, a, st) : launch_merged_t<2, 4, 2>(m, a, st);
}

}  // namespace srbcrs
