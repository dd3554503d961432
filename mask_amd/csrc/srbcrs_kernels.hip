// Host launchers of the SR-BCRS kernels (templates in srbcrs_stream.hpp).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "srbcrs_kernels.h"
#include "srbcrs_stream.hpp"  // segment_reduce, zero_rows, csr_spmm_rowwave

namespace srbcrs {

// ---------------------------------------------------------------------------
// Host launchers.

hipError_t launch_row(const StreamArgs& a, const int* soff, int Mo, int vec, const RunOpts& o,
                      hipStream_t st) {
  return (o.a_compact && a.a_words) ? launch_row_compact(a, soff, Mo, vec, o, st)
                                    : launch_row_dense(a, soff, Mo, vec, o, st);
}

hipError_t launch_tasks(const StreamArgs& a, const TaskTable& t, int vec, const RunOpts& o,
                        hipStream_t st) {
  return (o.a_compact && a.a_words) ? launch_tasks_compact(a, t, vec, o, st)
                                    : launch_tasks_dense(a, t, vec, o, st);
}

hipError_t launch_reduce(const ReduceArgs& a, int vec, hipStream_t st) {
  if (a.n_red == 0) return hipSuccess;
  const int64_t total = (int64_t)a.n_red * a.tile_rows * (a.N / vec);
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (vec == 4)
    hipLaunchKernelGGL(segment_reduce<4>, dim3((unsigned)blocks), dim3(256), 0, st, a.partial, a.C,
                       a.red_window, a.red_slot_off, a.n_red, a.tile_rows, a.M, a.N, a.ldc, a.rowmap, a.relu);
  else if (vec == 2)
    hipLaunchKernelGGL(segment_reduce<2>, dim3((unsigned)blocks), dim3(256), 0, st, a.partial, a.C,
                       a.red_window, a.red_slot_off, a.n_red, a.tile_rows, a.M, a.N, a.ldc, a.rowmap, a.relu);
  else
    hipLaunchKernelGGL(segment_reduce<1>, dim3((unsigned)blocks), dim3(256), 0, st, a.partial, a.C,
                       a.red_window, a.red_slot_off, a.n_red, a.tile_rows, a.M, a.N, a.ldc, a.rowmap, a.relu);
  return hipGetLastError();
}

// vec: columns per lane per pass (64*vec divides N, or 1).
hipError_t launch_csr(const CsrArgs& a, int vec, hipStream_t st) {
  const int n_chunks = (a.N + 64 * vec - 1) / (64 * vec);
  const int64_t nwg = ((int64_t)a.M + 3) / 4 * n_chunks;
  if (nwg == 0) return hipSuccess;
  if (nwg > INT32_MAX) return hipErrorInvalidConfiguration;
  dim3 grid((unsigned)nwg);
  if (vec == 4)
    hipLaunchKernelGGL((csr_spmm_rowwave<4, 8>), grid, dim3(256), 0, st, a.rowptr, a.colind,
                       a.values, a.B, a.C, a.M, a.N, a.ldb, a.ldc, n_chunks);
  else if (vec == 2)
    hipLaunchKernelGGL((csr_spmm_rowwave<2, 8>), grid, dim3(256), 0, st, a.rowptr, a.colind,
                       a.values, a.B, a.C, a.M, a.N, a.ldb, a.ldc, n_chunks);
  else
    hipLaunchKernelGGL((csr_spmm_rowwave<1, 8>), grid, dim3(256), 0, st, a.rowptr, a.colind,
                       a.values, a.B, a.C, a.M, a.N, a.ldb, a.ldc, n_chunks);
  return hipGetLastError();
}

hipError_t launch_zero_rows(float* C, const int* rows, int n_rows, int N, int64_t ldc, hipStream_t st) {
  if (n_rows == 0 || N == 0) return hipSuccess;
  const int64_t total = (int64_t)n_rows * N;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(zero_rows<float>, dim3((unsigned)blocks), dim3(256), 0, st, C, rows, n_rows, N, ldc);
  return hipGetLastError();
}

}  // namespace srbcrs
