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
                       a.red_window, a.red_slot_off, a.n_red, a.tile_rows, a.M, a.N, a.ldc, a.rowmap);
  else if (vec == 2)
    hipLaunchKernelGGL(segment_reduce<2>, dim3((unsigned)blocks), dim3(256), 0, st, a.partial, a.C,
                       a.red_window, a.red_slot_off, a.n_red, a.tile_rows, a.M, a.N, a.ldc, a.rowmap);
  else
    hipLaunchKernelGGL(segment_reduce<1>, dim3((unsigned)blocks), dim3(256), 0, st, a.partial, a.C,
                       a.red_window, a.red_slot_off, a.n_red, a.tile_rows, a.M, a.N, a.ldc, a.rowmap);
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

// Streaming-rate probes: what plain float4 streams move on this GPU, the
// context bench.py reports next to the SpMM's own HBM-side rate.  Grid-stride
// loops (every thread ends after ceil(n4 / threads) iterations).
namespace {
typedef float pf4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void k_probe_copy(const pf4* __restrict__ a, pf4* __restrict__ b, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    __builtin_nontemporal_store(a[i], b + i);
}
__global__ __launch_bounds__(256) void k_probe_read(const pf4* __restrict__ a, float* __restrict__ sink, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  pf4 s = {0.f, 0.f, 0.f, 0.f};
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) s += a[i];
  // a data-dependent store the compiler cannot drop; taken only for a NaN sum
  if (s.x + s.y + s.z + s.w != s.x + s.y + s.z + s.w) sink[0] = s.x;
}
__global__ __launch_bounds__(256) void k_probe_write(pf4* __restrict__ b, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const pf4 v = {1.f, 2.f, 3.f, 4.f};
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    __builtin_nontemporal_store(v, b + i);
}
}  // namespace

hipError_t launch_stream_probe(int kind, const float* a, float* b, int64_t n4, int blocks, hipStream_t st) {
  if (n4 <= 0) return hipSuccess;
  const auto* av = reinterpret_cast<const pf4*>(a);
  auto* bv = reinterpret_cast<pf4*>(b);
  if (kind == 0) hipLaunchKernelGGL(k_probe_copy, dim3(blocks), dim3(256), 0, st, av, bv, n4);
  else if (kind == 1) hipLaunchKernelGGL(k_probe_read, dim3(blocks), dim3(256), 0, st, av, b, n4);
  else hipLaunchKernelGGL(k_probe_write, dim3(blocks), dim3(256), 0, st, bv, n4);
  return hipGetLastError();
}

}  // namespace srbcrs
