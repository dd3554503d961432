// Measurement probes (declared in srbcrs_probe.h, bound by bench.py only):
// what plain streams and plain gathers move on this GPU, the reference
// points of the SpMM's roofline.  They compute nothing a caller uses.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "srbcrs_kernels.h"
#include "srbcrs_stream.hpp"   // xcd_remap, kNumXcd

namespace srbcrs {
namespace {
typedef float pf4 __attribute__((ext_vector_type(4)));

// Streaming rates: grid-stride loops (every thread ends after
// ceil(n4 / threads) iterations).
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

// Gather probe: one wave per workgroup walks its group's row list and reads
// one 1 KB load instruction per RPI rows (lane l: row sub = l / LPR of the
// instruction, 16 bytes at column chunk*SEG + 4*(l % LPR)), eight
// instructions in flight, the next eight rows' indices prefetched (clamped
// to the list, so the loop body has no branch).  Row counts are multiples
// of 8, so whole instructions cover every list.
template <int RPI>
__global__ __launch_bounds__(64) void k_gather_probe(const int* __restrict__ rows, const int64_t* __restrict__ row_off,
                                                     int n_groups, const float* __restrict__ B, int64_t ldb,
                                                     int n_chunks, int mapping, float* __restrict__ out) {
  constexpr int SEG = 256 / RPI;   // floats per row segment
  constexpr int LPR = 64 / RPI;    // lanes per row segment
  const int64_t bid = blockIdx.x;
  const int64_t work = (int64_t)n_groups * n_chunks;
  int64_t g;
  int c;
  if (mapping == 2) {
    const int x = (int)(bid % kNumXcd), per = kNumXcd / n_chunks;
    c = x % n_chunks;
    g = (bid / kNumXcd) * per + x / n_chunks;
  } else {
    const int64_t lid = mapping == 1 ? xcd_remap(bid, (int64_t)gridDim.x) : bid;
    c = (int)(lid / n_groups);
    g = lid % n_groups;
    if (lid >= work) g = n_groups;
  }
  const int lane = threadIdx.x;
  pf4 acc = {0.f, 0.f, 0.f, 0.f};
  if (g < n_groups) {
    const int sub = lane / LPR;
    const float* base = B + (int64_t)c * SEG + 4 * (lane % LPR);
    int64_t i = row_off[g];
    const int64_t e = row_off[g + 1];
    int nxt[8];
    auto ld_idx = [&](int64_t j) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t k = j + u * RPI + sub;
        nxt[u] = rows[k < e ? k : e - 1];
      }
    };
    if (i < e) ld_idx(i);
    for (; i + 8 * RPI <= e; i += 8 * RPI) {
      int cur[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) cur[u] = nxt[u];
      pf4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const pf4*>(base + (int64_t)cur[u] * ldb);
      ld_idx(i + 8 * RPI);
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += v[u];
    }
    for (; i < e; i += RPI) acc += *reinterpret_cast<const pf4*>(base + (int64_t)rows[i + sub] * ldb);
  }
  out[bid * 64 + lane] = acc.x + acc.y + acc.z + acc.w;
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

hipError_t launch_gather_probe(const int* rows, const int64_t* row_off, int n_groups, int rows_per_instr,
                               const float* B, int64_t ldb, int n_chunks, int mapping, float* out,
                               hipStream_t st) {
  const int64_t nwg = ((int64_t)n_groups * n_chunks + kNumXcd - 1) / kNumXcd * kNumXcd;
  if (nwg == 0) return hipSuccess;
  const dim3 grid((unsigned)nwg);
#define SRBCRS_GATHER(R) \
  hipLaunchKernelGGL(k_gather_probe<R>, grid, dim3(64), 0, st, rows, row_off, n_groups, B, ldb, n_chunks, mapping, out)
  switch (rows_per_instr) {
    case 1: SRBCRS_GATHER(1); break;
    case 2: SRBCRS_GATHER(2); break;
    case 4: SRBCRS_GATHER(4); break;
    default: SRBCRS_GATHER(8); break;
  }
#undef SRBCRS_GATHER
  return hipGetLastError();
}

}  // namespace srbcrs
