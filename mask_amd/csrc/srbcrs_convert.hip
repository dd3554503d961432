// Device-side CSR -> SR-BCRS conversion (canonical preprocess_gpu rules),
// bit-exact with the host converter and with the reference's
// preprocess_gpu_srcfp32_srbcrs (examples/src_fp32/sr_bcrs/testbed/
// SRBCRSSpMM_kernel.cu:226-340): per BH-row window the sorted distinct
// columns, cut into BW-column blocks padded with the window's last column;
// values at the swizzled block offset, the last write winning for duplicate
// (row, column) pairs; edge_to_row / edge_to_col / block_partition.
//
// The reference copies the CSR to the host and converts there.  Here the CSR
// stays in HBM: edges are keyed (window << 32 | column), radix-sorted with
// their edge index (stable, so duplicates keep edge order), and the distinct
// keys are ranked with a scan.  Every write has a single owner (no atomics):
// a duplicate run's last entry writes the value.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>
#include <stdint.h>

#include "srbcrs_convert.h"

namespace srbcrs {

namespace {

__device__ __forceinline__ int swz(int o) { return o ^ ((o & 0x60) >> 3); }

// flag[0] = 1 when the CSR is malformed (rowptr decreasing / out of range,
// negative column); flag[1] = max column (as int, -1 if none).
__global__ void k_validate_rowptr(const int* __restrict__ rowptr, int num_nodes, int64_t nnz,
                                  int* __restrict__ flag) {
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r <= num_nodes;
       r += (int64_t)gridDim.x * blockDim.x) {
    const int v = rowptr[r];
    bool bad = v < 0 || v > nnz;
    if (r < num_nodes && rowptr[r + 1] < v) bad = true;
    if (bad) flag[0] = 1;   // plain store: every writer writes the same value
  }
}

// Row ids of the edges in two parallel passes (a per-row loop serialises on
// hub rows): each non-empty row marks its first edge (one writer per edge:
// rows with the same start are empty but the last), then an inclusive max
// scan over the zero-filled edge range carries each mark forward.
__global__ void k_row_starts(const int* __restrict__ rowptr, int num_nodes, int* __restrict__ e2r) {
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < num_nodes;
       r += (int64_t)gridDim.x * blockDim.x)
    if (rowptr[r + 1] > rowptr[r]) e2r[rowptr[r]] = (int)r;
}

__global__ void k_make_keys(const int* __restrict__ colind, const int* __restrict__ e2r, int e0,
                            int n, int bh, uint64_t* __restrict__ keys, int* __restrict__ idx,
                            int* __restrict__ neg) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int e = e0 + (int)i;
    const int c = colind[e];
    if (c < 0) neg[0] = 1;
    keys[i] = ((uint64_t)(uint32_t)(e2r[e] / bh) << 32) | (uint32_t)c;
    idx[i] = e;
  }
}

__global__ void k_flags(const uint64_t* __restrict__ keys, int n, int* __restrict__ flags) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    flags[i] = (i == 0 || keys[i] != keys[i - 1]) ? 1 : 0;
}

// rank[i] = inclusive count of distinct keys up to i (1-based)
__global__ void k_unique(const uint64_t* __restrict__ keys, const int* __restrict__ rank, int n,
                         int* __restrict__ ucol, int* __restrict__ uwin) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    if (i == 0 || keys[i] != keys[i - 1]) {
      const int u = rank[i] - 1;
      ucol[u] = (int)(uint32_t)keys[i];
      uwin[u] = (int)(keys[i] >> 32);
    }
  }
}

// ufirst[w] = first distinct-key index of window w (lower bound), w in [0, Mo]
__global__ void k_window_first(const int* __restrict__ uwin, int nu, int Mo, int* __restrict__ ufirst) {
  for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w <= Mo;
       w += (int64_t)gridDim.x * blockDim.x) {
    int lo = 0, hi = nu;
    while (lo < hi) {
      const int mid = lo + (hi - lo) / 2;
      if (uwin[mid] < w) lo = mid + 1; else hi = mid;
    }
    ufirst[w] = lo;
  }
}

__global__ void k_block_counts(const int* __restrict__ ufirst, int Mo, int bw, int* __restrict__ nb,
                               int* __restrict__ bp) {
  for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w <= Mo;
       w += (int64_t)gridDim.x * blockDim.x) {
    const int c = w < Mo ? (ufirst[w + 1] - ufirst[w] + bw - 1) / bw : 0;
    nb[w] = c;
    if (bp && w < Mo) bp[w] = c;
  }
}

// sidx slot s (block b = s / bw): window by upper bound in soff, then the
// window's distinct column at min(position, count - 1)
__global__ void k_fill_sidx(const int* __restrict__ soff, const int* __restrict__ ufirst,
                            const int* __restrict__ ucol, int Mo, int bw, int64_t nslots,
                            int* __restrict__ sidx) {
  for (int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; s < nslots;
       s += (int64_t)gridDim.x * blockDim.x) {
    const int b = (int)(s / bw);
    int lo = 0, hi = Mo;   // last w with soff[w] <= b
    while (hi - lo > 1) {
      const int mid = lo + (hi - lo) / 2;
      if (soff[mid] <= b) lo = mid; else hi = mid;
    }
    const int w = lo;   // the window holding block b (empty windows have soff[w] == soff[w+1])
    const int64_t pos = s - (int64_t)soff[w] * bw;
    const int cnt = ufirst[w + 1] - ufirst[w];
    sidx[s] = ucol[ufirst[w] + (pos < cnt ? (int)pos : cnt - 1)];
  }
}

__global__ void k_zero(float* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0.f;
}

__global__ void k_scatter(const uint64_t* __restrict__ keys, const int* __restrict__ idx,
                          const int* __restrict__ rank, int n, const int* __restrict__ e2r,
                          const float* __restrict__ values, const int* __restrict__ ufirst,
                          const int* __restrict__ soff, int bh, int bw, float* __restrict__ val,
                          int* __restrict__ e2c) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int e = idx[i];
    const int w = (int)(keys[i] >> 32);
    const int p = rank[i] - 1 - ufirst[w];
    if (e2c) e2c[e] = p;
    const int row = e2r[e];
    // last entry of its (row, column) run: entries of one key are in edge
    // order and a row's edges are contiguous, so the run ends where the key
    // or the row changes
    const bool last = i + 1 == n || keys[i + 1] != keys[i] || e2r[idx[i + 1]] != row;
    if (last) {
      const int lr = row - w * bh;
      val[((int64_t)soff[w] + p / bw) * bh * bw + swz(lr * bw + p % bw)] = values[e];
    }
  }
}

inline unsigned grid_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  if (b < 1) b = 1;
  if (b > 65536) b = 65536;
  return (unsigned)b;
}

int bits_for(int64_t v) {
  int b = 0;
  while ((int64_t(1) << b) <= v) ++b;
  return b < 1 ? 1 : b;
}

}  // namespace

#define SRBCRS_TRY(x)                        \
  do {                                       \
    hipError_t e__ = (x);                    \
    if (e__ != hipSuccess) return e__;       \
  } while (0)

hipError_t device_convert(const DeviceConvertIn& in, DeviceConvertOut& out, DeviceAlloc alloc,
                          DeviceFree dfree, void* ctx, hipStream_t st) {
  const int bh = in.blk_h, bw = in.blk_w;
  const int Mo = (in.num_nodes + bh - 1) / bh;
  out.Mo = Mo;
  out.total = 0;
  out.bad = 0;
  out.max_col = -1;
  // 1. validate rowptr before trusting it for any edge access
  int* d_flag = (int*)alloc(ctx, 2 * sizeof(int));
  if (!d_flag) return hipErrorOutOfMemory;
  int h_flag[2] = {0, -1};
  SRBCRS_TRY(hipMemcpyAsync(d_flag, h_flag, sizeof(h_flag), hipMemcpyHostToDevice, st));
  hipLaunchKernelGGL(k_validate_rowptr, dim3(grid_for(in.num_nodes + 1)), dim3(256), 0, st, in.rowptr,
                     in.num_nodes, in.nnz, d_flag);
  SRBCRS_TRY(hipGetLastError());
  int h_rp[2];
  SRBCRS_TRY(hipMemcpyAsync(h_flag, d_flag, sizeof(h_flag), hipMemcpyDeviceToHost, st));
  SRBCRS_TRY(hipMemcpyAsync(&h_rp[0], in.rowptr, sizeof(int), hipMemcpyDeviceToHost, st));
  SRBCRS_TRY(hipMemcpyAsync(&h_rp[1], in.rowptr + in.num_nodes, sizeof(int), hipMemcpyDeviceToHost, st));
  SRBCRS_TRY(hipStreamSynchronize(st));
  if (h_flag[0]) {
    out.bad = 1;
    dfree(ctx, d_flag);
    return hipSuccess;
  }
  const int e0 = h_rp[0];
  const int n = h_rp[1] - h_rp[0];
  // 2. row ids (also edge_to_row), keys
  int* e2r = in.edge_to_row;
  SRBCRS_TRY(hipGetLastError());
  hipLaunchKernelGGL(k_row_starts, dim3(grid_for(in.num_nodes)), dim3(256), 0, st, in.rowptr, in.num_nodes, e2r);
  SRBCRS_TRY(hipGetLastError());
  if (n > 0) {   // carry the marks over [e0, e0 + n) (the caller zero-filled edge_to_row)
    int* scanned = (int*)alloc(ctx, (size_t)n * 4);
    void* scan_tmp = nullptr;
    size_t scan_bytes = 0;
    hipError_t e = scanned ? hipSuccess : hipErrorOutOfMemory;
    if (e == hipSuccess)
      e = hipcub::DeviceScan::InclusiveScan(nullptr, scan_bytes, e2r + e0, scanned, hipcub::Max(), n, st);
    if (e == hipSuccess) {
      scan_tmp = alloc(ctx, scan_bytes ? scan_bytes : 1);
      if (!scan_tmp) e = hipErrorOutOfMemory;
    }
    if (e == hipSuccess)
      e = hipcub::DeviceScan::InclusiveScan(scan_tmp, scan_bytes, e2r + e0, scanned, hipcub::Max(), n, st);
    if (e == hipSuccess) e = hipMemcpyAsync(e2r + e0, scanned, (size_t)n * 4, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (scanned) dfree(ctx, scanned);
    if (scan_tmp) dfree(ctx, scan_tmp);
    if (e != hipSuccess) {
      dfree(ctx, d_flag);
      return e;
    }
  }
  uint64_t *k0 = nullptr, *k1 = nullptr;
  int *i0 = nullptr, *i1 = nullptr, *flags = nullptr, *rank = nullptr;
  int *ucol = nullptr, *uwin = nullptr, *ufirst = nullptr, *nb = nullptr;
  void* tmp = nullptr;
  const size_t N = (size_t)(n > 0 ? n : 1);
  k0 = (uint64_t*)alloc(ctx, N * 8);
  k1 = (uint64_t*)alloc(ctx, N * 8);
  i0 = (int*)alloc(ctx, N * 4);
  i1 = (int*)alloc(ctx, N * 4);
  flags = (int*)alloc(ctx, N * 4);
  rank = (int*)alloc(ctx, N * 4);
  ucol = (int*)alloc(ctx, N * 4);
  uwin = (int*)alloc(ctx, N * 4);
  ufirst = (int*)alloc(ctx, ((size_t)Mo + 1) * 4);
  nb = (int*)alloc(ctx, ((size_t)Mo + 1) * 4);
  hipError_t err = hipSuccess;
  auto cleanup = [&] {
    for (void* p : {(void*)k0, (void*)k1, (void*)i0, (void*)i1, (void*)flags, (void*)rank, (void*)ucol,
                    (void*)uwin, (void*)ufirst, (void*)nb, tmp, (void*)d_flag})
      if (p) dfree(ctx, p);
  };
  if (!k0 || !k1 || !i0 || !i1 || !flags || !rank || !ucol || !uwin || !ufirst || !nb) {
    cleanup();
    return hipErrorOutOfMemory;
  }
#define SRBCRS_STEP(x)        \
  do {                        \
    err = (x);                \
    if (err != hipSuccess) {  \
      cleanup();              \
      return err;             \
    }                         \
  } while (0)
  int nu = 0;
  if (n > 0) {
    hipLaunchKernelGGL(k_make_keys, dim3(grid_for(n)), dim3(256), 0, st, in.colind, e2r, e0, n, bh, k0, i0,
                       d_flag);
    SRBCRS_STEP(hipGetLastError());
    // 3. stable radix sort of (window, column) keys with their edge index
    hipcub::DoubleBuffer<uint64_t> kb(k0, k1);
    hipcub::DoubleBuffer<int> ib(i0, i1);
    const int end_bit = 32 + bits_for(Mo);
    size_t tmp_bytes = 0;
    SRBCRS_STEP(hipcub::DeviceRadixSort::SortPairs(nullptr, tmp_bytes, kb, ib, n, 0, end_bit, st));
    size_t scan_bytes = 0;
    SRBCRS_STEP(hipcub::DeviceScan::InclusiveSum(nullptr, scan_bytes, flags, rank, n, st));
    size_t ex_bytes = 0;
    SRBCRS_STEP(hipcub::DeviceScan::ExclusiveSum(nullptr, ex_bytes, nb, out.soff, Mo + 1, st));
    size_t need = tmp_bytes > scan_bytes ? tmp_bytes : scan_bytes;
    if (ex_bytes > need) need = ex_bytes;
    tmp = alloc(ctx, need ? need : 1);
    if (!tmp) {
      cleanup();
      return hipErrorOutOfMemory;
    }
    SRBCRS_STEP(hipcub::DeviceRadixSort::SortPairs(tmp, tmp_bytes, kb, ib, n, 0, end_bit, st));
    const uint64_t* keys = kb.Current();
    const int* idx = ib.Current();
    hipLaunchKernelGGL(k_flags, dim3(grid_for(n)), dim3(256), 0, st, keys, n, flags);
    SRBCRS_STEP(hipGetLastError());
    SRBCRS_STEP(hipcub::DeviceScan::InclusiveSum(tmp, scan_bytes, flags, rank, n, st));
    hipLaunchKernelGGL(k_unique, dim3(grid_for(n)), dim3(256), 0, st, keys, rank, n, ucol, uwin);
    SRBCRS_STEP(hipGetLastError());
    SRBCRS_STEP(hipMemcpyAsync(&nu, rank + (n - 1), sizeof(int), hipMemcpyDeviceToHost, st));
    SRBCRS_STEP(hipStreamSynchronize(st));
    // negative column seen?
    SRBCRS_STEP(hipMemcpyAsync(h_flag, d_flag, sizeof(int), hipMemcpyDeviceToHost, st));
    SRBCRS_STEP(hipStreamSynchronize(st));
    if (h_flag[0]) {
      out.bad = 2;
      cleanup();
      return hipSuccess;
    }
    // max column: the largest column among the distinct keys
    int* d_max = flags;   // reuse
    size_t mx_bytes = 0;
    SRBCRS_STEP(hipcub::DeviceReduce::Max(nullptr, mx_bytes, ucol, d_max, nu, st));
    if (mx_bytes > need) {
      dfree(ctx, tmp);
      tmp = alloc(ctx, mx_bytes);
      need = mx_bytes;
      if (!tmp) {
        cleanup();
        return hipErrorOutOfMemory;
      }
    }
    SRBCRS_STEP(hipcub::DeviceReduce::Max(tmp, mx_bytes, ucol, d_max, nu, st));
    SRBCRS_STEP(hipMemcpyAsync(&out.max_col, d_max, sizeof(int), hipMemcpyDeviceToHost, st));
    // 4. windows: first distinct key, block counts, offsets
    hipLaunchKernelGGL(k_window_first, dim3(grid_for(Mo + 1)), dim3(256), 0, st, uwin, nu, Mo, ufirst);
    SRBCRS_STEP(hipGetLastError());
    hipLaunchKernelGGL(k_block_counts, dim3(grid_for(Mo + 1)), dim3(256), 0, st, ufirst, Mo, bw, nb,
                       in.block_partition);
    SRBCRS_STEP(hipGetLastError());
    SRBCRS_STEP(hipcub::DeviceScan::ExclusiveSum(tmp, ex_bytes, nb, out.soff, Mo + 1, st));
    int total = 0;
    SRBCRS_STEP(hipMemcpyAsync(&total, out.soff + Mo, sizeof(int), hipMemcpyDeviceToHost, st));
    SRBCRS_STEP(hipStreamSynchronize(st));
    out.total = total;
    // 5. arrays sized by the total
    const int64_t nslots = (int64_t)total * bw, nval = (int64_t)total * bh * bw;
    out.sidx = (int*)alloc(ctx, (size_t)(nslots > 0 ? nslots : 1) * 4);
    out.val = (float*)alloc(ctx, (size_t)(nval > 0 ? nval : 1) * 4);
    if (!out.sidx || !out.val) {
      cleanup();
      return hipErrorOutOfMemory;
    }
    if (nslots) {
      hipLaunchKernelGGL(k_fill_sidx, dim3(grid_for(nslots)), dim3(256), 0, st, out.soff, ufirst, ucol, Mo, bw,
                         nslots, out.sidx);
      SRBCRS_STEP(hipGetLastError());
      hipLaunchKernelGGL(k_zero, dim3(grid_for(nval)), dim3(256), 0, st, out.val, nval);
      SRBCRS_STEP(hipGetLastError());
      hipLaunchKernelGGL(k_scatter, dim3(grid_for(n)), dim3(256), 0, st, keys, idx, rank, n, e2r, in.values,
                         ufirst, out.soff, bh, bw, out.val, in.edge_to_col);
      SRBCRS_STEP(hipGetLastError());
    }
  } else {
    // no edges: all windows empty
    hipLaunchKernelGGL(k_window_first, dim3(grid_for(Mo + 1)), dim3(256), 0, st, uwin, 0, Mo, ufirst);
    SRBCRS_STEP(hipGetLastError());
    hipLaunchKernelGGL(k_block_counts, dim3(grid_for(Mo + 1)), dim3(256), 0, st, ufirst, Mo, bw, nb,
                       in.block_partition);
    SRBCRS_STEP(hipGetLastError());
    size_t ex_bytes = 0;
    SRBCRS_STEP(hipcub::DeviceScan::ExclusiveSum(nullptr, ex_bytes, nb, out.soff, Mo + 1, st));
    tmp = alloc(ctx, ex_bytes ? ex_bytes : 1);
    SRBCRS_STEP(hipcub::DeviceScan::ExclusiveSum(tmp, ex_bytes, nb, out.soff, Mo + 1, st));
    out.sidx = (int*)alloc(ctx, 4);
    out.val = (float*)alloc(ctx, 4);
  }
  SRBCRS_STEP(hipStreamSynchronize(st));
#undef SRBCRS_STEP
  cleanup();
  return hipSuccess;
}

}  // namespace srbcrs
