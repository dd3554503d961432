// Internal launch interface between the C-ABI layer and the HIP kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace srbcrs {

constexpr int kNumXcd = 8;   // MI355X: 8 XCDs, 32 CUs each
constexpr int kDepth = 4;    // blocks in flight per wave in the SR-BCRS kernels

struct RowArgs {
  const float* B;
  float* C;
  const int* soff;
  const int* sidx;
  const float* val;
  int M, N, Mo;
  int64_t ldb, ldc;
};

struct TaskArgs {
  const float* B;
  float* C;
  float* partial;
  const int* sidx;
  const float* val;
  const int* group_off;
  const int* task_begin;
  const int* task_end;
  const int* task_window;
  const int* task_slot;
  int n_groups;
  int M, N;
  int64_t ldb, ldc;
};

struct ReduceArgs {
  const float* partial;
  float* C;
  const int* red_window;
  const int* red_slot_off;
  int n_red;
  int M, N;
  int64_t ldc;
};

struct CsrArgs {
  const int* rowptr;
  const int* colind;
  const float* values;
  const float* B;
  float* C;
  int M, N;
  int64_t ldb, ldc;
};

hipError_t launch_row(const RowArgs& a, int vec, hipStream_t st);
hipError_t launch_tasks(const TaskArgs& a, int vec, hipStream_t st);
hipError_t launch_reduce(const ReduceArgs& a, int vec, hipStream_t st);
hipError_t launch_csr(const CsrArgs& a, int vec, hipStream_t st);

}  // namespace srbcrs
