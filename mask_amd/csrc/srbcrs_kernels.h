// Internal launch interface between the C-ABI layer and the HIP kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace srbcrs {



// Launch knobs (template / runtime parameters of the SR-BCRS kernels).
struct RunOpts {
  int depth = 2;             // units in flight per wave: 2, 4 or 8
  int wg_cols = 128;         // columns per workgroup (0 = up to 4 waves)
  int chunk_major = 1;       // grid order: 0 window-major, 1 chunk-major, 2 chunk sweep (no XCD blocking)
  int windows_per_wave = 1;  // row schedule: consecutive windows streamed per wave
  int a_compact = 1;         // read A from the compact copy when the plan has one
  int b_lds = 0;             // stage B through LDS (direct-to-LDS loads; vector width 4 only)
};

// Operands shared by every SR-BCRS launch.
struct StreamArgs {
  const float* B;
  float* C;
  float* partial;   // partial tiles of split schedules (may be null for "row")
  const int* sidx;
  const float* val;
  int M, N;
  int64_t ldb, ldc;
  int blk_h;        // 16 (16x8 blocks) or 32 (32x32 blocks)
  const int* rowmap = nullptr;  // packed row -> output row (null = identity); M counts packed rows
  const uint2* a_words = nullptr;   // compact A (null = read val)
  const float* a_packed = nullptr;
  int relu = 0;     // relu epilogue on the values written to C (not on partial tiles)
};

// Merged-window operands (spmm_merged): the row schedule's windows in groups
// of W; group g's unit stream is [moff[g], moff[g+1]) of the interleaved
// copies of sidx (8 per unit, -1 for null units) and of the compact A words.
struct MergedArgs {
  const int* moff;
  int Mo;
  int W;
  const int* sidx;
  const uint2* words;
};

// Nonzero-sweep operands (spmm_nzsweep): group g of W row windows owns the
// (entry, value) pairs [eoff[g], eoff[g+1]), entry = (B row << 9) | tile
// row, laid out for one launch setting (sub-batch size and ring depth).
struct NzArgs {
  const int* eoff;
  int Mo;
  int W;
  const uint2* pairs;
};

struct TaskTable {
  const int* group_off;
  const int* task_begin;
  const int* task_end;
  const int* task_window;
  const int* task_slot;
  int n_groups;
};

struct ReduceArgs {
  const float* partial;
  float* C;
  const int* red_window;
  const int* red_slot_off;
  int n_red;
  int tile_rows;    // rows per window (the block height)
  int M, N;         // M counts packed rows
  int64_t ldc;
  const int* rowmap = nullptr;
  int relu = 0;     // relu epilogue on the sums
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

hipError_t launch_row(const StreamArgs& a, const int* soff, int Mo, int vec, const RunOpts& o,
                      hipStream_t st);
hipError_t launch_tasks(const StreamArgs& a, const TaskTable& t, int vec, const RunOpts& o,
                        hipStream_t st);
// per A source (srbcrs_stream_dense.hip / srbcrs_stream_compact.hip)
hipError_t launch_row_dense(const StreamArgs& a, const int* soff, int Mo, int vec, const RunOpts& o,
                            hipStream_t st);
hipError_t launch_tasks_dense(const StreamArgs& a, const TaskTable& t, int vec, const RunOpts& o,
                              hipStream_t st);
hipError_t launch_row_compact(const StreamArgs& a, const int* soff, int Mo, int vec, const RunOpts& o,
                              hipStream_t st);
hipError_t launch_tasks_compact(const StreamArgs& a, const TaskTable& t, int vec, const RunOpts& o,
                                hipStream_t st);
// spmm_merged at a setting merged_setting_ok accepts, vector width 4, a.N /
// cols column chunks, which merged_chunks_ok must accept.
hipError_t launch_merged(const MergedArgs& m, const StreamArgs& a, int cols, int depth, hipStream_t st);
bool merged_setting_ok(int cols, int W, int depth);
bool merged_chunks_ok(int n_chunks);
// grid of the merged-window kernels: rounds of 8 workgroups, one per XCD,
// for chunk counts merged_chunks_ok accepts; one workgroup per (group, chunk)
// otherwise
int64_t merged_grid(int64_t n_groups, int n_chunks);
// spmm_nzsweep: W 4 or 8, (U, D) = (tile_b, depth) one of nz_setting_ok's,
// a.N / 64 column chunks (XCD-pinned when merged_chunks_ok accepts the count).
hipError_t launch_nzsweep(const NzArgs& z, const StreamArgs& a, int U, int D, hipStream_t st);
bool nz_setting_ok(int W, int U, int D);
hipError_t launch_reduce(const ReduceArgs& a, int vec, hipStream_t st);
hipError_t launch_csr(const CsrArgs& a, int vec, hipStream_t st);
hipError_t launch_zero_rows(float* C, const int* rows, int n_rows, int N, int64_t ldc, hipStream_t st);
// Measurement probes (srbcrs_probe.hip): streaming rates (kind 0 copy a -> b,
// 1 read a, 2 write b, n4 float4 elements) and the gather probe.
hipError_t launch_stream_probe(int kind, const float* a, float* b, int64_t n4, int blocks, hipStream_t st);
hipError_t launch_gather_probe(const int* rows, const int64_t* row_off, int n_groups, int rows_per_instr,
                               const float* B, int64_t ldb, int n_chunks, int mapping, float* out,
                               hipStream_t st);

}  // namespace srbcrs
