// Launch templates of spmm_stream, shared by the per-A-source translation
// units srbcrs_stream_dense.hip and srbcrs_stream_compact.hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "srbcrs_kernels.h"
#include "srbcrs_stream.hpp"

namespace srbcrs {

static int pick_waves(int N, int wcols, int wg_cols) {
  int cap = 4;
  if (wg_cols > 0) cap = wg_cols / wcols < 1 ? 1 : wg_cols / wcols;
  int w = (N + wcols - 1) / wcols;
  if (w > cap) w = cap;
  return w >= 4 ? 4 : (w >= 2 ? 2 : 1);
}

template <class AF, class Src, int BH, int BW, int VEC, int G, int DEPTH, int BSTAGE = 0>
static hipError_t launch_vg(const Src& src, const AF& af, int n_groups, const StreamArgs& a, const RunOpts& o,
                            hipStream_t st) {
  constexpr int WCOLS = 16 * VEC * G;
  const int waves = pick_waves(a.N, WCOLS, o.wg_cols);
  const int chunk_cols = waves * WCOLS;
  const int n_chunks = (a.N + chunk_cols - 1) / chunk_cols;
  const int64_t nwg = (int64_t)n_groups * n_chunks;
  if (nwg == 0) return hipSuccess;
  if (nwg > INT32_MAX) return hipErrorInvalidConfiguration;
  dim3 grid((unsigned)nwg);
#define SRBCRS_LAUNCH(W)                                                                       \
  hipLaunchKernelGGL((spmm_stream<Src, BH, BW, VEC, G, W, DEPTH, AF, BSTAGE>), grid, dim3(64 * W), 0, st, \
                     src, a.B, a.C, a.partial, a.sidx, af, a.M, a.N, a.ldb, a.ldc,          \
                     n_chunks, o.chunk_major)
  switch (waves) {
    case 4: SRBCRS_LAUNCH(4); break;
    case 2: SRBCRS_LAUNCH(2); break;
    default: SRBCRS_LAUNCH(1); break;
  }
#undef SRBCRS_LAUNCH
  return hipGetLastError();
}

// b_lds selects the LDS-staged B ring (BSTAGE 1) at vector width 4; other
// widths keep the register ring.
// vec (4, 2 or 1; 16*vec divides N) is chosen by the caller from N, the
// leading dimensions and pointer alignment.  16x8: G = 2 column groups per
// wave when the 128-column wave tile divides N and wider-than-64 workgroups
// are allowed.  32x32 (four units and two row halves per block) runs G = 2
// only in workgroups of 256 columns or more: it halves the A loads per MFMA
// (banded, full blocks: 0.72 -> 0.61 ms) but its register ring leaves 2
// waves per SIMD, and at 3 % block fill (uniform, GCN, R-MAT) two 64-column
// waves of G = 1 in a 128-column workgroup are faster (0.38 vs 0.42 ms).
template <class AF, class Src, int DEPTH>
static hipError_t launch_d(const Src& src, const AF& af, int n_groups, const StreamArgs& a, int vec,
                           const RunOpts& o, hipStream_t st) {
  if (a.blk_h == 32) {
    if (vec == 4 && o.b_lds)
      return (a.N % 128 == 0 && o.wg_cols >= 256) ? launch_vg<AF, Src, 32, 32, 4, 2, DEPTH, 1>(src, af, n_groups, a, o, st)
                                                 : launch_vg<AF, Src, 32, 32, 4, 1, DEPTH, 1>(src, af, n_groups, a, o, st);
    if (vec == 4)
      return (a.N % 128 == 0 && o.wg_cols >= 256) ? launch_vg<AF, Src, 32, 32, 4, 2, DEPTH>(src, af, n_groups, a, o, st)
                                                 : launch_vg<AF, Src, 32, 32, 4, 1, DEPTH>(src, af, n_groups, a, o, st);
    if (vec == 2) return launch_vg<AF, Src, 32, 32, 2, 1, DEPTH>(src, af, n_groups, a, o, st);
    return launch_vg<AF, Src, 32, 32, 1, 1, DEPTH>(src, af, n_groups, a, o, st);
  }
  if (vec == 4 && o.b_lds)
    return (a.N % 128 == 0 && o.wg_cols != 64) ? launch_vg<AF, Src, 16, 8, 4, 2, DEPTH, 1>(src, af, n_groups, a, o, st)
                                              : launch_vg<AF, Src, 16, 8, 4, 1, DEPTH, 1>(src, af, n_groups, a, o, st);
  if (vec == 4 && a.N % 256 == 0 && o.wg_cols >= 256)   // 256-column waves (G = 4)
    return launch_vg<AF, Src, 16, 8, 4, 4, DEPTH>(src, af, n_groups, a, o, st);
  if (vec == 4)
    return (a.N % 128 == 0 && o.wg_cols != 64) ? launch_vg<AF, Src, 16, 8, 4, 2, DEPTH>(src, af, n_groups, a, o, st)
                                              : launch_vg<AF, Src, 16, 8, 4, 1, DEPTH>(src, af, n_groups, a, o, st);
  if (vec == 2) return launch_vg<AF, Src, 16, 8, 2, 1, DEPTH>(src, af, n_groups, a, o, st);
  return launch_vg<AF, Src, 16, 8, 1, 1, DEPTH>(src, af, n_groups, a, o, st);
}

template <class AF, class Src>
static hipError_t launch_src(const Src& src, const AF& af, int n_groups, const StreamArgs& a, int vec,
                             const RunOpts& o, hipStream_t st) {
  switch (o.depth) {
    case 4: return launch_d<AF, Src, 4>(src, af, n_groups, a, vec, o, st);
    case 8: return launch_d<AF, Src, 8>(src, af, n_groups, a, vec, o, st);
    default: return launch_d<AF, Src, 2>(src, af, n_groups, a, vec, o, st);
  }
}

template <class AF>
static hipError_t launch_row_af(const AF& af, const StreamArgs& a, const int* soff, int Mo, int vec,
                                const RunOpts& o, hipStream_t st) {
  const int wpw = o.windows_per_wave > 0 ? o.windows_per_wave : 1;
  RowTasks src{soff, Mo, wpw, a.rowmap, a.relu};
  return launch_src(src, af, (Mo + wpw - 1) / wpw, a, vec, o, st);
}

template <class AF>
static hipError_t launch_tasks_af(const AF& af, const StreamArgs& a, const TaskTable& t, int vec,
                                  const RunOpts& o, hipStream_t st) {
  TableTasks src{t.group_off, t.task_begin, t.task_end, t.task_window, t.task_slot, a.rowmap, a.relu};
  return launch_src(src, af, t.n_groups, a, vec, o, st);
}

}  // namespace srbcrs
