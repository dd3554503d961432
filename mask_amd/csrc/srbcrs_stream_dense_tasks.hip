// spmm_stream instantiations reading A through DenseA, task-table schedules
// (split / strict_lb / multi_bind); a translation unit of its own so that the
// two halves of the instantiations compile in parallel.
#include "srbcrs_stream_launch.hpp"

namespace srbcrs {

hipError_t launch_tasks_dense(const StreamArgs& a, const TaskTable& t, int vec, const RunOpts& o,
                        hipStream_t st) {
  return launch_tasks_af(DenseA{a.val}, a, t, vec, o, st);
}

}  // namespace srbcrs
