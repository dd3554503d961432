// spmm_stream instantiations reading A through DenseA, row-window schedule.
#include "srbcrs_stream_launch.hpp"

namespace srbcrs {

hipError_t launch_row_dense(const StreamArgs& a, const int* soff, int Mo, int vec, const RunOpts& o,
                      hipStream_t st) {
  return launch_row_af(DenseA{a.val}, a, soff, Mo, vec, o, st);
}

}  // namespace srbcrs
