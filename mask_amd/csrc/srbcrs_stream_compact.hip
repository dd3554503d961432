// spmm_stream instantiations reading A through CompactA, row-window schedule.
#include "srbcrs_stream_launch.hpp"

namespace srbcrs {

hipError_t launch_row_compact(const StreamArgs& a, const int* soff, int Mo, int vec, const RunOpts& o,
                      hipStream_t st) {
  return launch_row_af(CompactA{a.a_words, a.a_packed}, a, soff, Mo, vec, o, st);
}

}  // namespace srbcrs
