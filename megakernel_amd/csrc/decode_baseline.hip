// The batch-1 decode kernel instantiations for the ShapeBaseline preset: the spread
// kernel's 16 modes and the
// class kernel's 8.
#define MK_DECODE_INSTANTIATE 1
#include "mk_launch.h"

namespace mk {
hipError_t launch_decode_baseline(int grid, hipStream_t stream, const Params& p, bool lc, bool cls) {
  return launch_decode<ShapeBaseline, true>(grid, stream, p, lc, cls);
}
int occupancy_decode_baseline() { return occupancy_min<ShapeBaseline, true>(); }
}  // namespace mk
