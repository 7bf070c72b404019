// The batch-1 decode kernel instantiations for the ShapeTiny preset: the spread
// kernel's 16 modes and the
// class kernel's 8.
#define MK_DECODE_INSTANTIATE 1
#include "mk_launch.h"

namespace mk {
hipError_t launch_decode_tiny(int grid, hipStream_t stream, const Params& p, bool lc, bool cls) {
  return launch_decode<ShapeTiny, true>(grid, stream, p, lc, cls);
}
int occupancy_decode_tiny() { return occupancy_min<ShapeTiny, true>(); }
}  // namespace mk
