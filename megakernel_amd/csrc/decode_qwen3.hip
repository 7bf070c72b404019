// The batch-1 decode kernel instantiations for the ShapeQwen3 preset: the
// spread kernel's 16 modes (the class kernel does not fit this shape: its
// QKV, gate/up, O and down blocks need more than two roles per workgroup).
#define MK_DECODE_INSTANTIATE 1
#include "mk_launch.h"

namespace mk {
hipError_t launch_decode_qwen3(int grid, hipStream_t stream, const Params& p, bool lc, bool cls) {
  return launch_decode<ShapeQwen3, false>(grid, stream, p, lc, cls);
}
int occupancy_decode_qwen3() { return occupancy_min<ShapeQwen3, false>(); }
}  // namespace mk
