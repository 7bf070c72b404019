// Launch and occupancy of the batch-1 decode kernel, one translation unit per
// shape preset (decode_<preset>.hip) so the kernel instantiations of each
// preset compile in parallel.  MODE bits pick the instantiation per launch:
// 1 the launch reaches more than merge_min attention splits per kv head, 2
// timestamps or validation outputs are recorded, 4 the FP8 LM head, 8 the FP8
// KV cache, 16 FP8 layer weights (class kernel only).
#pragma once
#include <hip/hip_runtime.h>

#include "mk_cls.h"
#include "mk_kernel.h"

namespace mk {

// cls: the class-specialised kernel (mk_cls.h; p.roles set), else the spread
// kernel (decode_kernel).
typedef hipError_t (*DecodeLaunch)(int grid, hipStream_t stream, const Params& p, bool lc, bool cls);

hipError_t launch_decode_baseline(int grid, hipStream_t stream, const Params& p, bool lc, bool cls);
hipError_t launch_decode_qwen3(int grid, hipStream_t stream, const Params& p, bool lc, bool cls);
hipError_t launch_decode_tiny(int grid, hipStream_t stream, const Params& p, bool lc, bool cls);
// Workgroups of 512 threads resident per CU for every instantiation (the
// minimum over the modes of both kernels); the persistent kernel needs at
// least one.
int occupancy_decode_baseline();
int occupancy_decode_qwen3();
int occupancy_decode_tiny();

#ifdef MK_DECODE_INSTANTIATE
template <class S, int MODE>
static void launch_mode(int grid, hipStream_t stream, const Params& p) {
  hipLaunchKernelGGL((decode_kernel<S, MODE>), dim3(grid), dim3(NT), 0, stream, p);
}

template <class S, int MODE>
static void launch_cls(int grid, hipStream_t stream, const Params& p) {
  hipLaunchKernelGGL((decode_cls_kernel<S, MODE>), dim3(grid), dim3(NT), 0, stream, p);
}

template <class S, bool HAS_CLS>
static hipError_t launch_decode(int grid, hipStream_t stream, const Params& p, bool lc, bool cls) {
  const int mode = (lc ? 1 : 0) | (p.trace || p.dbg_layers || p.dbg_logits ? 2 : 0) | (p.lmhead8 ? 4 : 0) |
                   (p.kscale ? 8 : 0);
  if constexpr (HAS_CLS) {
    if (cls && !lc) {
      switch (mode | (p.layers8 ? 16 : 0)) {
        case 0: launch_cls<S, 0>(grid, stream, p); break;
        case 2: launch_cls<S, 2>(grid, stream, p); break;
        case 4: launch_cls<S, 4>(grid, stream, p); break;
        case 6: launch_cls<S, 6>(grid, stream, p); break;
        case 8: launch_cls<S, 8>(grid, stream, p); break;
        case 10: launch_cls<S, 10>(grid, stream, p); break;
        case 12: launch_cls<S, 12>(grid, stream, p); break;
        case 14: launch_cls<S, 14>(grid, stream, p); break;
        case 16: launch_cls<S, 16>(grid, stream, p); break;
        case 18: launch_cls<S, 18>(grid, stream, p); break;
        case 20: launch_cls<S, 20>(grid, stream, p); break;
        case 22: launch_cls<S, 22>(grid, stream, p); break;
        case 24: launch_cls<S, 24>(grid, stream, p); break;
        case 26: launch_cls<S, 26>(grid, stream, p); break;
        case 28: launch_cls<S, 28>(grid, stream, p); break;
        default: launch_cls<S, 30>(grid, stream, p); break;
      }
      return hipGetLastError();
    }
  }
  if (p.layers8) return hipErrorInvalidValue;  // the spread kernel reads bf16 layer weights only
  switch (mode) {
    case 0: launch_mode<S, 0>(grid, stream, p); break;
    case 1: launch_mode<S, 1>(grid, stream, p); break;
    case 2: launch_mode<S, 2>(grid, stream, p); break;
    case 3: launch_mode<S, 3>(grid, stream, p); break;
    case 4: launch_mode<S, 4>(grid, stream, p); break;
    case 5: launch_mode<S, 5>(grid, stream, p); break;
    case 6: launch_mode<S, 6>(grid, stream, p); break;
    case 7: launch_mode<S, 7>(grid, stream, p); break;
    case 8: launch_mode<S, 8>(grid, stream, p); break;
    case 9: launch_mode<S, 9>(grid, stream, p); break;
    case 10: launch_mode<S, 10>(grid, stream, p); break;
    case 11: launch_mode<S, 11>(grid, stream, p); break;
    case 12: launch_mode<S, 12>(grid, stream, p); break;
    case 13: launch_mode<S, 13>(grid, stream, p); break;
    case 14: launch_mode<S, 14>(grid, stream, p); break;
    default: launch_mode<S, 15>(grid, stream, p); break;
  }
  return hipGetLastError();
}

template <class S, int MODE>
static int occupancy_of() {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_kernel<S, MODE>, NT, 0) != hipSuccess) return 0;
  return n;
}

template <class S, int MODE>
static int occupancy_cls() {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_cls_kernel<S, MODE>, NT, 0) != hipSuccess) return 0;
  return n;
}

template <class S, bool HAS_CLS>
static int occupancy_min() {
  const int n[16] = {occupancy_of<S, 0>(),  occupancy_of<S, 1>(),  occupancy_of<S, 2>(),  occupancy_of<S, 3>(),
                     occupancy_of<S, 4>(),  occupancy_of<S, 5>(),  occupancy_of<S, 6>(),  occupancy_of<S, 7>(),
                     occupancy_of<S, 8>(),  occupancy_of<S, 9>(),  occupancy_of<S, 10>(), occupancy_of<S, 11>(),
                     occupancy_of<S, 12>(), occupancy_of<S, 13>(), occupancy_of<S, 14>(), occupancy_of<S, 15>()};
  int m = n[0];
  for (int i = 1; i < 16; ++i) m = n[i] < m ? n[i] : m;
  if constexpr (HAS_CLS) {
    const int c[16] = {occupancy_cls<S, 0>(),  occupancy_cls<S, 2>(),  occupancy_cls<S, 4>(),  occupancy_cls<S, 6>(),
                       occupancy_cls<S, 8>(),  occupancy_cls<S, 10>(), occupancy_cls<S, 12>(), occupancy_cls<S, 14>(),
                       occupancy_cls<S, 16>(), occupancy_cls<S, 18>(), occupancy_cls<S, 20>(), occupancy_cls<S, 22>(),
                       occupancy_cls<S, 24>(), occupancy_cls<S, 26>(), occupancy_cls<S, 28>(), occupancy_cls<S, 30>()};
    for (int i = 0; i < 16; ++i) m = c[i] < m ? c[i] : m;
  }
  return m;
}
#endif

}  // namespace mk
