// Self-test of the dataflow hand-off on the device: the memory-model choice
// of the decode kernel (agent-scope write-through stores of 64-bit
// value|tag words, agent-scope polling loads, no fences) exercised on its
// own, across every CU and XCD.
//
// One workgroup per CU runs `rounds` all-gather rounds: in round r every
// workgroup publishes one word -- a full-tag word (tag r + 1) and a packed
// pair with the 4-bit tag tag4(r + 1) -- into the buffer of parity r % 2, then
// polls every other workgroup's words of round r and checks their values,
// which are a known function of (round, workgroup).  Double buffering by
// round parity is the decode kernel's argmax-slot scheme: a workgroup can
// only overwrite round r's buffer (in round r + 2) after every workgroup has
// published round r + 1, which each does only after reading all of round r.
// A word with the right tag and a wrong value (stale, torn, or reordered
// ahead of its value) counts as a mismatch.  Waits are bounded like the
// decode kernel's; a timeout sets the error word and every workgroup unwinds.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "megakernel.h"
#include "mk_host.h"

namespace mk {
namespace selftest {

constexpr int ST = 256;  // threads per workgroup

__device__ __forceinline__ float word_val(int r, int wg) { return (float)((r * 257 + wg * 31) % 65521); }

__global__ __launch_bounds__(ST) void dataflow_kernel(u64* full, u64* pairs, int rounds, int* mismatches, int* err,
                                                      u64 timeout_ticks, unsigned long long* t_out) {
  const int G = gridDim.x, wg = blockIdx.x, tid = threadIdx.x;
  __shared__ int bad, abort_;
  if (tid == 0) bad = 0, abort_ = 0;
  __syncthreads();
  const unsigned long long t0 = wall_clock64();
  for (int r = 0; r < rounds; ++r) {
    u64* fb = full + (r & 1) * G;
    u64* pb = pairs + (r & 1) * G;
    const unsigned tag = (unsigned)r + 1u, t4 = tag4(tag);
    if (tid == 0) {
      ll_put(fb + wg, ll_pack(word_val(r, wg), tag));
      ll_put(pb + wg, pk_pack(word_val(r, wg), word_val(r + 1, wg), t4));
    }
    int failed = 0;
    for (int src = tid; src < G; src += ST) {
      Spin sp;
      u64 a, b;
      while (true) {
        a = ll_get(fb + src);
        b = ll_get(pb + src);
        if (ll_tag(a) == tag && pk_ready(b, t4)) break;
        if (!sp.step(err, timeout_ticks)) {
          failed = 1;
          break;
        }
      }
      if (failed) break;
      if (ll_val(a) != word_val(r, src) || pk_lo(b) != word_val(r, src) || pk_hi(b) != word_val(r + 1, src))
        atomicAdd(&bad, 1);
    }
    if (failed) abort_ = 1;
    __syncthreads();
    if (*static_cast<volatile int*>(&abort_)) break;
  }
  __syncthreads();
  if (tid == 0) {
    if (bad) atomicAdd(mismatches, bad);
    if (wg == 0) t_out[0] = wall_clock64() - t0;
  }
}

}  // namespace selftest
}  // namespace mk

extern "C" {

int megakernel_selftest_dataflow(int rounds, int* mismatches, float* us_per_round) {
  using namespace mk;
  if (rounds < 1 || rounds > (1 << 24) || !mismatches) {
    set_err("selftest: rounds %d outside [1, 2^24] or null output", rounds);
    return -1;
  }
  int dev = 0, cus = 0, khz = 0;
  HIPCHK(hipGetDevice(&dev), -1);
  HIPCHK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), -1);
  HIPCHK(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev), -1);
  int occ = 0;
  HIPCHK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, selftest::dataflow_kernel, selftest::ST, 0), -1);
  if (occ < 1) {
    set_err("selftest: kernel cannot be resident");
    return -1;
  }
  const int G = cus;  // one workgroup per CU: every workgroup resident, every XCD involved
  char* mem = nullptr;
  const size_t words = (size_t)4 * G;
  HIPCHK(hipMalloc(&mem, words * 8 + 64), -1);
  int rc = -1;
  do {
    if (hipMemset(mem, 0, words * 8 + 64) != hipSuccess) {
      set_err("selftest: memset failed");
      break;
    }
    u64* full = reinterpret_cast<u64*>(mem);
    u64* pairs = full + 2 * G;
    int* counters = reinterpret_cast<int*>(mem + words * 8);  // [0] mismatches, [1] error word
    unsigned long long* t = reinterpret_cast<unsigned long long*>(mem + words * 8 + 8);
    const u64 timeout = (u64)(khz > 0 ? khz : 100000) * 2000ull;  // 2 s
    hipLaunchKernelGGL(selftest::dataflow_kernel, dim3(G), dim3(selftest::ST), 0, 0, full, pairs, rounds, counters,
                       counters + 1, timeout, t);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
      set_err("selftest kernel failed: %s", hipGetErrorString(e));
      break;
    }
    int host[2] = {0, 0};
    unsigned long long ticks = 0;
    if (hipMemcpy(host, counters, 8, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(&ticks, t, 8, hipMemcpyDeviceToHost) != hipSuccess) {
      set_err("selftest: copy-back failed");
      break;
    }
    *mismatches = host[0];
    if (us_per_round) *us_per_round = (float)((double)ticks * 1e3 / (khz > 0 ? khz : 100000) / rounds);
    if (host[1] != MK_OK) {
      set_err("selftest: a hand-off wait timed out");
      break;
    }
    rc = 0;
  } while (0);
  (void)hipFree(mem);
  return rc;
}

}  // extern "C"
