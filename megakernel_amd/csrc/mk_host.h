// Host-side helpers shared by the translation units of megakernel.so: the
// thread-local error message, the HIP error check, and the set-up kernels
// (weight repacking, synthetic data, KV layout conversion) that both the
// batch-1 decode handle and the batched-decode handle launch.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mk_device.h"

namespace mk {

extern thread_local char g_err[512];
void set_err(const char* fmt, ...);

#define HIPCHK(expr, ret)                                                                  \
  do {                                                                                     \
    hipError_t e_ = (expr);                                                                \
    if (e_ != hipSuccess) {                                                                \
      ::mk::set_err("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, __LINE__); \
      return ret;                                                                          \
    }                                                                                      \
  } while (0)

// Device KV cache addressing of one sequence: K [L][NKV][s_pad][D], V^T
// blocks [L][NKV][s_pad/32][D][32], both bf16; kv points at K, kvt at V^T.
__device__ __forceinline__ long long k_index(int l, int g, long long t, int d, int NKV, int s_pad, int D) {
  return (((long long)l * NKV + g) * s_pad + t) * D + d;
}
__device__ __forceinline__ long long vt_index(int l, int g, long long t, int d, int NKV, int s_pad, int D) {
  return ((long long)l * NKV + g) * (long long)s_pad * D + (t / 32) * 32LL * D + (long long)d * 32 + (t % 32);
}

__global__ void repack_kernel(const u32x4* __restrict__ src, int R, int K, u32x4* __restrict__ dst,
                              int blk_stride, int blk_off);
__global__ void synth_kv_kernel(uint16_t* __restrict__ kv, uint16_t* __restrict__ kvt, int L, int NKV, int s_pad,
                                int D, int len, unsigned long long seed, float c);
__global__ void kv_convert_kernel(uint16_t* __restrict__ buf, uint16_t* __restrict__ kv, uint16_t* __restrict__ kvt,
                                  int L, int NKV, int s_pad, int D, int len, int to_cache);
// FP8 cache conversions of one sequence (reference layout buf <-> codes + row scales)
__global__ void kv_quant_kernel(const uint16_t* __restrict__ buf, uint8_t* __restrict__ k8, uint8_t* __restrict__ v8,
                                float* __restrict__ ks, float* __restrict__ vs, int L, int NKV, int s_pad, int D,
                                int len);
__global__ void kv_dequant_kernel(uint16_t* __restrict__ buf, const uint8_t* __restrict__ k8,
                                  const uint8_t* __restrict__ v8, const float* __restrict__ ks,
                                  const float* __restrict__ vs, int L, int NKV, int s_pad, int D, int len);
__global__ void lmhead_fp8_kernel(const u32x4* __restrict__ src, int K, unsigned char* __restrict__ dst,
                                  float* __restrict__ scales, float* __restrict__ err);
__global__ void synth_kv_ref_kernel(uint16_t* __restrict__ buf, int L, int NKV, int D, int len,
                                    unsigned long long seed, float c);

// Prefill context of a batch-1 handle (batch.hip): the batched kernels'
// matrix-core weight copy and work buffers, bound to an external KV cache in
// the decode kernel's layout (K [L][NKV][s_pad][D], V^T blocks).
namespace batch {
struct BHandle;
BHandle* create_prefill_context(int preset, int vocab, int max_seq, const char* d_weights, const long long* offsets,
                                int num_offsets, uint16_t* kv, uint16_t* kvt);
// n prompt tokens at positions pos0 .. pos0 + n - 1 of the bound cache;
// next_token (may be null) receives the greedy token after the last one.
int prefill_context_run(BHandle* h, const int* tokens, int n, int pos0, int* next_token, float* logits,
                        float* kscale, float* vscale);
float prefill_context_ms(BHandle* h);
void destroy_prefill_context(BHandle* h);
}  // namespace batch

}  // namespace mk
