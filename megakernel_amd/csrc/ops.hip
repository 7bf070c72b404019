// Operator microbench: every op of one decode step as a
// standalone launch at the decoder's shapes.  Each call runs `reps`
// independent instances of the op in ONE launch (in-kernel repetition: a
// single op takes 0.3-40 us, below the cost of a launch); instance r reads
// weight copy r % n_copies, input r % n_in and writes output slot r % n_out,
// so a caller that rotates >= 512 MB of weight copies defeats every cache.
//
// The GEMVs use the persistent kernel's own packed layouts and inner loops
// (tile blocks with Blk / blk_load / blk_mma, the LM head's tile stream), so
// their numbers measure the code the decode runs.  Reference device code
// each op restates:
//   rmsnorm            src/rmsnorm.cuh:87-108   (rmsnorm_float_in)
//   gemv (QKV / O)     src/gemv.cuh:118-199, src/gemv.cuh:36-104
//   gemv + residual    src/gemv.cuh:36-104 with src/megakernel.cu:288-290 (down)
//   gate/up + SiLU     src/gemv.cuh:212-279, src/utils.cuh:47-61
//   rope               src/attention.cuh:22-44  (apply_rope_inplace)
//   lm head + argmax   src/sampling.cuh:32-117  (lowest index on ties)
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <mutex>

#include "megakernel.h"
#include "mk_host.h"
#include "mk_kernel.h"

namespace mk {
namespace ops {

enum GemvKind : int { GEMV_PLAIN = 0, GEMV_RESIDUAL = 1, GEMV_GATE_UP = 2 };

// ------------------------------------------------------------------ GEMVs
// Work item = (instance r, 16-row block b), items r-major and dealt to
// workgroups round-robin, so the workgroups in flight stream neighbouring
// blocks of one weight copy.  The input vector of the item's instance is
// staged in LDS (split-bf16 pairs, as the decode kernel's GEMVs read it) and
// only reloaded when the instance's input changes; the block product is the
// decode kernel's (blk_mma on tile-layout blocks, wave shares summed in LDS).
// Loads are issued vector first (L2-resident pool), weights second, so the
// vector's wait does not wait for the weight block (loads return in order).
template <int KC, int KIND>
__global__ __launch_bounds__(NT) void gemv_kernel(const u32x4* __restrict__ w, long long copy_units, int n_copies,
                                                  int rows, const float* __restrict__ x,
                                                  const float* __restrict__ res, int n_in, float* __restrict__ y,
                                                  int n_out, int reps) {
  constexpr int K = KC * 256, KT = K / 32, PER = (K + NT - 1) / NT;
  __shared__ float vec[K];
  __shared__ float red[2][NW * 16];
  const int RB = rows / 16;
  const long long items = (long long)reps * RB;
  int have = -1;  // input index staged in vec (uniform across the workgroup)
  for (long long it = blockIdx.x; it < items; it += gridDim.x) {
    const int r = (int)(it / RB), b = (int)(it % RB);
    const int in = r % n_in;
    const bool reload = in != have;
    float xv[PER];
    if (reload) {
      const float* xs = x + (long long)in * K;
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const int i = (int)threadIdx.x + k * NT;
        xv[k] = xs[i < K ? i : K - 1];
      }
    }
    const u32x4* wc = w + (long long)(r % n_copies) * copy_units;
    Blk<KC> bg, bu;
    if (KIND == GEMV_GATE_UP) {
      blk_load(bg, wc + (long long)(2 * b) * KT * 64);
      blk_load(bu, wc + (long long)(2 * b + 1) * KT * 64);
    } else {
      blk_load(bg, wc + (long long)b * KT * 64);
    }
    __syncthreads();  // the previous item's reads of vec and red are done
    if (reload) {
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const int i = (int)threadIdx.x + k * NT;
        if (i < K) xs_put(reinterpret_cast<uint32_t*>(vec), i, xv[k]);
      }
      __syncthreads();
      have = in;
    }
    blk_mma(bg, vec, red[0]);
    if (KIND == GEMV_GATE_UP) blk_mma(bu, vec, red[1]);
    __syncthreads();
    if (threadIdx.x < 16) {
      const int t = (int)threadIdx.x, row = b * 16 + t;
      float v = red_sum(red[0], t);
      if (KIND == GEMV_GATE_UP) v = silu_mul(v, red_sum(red[1], t));
      if (KIND == GEMV_RESIDUAL) v += res[(long long)in * rows + row];
      y[(long long)(r % n_out) * rows + row] = v;
    }
  }
}

// ------------------------------------------------------- LM head + argmax
// Tile layout (mk_config.h): a wave reduces whole 16-row blocks, 16 KiB of
// loads in flight per wave, exactly the persistent kernel's LM-head loop.
// Work item = (instance r, chunk of chb blocks, a multiple of the wave count
// sized so one instance covers the resident grid).  A workgroup carries its
// best (logit, index) key across its items of one instance and folds it into
// keys[r % n_out] with one 64-bit atomic max when the instance changes.

template <int KT>
__global__ __launch_bounds__(NT) void lmhead_kernel(const u32x4* __restrict__ w, long long copy_units,
                                                    int n_copies, int vocab, const float* __restrict__ h, int n_in,
                                                    float* __restrict__ logits, unsigned long long* __restrict__ keys,
                                                    int n_out, int reps, int chb) {
  constexpr int K = KT * 32, PER = (K + NT - 1) / NT;
  __shared__ float vec[K];
  __shared__ unsigned long long wbest[NW];
  const int nb = vocab / 16, nch = (nb + chb - 1) / chb;
  const long long items = (long long)reps * nch;
  const unsigned lo = lane_id();
  int have = -1;
  unsigned long long best = 0ull;  // this lane's best key of the current instance
  for (long long it = blockIdx.x; it < items; it += gridDim.x) {
    const int r = (int)(it / nch), c = (int)(it % nch);
    const int in = r % n_in;
    if (in != have) {
      float xv[PER];
      const float* hs = h + (long long)in * K;
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const int i = (int)threadIdx.x + k * NT;
        xv[k] = hs[i < K ? i : K - 1];
      }
      __syncthreads();
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const int i = (int)threadIdx.x + k * NT;
        if (i < K) vec[i] = xv[k];
      }
      __syncthreads();
      have = in;
    }
    const u32x4* wc = w + (long long)(r % n_copies) * copy_units;
    float* lg = logits ? logits + (long long)(r % n_out) * vocab : nullptr;
    const int b1 = (c + 1) * chb < nb ? (c + 1) * chb : nb;
    for (int b = c * chb + wave_id(); b < b1; b += NW) {
      const float* hv = vec + (lo >> 4) * 8;
      const auto rs = make_rsrc(wc + (long long)b * KT * 64);
      float acc = 0.f;
      constexpr int U = KT < 16 ? KT : 16;
#pragma unroll 1
      for (int k0 = 0; k0 < KT; k0 += U) {
        u32x4 wv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) wv[u] = buf_ld_nt(rs, lo * 16u, (unsigned)(k0 + u) * 1024u);
#pragma unroll
        for (int u = 0; u < U; ++u) acc = dot8(wv[u], hv + (k0 + u) * 32, acc);
      }
      acc = stride_sum<16>(acc);
      if (lo < 16) {
        const unsigned idx = (unsigned)(b * 16) + lo;
        if (lg) lg[idx] = acc;
        const unsigned long long key = argmax_key(acc, idx);
        best = key > best ? key : best;
      }
    }
    const long long nx = it + gridDim.x;
    if (nx >= items || nx / nch != r) {  // last item of this instance here: publish
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) {
        const unsigned long long o = __shfl_xor(best, m);
        best = o > best ? o : best;
      }
      if (lo == 0) wbest[wave_id()] = best;
      __syncthreads();
      if (threadIdx.x == 0) {
        unsigned long long m = 0ull;
        for (int i = 0; i < NW; ++i) m = wbest[i] > m ? wbest[i] : m;
        atomicMax(keys + (r % n_out), m);
      }
      __syncthreads();  // wbest is rewritten by the next publish
      best = 0ull;
    }
  }
}

__global__ void keys_clear_kernel(unsigned long long* keys, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) keys[i] = 0ull;
}

__global__ void keys_to_tokens_kernel(const unsigned long long* keys, int* tokens, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) tokens[i] = (int)argmax_key_index(keys[i]);
}

// ---------------------------------------------------------------- RMSNorm
// One wave per instance: lane l holds elements 512j + 8l .. +7 (one 16-byte
// load each), the sum of squares is a wave reduction (no LDS, no barrier),
// and each lane writes its 8 outputs as two 16-byte stores.
// y = x * rsqrt(mean(x^2) + eps) * gain, x and gain bf16, y fp32.
template <int NJ>
__global__ __launch_bounds__(NT) void rmsnorm_kernel(const u32x4* __restrict__ x, const u32x4* __restrict__ gain,
                                                     float* __restrict__ y, int n_in, int n_out, int reps,
                                                     float eps) {
  constexpr int N = NJ * 512;
  const unsigned l = lane_id();
  const int wv = (int)blockIdx.x * NW + wave_id(), nwv = (int)gridDim.x * NW;
  float g[NJ][8];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const u32x4 gw = gain[64 * j + l];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      g[j][2 * e] = bf16_lo(gw[e]);
      g[j][2 * e + 1] = bf16_hi(gw[e]);
    }
  }
  for (int r = wv; r < reps; r += nwv) {
    const auto rs = make_rsrc(x + (long long)(r % n_in) * (N / 8));
    u32x4 v[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) v[j] = buf_ld_nt(rs, l * 16u, (unsigned)j * 1024u);
    float f[NJ][8];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f[j][2 * e] = bf16_lo(v[j][e]);
        f[j][2 * e + 1] = bf16_hi(v[j][e]);
        ss += f[j][2 * e] * f[j][2 * e] + f[j][2 * e + 1] * f[j][2 * e + 1];
      }
    ss = wave_sum(ss);
    const float rn = rsqrtf(ss / (float)N + eps);
    float4* yr = reinterpret_cast<float4*>(y + (long long)(r % n_out) * N);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = f[j][e] * rn * g[j][e];
      yr[(512 * j + 8 * l) / 4] = make_float4(o[0], o[1], o[2], o[3]);
      yr[(512 * j + 8 * l) / 4 + 1] = make_float4(o[4], o[5], o[6], o[7]);
    }
  }
}

// ------------------------------------------------------------------- RoPE
// NeoX rotate-half on n_heads heads of D at position pos:
// (x_i, x_{i+D/2}) -> (x_i c - x_{i+D/2} s, x_{i+D/2} c + x_i s),
// angle = pos * inv_freq[i] in fp32 (the HF / persistent-kernel convention).
// One wave per instance; lane l owns pair i = l % (D/2) of heads
// l / (D/2) + k * (64 / (D/2)), so each lane computes one sincos.
struct InvFreq {
  float v[64];
};

template <int D>
__global__ __launch_bounds__(NT) void rope_kernel(const float* __restrict__ x, const int* __restrict__ pos,
                                                  float* __restrict__ y, int n_heads, int n_in, int n_out,
                                                  int reps, InvFreq invf) {
  constexpr int P = D / 2, HPW = kWave / P;  // pairs per head, heads per wave pass
  const unsigned l = lane_id();
  const int i = (int)(l % P), h0 = (int)(l / P);
  const int wv = (int)blockIdx.x * NW + wave_id(), nwv = (int)gridDim.x * NW;
  const long long n = (long long)n_heads * D;
  for (int r = wv; r < reps; r += nwv) {
    const int in = r % n_in;
    float sn, cs;
    sincosf((float)pos[in] * invf.v[i], &sn, &cs);
    const float* xr = x + in * n;
    float* yr = y + (long long)(r % n_out) * n;
    for (int hd = h0; hd < n_heads; hd += HPW) {
      const float a = xr[hd * D + i], b = xr[hd * D + i + P];
      yr[hd * D + i] = a * cs - b * sn;
      yr[hd * D + i + P] = b * cs + a * sn;
    }
  }
}

// ------------------------------------------------------------- host side
thread_local float g_last_ms = 0.f;

template <class Kern>
static int grid_for(Kern k, int smem, long long items) {
  int dev = 0, cus = 0, occ = 0;
  HIPCHK(hipGetDevice(&dev), -1);
  HIPCHK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), -1);
  HIPCHK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k, NT, smem), -1);
  if (occ < 1) occ = 1;
  const long long g = (long long)cus * occ;
  return (int)(items < g ? (items > 0 ? items : 1) : g);
}

// Runs launch() on the null stream between two events; blocking.
template <class F>
static int timed(F launch) {
  hipEvent_t e0 = nullptr, e1 = nullptr;
  HIPCHK(hipEventCreate(&e0), -1);
  if (hipEventCreate(&e1) != hipSuccess) {
    (void)hipEventDestroy(e0);
    set_err("hipEventCreate failed");
    return -1;
  }
  int rc = -1;
  do {
    if (hipEventRecord(e0, 0) != hipSuccess) { set_err("hipEventRecord failed"); break; }
    if (launch() != 0) break;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) { set_err("op launch failed: %s", hipGetErrorString(e)); break; }
    if (hipEventRecord(e1, 0) != hipSuccess) { set_err("hipEventRecord failed"); break; }
    e = hipEventSynchronize(e1);
    if (e != hipSuccess) { set_err("op kernel failed: %s", hipGetErrorString(e)); break; }
    float ms = 0.f;
    (void)hipEventElapsedTime(&ms, e0, e1);
    g_last_ms = ms;
    rc = 0;
  } while (0);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return rc;
}

static bool common_ok(int n_in, int n_out, int reps) {
  if (n_in < 1 || n_out < 1 || reps < 1) {
    set_err("n_in, n_out and reps must be >= 1 (got %d, %d, %d)", n_in, n_out, reps);
    return false;
  }
  return true;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <int KC, int KIND>
static int launch_gemv(const u32x4* w, long long cu, int nc, int rows, const float* x, const float* res, int n_in,
                       float* y, int n_out, int reps) {
  auto k = gemv_kernel<KC, KIND>;
  const int g = grid_for(k, 0, (long long)reps * (rows / 16));
  if (g < 0) return -1;
  hipLaunchKernelGGL(k, dim3(g), dim3(NT), 0, 0, w, cu, nc, rows, x, res, n_in, y, n_out, reps);
  return 0;
}

template <int KIND>
static int gemv_dispatch(int k, const u32x4* w, long long cu, int nc, int rows, const float* x, const float* res,
                         int n_in, float* y, int n_out, int reps) {
  switch (k / 256) {
    case 1: return launch_gemv<1, KIND>(w, cu, nc, rows, x, res, n_in, y, n_out, reps);
    case 2: return launch_gemv<2, KIND>(w, cu, nc, rows, x, res, n_in, y, n_out, reps);
    case 4: return launch_gemv<4, KIND>(w, cu, nc, rows, x, res, n_in, y, n_out, reps);
    case 8: return launch_gemv<8, KIND>(w, cu, nc, rows, x, res, n_in, y, n_out, reps);
    case 11: return launch_gemv<11, KIND>(w, cu, nc, rows, x, res, n_in, y, n_out, reps);
    case 12: return launch_gemv<12, KIND>(w, cu, nc, rows, x, res, n_in, y, n_out, reps);
    default: set_err("gemv: k=%d not supported", k); return -1;
  }
}

static bool gemv_k_ok(int k) {
  const int c = k / 256;
  return k % 256 == 0 && (c == 1 || c == 2 || c == 4 || c == 8 || c == 11 || c == 12);
}


static bool lmhead_args_ok(const void* w, long long copy_bytes, int n_copies, int vocab, int k, const float* h,
                           int n_in, const int* tokens, int n_out, int reps) {
  if (!common_ok(n_in, n_out, reps)) return false;
  if (!w || !h || !tokens || !aligned16(w) || n_copies < 1 || copy_bytes < 0 || copy_bytes % 16) {
    set_err("op_lmhead_argmax: null/unaligned pointer, n_copies < 1 or copy_bytes not a multiple of 16");
    return false;
  }
  if (vocab <= 0 || vocab % 16 || vocab > (1 << 30) || (k != 256 && k != 512 && k != 1024)) {
    set_err("op_lmhead_argmax: vocab=%d (multiple of 16), k=%d (256, 512 or 1024)", vocab, k);
    return false;
  }
  if (n_copies > 1 && copy_bytes < (long long)vocab * k * 2) {
    set_err("op_lmhead_argmax: copy_bytes %lld < packed matrix bytes %lld", copy_bytes, (long long)vocab * k * 2);
    return false;
  }
  return true;
}

// Clear the keys (a fill kernel, no memset node), score every row and fold
// the keys into tokens, on the null stream (not waited for).
static int lmhead_argmax_enqueue(const void* w, long long copy_bytes, int n_copies, int vocab, int k, const float* h,
                                 int n_in, float* logits, unsigned long long* keys, int* tokens, int n_out,
                                 int reps) {
  const u32x4* wp = static_cast<const u32x4*>(w);
  const long long cu = copy_bytes / 16;
  const int tb = 256, nb = (n_out + tb - 1) / tb;
  hipLaunchKernelGGL(keys_clear_kernel, dim3(nb), dim3(tb), 0, 0, keys, n_out);
  auto run = [&](auto kern) -> int {
    const int nb16 = vocab / 16;
    const int full = grid_for(kern, 0, 1LL << 30);  // resident workgroups
    if (full < 0) return -1;
    const int chb = NW * ((nb16 + full * NW - 1) / (full * NW));
    const int nch = (nb16 + chb - 1) / chb;
    const int g = full < (long long)reps * nch ? full : (int)((long long)reps * nch);
    hipLaunchKernelGGL(kern, dim3(g), dim3(NT), 0, 0, wp, cu, n_copies, vocab, h, n_in, logits, keys, n_out, reps,
                       chb);
    return 0;
  };
  const int rc = k == 256 ? run(lmhead_kernel<8>) : k == 512 ? run(lmhead_kernel<16>) : run(lmhead_kernel<32>);
  if (rc) return rc;
  hipLaunchKernelGGL(keys_to_tokens_kernel, dim3(nb), dim3(tb), 0, 0, keys, tokens, n_out);
  return 0;
}

// ------------------------------------------- allocation-free LM head argmax
// The argmax keys of megakernel_op_lmhead_argmax_noalloc live in this
// file-scope device array instead of a caller workspace.  Every GPU the
// library runs on holds its own copy until the process ends.  In host code
// the name `scratch` is only a host-side stand-in: the device address of the
// current GPU's copy comes from hipGetSymbolAddress, once per device, and is
// the only form host code passes to kernels.  Calls on one GPU share the
// array (it keeps the last call's keys; each call clears what it uses), so
// calls that overlap on one GPU race.
static __device__ __align__(256) unsigned long long scratch[MK_NOALLOC_KEYS_MAX];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static unsigned long long* g_scratch_dev[kMaxDevices] = {};

static unsigned long long* scratch_keys() {
  int dev = -1;
  HIPCHK(hipGetDevice(&dev), nullptr);
  if (dev < 0 || dev >= kMaxDevices) {
    set_err("device index %d out of range", dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* ptr = nullptr;
    HIPCHK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), nullptr);
    g_scratch_dev[dev] = static_cast<unsigned long long*>(ptr);
  }
  return g_scratch_dev[dev];
}

}  // namespace ops
}  // namespace mk

using namespace mk;
using namespace mk::ops;

extern "C" {

long long megakernel_op_packed_bytes(int rows, int k) {
  if (rows <= 0 || k <= 0 || rows % 16 || k % 32) {
    set_err("rows must be a positive multiple of 16 and k of 32 (got %d, %d)", rows, k);
    return -1;
  }
  return (long long)rows * k * 2;
}

int megakernel_op_pack(const void* d_src, int rows, int k, int layout, void* d_dst) {
  if (!d_src || !d_dst || !aligned16(d_src) || !aligned16(d_dst)) {
    set_err("op_pack: null or unaligned pointer");
    return -1;
  }
  if (layout != MK_OP_LAYOUT_TILE && layout != MK_OP_LAYOUT_GATE_UP) {
    set_err("op_pack: unknown layout %d", layout);
    return -1;
  }
  if (rows <= 0 || rows % 16 || k <= 0 || k % 32 || (layout == MK_OP_LAYOUT_GATE_UP && rows % 32)) {
    set_err("op_pack: rows=%d k=%d do not fit layout %d", rows, k, layout);
    return -1;
  }
  const u32x4* src = static_cast<const u32x4*>(d_src);
  u32x4* dst = static_cast<u32x4*>(d_dst);
  return timed([&]() -> int {
    const long long units = (long long)rows * k / 8;
    const int threads = 256;
    const int blocks = (int)((units + threads - 1) / threads < 65536 ? (units + threads - 1) / threads : 65536);
    if (layout == MK_OP_LAYOUT_GATE_UP) {  // gate rows [0, rows/2), up rows [rows/2, rows): blocks interleaved
      const int half = rows / 2;
      const long long hu = (long long)half * k / 8;
      hipLaunchKernelGGL(repack_kernel, dim3(blocks), dim3(threads), 0, 0, src, half, k, dst, 2, 0);
      hipLaunchKernelGGL(repack_kernel, dim3(blocks), dim3(threads), 0, 0, src + hu, half, k, dst, 2, 1);
    } else {
      hipLaunchKernelGGL(repack_kernel, dim3(blocks), dim3(threads), 0, 0, src, rows, k, dst, 1, 0);
    }
    return 0;
  });
}

int megakernel_op_rmsnorm(const void* x, const void* gain, float* y, int n, int n_in, int n_out, int reps,
                          float eps) {
  if (!common_ok(n_in, n_out, reps)) return -1;
  if (!x || !gain || !y || !aligned16(x) || !aligned16(gain) || !aligned16(y)) {
    set_err("op_rmsnorm: null or unaligned pointer");
    return -1;
  }
  if (n != 512 && n != 1024 && n != 2048) {
    set_err("op_rmsnorm: n=%d not supported (512, 1024, 2048)", n);
    return -1;
  }
  const u32x4* xs = static_cast<const u32x4*>(x);
  const u32x4* gs = static_cast<const u32x4*>(gain);
  return timed([&]() -> int {
    const long long waves = reps;
    auto run = [&](auto kern) -> int {
      const int g = grid_for(kern, 0, (waves + NW - 1) / NW);
      if (g < 0) return -1;
      hipLaunchKernelGGL(kern, dim3(g), dim3(NT), 0, 0, xs, gs, y, n_in, n_out, reps, eps);
      return 0;
    };
    return n == 512 ? run(rmsnorm_kernel<1>) : n == 1024 ? run(rmsnorm_kernel<2>) : run(rmsnorm_kernel<4>);
  });
}

int megakernel_op_gemv(const void* w, long long copy_bytes, int n_copies, int rows, int k, int kind, const float* x,
                       const float* res, int n_in, float* y, int n_out, int reps) {
  if (!common_ok(n_in, n_out, reps)) return -1;
  if (!w || !x || !y || !aligned16(w) || n_copies < 1 || copy_bytes < 0 || copy_bytes % 16) {
    set_err("op_gemv: null/unaligned pointer, n_copies < 1 or copy_bytes not a multiple of 16");
    return -1;
  }
  if (kind < GEMV_PLAIN || kind > GEMV_GATE_UP) {
    set_err("op_gemv: unknown kind %d", kind);
    return -1;
  }
  if (kind == GEMV_RESIDUAL && !res) {
    set_err("op_gemv: residual kind needs res");
    return -1;
  }
  if (rows <= 0 || rows % 16 || !gemv_k_ok(k)) {
    set_err("op_gemv: rows=%d must be a multiple of 16, k=%d one of 256/512/1024/2048/2816/3072", rows, k);
    return -1;
  }
  const long long need = (long long)rows * k * 2 * (kind == GEMV_GATE_UP ? 2 : 1);
  if (n_copies > 1 && copy_bytes < need) {
    set_err("op_gemv: copy_bytes %lld < packed matrix bytes %lld", copy_bytes, need);
    return -1;
  }
  const u32x4* wp = static_cast<const u32x4*>(w);
  const long long cu = copy_bytes / 16;
  return timed([&]() -> int {
    switch (kind) {
      case GEMV_PLAIN: return gemv_dispatch<GEMV_PLAIN>(k, wp, cu, n_copies, rows, x, res, n_in, y, n_out, reps);
      case GEMV_RESIDUAL:
        return gemv_dispatch<GEMV_RESIDUAL>(k, wp, cu, n_copies, rows, x, res, n_in, y, n_out, reps);
      default: return gemv_dispatch<GEMV_GATE_UP>(k, wp, cu, n_copies, rows, x, res, n_in, y, n_out, reps);
    }
  });
}

int megakernel_op_rope(const float* x, const int* pos, float* y, int n_heads, int head_dim, int n_in, int n_out,
                       int reps, float theta) {
  if (!common_ok(n_in, n_out, reps)) return -1;
  if (!x || !pos || !y) {
    set_err("op_rope: null pointer");
    return -1;
  }
  if ((head_dim != 64 && head_dim != 128) || n_heads < 1 || n_heads > 256 || !(theta > 1.0f)) {
    set_err("op_rope: head_dim %d (64 or 128), n_heads %d (1..256), theta %g (> 1)", head_dim, n_heads, theta);
    return -1;
  }
  InvFreq invf{};
  for (int i = 0; i < head_dim / 2; ++i) invf.v[i] = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
  return timed([&]() -> int {
    auto run = [&](auto kern) -> int {
      const int g = grid_for(kern, 0, ((long long)reps + NW - 1) / NW);
      if (g < 0) return -1;
      hipLaunchKernelGGL(kern, dim3(g), dim3(NT), 0, 0, x, pos, y, n_heads, n_in, n_out, reps, invf);
      return 0;
    };
    return head_dim == 64 ? run(rope_kernel<64>) : run(rope_kernel<128>);
  });
}

int megakernel_op_lmhead_argmax(const void* w, long long copy_bytes, int n_copies, int vocab, int k, const float* h,
                                int n_in, float* logits, unsigned long long* keys, int* tokens, int n_out,
                                int reps) {
  if (!lmhead_args_ok(w, copy_bytes, n_copies, vocab, k, h, n_in, tokens, n_out, reps)) return -1;
  if (!keys) {
    set_err("op_lmhead_argmax: null keys workspace");
    return -1;
  }
  return timed([&]() -> int {
    return lmhead_argmax_enqueue(w, copy_bytes, n_copies, vocab, k, h, n_in, logits, keys, tokens, n_out, reps);
  });
}

int megakernel_op_lmhead_argmax_noalloc(const void* w, long long copy_bytes, int n_copies, int vocab, int k,
                                        const float* h, int n_in, float* logits, int* tokens, int n_out, int reps) {
  if (!lmhead_args_ok(w, copy_bytes, n_copies, vocab, k, h, n_in, tokens, n_out, reps)) return -1;
  if (n_out > MK_NOALLOC_KEYS_MAX) {
    set_err("op_lmhead_argmax_noalloc: n_out=%d exceeds the static key array (%d entries)", n_out,
            MK_NOALLOC_KEYS_MAX);
    return -1;
  }
  unsigned long long* keys = scratch_keys();
  if (!keys) return -1;
  if (lmhead_argmax_enqueue(w, copy_bytes, n_copies, vocab, k, h, n_in, logits, keys, tokens, n_out, reps)) return -1;
  HIPCHK(hipGetLastError(), -1);
  return 0;
}

float megakernel_op_last_ms(void) { return g_last_ms; }

}  // extern "C"
