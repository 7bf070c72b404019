// megakernel.so: host runtime and C ABI of the MI355X persistent decode
// megakernel.  The six reference entry points keep their exact signatures and
// meaning (/root/reference/src/megakernel.cu:535-624); everything else is an
// additive extension declared in include/megakernel.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <vector>

#include "mk_config.h"
#include "mk_device.h"
#include "mk_host.h"
#include "mk_kernel.h"
#include "mk_launch.h"

#include "../../include/megakernel.h"

namespace mk {

// ------------------------------------------------------------ error state
thread_local char g_err[512] = "";

// ------------------------------------------- uncached hand-off word buffers
// The tagged hand-off words (x, qkv, part, act, argmax slots) live in
// uncached device memory: their stores and polls skip the per-XCD L2s and go
// straight to the device's coherence point, which shortens every
// cross-workgroup hand-off (measured: 2,711 -> 2,792 tok/s at ctx 1024).
// Uncached memory that a kernel has read must not be freed before the
// process ends (allocations made after such a free have held wrong values
// on this platform), so these buffers come from a process-wide pool: a
// handle takes blocks at init and gives them back at free, and a block is
// only ever reused, never released.  The pool is small: five buffers of at
// most a few hundred KB per live handle.
struct UcBlock {
  int device;
  size_t bytes;
  void* ptr;
  bool busy;
};
static std::mutex g_uc_mu;
static std::vector<UcBlock> g_uc_pool;

static void* uc_acquire(int device, size_t bytes) {
  std::lock_guard<std::mutex> lk(g_uc_mu);
  for (UcBlock& b : g_uc_pool)
    if (!b.busy && b.device == device && b.bytes >= bytes) {
      b.busy = true;
      return b.ptr;
    }
  void* p = nullptr;
  const size_t sz = (bytes + 4095) / 4096 * 4096;
  if (hipExtMallocWithFlags(&p, sz, hipDeviceMallocUncached) != hipSuccess || !p) {
    (void)hipGetLastError();
    return nullptr;
  }
  g_uc_pool.push_back(UcBlock{device, sz, p, true});
  return p;
}
static void uc_release(void* p) {
  if (!p) return;
  std::lock_guard<std::mutex> lk(g_uc_mu);
  for (UcBlock& b : g_uc_pool)
    if (b.ptr == p) b.busy = false;
}

void set_err(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

// --------------------------------------------------------- device helpers
// Repack a row-major bf16 matrix W[R][K] into the packed tile layout of
// mk_config.h.  Destination 16-row block of source block rb is
// rb * blk_stride + blk_off, so gate/up can be interleaved.  One thread per
// 16-byte unit.
__global__ void repack_kernel(const u32x4* __restrict__ src, int R, int K, u32x4* __restrict__ dst,
                              int blk_stride, int blk_off) {
  const int KT = K / 32;
  const long long units = (long long)R * K / 8;
  for (long long u = (long long)blockIdx.x * blockDim.x + threadIdx.x; u < units;
       u += (long long)gridDim.x * blockDim.x) {
    const int lane = (int)(u % 64);
    const long long t = u / 64;
    const int tin = (int)(t % KT);  // 1 KiB unit (16 x 32 tile) inside the block
    const long long rb = t / KT;
    const long long row = rb * 16 + (lane & 15), chunk = (long long)tin * 4 + (lane >> 4);
    dst[((rb * blk_stride + blk_off) * KT + tin) * 64 + lane] = src[row * (K / 8) + chunk];
  }
}

// FP8 copy of the LM head (no counterpart in the reference kernel; the
// reference plans FP8 weights in RESEARCH.md:434-436,463).  One workgroup per
// 16-row block of the bf16 tiles: row r gets the power-of-two scale 2^e with
// the smallest e such that max|W[r]| <= 448 * 2^e, and each weight becomes
// e4m3(W[r][c] * 2^-e) (exact scaling, then round to nearest even).  Output
// tiles: 1 KiB units of 64 lanes x 16 bytes, lane (q, r) holding row r,
// columns 64u + 16q .. +15 of unit u.
// err (optional): per row an upper bound B_r on |W[r] . h - Q[r] . h| / ||h||
// for any h, Q[r] the dequantised FP8 row, including both products' fp32
// summation error: B_r = (||W[r] - Q[r]|| + 3 g (||W[r]|| + ||W[r] - Q[r]||))
// (1 + 2^-12), g = 1.1 (K + 64) 2^-24 (the bound gamma_n n u / (1 - n u) on a
// length-n fp32 sum, with room); the screened LM head uses it to skip rows.
__global__ __launch_bounds__(256) void lmhead_fp8_kernel(const u32x4* __restrict__ src, int K,
                                                         unsigned char* __restrict__ dst, float* __restrict__ scales,
                                                         float* __restrict__ err) {
  const int r = threadIdx.x >> 4, j = threadIdx.x & 15;  // 16 threads per row (one lane group)
  const long long rb = blockIdx.x, row = rb * 16 + r;
  const int KT = K / 32, KT8 = K / 64;
  const uint16_t* s16 = reinterpret_cast<const uint16_t*>(src + rb * KT * 64);
  auto elem = [&](int c) {  // bf16 tile layout: unit c/32, lane ((c/8)%4)*16 + r, element c%8
    return bf16_to_f32(s16[(((c >> 5) * 64) + ((c >> 3) & 3) * 16 + r) * 8 + (c & 7)]);
  };
  float amax = 0.f;
  for (int c = j; c < K; c += 16) amax = fmaxf(amax, fabsf(elem(c)));
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m));
  const int e = e4m3_row_exp(amax);
  unsigned char* d = dst + rb * KT8 * 1024;
  double rr = 0.0, ww = 0.0;  // squared norms of W[r] - Q[r] and of W[r]
  for (int c = j; c < K; c += 16) {
    const int code = e4m3_encode(ldexpf(elem(c), -e));
    d[(c >> 6) * 1024 + (((c >> 4) & 3) * 16 + r) * 16 + (c & 15)] = (unsigned char)code;
    const double w = elem(c), q = (double)__builtin_amdgcn_cvt_pk_f32_fp8(code, false)[0] * ldexp(1.0, e);
    rr += (w - q) * (w - q);
    ww += w * w;
  }
  if (j == 0) scales[row] = ldexpf(1.f, e);
  if (err) {
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) {
      rr += __shfl_xor(rr, m);
      ww += __shfl_xor(ww, m);
    }
    if (j == 0) {
      const double g = 1.1 * (K + 64) * ldexp(1.0, -24), rn = sqrt(rr), wn = sqrt(ww);
      err[row] = (float)((rn + 3.0 * g * (wn + rn)) * (1.0 + ldexp(1.0, -12)));
    }
  }
}

// FP8 copy of the layer weights (opt-in; the same quantisation as the LM
// head's: power-of-two row scale 2^e, e the smallest with max|W[r]| <= 448 *
// 2^e, codes e4m3(W[r][c] * 2^-e) rounded to nearest even).  One workgroup per
// 16-row block (blockIdx.x) of one matrix region of layer blockIdx.y; the
// region starts at unit `off` of the layer in both formats (bf16: 16-byte
// units, FP8: 8-byte units) and its blocks hold K / 32 tiles each.  FP8 tile:
// 512 bytes, lane ((c >> 3) & 3) * 16 + r holding row r, columns 32 u + 8
// ((c >> 3) & 3) .. +7 of tile u as 8 consecutive bytes.  Scale of block row r
// at scales[layer * srows_layer + srow + 16 rb + r].
__global__ __launch_bounds__(256) void layer_fp8_kernel(const u32x4* __restrict__ layers, long long u_layer,
                                                        long long off, int K, unsigned char* __restrict__ dst8,
                                                        float* __restrict__ scales, int srows_layer, int srow) {
  const int r = threadIdx.x >> 4, j = threadIdx.x & 15;  // 16 threads per row
  const long long rb = blockIdx.x, layer = blockIdx.y;
  const int KT = K / 32;
  const long long blk_units = layer * u_layer + off + rb * KT * 64;
  const uint16_t* s16 = reinterpret_cast<const uint16_t*>(layers + blk_units);
  auto lane_of = [&](int c) { return ((c >> 3) & 3) * 16 + r; };
  auto elem = [&](int c) { return bf16_to_f32(s16[((c >> 5) * 64 + lane_of(c)) * 8 + (c & 7)]); };
  float amax = 0.f;
  for (int c = j; c < K; c += 16) amax = fmaxf(amax, fabsf(elem(c)));
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m));
  const int e = e4m3_row_exp(amax);
  unsigned char* d = dst8 + blk_units * 8;
  for (int c = j; c < K; c += 16)
    d[(c >> 5) * 512 + lane_of(c) * 8 + (c & 7)] = (unsigned char)e4m3_encode(ldexpf(elem(c), -e));
  if (j == 0) scales[layer * srows_layer + srow + rb * 16 + r] = ldexpf(1.f, e);
}

__global__ void synth_fill_kernel(uint16_t* __restrict__ dst, unsigned long long n, unsigned long long key,
                                  float c, int add_one) {
  for (unsigned long long i = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (unsigned long long)gridDim.x * blockDim.x)
    dst[i] = synth_bf16(key, i, c, add_one);
}


// Synthetic KV prefill of positions [0, len).  Stream id KV_ID_BASE +
// 2*layer + kv; element index (t * NKV + g) * D + d (matches
// oracle/synth.py:kv_prefill_bits).
__global__ void synth_kv_kernel(uint16_t* __restrict__ kv, uint16_t* __restrict__ kvt, int L, int NKV, int s_pad,
                                int D, int len, unsigned long long seed, float c) {
  const unsigned long long per = (unsigned long long)len * NKV * D;
  const unsigned long long total = per * 2ull * L;
  for (unsigned long long i = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (unsigned long long)gridDim.x * blockDim.x) {
    const unsigned long long plane = i / per;  // layer*2 + kv
    const unsigned long long e = i % per;      // (t*NKV + g)*D + d
    const int d = (int)(e % D);
    const int g = (int)((e / D) % NKV);
    const long long t = (long long)(e / ((unsigned long long)D * NKV));
    const unsigned long long key = sm_h(seed, 0x40000000ull + plane);
    const int l = (int)(plane / 2);
    const uint16_t v = synth_bf16(key, e, c, 0);
    if (plane % 2 == 0) kv[k_index(l, g, t, d, NKV, s_pad, D)] = v;
    else kvt[vt_index(l, g, t, d, NKV, s_pad, D)] = v;
  }
}

// Copy between the reference layout [L][2][NKV][len][D] (buf) and the cache:
// to_cache = 1 imports, 0 exports.
__global__ void kv_convert_kernel(uint16_t* __restrict__ buf, uint16_t* __restrict__ kv, uint16_t* __restrict__ kvt,
                                  int L, int NKV, int s_pad, int D, int len, int to_cache) {
  const unsigned long long total = 2ull * L * NKV * (unsigned long long)len * D;
  for (unsigned long long i = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (unsigned long long)gridDim.x * blockDim.x) {
    const int d = (int)(i % D);
    const long long t = (long long)((i / D) % len);
    const int g = (int)((i / ((unsigned long long)D * len)) % NKV);
    const unsigned long long plane = i / ((unsigned long long)D * len * NKV);  // layer*2 + kv
    const int l = (int)(plane / 2);
    uint16_t* c = plane % 2 == 0 ? kv + k_index(l, g, t, d, NKV, s_pad, D) : kvt + vt_index(l, g, t, d, NKV, s_pad, D);
    if (to_cache) *c = buf[i];
    else buf[i] = *c;
  }
}

// FP8 KV cache (no counterpart in the reference, which plans FP8 KV in
// RESEARCH.md:434-436,463): rows of the reference layout buf [L][2][NKV][len][D]
// (bf16) <-> e4m3 codes at the cache's element indices read as byte indices,
// one power-of-two scale per (layer, kv head, position) row of K and of V.
// Quantisation as the kernel's append: 2^e with the smallest e such that
// max|row| <= 448 * 2^e, codes rounded to nearest even after exact scaling.
__global__ void kv_quant_kernel(const uint16_t* __restrict__ buf, uint8_t* __restrict__ k8, uint8_t* __restrict__ v8,
                                float* __restrict__ ks, float* __restrict__ vs, int L, int NKV, int s_pad, int D,
                                int len) {
  const unsigned long long rows = 2ull * L * NKV * (unsigned long long)len;
  for (unsigned long long r = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x; r < rows;
       r += (unsigned long long)gridDim.x * blockDim.x) {
    const long long t = (long long)(r % len);
    const int g = (int)((r / len) % NKV);
    const unsigned long long plane = r / ((unsigned long long)len * NKV);  // layer*2 + kv
    const int l = (int)(plane / 2), kv = (int)(plane % 2);
    const uint16_t* src = buf + r * D;
    float amax = 0.f;
    for (int d = 0; d < D; ++d) amax = fmaxf(amax, fabsf(bf16_to_f32(src[d])));
    const int e = e4m3_row_exp(amax);
    for (int d = 0; d < D; ++d) {
      const uint8_t code = (uint8_t)e4m3_encode(ldexpf(bf16_to_f32(src[d]), -e));
      if (kv == 0) k8[k_index(l, g, t, d, NKV, s_pad, D)] = code;
      else v8[vt_index(l, g, t, d, NKV, s_pad, D)] = code;
    }
    (kv == 0 ? ks : vs)[((long long)l * NKV + g) * s_pad + t] = ldexpf(1.f, e);
  }
}

// FP8 cache -> reference layout, bf16 of code x scale (exact).
__global__ void kv_dequant_kernel(uint16_t* __restrict__ buf, const uint8_t* __restrict__ k8,
                                  const uint8_t* __restrict__ v8, const float* __restrict__ ks,
                                  const float* __restrict__ vs, int L, int NKV, int s_pad, int D, int len) {
  const unsigned long long total = 2ull * L * NKV * (unsigned long long)len * D;
  for (unsigned long long i = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (unsigned long long)gridDim.x * blockDim.x) {
    const int d = (int)(i % D);
    const long long t = (long long)((i / D) % len);
    const int g = (int)((i / ((unsigned long long)D * len)) % NKV);
    const unsigned long long plane = i / ((unsigned long long)D * len * NKV);
    const int l = (int)(plane / 2), kv = (int)(plane % 2);
    const unsigned code = kv == 0 ? k8[k_index(l, g, t, d, NKV, s_pad, D)] : v8[vt_index(l, g, t, d, NKV, s_pad, D)];
    const float sc = (kv == 0 ? ks : vs)[((long long)l * NKV + g) * s_pad + t];
    buf[i] = f32_to_bf16(__builtin_amdgcn_cvt_pk_f32_fp8((int)code, false)[0] * sc);
  }
}

// Synthetic KV of positions [0, len) in the reference layout (the values of
// synth_kv_kernel).
__global__ void synth_kv_ref_kernel(uint16_t* __restrict__ buf, int L, int NKV, int D, int len,
                                    unsigned long long seed, float c) {
  const unsigned long long per = (unsigned long long)len * NKV * D;
  const unsigned long long total = per * 2ull * L;
  for (unsigned long long i = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (unsigned long long)gridDim.x * blockDim.x) {
    const unsigned long long plane = i / per;
    const unsigned long long e = i % per;  // (t*NKV + g)*D + d
    const int d = (int)(e % D);
    const int g = (int)((e / D) % NKV);
    const long long t = (long long)(e / ((unsigned long long)D * NKV));
    buf[((plane * NKV + g) * (unsigned long long)len + t) * D + d] = synth_bf16(sm_h(seed, 0x40000000ull + plane), e, c, 0);
  }
}

// -------------------------------------------------------------- the handle
struct ShapeInfo {
  int H, NQ, NKV, D, F, QD, KVD, QKV, GQA;
  long long u_layer, off_qkv, off_o, off_gu, off_down;
  int srows_layer, srow_qkv, srow_o, srow_gu, srow_down;  // FP8 row-scale offsets per layer
  int norm_stride, norm_attn, norm_q, norm_k, norm_ffn;
  int part_words;  // words of one attention item's published partial
};

template <class S>
static ShapeInfo shape_info() {
  return ShapeInfo{S::H, S::NQ, S::NKV, S::D, S::F, S::QD, S::KVD, S::QKV, S::GQA,
                   S::U_LAYER, S::OFF_QKV, S::OFF_O, S::OFF_GU, S::OFF_DOWN,
                   S::SROWS_LAYER, S::SROW_QKV, S::SROW_O, S::SROW_GU, S::SROW_DOWN,
                   S::NORM_STRIDE, S::NORM_ATTN, S::NORM_Q, S::NORM_K, S::NORM_FFN, part_words<S>()};
}

// Attention splits per kv head up to which the class kernel has role tables
// (eight splits of eight kv heads: the attention workgroups and the other
// roles of a BASELINE layer just fit 256 workgroups).
constexpr int kMaxClsSplit = 8;
// Largest attention chunk a launch takes to stay in the class kernel (see
// launch_chunk; measured at ctx 4,096: eight splits of 544 positions in the
// class kernel 2,451 tok/s, nine of 512 in the spread kernel 2,261; at 8,192
// eight of 1,088 lose, 1,957 vs 2,104).
constexpr int kClsChunkMax = 640;

// Role table of the class kernel (mk_cls.h) for `nsplit` attention splits
// per kv head on G workgroups: attention items (att_o: each with an O block)
// on workgroups [0, NKV*nsplit) (item (g, s) on workgroup s*NKV + g: XCD g
// for 8 kv heads), then QKV + gate/up pairs with kv head g's QKV blocks on
// XCD g % 8, then gate/up + down, down + O, O (one or two blocks), single
// roles for whatever has no partner.  False when the shape's blocks do not
// fit G workgroups this way.
static bool build_roles_as(const ShapeInfo& s, int G, int nsplit, bool att_o, std::vector<int>& rows) {
  const int NA = s.NKV * nsplit, RBQ = s.QKV / 16, RBF = s.F / 16, RBH = s.H / 16;
  rows.assign((size_t)G * ROLE_INTS, -1);
  for (int w = 0; w < G; ++w) rows[(size_t)w * ROLE_INTS + RF_CLS] = CLS_IDLE;
  auto at = [&](int w, int f) -> int& { return rows[(size_t)w * ROLE_INTS + f]; };
  if (NA > G) return false;
  int w = 0, o = 0;
  for (; w < NA; ++w) {  // attention items, each with an O block while they last (att_o)
    at(w, RF_CLS) = att_o ? CLS_ATT : CLS_A;
    at(w, RF_ATT) = w;
    if (att_o && o < RBH) at(w, RF_O0) = o++;
  }
  // QKV blocks grouped by the XCD of their kv head
  std::vector<int> by_xcd[8];
  for (int b = 0; b < RBQ; ++b) {
    const int row = 16 * b;
    const int g = row < s.QD ? (row / s.D) / s.GQA : (row < s.QD + s.KVD ? (row - s.QD) / s.D : (row - s.QD - s.KVD) / s.D);
    by_xcd[g % 8].push_back(b);
  }
  size_t next_any = 0;
  std::vector<char> used(RBQ, 0);
  auto take_q = [&](int wg) -> int {
    auto& v = by_xcd[wg % 8];
    for (int b : v)
      if (!used[b]) return used[b] = 1, b;
    for (; next_any < (size_t)RBQ; ++next_any)
      if (!used[next_any]) return used[next_any] = 1, (int)next_any;
    return -1;
  };
  const int nqg = RBQ < RBF ? RBQ : RBF;
  if (w + nqg > G) return false;
  for (int i = 0; i < nqg; ++i, ++w) {
    at(w, RF_CLS) = CLS_QG;
    at(w, RF_Q) = take_q(w);
    at(w, RF_G) = i;
  }
  for (int i = nqg; i < RBQ; ++i, ++w) {  // QKV blocks without a gate/up partner
    if (w >= G) return false;
    at(w, RF_CLS) = CLS_Q;
    at(w, RF_Q) = take_q(w);
  }
  int d = 0;
  for (int gi = nqg; gi < RBF; ++gi, ++w) {  // gate/up pairs: with a down block while they last
    if (w >= G) return false;
    at(w, RF_G) = gi;
    if (d < RBH) {
      at(w, RF_CLS) = CLS_DG;
      at(w, RF_D) = d++;
    } else {
      at(w, RF_CLS) = CLS_G;
    }
  }
  for (; d < RBH; ++d, ++w) {  // down blocks: with an O block while they last
    if (w >= G) return false;
    at(w, RF_D) = d;
    if (o < RBH) {
      at(w, RF_CLS) = CLS_DO;
      at(w, RF_O0) = o++;
    } else {
      at(w, RF_CLS) = CLS_D;
    }
  }
  const int rem_o = RBH - o, rem_w = G - w;
  if (rem_o > 2 * rem_w) return false;
  const int two = rem_o > rem_w ? rem_o - rem_w : 0;  // workgroups that take two O blocks
  for (int i = 0; o < RBH; ++i, ++w) {
    at(w, RF_CLS) = CLS_O;
    at(w, RF_O0) = o++;
    if (i < two) at(w, RF_O1) = o++;
  }
  return true;
}

// Attention-only workgroups when the O blocks fit on the other workgroups
// (3,133 -> 3,146 tok/s at ctx 1024, alternating runs), else attention
// workgroups that also take an O block.
static bool build_roles(const ShapeInfo& s, int G, int nsplit, std::vector<int>& rows) {
  return build_roles_as(s, G, nsplit, false, rows) || build_roles_as(s, G, nsplit, true, rows);
}

struct Handle {
  int device = 0, preset = 0, G = 0;
  ShapeInfo sh{};
  int L = 0, V = 0, S = 0;
  int max_launch_tokens = 0;
  int nsplit_max = 1, chunk_min = 256 * KVB;  // one 32-position block per wave and register set
  int chunk_eff = 0;                           // the attention chunk of the last launch (launch_chunk)
  int merge_min = 20;  // above this many splits per kv head the first split's workgroup merges them
  hipStream_t stream = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  float last_ms = 0.f;
  unsigned long long timeout_ticks = 0;
  // device memory (owned)
  u32x4* layers = nullptr;
  uint16_t* norms = nullptr;
  uint16_t* final_norm = nullptr;
  u32x4* lmhead = nullptr;
  u32x4* lmhead8 = nullptr;  // optional FP8 copy of the LM head, built on request
  float* lm_scale = nullptr;
  float* lm_err = nullptr;   // per-row bound of the FP8 rows' error (lmhead_fp8_kernel)
  int lm_mode = MK_LMHEAD_BF16;  // bf16, FP8, or FP8 screening + exact bf16 rescoring
  u32x2* layers8 = nullptr;  // optional FP8 copy of the layer weights (same unit offsets, 8-byte units)
  float* lscale = nullptr;   // its row scales [L][srows_layer]
  bool layer_fp8 = false;    // the class kernel reads layers8
  float *kscale = nullptr, *vscale = nullptr;  // FP8 KV cache: row scales [L][NKV][s_pad]
  bool kv_fp8 = false;       // the cache holds e4m3 codes (byte index = bf16 element index)
  uint16_t* kv = nullptr;
  u64 *x = nullptr, *qkv = nullptr, *part = nullptr, *act = nullptr;
  u64* amax = nullptr;
  size_t tagged_bytes[5] = {0, 0, 0, 0, 0};
  int* out_tokens = nullptr;
  int* err = nullptr;
  int* host_io = nullptr;  // pinned copy of err and out_tokens (same offsets) after a launch
  u64* trace = nullptr;
  float* inv_freq = nullptr;
  float* dbg_layers = nullptr;
  float* dbg_logits = nullptr;
  void* owned_flat = nullptr;
  std::vector<long long> offsets;         // the init offsets (a prefill context built later reuses them)
  batch::BHandle* prefill = nullptr;      // optional prefill context bound to this handle's KV cache
  unsigned tag_base = 1;  // tag of the next launch's first phase (0 never valid)
  int pos = 0;
  long long kv_bytes = 0;
  int s_pad = 0;               // KV capacity rounded up to whole 32-position blocks
  uint16_t* kvt = nullptr;     // V^T region inside the kv allocation
  DecodeLaunch launch = nullptr;
  // class kernel role tables for 1..kMaxClsSplit attention splits per kv head
  // ([kMaxClsSplit][G][ROLE_INTS] ints); roles_ok[k]: a table for k splits exists
  int* roles = nullptr;
  bool roles_ok[kMaxClsSplit + 1] = {};
  int kernel_variant = MK_KERNEL_AUTO;
  bool has_cls = false;  // the preset has class-kernel instantiations
  int pace_pct = 100;  // class kernel prefetch pacing (environment MK_PACE_PCT at init; 0 = bursts)
};

static void free_all(Handle* h) {
  if (h->roles) (void)hipFree(h->roles);
  h->roles = nullptr;
  batch::destroy_prefill_context(h->prefill);
  h->prefill = nullptr;
  // the hand-off words go back to the uncached pool (never freed)
  for (void* q : {(void*)h->x, (void*)h->qkv, (void*)h->part, (void*)h->act, (void*)h->amax}) uc_release(q);
  void* ptrs[] = {h->layers, h->norms, h->final_norm, h->lmhead, h->lmhead8, h->lm_scale, h->lm_err, h->layers8, h->lscale, h->kscale, h->vscale, h->kv,
                  h->err, h->inv_freq, h->dbg_layers,
                  h->dbg_logits, h->trace, h->owned_flat};
  for (void* q : ptrs)
    if (q) (void)hipFree(q);
  if (h->host_io) (void)hipHostFree(h->host_io);
  if (h->ev0) (void)hipEventDestroy(h->ev0);
  if (h->ev1) (void)hipEventDestroy(h->ev1);
  if (h->stream) (void)hipStreamDestroy(h->stream);
}

static int repack(Handle* h, const char* base, long long off, int R, int K, u32x4* dst, int stride,
                  int blk_off) {
  if (off < 0 || (off & 15)) {
    set_err("weight offset %lld is negative or not 16-byte aligned", off);
    return -1;
  }
  const long long units = (long long)R * K / 8;
  const int threads = 256;
  const int blocks = (int)((units + threads - 1) / threads < 65536 ? (units + threads - 1) / threads : 65536);
  hipLaunchKernelGGL(repack_kernel, dim3(blocks), dim3(threads), 0, h->stream,
                     reinterpret_cast<const u32x4*>(base + off), R, K, dst, stride, blk_off);
  HIPCHK(hipGetLastError(), -1);
  return 0;
}

static int init_device_state(Handle* h, const char* base, const long long* off, int n_off) {
  const ShapeInfo& s = h->sh;
  if (n_off < 13 || (n_off - 2) % 11 != 0) {
    set_err("num_offsets=%d is not 2 + 11*layers", n_off);
    return -1;
  }
  h->L = (n_off - 2) / 11;
  if (h->V <= 0 || h->V % 16 || h->V > (int)IDX_MAX + 1) {
    set_err("vocab %d must be a positive multiple of 16 and at most %u", h->V, IDX_MAX + 1);
    return -1;
  }
  HIPCHK(hipGetDevice(&h->device), -1);
  hipDeviceProp_t prop;
  HIPCHK(hipGetDeviceProperties(&prop, h->device), -1);
  h->G = prop.multiProcessorCount;
  int wall_khz = 0;
  HIPCHK(hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, h->device), -1);
  h->timeout_ticks = (unsigned long long)(wall_khz > 0 ? wall_khz : 100000) * 10000ull;  // 10 s
  h->nsplit_max = h->G / s.NKV > 0 ? h->G / s.NKV : 1;
  if (h->nsplit_max > NSPLIT_CAP) h->nsplit_max = NSPLIT_CAP;
  HIPCHK(hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking), -1);
  HIPCHK(hipEventCreate(&h->ev0), -1);
  HIPCHK(hipEventCreate(&h->ev1), -1);

  const long long layer_bytes = s.u_layer * 16;
  HIPCHK(hipMalloc(&h->layers, layer_bytes * h->L), -1);
  HIPCHK(hipMalloc(&h->norms, (size_t)s.norm_stride * 2 * h->L), -1);
  HIPCHK(hipMalloc(&h->final_norm, (size_t)s.H * 2), -1);
  HIPCHK(hipMalloc(&h->lmhead, (size_t)h->V * s.H * 2), -1);
  h->s_pad = (h->S + 31) / 32 * 32;
  h->kv_bytes = 2LL * h->L * s.NKV * (long long)h->s_pad * s.D * 2;
  HIPCHK(hipMalloc(&h->kv, h->kv_bytes), -1);
  h->kvt = h->kv + (long long)h->L * s.NKV * h->s_pad * s.D;
  HIPCHK(hipMemsetAsync(h->kv, 0, h->kv_bytes, h->stream), -1);
  // tagged activation words (zero = tag 0, never a valid tag)
  u64** tagged[5] = {&h->x, &h->qkv, &h->part, &h->act, &h->amax};
  // part: the splits' partials, then one row for a long context's merged partial
  const size_t words[5] = {(size_t)s.H / 2, (size_t)s.QKV,
                           (size_t)(h->nsplit_max + 1) * s.NKV * s.part_words, (size_t)s.F / 2,
                           (size_t)4 * h->G};  // amax: [2][G] argmax words, then [2][G] screening thresholds
  for (int i = 0; i < 5; ++i) {
    h->tagged_bytes[i] = words[i] * 8;
    *tagged[i] = static_cast<u64*>(uc_acquire(h->device, h->tagged_bytes[i]));
    if (!*tagged[i]) {
      set_err("uncached device allocation of %zu bytes failed", h->tagged_bytes[i]);
      return -1;
    }
    HIPCHK(hipMemsetAsync(*tagged[i], 0, h->tagged_bytes[i], h->stream), -1);
  }
  // role tables of the class kernel (kept on the device; a launch points at one)
  {
    std::vector<int> all((size_t)kMaxClsSplit * h->G * ROLE_INTS, 0), one;
    for (int k = 1; k <= kMaxClsSplit; ++k) {
      h->roles_ok[k] = build_roles(s, h->G, k, one);
      if (h->roles_ok[k]) std::copy(one.begin(), one.end(), all.begin() + (size_t)(k - 1) * h->G * ROLE_INTS);
    }
    HIPCHK(hipMalloc(&h->roles, all.size() * sizeof(int)), -1);
    HIPCHK(hipMemcpyAsync(h->roles, all.data(), all.size() * sizeof(int), hipMemcpyHostToDevice, h->stream), -1);
    HIPCHK(hipStreamSynchronize(h->stream), -1);
  }
  h->max_launch_tokens = 1 << 20;
  HIPCHK(hipMalloc(&h->trace, ((size_t)(5 * h->L + 1) * 2 + EVT_N) * h->G * 8), -1);
  // error word (256 bytes), then the output tokens: one copy brings both back
  HIPCHK(hipMalloc(&h->err, 256 + (size_t)h->max_launch_tokens * 4), -1);
  h->out_tokens = h->err + 64;
  HIPCHK(hipHostMalloc(reinterpret_cast<void**>(&h->host_io), 256 + (size_t)h->max_launch_tokens * 4), -1);
  HIPCHK(hipMemsetAsync(h->err, 0, 256, h->stream), -1);
  HIPCHK(hipMalloc(&h->dbg_layers, (size_t)(h->L + 1) * s.H * 4), -1);
  HIPCHK(hipMalloc(&h->dbg_logits, (size_t)h->V * 4), -1);

  // RoPE inverse frequencies, computed as HF does in fp32:
  // 1 / theta ** (float(2i) / D)  (transformers Qwen3RotaryEmbedding).
  std::vector<float> invf(s.D / 2);
  for (int i = 0; i < s.D / 2; ++i) invf[i] = 1.0f / powf((float)kRopeTheta, (float)(2 * i) / (float)s.D);
  HIPCHK(hipMalloc(&h->inv_freq, invf.size() * 4), -1);
  HIPCHK(hipMemcpyAsync(h->inv_freq, invf.data(), invf.size() * 4, hipMemcpyHostToDevice, h->stream), -1);

  // Repack matrices (offset order: reference megakernel.cu:518-532).
  const int KTH = s.H / 32;
  if (repack(h, base, off[0], h->V, s.H, h->lmhead, 1, 0)) return -1;
  HIPCHK(hipMemcpyAsync(h->final_norm, base + off[1], (size_t)s.H * 2, hipMemcpyDeviceToDevice, h->stream), -1);
  for (int i = 0; i < h->L; ++i) {
    const long long* o = off + 2 + 11 * i;
    u32x4* wl = h->layers + (long long)i * s.u_layer;
    uint16_t* nl = h->norms + (long long)i * s.norm_stride;
    HIPCHK(hipMemcpyAsync(nl + s.norm_attn, base + o[0], (size_t)s.H * 2, hipMemcpyDeviceToDevice, h->stream), -1);
    HIPCHK(hipMemcpyAsync(nl + s.norm_q, base + o[4], (size_t)s.D * 2, hipMemcpyDeviceToDevice, h->stream), -1);
    HIPCHK(hipMemcpyAsync(nl + s.norm_k, base + o[5], (size_t)s.D * 2, hipMemcpyDeviceToDevice, h->stream), -1);
    HIPCHK(hipMemcpyAsync(nl + s.norm_ffn, base + o[7], (size_t)s.H * 2, hipMemcpyDeviceToDevice, h->stream), -1);
    u32x4* qkv = wl + s.off_qkv;
    if (repack(h, base, o[1], s.QD, s.H, qkv, 1, 0)) return -1;
    if (repack(h, base, o[2], s.KVD, s.H, qkv, 1, s.QD / 16)) return -1;
    if (repack(h, base, o[3], s.KVD, s.H, qkv, 1, (s.QD + s.KVD) / 16)) return -1;
    if (repack(h, base, o[6], s.H, s.QD, wl + s.off_o, 1, 0)) return -1;
    if (repack(h, base, o[8], s.F, s.H, wl + s.off_gu, 2, 0)) return -1;
    if (repack(h, base, o[9], s.F, s.H, wl + s.off_gu, 2, 1)) return -1;
    if (repack(h, base, o[10], s.H, s.F, wl + s.off_down, 1, 0)) return -1;
  }
  (void)KTH;
  HIPCHK(hipStreamSynchronize(h->stream), -1);
  return 0;
}

static Handle* create(int preset, int vocab, int max_seq) {
  Handle* h = new (std::nothrow) Handle();
  if (!h) {
    set_err("out of host memory");
    return nullptr;
  }
  h->preset = preset;
  h->V = vocab;
  h->S = max_seq;
  if (const char* e = getenv("MK_PACE_PCT")) h->pace_pct = atoi(e) < 0 ? 0 : atoi(e);
  switch (preset) {
    case PRESET_BASELINE:
      h->sh = shape_info<ShapeBaseline>();
      h->launch = launch_decode_baseline;
      h->has_cls = true;
      break;
    case PRESET_QWEN3_06B:
      h->sh = shape_info<ShapeQwen3>();
      h->launch = launch_decode_qwen3;
      break;
    case PRESET_TINY:
      h->sh = shape_info<ShapeTiny>();
      h->launch = launch_decode_tiny;
      h->has_cls = true;
      break;
    default:
      set_err("unknown preset %d", preset);
      delete h;
      return nullptr;
  }
  if (max_seq <= 0) {
    set_err("max_seq must be positive");
    delete h;
    return nullptr;
  }
  return h;
}

static int check_occupancy(Handle* h) {
  int nblk = 0;
  switch (h->preset) {
    case PRESET_BASELINE: nblk = occupancy_decode_baseline(); break;
    case PRESET_QWEN3_06B: nblk = occupancy_decode_qwen3(); break;
    default: nblk = occupancy_decode_tiny(); break;
  }
  if (nblk < 1) {
    set_err("persistent kernel cannot keep one workgroup resident per CU (occupancy %d)", nblk);
    return -1;
  }
  return 0;
}

// Clear every tagged word (tag 0 is never expected) and the error word.
static int clear_tagged_state(Handle* h) {
  u64* bufs[5] = {h->x, h->qkv, h->part, h->act, h->amax};
  for (int i = 0; i < 5; ++i) HIPCHK(hipMemsetAsync(bufs[i], 0, h->tagged_bytes[i], h->stream), -1);
  HIPCHK(hipMemsetAsync(h->err, 0, 256, h->stream), -1);
  HIPCHK(hipStreamSynchronize(h->stream), -1);
  return 0;
}

// The packed-pair words (x, part, act) carry 4-bit tags, so a stale word can
// look current when its tag is a multiple of 15 phases old.  While the
// position only grows and the split configuration is fixed, that never
// happens: every act word and every active split slot is rewritten at each
// layer (5 phases apart, 6 across a token boundary), and split counts never
// shrink, so a slot that becomes active still holds zeros.  A position that
// moves backwards, a new cache, or a new split / merge configuration breaks
// that, and clears them.  x needs no such clear: its words are rewritten twice
// a layer (after O and after down, 2 and 3 phases apart; the tag sequence
// runs on across launches), and every reader of x depends on a phase that
// consumed the whole previous-layer x, so it waits for a write 2 to 6 phases
// after the word's current one -- never a multiple of 15.
static int clear_pair_words(Handle* h) {
  HIPCHK(hipMemsetAsync(h->part, 0, h->tagged_bytes[2], h->stream), -1);
  HIPCHK(hipMemsetAsync(h->act, 0, h->tagged_bytes[3], h->stream), -1);
  HIPCHK(hipStreamSynchronize(h->stream), -1);
  return 0;
}

// The attention chunk of a launch whose last token sits at position end - 1:
// the handle's, or, when that needs more splits per kv head than the class
// kernel's role tables hold while a chunk of at most kClsChunkMax positions
// would not, the smallest multiple of 32 positions that gives kMaxClsSplit
// splits (a few longer splits in the class kernel beat more splits in the
// spread kernel).
static int launch_chunk(const Handle* h, int end) {
  const int c = h->chunk_min;
  if (!h->has_cls || h->kernel_variant != MK_KERNEL_AUTO || !h->roles_ok[kMaxClsSplit] ||
      split_count(end, c, h->nsplit_max) <= kMaxClsSplit)
    return c;
  const int c8 = ((end + kMaxClsSplit - 1) / kMaxClsSplit + 31) / 32 * 32;
  return c8 > c && c8 <= kClsChunkMax ? c8 : c;
}

// One resident launch decoding n tokens starting at h->pos.
static int run(Handle* h, int first_token, int n, int* out_host, bool debug, int trace_token = -1) {
  if (n <= 0 || n > h->max_launch_tokens) {
    set_err("token count %d outside [1, %d]", n, h->max_launch_tokens);
    return -1;
  }
  if (first_token < 0 || first_token >= h->V) {
    set_err("token id %d outside [0, %d)", first_token, h->V);
    return -1;
  }
  if (h->pos + n > h->S) {
    set_err("position %d + %d tokens exceeds KV capacity %d", h->pos, n, h->S);
    return -1;
  }
  Params p{};
  p.layers = h->layers;
  p.norms = h->norms;
  p.final_norm = h->final_norm;
  p.lmhead = h->lmhead;
  p.lmhead8 = h->lm_mode != MK_LMHEAD_BF16 ? h->lmhead8 : nullptr;
  p.lm_scale = h->lm_mode != MK_LMHEAD_BF16 ? h->lm_scale : nullptr;
  p.lm_err = nullptr;
  p.layers8 = h->layer_fp8 ? h->layers8 : nullptr;
  p.lscale = h->layer_fp8 ? h->lscale : nullptr;
  p.kscale = h->kv_fp8 ? h->kscale : nullptr;
  p.vscale = h->kv_fp8 ? h->vscale : nullptr;
  p.kv = h->kv;
  p.kvt = h->kvt;
  p.s_pad = h->s_pad;
  const unsigned per_token = (unsigned)(5 * h->L + 1);
  if ((unsigned long long)h->tag_base + (unsigned long long)n * per_token >= 0x7fffffffull) {
    if (clear_tagged_state(h)) return -1;  // restart the tag sequence well before it wraps
    h->tag_base = 1;
  }
  p.x = h->x;
  p.qkv = h->qkv;
  p.part = h->part;
  p.act = h->act;
  p.amax = h->amax;
  p.out_tokens = h->out_tokens;
  p.err = h->err;
  p.trace = trace_token >= 0 ? h->trace : nullptr;
  p.trace_token = trace_token;
  p.trace_layer = h->L / 2;
  p.dbg_layers = debug ? h->dbg_layers : nullptr;
  p.dbg_logits = debug ? h->dbg_logits : nullptr;
  p.inv_freq = h->inv_freq;
  p.timeout_ticks = h->timeout_ticks;
  p.tag_base = h->tag_base;
  p.n_layers = h->L;
  p.vocab = h->V;
  p.max_seq = h->S;
  p.pos0 = h->pos;
  p.n_tokens = n;
  p.first_token = first_token;
  p.nsplit_max = h->nsplit_max;
  // a new split layout starts from cleared pair words (their 4-bit tags are
  // only unambiguous while a layout's split counts grow)
  const int chunk = launch_chunk(h, h->pos + n);
  if (chunk != h->chunk_eff) {
    if (clear_pair_words(h)) return -1;
    h->chunk_eff = chunk;
  }
  p.chunk_min = chunk;
  p.merge_min = h->merge_min;
  p.pace_pct = h->pace_pct;
  HIPCHK(hipEventRecord(h->ev0, h->stream), -1);
  // the long-context instantiation when the launch's last token has more
  // than merge_min splits per kv head (split counts grow with the position)
  const int ns_last = split_count(h->pos + n, chunk, h->nsplit_max);
  const bool lc = ns_last > h->merge_min;
  // the class kernel when a role table holds every attention item of the
  // launch (its attention workgroups serve the last token's split count)
  const bool cls =
      h->has_cls && h->kernel_variant == MK_KERNEL_AUTO && !lc && ns_last <= kMaxClsSplit && h->roles_ok[ns_last];
  p.roles = cls ? h->roles + (size_t)(ns_last - 1) * h->G * ROLE_INTS : nullptr;
  if (h->lm_mode == MK_LMHEAD_SCREENED) {
    // the screened LM head runs in the class kernel, and not for validation
    // outputs (they report every row's bf16 logit); elsewhere the bf16 head
    // gives the same tokens
    if (cls && !p.dbg_logits && (h->V / 16 + h->G - 1) / h->G * 16 <= LM_ROWS_MAX) {
      p.lm_err = h->lm_err;
    } else {
      p.lmhead8 = nullptr;
      p.lm_scale = nullptr;
    }
  }
  if (h->layer_fp8 && !cls) {
    set_err("FP8 layer weights need the class kernel (automatic variant, at most %d attention splits per kv head; "
            "this launch needs %d)", kMaxClsSplit, ns_last);
    return -1;
  }
  HIPCHK(h->launch(h->G, h->stream, p, lc, cls), -1);
  HIPCHK(hipEventRecord(h->ev1, h->stream), -1);
  // error word and tokens come back in one copy into pinned memory
  HIPCHK(hipMemcpyAsync(h->host_io, h->err, 256 + (out_host ? (size_t)n * 4 : 0), hipMemcpyDeviceToHost, h->stream),
         -1);
  HIPCHK(hipStreamSynchronize(h->stream), -1);
  HIPCHK(hipEventElapsedTime(&h->last_ms, h->ev0, h->ev1), -1);
  const int err = h->host_io[0];
  h->tag_base += (unsigned)n * per_token;  // tags of this launch are never expected again
  if (err != MK_OK) {
    clear_tagged_state(h);
    set_err("decode kernel aborted: %s", err == MK_ERR_TIMEOUT ? "a dataflow wait timed out" : "device error");
    return -1;
  }
  if (out_host) memcpy(out_host, h->host_io + 64, (size_t)n * 4);
  h->pos += n;
  return 0;
}

// Byte sizes of the tensors of one layer of shape S, in the reference's offset
// order (attn_norm, w_q, w_k, w_v, q_norm, k_norm, w_o, ffn_norm, w_gate, w_up,
// w_down; /root/reference/host/weight_loader.py:141-192, bridge.py:86-93).
template <class S>
static void layer_tensor_bytes(long long b[11]) {
  const long long H = S::H, QD = S::QD, KVD = S::KVD, D = S::D, F = S::F;
  const long long v[11] = {H, QD * H, KVD * H, KVD * H, D, D, H * QD, H, F * H, F * H, H * F};
  for (int i = 0; i < 11; ++i) b[i] = 2 * v[i];
}

template <class S>
static bool contiguous_for(const long long* off, int n_off, int* vocab) {
  if (n_off < 13 || (n_off - 2) % 11 != 0) return false;
  long long b[11];
  layer_tensor_bytes<S>(b);
  const long long emb = off[1] - off[0];
  if (emb <= 0 || emb % (2LL * S::H) != 0 || off[2] - off[1] != 2LL * S::H) return false;
  const int L = (n_off - 2) / 11;
  for (int l = 0; l < L; ++l) {
    const long long* o = off + 2 + 11 * l;
    for (int k = 0; k < 10; ++k)
      if (o[k + 1] - o[k] != b[k]) return false;
    if (l + 1 < L && o[11] - o[10] != b[10]) return false;
  }
  *vocab = (int)(emb / (2LL * S::H));
  return true;
}

// The preset (and vocabulary) whose contiguous weights.bin the offsets
// describe exactly -- the file the reference's weight loader writes -- or -1.
static int contiguous_preset(const long long* off, int n_off, int* vocab) {
  if (contiguous_for<ShapeBaseline>(off, n_off, vocab)) return PRESET_BASELINE;
  if (contiguous_for<ShapeQwen3>(off, n_off, vocab)) return PRESET_QWEN3_06B;
  if (contiguous_for<ShapeTiny>(off, n_off, vocab)) return PRESET_TINY;
  return -1;
}

static const char* preset_name(int p) {
  return p == PRESET_BASELINE ? "BASELINE (head_dim 64, ffn 2816)"
                              : p == PRESET_QWEN3_06B ? "QWEN3_06B (head_dim 128, ffn 3072)" : "TINY";
}

// Tensors of a non-contiguous layout must not overlap at the preset's sizes
// (a preset larger than the file's tensors would read into its neighbours).
template <class S>
static bool disjoint_for(const long long* off, int n_off, int vocab) {
  std::vector<std::pair<long long, long long>> iv;
  iv.reserve(n_off);
  long long b[11];
  layer_tensor_bytes<S>(b);
  iv.push_back({off[0], 2LL * vocab * S::H});
  iv.push_back({off[1], 2LL * S::H});
  for (int i = 2; i < n_off; ++i) iv.push_back({off[i], b[(i - 2) % 11]});
  std::sort(iv.begin(), iv.end());
  for (size_t i = 1; i < iv.size(); ++i)
    if (iv[i - 1].first + iv[i - 1].second > iv[i].first) return false;
  return true;
}

static bool disjoint(int preset, const long long* off, int n_off, int vocab) {
  switch (preset) {
    case PRESET_BASELINE: return disjoint_for<ShapeBaseline>(off, n_off, vocab);
    case PRESET_QWEN3_06B: return disjoint_for<ShapeQwen3>(off, n_off, vocab);
    default: return disjoint_for<ShapeTiny>(off, n_off, vocab);
  }
}

// preset < 0: infer preset and vocabulary from the offsets (the reference's
// megakernel_init passes no shape).  An explicit preset must agree with what
// a contiguous file's offsets imply.
static Handle* init_common(const void* d_weights, const long long* offsets, int n_off, int preset, int vocab,
                           int max_seq, void* owned) {
  if (!d_weights || !offsets) {
    set_err("null weights or offsets");
    return nullptr;
  }
  if (n_off < 13 || (n_off - 2) % 11 != 0) {
    set_err("num_offsets=%d is not 2 + 11*layers", n_off);
    return nullptr;
  }
  int inf_vocab = 0;
  const int inf = contiguous_preset(offsets, n_off, &inf_vocab);
  if (preset < 0) {
    if (inf < 0) {
      set_err("offsets do not describe a contiguous weights.bin of a supported shape (BASELINE, QWEN3_06B, TINY); "
              "use megakernel_init_ex with an explicit preset");
      return nullptr;
    }
    preset = inf;
    vocab = inf_vocab;
  } else if (inf >= 0 && (inf != preset || inf_vocab != vocab)) {
    set_err("offsets describe a %s file with vocab %d, not preset %s with vocab %d", preset_name(inf), inf_vocab,
            preset_name(preset), vocab);
    return nullptr;
  } else if (inf < 0 && (preset == PRESET_BASELINE || preset == PRESET_QWEN3_06B || preset == PRESET_TINY) &&
             vocab > 0 && !disjoint(preset, offsets, n_off, vocab)) {
    set_err("tensors overlap at the sizes of preset %s with vocab %d", preset_name(preset), vocab);
    return nullptr;
  }
  Handle* h = create(preset, vocab, max_seq);
  if (!h) return nullptr;
  h->owned_flat = owned;
  if (n_off > 0) h->offsets.assign(offsets, offsets + n_off);
  if (check_occupancy(h) || init_device_state(h, static_cast<const char*>(d_weights), offsets, n_off)) {
    h->owned_flat = nullptr;  // the caller still owns (and frees) the uploaded copy
    free_all(h);
    delete h;
    return nullptr;
  }
  return h;
}

}  // namespace mk

using mk::Handle;

// =========================================================================
// C ABI
// =========================================================================
extern "C" {

void* megakernel_init(void* d_weights, long long* offsets, int num_offsets) {
  // shape and vocabulary from the offsets of the reference's contiguous file
  return mk::init_common(d_weights, offsets, num_offsets, -1, 0, MK_DEFAULT_MAX_SEQ, nullptr);
}

int megakernel_decode(void* handle, int input_token) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) {
    mk::set_err("null handle");
    return -1;
  }
  int out = -1;
  if (mk::run(h, input_token, 1, &out, false)) return -1;
  return out;
}

void megakernel_reset(void* handle) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) return;
  (void)hipMemsetAsync(h->kv, 0, h->kv_bytes, h->stream);
  if (h->kscale) {
    const size_t sb = (size_t)h->L * h->sh.NKV * h->s_pad * 4;
    (void)hipMemsetAsync(h->kscale, 0, sb, h->stream);
    (void)hipMemsetAsync(h->vscale, 0, sb, h->stream);
  }
  (void)mk::clear_pair_words(h);
  h->pos = 0;
}

int megakernel_get_pos(void* handle) {
  Handle* h = static_cast<Handle*>(handle);
  return h ? h->pos : -1;
}

void megakernel_free(void* handle) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) return;
  (void)hipStreamSynchronize(h->stream);
  mk::free_all(h);
  delete h;
}

void megakernel_sync(void) { (void)hipDeviceSynchronize(); }

// ------------------------------------------------------------- extensions
const char* megakernel_last_error(void) { return mk::g_err; }

void* megakernel_init_ex(void* d_weights, const long long* offsets, int num_offsets, int preset, int vocab,
                         int max_seq) {
  return mk::init_common(d_weights, offsets, num_offsets, preset, vocab, max_seq, nullptr);
}

void* megakernel_init_from_host(const void* host_weights, unsigned long long nbytes, const long long* offsets,
                                int num_offsets, int preset, int vocab, int max_seq) {
  if (!host_weights || nbytes == 0) {
    mk::set_err("null or empty host weight buffer");
    return nullptr;
  }
  void* d = nullptr;
  hipError_t e = hipMalloc(&d, nbytes);
  if (e != hipSuccess) {
    mk::set_err("hipMalloc(%llu) failed: %s", nbytes, hipGetErrorString(e));
    return nullptr;
  }
  e = hipMemcpy(d, host_weights, nbytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    mk::set_err("weight upload failed: %s", hipGetErrorString(e));
    (void)hipFree(d);
    return nullptr;
  }
  void* h = mk::init_common(d, offsets, num_offsets, preset, vocab, max_seq, d);
  if (!h) (void)hipFree(d);
  return h;
}

int megakernel_generate(void* handle, int first_token, int n, int* out_tokens) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) {
    mk::set_err("null handle");
    return -1;
  }
  return mk::run(h, first_token, n, out_tokens, false);
}

int megakernel_debug_forward(void* handle, int token, float* layers_out, float* logits_out) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) {
    mk::set_err("null handle");
    return -1;
  }
  int out = -1;
  if (mk::run(h, token, 1, &out, true)) return -1;
  if (layers_out &&
      hipMemcpy(layers_out, h->dbg_layers, (size_t)(h->L + 1) * h->sh.H * 4, hipMemcpyDeviceToHost) != hipSuccess) {
    mk::set_err("debug copy failed");
    return -1;
  }
  if (logits_out && hipMemcpy(logits_out, h->dbg_logits, (size_t)h->V * 4, hipMemcpyDeviceToHost) != hipSuccess) {
    mk::set_err("debug copy failed");
    return -1;
  }
  return out;
}

int megakernel_set_pos(void* handle, int pos) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || pos < 0 || pos > h->S) {
    mk::set_err("invalid handle or position %d", pos);
    return -1;
  }
  if (pos < h->pos && mk::clear_pair_words(h)) return -1;
  h->pos = pos;
  return 0;
}

// Converts through a device staging buffer in the reference layout.
static int kv_transfer(Handle* h, void* host_kv, int len, int to_cache) {
  const size_t bytes = (size_t)2 * h->L * h->sh.NKV * (size_t)len * h->sh.D * 2;
  void* stage = nullptr;
  HIPCHK(hipMalloc(&stage, bytes), -1);
  int rc = -1;
  do {
    if (to_cache && hipMemcpy(stage, host_kv, bytes, hipMemcpyHostToDevice) != hipSuccess) {
      mk::set_err("KV upload failed");
      break;
    }
    if (h->kv_fp8 && to_cache)
      hipLaunchKernelGGL(mk::kv_quant_kernel, dim3(2048), dim3(256), 0, h->stream, static_cast<uint16_t*>(stage),
                         reinterpret_cast<uint8_t*>(h->kv), reinterpret_cast<uint8_t*>(h->kvt), h->kscale, h->vscale,
                         h->L, h->sh.NKV, h->s_pad, h->sh.D, len);
    else if (h->kv_fp8)
      hipLaunchKernelGGL(mk::kv_dequant_kernel, dim3(2048), dim3(256), 0, h->stream, static_cast<uint16_t*>(stage),
                         reinterpret_cast<const uint8_t*>(h->kv), reinterpret_cast<const uint8_t*>(h->kvt), h->kscale,
                         h->vscale, h->L, h->sh.NKV, h->s_pad, h->sh.D, len);
    else
      hipLaunchKernelGGL(mk::kv_convert_kernel, dim3(2048), dim3(256), 0, h->stream, static_cast<uint16_t*>(stage),
                         h->kv, h->kvt, h->L, h->sh.NKV, h->s_pad, h->sh.D, len, to_cache);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(h->stream) != hipSuccess) {
      mk::set_err("KV layout conversion failed");
      break;
    }
    if (!to_cache && hipMemcpy(host_kv, stage, bytes, hipMemcpyDeviceToHost) != hipSuccess) {
      mk::set_err("KV download failed");
      break;
    }
    rc = 0;
  } while (0);
  (void)hipFree(stage);
  return rc;
}

int megakernel_set_kv(void* handle, const void* host_kv, int len) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || !host_kv || len < 0 || len > h->S) {
    mk::set_err("invalid set_kv arguments (len %d)", len);
    return -1;
  }
  if (len > 0 && kv_transfer(h, const_cast<void*>(host_kv), len, 1)) return -1;
  if (mk::clear_pair_words(h)) return -1;
  h->pos = len;
  return 0;
}

int megakernel_get_kv(void* handle, void* host_kv, int len) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || !host_kv || len < 0 || len > h->S) {
    mk::set_err("invalid get_kv arguments (len %d)", len);
    return -1;
  }
  if (len > 0 && kv_transfer(h, host_kv, len, 0)) return -1;
  return 0;
}

int megakernel_fill_kv_synthetic(void* handle, int len, unsigned long long seed, float std) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || len < 0 || len > h->S) {
    mk::set_err("invalid fill_kv arguments (len %d)", len);
    return -1;
  }
  if (len > 0 && h->kv_fp8) {  // the bf16 values in the reference layout, then quantised rows
    const float c = (float)(std * sqrt(3.0) / 65536.0);
    void* stage = nullptr;
    HIPCHK(hipMalloc(&stage, (size_t)2 * h->L * h->sh.NKV * (size_t)len * h->sh.D * 2), -1);
    hipLaunchKernelGGL(mk::synth_kv_ref_kernel, dim3(4096), dim3(256), 0, h->stream, static_cast<uint16_t*>(stage),
                       h->L, h->sh.NKV, h->sh.D, len, seed, c);
    hipLaunchKernelGGL(mk::kv_quant_kernel, dim3(2048), dim3(256), 0, h->stream, static_cast<const uint16_t*>(stage),
                       reinterpret_cast<uint8_t*>(h->kv), reinterpret_cast<uint8_t*>(h->kvt), h->kscale, h->vscale,
                       h->L, h->sh.NKV, h->s_pad, h->sh.D, len);
    const hipError_t e = hipGetLastError() == hipSuccess ? hipStreamSynchronize(h->stream) : hipErrorLaunchFailure;
    (void)hipFree(stage);
    if (e != hipSuccess) {
      mk::set_err("FP8 KV fill failed: %s", hipGetErrorString(e));
      return -1;
    }
  } else if (len > 0) {
    const float c = (float)(std * sqrt(3.0) / 65536.0);
    hipLaunchKernelGGL(mk::synth_kv_kernel, dim3(4096), dim3(256), 0, h->stream, h->kv, h->kvt, h->L, h->sh.NKV,
                       h->s_pad, h->sh.D, len, seed, c);
    HIPCHK(hipGetLastError(), -1);
    HIPCHK(hipStreamSynchronize(h->stream), -1);
  }
  if (mk::clear_pair_words(h)) return -1;
  h->pos = len;
  return 0;
}

int megakernel_trace_generate(void* handle, int first_token, int n, int trace_token,
                              unsigned long long* host_trace) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || !host_trace || trace_token < 0 || trace_token >= n) {
    mk::set_err("invalid trace arguments");
    return -1;
  }
  if (h->L > mk::TRACE_MAX_LAYERS) {
    mk::set_err("tracing supports at most 48 layers");
    return -1;
  }
  const size_t bytes = ((size_t)(5 * h->L + 1) * 2 + mk::EVT_N) * h->G * 8;
  if (hipMemsetAsync(h->trace, 0, bytes, h->stream) != hipSuccess) {
    mk::set_err("trace clear failed");
    return -1;
  }
  if (mk::run(h, first_token, n, nullptr, false, trace_token)) return -1;
  if (hipMemcpy(host_trace, h->trace, bytes, hipMemcpyDeviceToHost) != hipSuccess) {
    mk::set_err("trace copy failed");
    return -1;
  }
  return ((5 * h->L + 1) * 2 + mk::EVT_N) * h->G;
}

float megakernel_last_kernel_ms(void* handle) {
  Handle* h = static_cast<Handle*>(handle);
  return h ? h->last_ms : -1.f;
}

int megakernel_grid_size(void* handle) {
  Handle* h = static_cast<Handle*>(handle);
  return h ? h->G : -1;
}

int megakernel_prefill_attach(void* handle, void* d_weights, const long long* offsets, int num_offsets) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) {
    mk::set_err("null handle");
    return -1;
  }
  if (h->prefill) return 0;
  const char* w = static_cast<const char*>(d_weights);
  if (!w) {  // the library's own upload (megakernel_init_from_host) with the init offsets
    if (!h->owned_flat) {
      mk::set_err("prefill_attach: no weight buffer (pass the flat device weights given to init)");
      return -1;
    }
    w = static_cast<const char*>(h->owned_flat);
    offsets = h->offsets.data();
    num_offsets = (int)h->offsets.size();
  }
  if (!offsets || num_offsets != (int)h->offsets.size()) {
    mk::set_err("prefill_attach: %d offsets, the handle was built from %zu", num_offsets, h->offsets.size());
    return -1;
  }
  h->prefill = mk::batch::create_prefill_context(h->preset, h->V, h->S, w, offsets, num_offsets, h->kv, h->kvt);
  return h->prefill ? 0 : -1;
}

int megakernel_prefill(void* handle, const int* tokens, int n, int* next_token) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || !tokens) {
    mk::set_err("null handle or tokens");
    return -1;
  }
  if (!h->prefill) {
    mk::set_err("prefill: no prefill context (call megakernel_prefill_attach)");
    return -1;
  }
  if (mk::batch::prefill_context_run(h->prefill, tokens, n, h->pos, next_token, nullptr,
                                     h->kv_fp8 ? h->kscale : nullptr, h->kv_fp8 ? h->vscale : nullptr)) return -1;
  h->pos += n;
  h->last_ms = mk::batch::prefill_context_ms(h->prefill);
  return 0;
}

int megakernel_set_attention_merge(void* handle, int merge_min) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || merge_min < 1) {
    mk::set_err("attention merge threshold %d must be >= 1", merge_min);
    return -1;
  }
  if (merge_min != h->merge_min && mk::clear_pair_words(h)) return -1;
  h->merge_min = merge_min;
  return 0;
}

int megakernel_set_decode_kernel(void* handle, int variant) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) {
    mk::set_err("null handle");
    return -1;
  }
  if (variant != MK_KERNEL_AUTO && variant != MK_KERNEL_SPREAD) {
    mk::set_err("unknown decode kernel variant %d", variant);
    return -1;
  }
  h->kernel_variant = variant;
  return 0;
}

int megakernel_decode_kernel_for(void* handle, int n_tokens) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || n_tokens < 1) {
    mk::set_err("null handle or token count < 1");
    return -1;
  }
  const int ns = mk::split_count(h->pos + n_tokens, mk::launch_chunk(h, h->pos + n_tokens), h->nsplit_max);
  const bool cls = h->has_cls && h->kernel_variant == MK_KERNEL_AUTO && ns <= h->merge_min &&
                   ns <= mk::kMaxClsSplit && h->roles_ok[ns];
  return cls ? MK_KERNEL_CLASS : MK_KERNEL_SPREAD;
}

int megakernel_set_attention_chunk(void* handle, int chunk_min) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || chunk_min < 1) {
    mk::set_err("attention chunk %d must be >= 1", chunk_min);
    return -1;
  }
  if (chunk_min != h->chunk_min && mk::clear_pair_words(h)) return -1;
  h->chunk_min = chunk_min;
  return 0;
}

int megakernel_set_lmhead_fp8(void* handle, int enable) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) {
    mk::set_err("null handle");
    return -1;
  }
  if (enable < MK_LMHEAD_BF16 || enable > MK_LMHEAD_SCREENED) {
    mk::set_err("unknown LM head mode %d", enable);
    return -1;
  }
  if (enable && !h->lmhead8) {
    const int K = h->sh.H;
    if (h->V % 16 || K % 64) {
      mk::set_err("FP8 LM head needs vocab %% 16 == 0 and hidden %% 64 == 0 (vocab %d, hidden %d)", h->V, K);
      return -1;
    }
    HIPCHK(hipMalloc(&h->lmhead8, (size_t)h->V * K), -1);
    HIPCHK(hipMalloc(&h->lm_scale, (size_t)h->V * 4), -1);
    HIPCHK(hipMalloc(&h->lm_err, (size_t)h->V * 4), -1);
    hipLaunchKernelGGL(mk::lmhead_fp8_kernel, dim3(h->V / 16), dim3(256), 0, h->stream, h->lmhead, K,
                       reinterpret_cast<unsigned char*>(h->lmhead8), h->lm_scale, h->lm_err);
    HIPCHK(hipGetLastError(), -1);
    HIPCHK(hipStreamSynchronize(h->stream), -1);
  }
  h->lm_mode = enable;
  return 0;
}

int megakernel_set_layer_fp8(void* handle, int enable) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) {
    mk::set_err("null handle");
    return -1;
  }
  if (enable && (!h->has_cls || !h->roles_ok[1])) {
    mk::set_err("FP8 layer weights need the class kernel, which this preset / device does not have");
    return -1;
  }
  if (enable && !h->layers8) {
    const mk::ShapeInfo& s = h->sh;
    HIPCHK(hipMalloc(&h->layers8, (size_t)s.u_layer * 8 * h->L), -1);
    HIPCHK(hipMalloc(&h->lscale, (size_t)s.srows_layer * 4 * h->L), -1);
    struct Region { long long off; int blocks, K, srow; };
    const Region reg[4] = {{s.off_qkv, s.QKV / 16, s.H, s.srow_qkv},
                           {s.off_o, s.H / 16, s.QD, s.srow_o},
                           {s.off_gu, 2 * (s.F / 16), s.H, s.srow_gu},
                           {s.off_down, s.H / 16, s.F, s.srow_down}};
    for (const Region& g : reg)
      hipLaunchKernelGGL(mk::layer_fp8_kernel, dim3(g.blocks, h->L), dim3(256), 0, h->stream, h->layers, s.u_layer,
                         g.off, g.K, reinterpret_cast<unsigned char*>(h->layers8), h->lscale, s.srows_layer, g.srow);
    HIPCHK(hipGetLastError(), -1);
    HIPCHK(hipStreamSynchronize(h->stream), -1);
  }
  h->layer_fp8 = enable != 0;
  return 0;
}

int megakernel_get_layer_fp8(void* handle, int layer, int which, unsigned char* codes, float* scales) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || !h->layers8 || !codes || !scales) {
    mk::set_err("FP8 layer weights not built (megakernel_set_layer_fp8) or null output");
    return -1;
  }
  if (layer < 0 || layer >= h->L || which < MK_LAYER_QKV || which > MK_LAYER_DOWN) {
    mk::set_err("layer %d / matrix %d outside [0, %d) / [%d, %d]", layer, which, h->L, MK_LAYER_QKV, MK_LAYER_DOWN);
    return -1;
  }
  const mk::ShapeInfo& s = h->sh;
  // rows, K, region offset, block stride / offset (gate and up interleave), scale rows
  int R = 0, K = 0, bs = 1, bo = 0, srow = 0;
  long long off = 0;
  switch (which) {
    case MK_LAYER_QKV: R = s.QKV, K = s.H, off = s.off_qkv, srow = s.srow_qkv; break;
    case MK_LAYER_O: R = s.H, K = s.QD, off = s.off_o, srow = s.srow_o; break;
    case MK_LAYER_GATE: R = s.F, K = s.H, off = s.off_gu, bs = 2, srow = s.srow_gu; break;
    case MK_LAYER_UP: R = s.F, K = s.H, off = s.off_gu, bs = 2, bo = 1, srow = s.srow_gu; break;
    default: R = s.H, K = s.F, off = s.off_down, srow = s.srow_down; break;
  }
  const int KT = K / 32;
  const size_t region = (size_t)R * K * (bs == 2 ? 2 : 1);
  std::vector<unsigned char> tiles(region);
  std::vector<float> sc((size_t)R * (bs == 2 ? 2 : 1));
  HIPCHK(hipMemcpy(tiles.data(), reinterpret_cast<const unsigned char*>(h->layers8 + (long long)layer * s.u_layer + off),
                   region, hipMemcpyDeviceToHost), -1);
  HIPCHK(hipMemcpy(sc.data(), h->lscale + (size_t)layer * s.srows_layer + srow, sc.size() * 4, hipMemcpyDeviceToHost),
         -1);
  for (long long row = 0; row < R; ++row) {
    const long long blk = (row >> 4) * bs + bo;
    scales[row] = sc[blk * 16 + (row & 15)];
    for (int c = 0; c < K; ++c)
      codes[row * K + c] = tiles[(blk * KT + (c >> 5)) * 512 + (((c >> 3) & 3) * 16 + (row & 15)) * 8 + (c & 7)];
  }
  return 0;
}

int megakernel_set_kv_fp8(void* handle, int enable) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h) {
    mk::set_err("null handle");
    return -1;
  }
  if (enable && !h->kscale) {
    const size_t sb = (size_t)h->L * h->sh.NKV * h->s_pad * 4;
    HIPCHK(hipMalloc(&h->kscale, sb), -1);
    HIPCHK(hipMalloc(&h->vscale, sb), -1);
  }
  h->kv_fp8 = enable != 0;
  megakernel_reset(h);  // a new, empty cache in the chosen format
  return 0;
}

int megakernel_get_lmhead_fp8(void* handle, unsigned char* codes, float* scales) {
  Handle* h = static_cast<Handle*>(handle);
  if (!h || !h->lmhead8 || !codes || !scales) {
    mk::set_err("FP8 LM head not built (megakernel_set_lmhead_fp8) or null output");
    return -1;
  }
  const int K = h->sh.H, KT8 = K / 64;
  std::vector<unsigned char> tiles((size_t)h->V * K);
  HIPCHK(hipMemcpy(tiles.data(), h->lmhead8, tiles.size(), hipMemcpyDeviceToHost), -1);
  HIPCHK(hipMemcpy(scales, h->lm_scale, (size_t)h->V * 4, hipMemcpyDeviceToHost), -1);
  for (long long row = 0; row < h->V; ++row)
    for (int c = 0; c < K; ++c)
      codes[row * K + c] =
          tiles[((row >> 4) * KT8 + (c >> 6)) * 1024 + (((c >> 4) & 3) * 16 + (row & 15)) * 16 + (c & 15)];
  return 0;
}

int megakernel_synth_fill(void* d_dst, unsigned long long n, unsigned long long key, float c, int add_one) {
  if (!d_dst) {
    mk::set_err("null destination");
    return -1;
  }
  if (n == 0) return 0;
  hipLaunchKernelGGL(mk::synth_fill_kernel, dim3(4096), dim3(256), 0, 0, static_cast<uint16_t*>(d_dst), n, key, c,
                     add_one);
  HIPCHK(hipGetLastError(), -1);
  HIPCHK(hipDeviceSynchronize(), -1);
  return 0;
}

unsigned long long megakernel_synth_key(unsigned long long seed, unsigned long long tensor_id) {
  return mk::sm_h(seed, tensor_id);
}

int megakernel_rope_inv_freq(int preset, float* out, int n) {
  int D = preset == mk::PRESET_QWEN3_06B ? 128 : 64;
  if (!out || n < D / 2) {
    mk::set_err("output buffer too small");
    return -1;
  }
  for (int i = 0; i < D / 2; ++i) out[i] = 1.0f / powf((float)mk::kRopeTheta, (float)(2 * i) / (float)D);
  return D / 2;
}

void* megakernel_device_alloc(unsigned long long nbytes) {
  void* d = nullptr;
  hipError_t e = hipMalloc(&d, nbytes);
  if (e != hipSuccess) {
    mk::set_err("hipMalloc(%llu) failed: %s", nbytes, hipGetErrorString(e));
    return nullptr;
  }
  return d;
}

void megakernel_device_free(void* d) {
  if (d) (void)hipFree(d);
}

int megakernel_memcpy(void* dst, const void* src, unsigned long long nbytes, int kind) {
  hipMemcpyKind k = kind == 0 ? hipMemcpyHostToDevice : kind == 1 ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
  hipError_t e = hipMemcpy(dst, src, nbytes, k);
  if (e != hipSuccess) {
    mk::set_err("hipMemcpy failed: %s", hipGetErrorString(e));
    return -1;
  }
  return 0;
}

int megakernel_device_info(int* cus, int* wall_clock_khz, char* name, int name_len) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    mk::set_err("no HIP device");
    return -1;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
    mk::set_err("hipGetDeviceProperties failed");
    return -1;
  }
  if (cus) *cus = prop.multiProcessorCount;
  if (wall_clock_khz) (void)hipDeviceGetAttribute(wall_clock_khz, hipDeviceAttributeWallClockRate, dev);
  if (name && name_len > 0)
    snprintf(name, name_len, "%s (%s)", prop.name[0] ? prop.name : "AMD Instinct GPU", prop.gcnArchName);
  return 0;
}

}  // extern "C"
