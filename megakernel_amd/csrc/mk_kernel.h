// The persistent decode megakernel for gfx950 (one resident launch decodes
// n_tokens greedy tokens; every workgroup stays resident for the whole launch).
//
// Per token (reference phase order: /root/reference/src/megakernel.cu:132-332):
//   for each layer:
//     P1  rmsnorm(x) -> fused QKV GEMV                          row-block owners
//     P2  QK-norm + RoPE + KV append + split-position GQA attention partials
//     P3  merge partials -> O GEMV -> x[rows] = x[rows] + o[rows] row-block owners
//     P4  rmsnorm(x) -> gate/up GEMV -> silu(g) * u               row-block owners
//     P5  down GEMV -> x[rows] += d[rows]                         row-block owners
//   final rmsnorm -> tied LM head -> per-workgroup argmax -> next token
//
// There is no grid barrier.  Each phase instance has a global number (its
// tag); every activation word carries the tag of the phase that wrote it, and
// a consumer waits for exactly the words it reads (tagged dataflow, see
// mk_device.h).  Every residual element has exactly one writer per phase (the
// owner of its 16-row block), so there is no read-modify-write race on x
// (unlike megakernel.cu:243-245,288-290), and the per-token tags make the
// reference's never-re-armed KV flag problem (barriers.cuh:112-134)
// impossible.  Buffers are single-buffered: every write of a buffer depends
// (through the phase chain) on every read of its previous contents.
#pragma once
#include "mk_config.h"
#include "mk_device.h"

namespace mk {

constexpr int NT = 512;               // threads per workgroup (8 waves)
constexpr int NW = NT / kWave;
constexpr int CHUNK_MAX = 2048;       // max positions per attention work item
constexpr int PHASES_PER_LAYER = 5;
constexpr int ML_CAP = 1024;          // LDS floats for split (max, sum): nsplit_max * NQ * 2
constexpr int TAG14 = 0x3FFF;         // argmax words carry a 14-bit tag, never 0
__device__ __forceinline__ unsigned tag14(unsigned tag) { return tag % 16383u + 1u; }
constexpr int IDX_BITS = 18;          // ... and an 18-bit vocabulary index
constexpr unsigned IDX_MAX = (1u << IDX_BITS) - 1;

struct Params {
  const u32x4* layers;        // packed per-layer weights (L * U_LAYER units)
  const uint16_t* norms;      // [L][NORM_STRIDE] bf16 gains
  const uint16_t* final_norm; // [H] bf16
  const u32x4* lmhead;        // packed tied embedding [V/16][KT_H][64]
  uint16_t* kv;               // [L][2][NKV][max_seq][D] bf16
  u64* x;                     // [H] residual stream (tagged)
  u64* qkv;                   // [QKV] projections of the current layer (tagged)
  u64* part_ml;               // [nsplit_max][NQ][2] split max / sum (tagged)
  u64* part_acc;              // [nsplit_max][NQ][D] split unnormalised outputs (tagged)
  u64* act;                   // [F] silu(gate)*up (tagged)
  u64* amax;                  // [2][G] per-workgroup argmax words (token parity)
  int* out_tokens;            // [n_tokens]
  int* err;                   // error word
  float* dbg_layers;          // optional [(L+1)][H]: embedding, then x after each layer
  float* dbg_logits;          // optional [V]
  u64* trace;                 // optional [(5L+1)][2][G] wall-clock ready/done per phase
  const float* inv_freq;      // [D/2] RoPE inverse frequencies
  u64 timeout_ticks;
  unsigned tag_base;          // tag of the first phase of this launch
  int n_layers, vocab, max_seq;
  int pos0, n_tokens, first_token;
  int nsplit_max, chunk_min;
  int trace_token;
};

template <class S>
struct Smem {
  static constexpr int VEC = (S::F > S::QD ? (S::F > S::H ? S::F : S::H) : (S::QD > S::H ? S::QD : S::H));
  float vec[VEC];                     // GEMV input vector
  float xin[S::H];                    // residual stream as read
  float red[2 * NW * 16];             // GEMV cross-wave partials
  float qk[(S::GQA + 1) * S::D];      // q heads, then k (normed + rotated in place)
  float vv[S::D];                     // v of the current position
  u32x4 kvcur[2][S::D / 8];           // bf16 K/V of the current position
  float sc[S::GQA * CHUNK_MAX];       // attention scores / probabilities
  float pv[NW * S::GQA * S::D];       // attention P*V cross-wave partials
  float ml[ML_CAP];                    // merge: per split/head (max, sum) -> (scale)
  float hl[S::NQ];                    // merge: per head 1 / total sum
  float rc[S::D / 2], rs[S::D / 2];   // RoPE cos / sin of this token
  float scratch[4 * NW];
  u64 amax[NW];
  int flag;
};

// Element `col` of row `row` of a packed [R][K] matrix (K = 32 * KT).
template <int KT>
__device__ __forceinline__ float packed_elem(const u32x4* base, int row, int col) {
  const int kt = col >> 5, q = (col >> 3) & 3, e = col & 7;
  const uint16_t* u = reinterpret_cast<const uint16_t*>(
      base + ((long long)(row >> 4) * KT + kt) * 64 + q * 16 + (row & 15));
  return bf16_to_f32(u[e]);
}

// y[r] = sum_k W[rb*16 + r][k] * vec[k] for one packed 16-row block.  Wave w
// takes k-tiles w, w+NW, ...; lane l covers row l & 15 and columns
// (l >> 4) * 8 .. +8 of each tile.  Result valid in threads 0..15.
template <int KT>
__device__ __forceinline__ float gemv16(const u32x4* __restrict__ tiles, const float* vec, float* red) {
  const int w = threadIdx.x / kWave, l = opaque_v(threadIdx.x % kWave);
  constexpr int PER = (KT + NW - 1) / NW;
  u32x4 wv[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int kt = w + i * NW;
    if (kt < KT) wv[i] = ld_nt(tiles + kt * 64 + l);
  }
  float acc = 0.f;
  const float* hv = vec + (l >> 4) * 8;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int kt = w + i * NW;
    if (kt < KT) acc = dot8(wv[i], hv + kt * 32, acc);
  }
  acc += __shfl_xor(acc, 16);
  acc += __shfl_xor(acc, 32);
  if (l < 16) red[w * 16 + l] = acc;
  __syncthreads();
  float y = 0.f;
  if (threadIdx.x < 16) {
#pragma unroll
    for (int i = 0; i < NW; ++i) y += red[i * 16 + threadIdx.x];
  }
  __syncthreads();
  return y;
}

// Two blocks (gate and up) against the same input vector.
template <int KT>
__device__ __forceinline__ void gemv16x2(const u32x4* __restrict__ ta, const u32x4* __restrict__ tb,
                                         const float* vec, float* red, float& ya, float& yb) {
  const int w = threadIdx.x / kWave, l = opaque_v(threadIdx.x % kWave);
  constexpr int PER = (KT + NW - 1) / NW;
  u32x4 wa[PER], wb[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int kt = w + i * NW;
    if (kt < KT) {
      wa[i] = ld_nt(ta + kt * 64 + l);
      wb[i] = ld_nt(tb + kt * 64 + l);
    }
  }
  float a = 0.f, b = 0.f;
  const float* hv = vec + (l >> 4) * 8;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int kt = w + i * NW;
    if (kt < KT) {
      a = dot8(wa[i], hv + kt * 32, a);
      b = dot8(wb[i], hv + kt * 32, b);
    }
  }
  a += __shfl_xor(a, 16);
  a += __shfl_xor(a, 32);
  b += __shfl_xor(b, 16);
  b += __shfl_xor(b, 32);
  if (l < 16) {
    red[w * 16 + l] = a;
    red[NW * 16 + w * 16 + l] = b;
  }
  __syncthreads();
  ya = 0.f;
  yb = 0.f;
  if (threadIdx.x < 16) {
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      ya += red[i * 16 + threadIdx.x];
      yb += red[NW * 16 + i * 16 + threadIdx.x];
    }
  }
  __syncthreads();
}

// out[i] = v[i] * rsqrt(mean(v^2) + eps) * gain[i]  (reference rmsnorm.cuh:87-108).
// The source is the residual stream in LDS, or (layer 0) the embedding row.
template <class S>
__device__ __forceinline__ void rmsnorm_to(Smem<S>& sm, const float* xl, const u32x4* emb, int tok,
                                           const uint16_t* gain, float* out) {
  constexpr int VPT = (S::H + NT - 1) / NT;
  float v[VPT];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < VPT; ++c) {
    const int i = threadIdx.x + c * NT;
    float t = 0.f;
    if (i < S::H) t = emb ? packed_elem<S::KT_H>(emb, tok, i) : xl[i];
    v[c] = t;
    ss = fmaf(t, t, ss);
  }
  ss = block_sum<NW>(ss, sm.scratch);
  const float r = rsqrtf(ss / (float)S::H + kRmsEps);
#pragma unroll
  for (int c = 0; c < VPT; ++c) {
    const int i = threadIdx.x + c * NT;
    if (i < S::H) out[i] = v[c] * r * bf16_to_f32(gain[i]);
  }
  __syncthreads();
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + __expf(-g)) * u; }

// Work item i of a phase runs on workgroup (i + off) mod G.
__device__ __forceinline__ int first_item(int wg, int off, int G) { return (wg + G - (off % G)) % G; }

__device__ __forceinline__ void trace_mark(const Params& p, int t, int slot, int which) {
  if (p.trace && t == p.trace_token && threadIdx.x == 0)
    p.trace[((long long)slot * 2 + which) * gridDim.x + blockIdx.x] = wall_clock64();
}

// ---------------------------------------------------------------- phase P2
// One attention work item: kv head g, positions [s*chunk, min((s+1)*chunk, pos+1)).
template <class S>
__device__ bool attention_item(const Params& p, Smem<S>& sm, int layer, int pos, int g, int s, int chunk,
                               unsigned tag_in, unsigned tag_out) {
  constexpr int D = S::D, GQA = S::GQA, LPP = D / 8, PPW = kWave / LPP;
  const int tid = threadIdx.x, w = tid / kWave, l = opaque_v(tid % kWave);
  const int n = pos + 1;
  // splits are never empty (nsplit = ceil(n / chunk)), so every item reads
  // its group's q/k/v before writing: no item can overwrite partials that an
  // O-projection owner of the previous layer is still merging.
  const int t0 = s * chunk, t1 = min(n, t0 + chunk);
  u64* mlw = p.part_ml + ((long long)s * S::NQ + g * GQA) * 2;
  u64* accw = p.part_acc + ((long long)s * S::NQ + g * GQA) * D;
  // inputs: the group's q heads, its k and v rows
  if (!ll_fetch<NT, 1>(p.qkv + g * GQA * D, GQA * D, tag_in, sm.qk, p.err, p.timeout_ticks)) return false;
  if (!ll_fetch<NT, 1>(p.qkv + S::QD + g * D, D, tag_in, sm.qk + GQA * D, p.err, p.timeout_ticks)) return false;
  if (!ll_fetch<NT, 1>(p.qkv + S::QD + S::KVD + g * D, D, tag_in, sm.vv, p.err, p.timeout_ticks)) return false;
  const uint16_t* nrm = p.norms + (long long)layer * S::NORM_STRIDE;
  // 1. per-head RMSNorm of the q heads and the k head (reference
  //    rmsnorm.cuh:57-84); one wave per head.
  if (w < GQA + 1) {
    const uint16_t* gain = nrm + (w < GQA ? S::NORM_Q : S::NORM_K);
    float v[D / kWave];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < D / kWave; ++c) {
      v[c] = sm.qk[w * D + l + c * kWave];
      ss = fmaf(v[c], v[c], ss);
    }
    ss = wave_sum(ss);
    const float r = rsqrtf(ss / (float)D + kRmsEps);
#pragma unroll
    for (int c = 0; c < D / kWave; ++c) sm.qk[w * D + l + c * kWave] = v[c] * r * bf16_to_f32(gain[l + c * kWave]);
  }
  __syncthreads();
  // 2. RoPE, rotate-half pairs (d, d + D/2) (reference attention.cuh:22-44).
  for (int e = tid; e < (GQA + 1) * (D / 2); e += NT) {
    const int hh = e / (D / 2), d = e % (D / 2);
    const float a = sm.qk[hh * D + d], b = sm.qk[hh * D + d + D / 2];
    const float c = sm.rc[d], sn = sm.rs[d];
    sm.qk[hh * D + d] = a * c - b * sn;
    sm.qk[hh * D + d + D / 2] = b * c + a * sn;
  }
  __syncthreads();
  uint16_t* kb = p.kv + ((long long)(layer * 2 + 0) * S::NKV + g) * (long long)p.max_seq * D;
  uint16_t* vb = p.kv + ((long long)(layer * 2 + 1) * S::NKV + g) * (long long)p.max_seq * D;
  // 3. bf16 K/V of the current position (reference kv_cache.cuh:58-78); the
  //    split that owns `pos` appends them to the cache with write-through
  //    stores and uses its LDS copy for this token.
  const bool own = (t0 <= pos && pos < t1);
  if (tid < D / 2) {
    const int d = 2 * tid;
    const unsigned kw = (unsigned)f32_to_bf16(sm.qk[GQA * D + d]) | ((unsigned)f32_to_bf16(sm.qk[GQA * D + d + 1]) << 16);
    const unsigned vw = (unsigned)f32_to_bf16(sm.vv[d]) | ((unsigned)f32_to_bf16(sm.vv[d + 1]) << 16);
    reinterpret_cast<unsigned*>(sm.kvcur[0])[tid] = kw;
    reinterpret_cast<unsigned*>(sm.kvcur[1])[tid] = vw;
    if (own) {
      __hip_atomic_store(reinterpret_cast<unsigned*>(kb + (long long)pos * D) + tid, kw, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(reinterpret_cast<unsigned*>(vb + (long long)pos * D) + tid, vw, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  // 4. scores s_j[t] = (q_j . K[t]) / sqrt(D); LPP lanes per position.
  const float scale = 1.0f / sqrtf((float)D);
  const int c = l % LPP, po = l / LPP;
  float qr[GQA][8];
#pragma unroll
  for (int j = 0; j < GQA; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) qr[j][e] = sm.qk[j * D + c * 8 + e];
  const int cnt = t1 - t0;
  constexpr int U = 4;
  for (int tb = t0 + w * PPW; tb < t1; tb += NW * PPW * U) {
    u32x4 kk[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = tb + u * NW * PPW + po;
      kk[u] = (t < t1 && t != pos) ? ld_nt(reinterpret_cast<const u32x4*>(kb + (long long)t * D + c * 8))
                                   : sm.kvcur[0][c];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = tb + u * NW * PPW + po;
#pragma unroll
      for (int j = 0; j < GQA; ++j) {
        float d = dot8(kk[u], qr[j], 0.f);
#pragma unroll
        for (int m = LPP / 2; m >= 1; m >>= 1) d += __shfl_xor(d, m);
        if (c == 0 && t < t1) sm.sc[j * CHUNK_MAX + (t - t0)] = d * scale;
      }
    }
  }
  __syncthreads();
  // 5. softmax statistics of this split (fp32).
  float mj[GQA], lj[GQA];
#pragma unroll
  for (int j = 0; j < GQA; ++j) {
    float m = -INFINITY;
    for (int i = tid; i < cnt; i += NT) m = fmaxf(m, sm.sc[j * CHUNK_MAX + i]);
    mj[j] = block_max<NW>(m, sm.scratch);
  }
#pragma unroll
  for (int j = 0; j < GQA; ++j) {
    float sum = 0.f;
    for (int i = tid; i < cnt; i += NT) {
      const float e = __expf(sm.sc[j * CHUNK_MAX + i] - mj[j]);
      sm.sc[j * CHUNK_MAX + i] = e;
      sum += e;
    }
    lj[j] = block_sum<NW>(sum, sm.scratch);
  }
  // 6. acc_j = sum_t p_j[t] V[t]  (unnormalised).
  float acc[GQA][8];
#pragma unroll
  for (int j = 0; j < GQA; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = 0.f;
  for (int tb = t0 + w * PPW; tb < t1; tb += NW * PPW * U) {
    u32x4 vk[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = tb + u * NW * PPW + po;
      vk[u] = (t < t1 && t != pos) ? ld_nt(reinterpret_cast<const u32x4*>(vb + (long long)t * D + c * 8))
                                   : sm.kvcur[1][c];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = tb + u * NW * PPW + po;
      if (t < t1) {
        float vf[8] = {bf16_lo(vk[u].x), bf16_hi(vk[u].x), bf16_lo(vk[u].y), bf16_hi(vk[u].y),
                       bf16_lo(vk[u].z), bf16_hi(vk[u].z), bf16_lo(vk[u].w), bf16_hi(vk[u].w)};
#pragma unroll
        for (int j = 0; j < GQA; ++j) {
          const float pj = sm.sc[j * CHUNK_MAX + (t - t0)];
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[j][e] = fmaf(pj, vf[e], acc[j][e]);
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < GQA; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = acc[j][e];
#pragma unroll
      for (int m = LPP; m < kWave; m <<= 1) v += __shfl_xor(v, m);
      acc[j][e] = v;
    }
  if (po == 0) {
#pragma unroll
    for (int j = 0; j < GQA; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) sm.pv[(w * GQA + j) * D + c * 8 + e] = acc[j][e];
  }
  __syncthreads();
  for (int e = tid; e < GQA * D; e += NT) {
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) v += sm.pv[i * GQA * D + e];
    ll_put(accw + e, ll_pack(v, tag_out));
  }
  if (tid < GQA * 2) ll_put(mlw + tid, ll_pack((tid & 1) ? lj[tid >> 1] : mj[tid >> 1], tag_out));
  return true;
}

// ---------------------------------------------------------------- phase P3
// Merge the split partials of every q head (log-sum-exp) into vec[QD].
template <class S>
__device__ bool merge_attention(const Params& p, Smem<S>& sm, int nsplit, unsigned tag) {
  constexpr int D = S::D, NQ = S::NQ;
  if (!ll_fetch<NT, 2>(p.part_ml, nsplit * NQ * 2, tag, sm.ml, p.err, p.timeout_ticks)) return false;
  if (threadIdx.x < NQ) {
    const int h = threadIdx.x;
    float M = -INFINITY;
    for (int s = 0; s < nsplit; ++s) M = fmaxf(M, sm.ml[(s * NQ + h) * 2]);
    float L = 0.f;
    for (int s = 0; s < nsplit; ++s) {
      const float f = __expf(sm.ml[(s * NQ + h) * 2] - M);
      L = fmaf(f, sm.ml[(s * NQ + h) * 2 + 1], L);
      sm.ml[(s * NQ + h) * 2] = f;  // becomes the split's scale
    }
    sm.hl[h] = 1.0f / L;
  }
  __syncthreads();
  int failed = 0;
  for (int e = threadIdx.x; e < S::QD && !failed; e += NT) {
    const int h = e / D;
    float o = 0.f;
    for (int s0 = 0; s0 < nsplit && !failed; s0 += 8) {
      u64 wv[8];
      Spin sp;
      while (true) {
        bool ready = true;
#pragma unroll
        for (int b = 0; b < 8; ++b)
          if (s0 + b < nsplit) {
            wv[b] = ll_get(p.part_acc + (long long)(s0 + b) * S::QD + e);
            ready = ready && ll_tag(wv[b]) == tag;
          }
        if (ready) break;
        if (!sp.step(p.err, p.timeout_ticks)) {
          failed = 1;
          break;
        }
      }
#pragma unroll
      for (int b = 0; b < 8; ++b)
        if (s0 + b < nsplit) o = fmaf(sm.ml[((s0 + b) * NQ + h) * 2], ll_val(wv[b]), o);
    }
    sm.vec[e] = o * sm.hl[h];
  }
  return __syncthreads_or(failed) == 0;
}

// ------------------------------------------------------------------ kernel
template <class S>
__global__ __launch_bounds__(NT) void decode_kernel(Params p) {
  __shared__ Smem<S> sm;
  const int G = gridDim.x, wg = blockIdx.x, tid = threadIdx.x;
  const int w = tid / kWave, l = tid % kWave;
  const int L = p.n_layers;
  const unsigned per_token = (unsigned)(PHASES_PER_LAYER * L + 1);
  // Phase -> workgroup offsets spread the per-layer byte load across CUs.
  const int off_qkv = G / 4, off_gu = G / 4, off_o = (3 * G) / 4, off_down = 0, off_att = 0;

  int tok = p.first_token;
  for (int t = 0; t < p.n_tokens; ++t) {
    const int pos = p.pos0 + t;
    const unsigned tb = p.tag_base + (unsigned)t * per_token;  // tag of this token's first phase
    if (t > 0) {
      // next token = argmax over every workgroup's word of the previous token
      const unsigned want = tag14(tb - 1u);
      u64* slots = p.amax + ((t - 1) & 1) * G;
      int failed = 0;
      u64 best = 0;
      for (int i = tid; i < G && !failed; i += NT) {
        Spin sp;
        u64 v;
        while (((v = ll_get(slots + i)) & TAG14) != want)
          if (!sp.step(p.err, p.timeout_ticks)) {
            failed = 1;
            break;
          }
        best = v > best ? v : best;
      }
      if (__syncthreads_or(failed)) return;
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) {
        const u64 o = __shfl_xor(best, m);
        best = o > best ? o : best;
      }
      if (l == 0) sm.amax[w] = best;
      __syncthreads();
      best = sm.amax[0];
      for (int i = 1; i < NW; ++i) best = sm.amax[i] > best ? sm.amax[i] : best;
      __syncthreads();
      const unsigned idx = IDX_MAX - (unsigned)((best >> 14) & IDX_MAX);
      tok = idx < (unsigned)p.vocab ? (int)idx : 0;
      if (wg == 0 && tid == 0) p.out_tokens[t - 1] = tok;
    }
    if (tid < S::D / 2) {
      float sn, cs;
      sincosf((float)pos * p.inv_freq[tid], &sn, &cs);
      sm.rc[tid] = cs;
      sm.rs[tid] = sn;
    }
    if (p.dbg_layers && wg == 0)
      for (int i = tid; i < S::H; i += NT) p.dbg_layers[i] = packed_elem<S::KT_H>(p.lmhead, tok, i);
    __syncthreads();
    const int n = pos + 1;
    int ns0 = (n + p.chunk_min - 1) / p.chunk_min;
    ns0 = ns0 < 1 ? 1 : (ns0 > p.nsplit_max ? p.nsplit_max : ns0);
    const int chunk = (n + ns0 - 1) / ns0;
    const int nsplit = (n + chunk - 1) / chunk;  // <= ns0, and no split is empty

    for (int layer = 0; layer < L; ++layer) {
      const u32x4* wl = p.layers + (long long)layer * S::U_LAYER;
      const uint16_t* nrm = p.norms + (long long)layer * S::NORM_STRIDE;
      const unsigned tg = tb + (unsigned)(PHASES_PER_LAYER * layer);  // tag of P1 of this layer
      const unsigned tg_x = tg - 1u;  // tag of the x rows this layer starts from (layer > 0)
      const int slot = PHASES_PER_LAYER * layer;
      // P1: QKV
      {
        bool have = false;
        for (int rb = first_item(wg, off_qkv, G); rb < S::RB_QKV; rb += G) {
          if (!have) {
            if (layer > 0 && !ll_fetch<NT, 2>(p.x, S::H, tg_x, sm.xin, p.err, p.timeout_ticks)) return;
            trace_mark(p, t, slot + 0, 0);
            rmsnorm_to<S>(sm, sm.xin, layer == 0 ? p.lmhead : nullptr, tok, nrm + S::NORM_ATTN, sm.vec);
            have = true;
          }
          const float y = gemv16<S::KT_H>(wl + S::OFF_QKV + (long long)rb * S::KT_H * 64, sm.vec, sm.red);
          if (tid < 16) ll_put(p.qkv + rb * 16 + tid, ll_pack(y, tg));
        }
        if (have) trace_mark(p, t, slot + 0, 1);
      }
      // P2: attention partials
      {
        bool any = false;
        for (int it = first_item(wg, off_att, G); it < S::NKV * nsplit; it += G) {
          if (!attention_item<S>(p, sm, layer, pos, it / nsplit, it % nsplit, chunk, tg, tg + 1u)) return;
          if (!any) trace_mark(p, t, slot + 1, 0);
          any = true;
        }
        if (any) trace_mark(p, t, slot + 1, 1);
      }
      // P3: O projection + residual
      {
        bool have = false;
        for (int rb = first_item(wg, off_o, G); rb < S::RB_H; rb += G) {
          if (!have) {
            if (!merge_attention<S>(p, sm, nsplit, tg + 1u)) return;
            trace_mark(p, t, slot + 2, 0);
            have = true;
          }
          const float y = gemv16<S::KT_Q>(wl + S::OFF_O + (long long)rb * S::KT_Q * 64, sm.vec, sm.red);
          int failed = 0;
          if (tid < 16) {
            const int row = rb * 16 + tid;
            float xo;
            if (layer == 0) xo = packed_elem<S::KT_H>(p.lmhead, tok, row);
            else failed = !ll_wait1(p.x + row, tg_x, &xo, p.err, p.timeout_ticks);
            if (!failed) ll_put(p.x + row, ll_pack(xo + y, tg + 2u));
          }
          if (__syncthreads_or(failed)) return;
        }
        if (have) trace_mark(p, t, slot + 2, 1);
      }
      // P4: gate/up + SiLU
      {
        bool have = false;
        for (int pr = first_item(wg, off_gu, G); pr < S::RB_F; pr += G) {
          if (!have) {
            if (!ll_fetch<NT, 2>(p.x, S::H, tg + 2u, sm.xin, p.err, p.timeout_ticks)) return;
            trace_mark(p, t, slot + 3, 0);
            rmsnorm_to<S>(sm, sm.xin, nullptr, tok, nrm + S::NORM_FFN, sm.vec);
            have = true;
          }
          float yg, yu;
          const u32x4* tgp = wl + S::OFF_GU + (long long)(2 * pr) * S::KT_H * 64;
          gemv16x2<S::KT_H>(tgp, tgp + S::KT_H * 64, sm.vec, sm.red, yg, yu);
          if (tid < 16) ll_put(p.act + pr * 16 + tid, ll_pack(silu_mul(yg, yu), tg + 3u));
        }
        if (have) trace_mark(p, t, slot + 3, 1);
      }
      // P5: down projection + residual
      {
        bool have = false;
        for (int rb = first_item(wg, off_down, G); rb < S::RB_H; rb += G) {
          if (!have) {
            if (!ll_fetch<NT, 6>(p.act, S::F, tg + 3u, sm.vec, p.err, p.timeout_ticks)) return;
            trace_mark(p, t, slot + 4, 0);
            have = true;
          }
          const float y = gemv16<S::KT_F>(wl + S::OFF_DOWN + (long long)rb * S::KT_F * 64, sm.vec, sm.red);
          int failed = 0;
          if (tid < 16) {
            const int row = rb * 16 + tid;
            float xo;
            failed = !ll_wait1(p.x + row, tg + 2u, &xo, p.err, p.timeout_ticks);
            if (!failed) {
              const float xn = xo + y;
              ll_put(p.x + row, ll_pack(xn, tg + 4u));
              if (p.dbg_layers) p.dbg_layers[(long long)(layer + 1) * S::H + row] = xn;
            }
          }
          if (__syncthreads_or(failed)) return;
        }
        if (have) trace_mark(p, t, slot + 4, 1);
      }
    }
    // Final norm + tied LM head + per-workgroup argmax (reference sampling.cuh:32-117).
    {
      const unsigned tl = tb + (unsigned)(PHASES_PER_LAYER * L);
      if (!ll_fetch<NT, 2>(p.x, S::H, tl - 1u, sm.xin, p.err, p.timeout_ticks)) return;
      trace_mark(p, t, PHASES_PER_LAYER * L, 0);
      rmsnorm_to<S>(sm, sm.xin, nullptr, tok, p.final_norm, sm.vec);
      const long long nb = p.vocab / 16;
      const long long b0 = (long long)wg * nb / G, b1 = (long long)(wg + 1) * nb / G;
      u64 best = 0ull;
      for (long long b = b0 + w; b < b1; b += NW) {
        // re-derived per block so the LDS reads of the hidden vector are not
        // hoisted out of the block loop (256 floats per lane would not fit)
        const int lo = opaque_v(l);
        const float* hv = sm.vec + (lo >> 4) * 8;
        const u32x4* tiles = p.lmhead + b * S::KT_H * 64 + lo;
        float acc = 0.f;
        constexpr int U = 16;
#pragma unroll 1
        for (int k0 = 0; k0 < S::KT_H; k0 += U) {
          u32x4 wv[U];
#pragma unroll
          for (int u = 0; u < U; ++u)
            if (k0 + u < S::KT_H) wv[u] = ld_nt(tiles + (k0 + u) * 64);
#pragma unroll
          for (int u = 0; u < U; ++u)
            if (k0 + u < S::KT_H) acc = dot8(wv[u], hv + (k0 + u) * 32, acc);
        }
        acc += __shfl_xor(acc, 16);
        acc += __shfl_xor(acc, 32);
        if (l < 16) {
          const unsigned idx = (unsigned)(b * 16 + l);
          if (p.dbg_logits) p.dbg_logits[idx] = acc;
          // key: ordered value | (IDX_MAX - idx) | tag: an unsigned max picks
          // the largest logit and, among equal logits, the lowest index
          // (torch.argmax semantics)
          const u64 key = ((u64)f32_order_key(acc) << 32) | ((u64)(IDX_MAX - idx) << 14);
          best = key > best ? key : best;
        }
      }
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) {
        const u64 o = __shfl_xor(best, m);
        best = o > best ? o : best;
      }
      if (l == 0) sm.amax[w] = best;
      __syncthreads();
      if (tid == 0) {
        u64 b = 0ull;
        for (int i = 0; i < NW; ++i) b = sm.amax[i] > b ? sm.amax[i] : b;
        ll_put(p.amax + (t & 1) * G + wg, b | (u64)tag14(tl));
      }
      trace_mark(p, t, PHASES_PER_LAYER * L, 1);
      __syncthreads();
    }
  }
  if (wg == 0) {  // the last token's id
    const int t = p.n_tokens;
    const unsigned want = tag14(p.tag_base + (unsigned)t * per_token - 1u);
    u64* slots = p.amax + ((t - 1) & 1) * G;
    int failed = 0;
    u64 best = 0;
    for (int i = tid; i < G && !failed; i += NT) {
      Spin sp;
      u64 v;
      while (((v = ll_get(slots + i)) & TAG14) != want)
        if (!sp.step(p.err, p.timeout_ticks)) {
          failed = 1;
          break;
        }
      best = v > best ? v : best;
    }
    if (__syncthreads_or(failed)) return;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      const u64 o = __shfl_xor(best, m);
      best = o > best ? o : best;
    }
    if (l == 0) sm.amax[w] = best;
    __syncthreads();
    if (tid == 0) {
      for (int i = 0; i < NW; ++i) best = sm.amax[i] > best ? sm.amax[i] : best;
      const unsigned idx = IDX_MAX - (unsigned)((best >> 14) & IDX_MAX);
      p.out_tokens[t - 1] = idx < (unsigned)p.vocab ? (int)idx : 0;
    }
  }
}

}  // namespace mk
