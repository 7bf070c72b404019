// The persistent decode megakernel for gfx950 (one resident launch decodes
// n_tokens greedy tokens; every workgroup stays resident for the whole launch).
//
// Per token (reference phase order: /root/reference/src/megakernel.cu:132-332):
//   for each layer:
//     P1  rmsnorm(x) -> fused QKV GEMV          owners of 16-row QKV blocks
//     P2  QK-norm + RoPE + KV append + split-position GQA attention partials
//     P3  combine partials -> O GEMV -> x[rows] = x[rows] + o[rows]  (row owners)
//     P4  rmsnorm(x) -> gate/up GEMV -> silu(g) * u                   (row owners)
//     P5  down GEMV -> x[rows] += d[rows]                             (row owners)
//   final rmsnorm -> tied LM head -> fused argmax (64-bit atomic max)
// Each phase ends at a grid sync point (5 * layers + 1 per token).  Every
// residual element has exactly one writer (the owner of its 16-row block), so
// there is no read-modify-write race on x (unlike megakernel.cu:243-245,288-290).
#pragma once
#include "mk_config.h"
#include "mk_device.h"

namespace mk {

constexpr int NT = 512;               // threads per workgroup (8 waves)
constexpr int NW = NT / kWave;
constexpr int CHUNK_MAX = 2048;       // max positions per attention work item
constexpr int PART_STRIDE_PAD = 4;    // partial row = m, l, pad, pad, acc[D]

struct Params {
  const u32x4* layers;        // packed per-layer weights (L * U_LAYER units)
  const uint16_t* norms;      // [L][NORM_STRIDE] bf16 gains
  const uint16_t* final_norm; // [H] bf16
  const u32x4* lmhead;        // packed tied embedding [V/16][KT_H][64]
  uint16_t* kv;               // [L][2][NKV][max_seq][D] bf16
  float* x;                   // [H] residual stream
  float* qkv;                 // [QKV] projections of the current layer
  float* part;                // attention partials [NKV*nsplit_max][GQA][PART_STRIDE]
  float* act;                 // [F] silu(gate)*up
  unsigned long long* amax;   // [n_tokens] argmax keys
  int* out_tokens;            // [n_tokens]
  unsigned* sync;             // grid arrival counter
  int* err;                   // error word
  float* dbg_layers;          // optional [(L+1)][H]: embedding, then x after each layer
  float* dbg_logits;          // optional [V]
  const float* inv_freq;      // [D/2] RoPE inverse frequencies
  unsigned long long timeout_ticks;
  unsigned sync_base;
  int n_layers, vocab, max_seq;
  int pos0, n_tokens, first_token;
  int nsplit_max, chunk_min;
};

template <class S>
struct Smem {
  static constexpr int VEC = (S::F > S::QD ? (S::F > S::H ? S::F : S::H) : (S::QD > S::H ? S::QD : S::H));
  float vec[VEC];                     // GEMV input vector
  float red[2 * NW * 16];             // GEMV cross-wave partials
  float qk[(S::GQA + 1) * S::D];      // normed + rotated q heads, then k
  float vv[S::D];                     // v of the current position
  float sc[S::GQA * CHUNK_MAX];       // attention scores / probabilities
  float pv[NW * S::GQA * S::D];       // attention P*V cross-wave partials
  float rc[S::D / 2], rs[S::D / 2];   // RoPE cos / sin of this token
  float scratch[4 * NW];
  unsigned long long amax[NW];
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
// The source is the fp32 residual stream, or (layer 0) the embedding row.
template <class S>
__device__ __forceinline__ void rmsnorm_to(Smem<S>& sm, const float* x, const u32x4* emb, int tok,
                                           const uint16_t* gain, float* out) {
  constexpr int VPT = (S::H + NT - 1) / NT;
  float v[VPT];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < VPT; ++c) {
    const int i = threadIdx.x + c * NT;
    float t = 0.f;
    if (i < S::H) t = emb ? packed_elem<S::KT_H>(emb, tok, i) : x[i];
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

template <class S>
__device__ __forceinline__ float silu_mul(float g, float u) {
  return g / (1.0f + __expf(-g)) * u;
}

// Work item i of a phase with `n` items runs on workgroup (i + off) mod G.
__device__ __forceinline__ int first_item(int wg, int off, int G) { return (wg + G - (off % G)) % G; }

// ---------------------------------------------------------------- phase P2
template <class S>
__device__ void attention_item(const Params& p, Smem<S>& sm, int layer, int pos, int g, int s,
                               int nsplit, int chunk) {
  constexpr int D = S::D, GQA = S::GQA, LPP = D / 8, PPW = kWave / LPP;
  constexpr int PS = D + PART_STRIDE_PAD;
  const int tid = threadIdx.x, w = tid / kWave, l = opaque_v(tid % kWave);
  const int n = pos + 1;
  const int t0 = s * chunk, t1 = min(n, t0 + chunk);
  float* prow = p.part + ((long long)(g * p.nsplit_max + s) * GQA) * PS;
  if (t0 >= t1) {  // empty split: neutral partial
    for (int e = tid; e < GQA * PS; e += NT) {
      const int j = e / PS, c = e % PS;
      prow[j * PS + c] = (c == 0) ? -INFINITY : 0.f;
    }
    return;
  }
  const uint16_t* nrm = p.norms + (long long)layer * S::NORM_STRIDE;
  // 1. per-head RMSNorm of the GQA q heads and the k head (reference
  //    rmsnorm.cuh:57-84), v copied; one wave per head.
  if (w < GQA + 1) {
    const float* src = (w < GQA) ? p.qkv + (g * GQA + w) * D : p.qkv + S::QD + g * D;
    const uint16_t* gain = nrm + (w < GQA ? S::NORM_Q : S::NORM_K);
    float v[D / kWave];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < D / kWave; ++c) {
      v[c] = src[l + c * kWave];
      ss = fmaf(v[c], v[c], ss);
    }
    ss = wave_sum(ss);
    const float r = rsqrtf(ss / (float)D + kRmsEps);
#pragma unroll
    for (int c = 0; c < D / kWave; ++c) sm.qk[w * D + l + c * kWave] = v[c] * r * bf16_to_f32(gain[l + c * kWave]);
  } else if (w == GQA + 1) {
#pragma unroll
    for (int c = 0; c < D / kWave; ++c) sm.vv[l + c * kWave] = p.qkv[S::QD + S::KVD + g * D + l + c * kWave];
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
  // 3. the split that owns position `pos` appends bf16 K/V (kv_cache.cuh:58-78).
  if (t0 <= pos && pos < t1) {
    for (int d = tid; d < D; d += NT) {
      kb[(long long)pos * D + d] = f32_to_bf16(sm.qk[GQA * D + d]);
      vb[(long long)pos * D + d] = f32_to_bf16(sm.vv[d]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
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
      kk[u] = (t < t1) ? ld_nt(reinterpret_cast<const u32x4*>(kb + (long long)t * D + c * 8))
                       : u32x4{0u, 0u, 0u, 0u};
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
      vk[u] = (t < t1) ? ld_nt(reinterpret_cast<const u32x4*>(vb + (long long)t * D + c * 8))
                       : u32x4{0u, 0u, 0u, 0u};
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
    const int j = e / D, d = e % D;
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) v += sm.pv[(i * GQA + j) * D + d];
    prow[j * PS + PART_STRIDE_PAD + d] = v;
  }
  if (tid < GQA) {
    prow[tid * PS + 0] = mj[tid];
    prow[tid * PS + 1] = lj[tid];
  }
}

// ---------------------------------------------------------------- phase P3
// Merge the split partials of every q head (log-sum-exp) into vec[QD].
template <class S>
__device__ void combine_attention(const Params& p, Smem<S>& sm, int nsplit) {
  constexpr int D = S::D, GQA = S::GQA, PS = D + PART_STRIDE_PAD;
  for (int e = threadIdx.x; e < S::QD; e += NT) {
    const int h = e / D, d = e % D, g = h / GQA, j = h % GQA;
    const float* base = p.part + ((long long)(g * p.nsplit_max) * GQA + j) * PS;
    float M = -INFINITY;
    for (int s = 0; s < nsplit; ++s) M = fmaxf(M, base[(long long)s * GQA * PS]);
    float L = 0.f, o = 0.f;
    for (int s = 0; s < nsplit; ++s) {
      const float* r = base + (long long)s * GQA * PS;
      const float f = __expf(r[0] - M);
      L = fmaf(f, r[1], L);
      o = fmaf(f, r[PART_STRIDE_PAD + d], o);
    }
    sm.vec[e] = o / L;
  }
  __syncthreads();
}

// ------------------------------------------------------------------ kernel
template <class S>
__global__ __launch_bounds__(NT) void decode_kernel(Params p) {
  __shared__ Smem<S> sm;
  const int G = gridDim.x, wg = blockIdx.x, tid = threadIdx.x;
  const int w = tid / kWave, l = tid % kWave;
  unsigned k = 0;  // sync points passed
  // Phase -> workgroup offsets spread the per-layer byte load across CUs.
  const int off_qkv = G / 4, off_gu = G / 4, off_o = (3 * G) / 4, off_down = 0, off_att = 0;

  if (wg == 0)
    for (int i = tid; i < p.n_tokens; i += NT) p.amax[i] = 0ull;

#define MK_SYNC()                                                                        \
  do {                                                                                   \
    grid_arrive(p.sync);                                                                 \
    ++k;                                                                                 \
    if (!grid_wait(p.sync, p.sync_base + k * (unsigned)G, p.err, p.timeout_ticks, &sm.flag)) \
      return;                                                                            \
  } while (0)

  int tok = p.first_token;
  for (int t = 0; t < p.n_tokens; ++t) {
    const int pos = p.pos0 + t;
    if (t > 0) {
      const unsigned idx = argmax_key_index(p.amax[t - 1]);
      tok = idx < (unsigned)p.vocab ? (int)idx : 0;  // always in range (keys are never 0)
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
    int nsplit = (n + p.chunk_min - 1) / p.chunk_min;
    nsplit = nsplit < 1 ? 1 : (nsplit > p.nsplit_max ? p.nsplit_max : nsplit);
    const int chunk = (n + nsplit - 1) / nsplit;

    for (int layer = 0; layer < p.n_layers; ++layer) {
      const u32x4* wl = p.layers + (long long)layer * S::U_LAYER;
      const uint16_t* nrm = p.norms + (long long)layer * S::NORM_STRIDE;
      const u32x4* emb0 = (layer == 0) ? p.lmhead : nullptr;
      // P1: QKV
      {
        bool have = false;
        for (int rb = first_item(wg, off_qkv, G); rb < S::RB_QKV; rb += G) {
          if (!have) {
            rmsnorm_to<S>(sm, p.x, emb0, tok, nrm + S::NORM_ATTN, sm.vec);
            have = true;
          }
          const float y = gemv16<S::KT_H>(wl + S::OFF_QKV + (long long)rb * S::KT_H * 64, sm.vec, sm.red);
          if (tid < 16) p.qkv[rb * 16 + tid] = y;
        }
      }
      MK_SYNC();
      // P2: attention partials
      for (int it = first_item(wg, off_att, G); it < S::NKV * nsplit; it += G)
        attention_item<S>(p, sm, layer, pos, it / nsplit, it % nsplit, nsplit, chunk);
      MK_SYNC();
      // P3: O projection + residual
      {
        bool have = false;
        for (int rb = first_item(wg, off_o, G); rb < S::RB_H; rb += G) {
          if (!have) {
            combine_attention<S>(p, sm, nsplit);
            have = true;
          }
          const float y = gemv16<S::KT_Q>(wl + S::OFF_O + (long long)rb * S::KT_Q * 64, sm.vec, sm.red);
          if (tid < 16) {
            const int row = rb * 16 + tid;
            const float xo = emb0 ? packed_elem<S::KT_H>(p.lmhead, tok, row) : p.x[row];
            p.x[row] = xo + y;
          }
        }
      }
      MK_SYNC();
      // P4: gate/up + SiLU
      {
        bool have = false;
        for (int pr = first_item(wg, off_gu, G); pr < S::RB_F; pr += G) {
          if (!have) {
            rmsnorm_to<S>(sm, p.x, nullptr, tok, nrm + S::NORM_FFN, sm.vec);
            have = true;
          }
          float yg, yu;
          const u32x4* tg = wl + S::OFF_GU + (long long)(2 * pr) * S::KT_H * 64;
          gemv16x2<S::KT_H>(tg, tg + S::KT_H * 64, sm.vec, sm.red, yg, yu);
          if (tid < 16) p.act[pr * 16 + tid] = silu_mul<S>(yg, yu);
        }
      }
      MK_SYNC();
      // P5: down projection + residual
      {
        bool have = false;
        for (int rb = first_item(wg, off_down, G); rb < S::RB_H; rb += G) {
          if (!have) {
            for (int i = tid; i < S::F; i += NT) sm.vec[i] = p.act[i];
            __syncthreads();
            have = true;
          }
          const float y = gemv16<S::KT_F>(wl + S::OFF_DOWN + (long long)rb * S::KT_F * 64, sm.vec, sm.red);
          if (tid < 16) {
            const int row = rb * 16 + tid;
            const float xn = p.x[row] + y;
            p.x[row] = xn;
            if (p.dbg_layers) p.dbg_layers[(long long)(layer + 1) * S::H + row] = xn;
          }
        }
      }
      MK_SYNC();
    }
    // Final norm + tied LM head + argmax (reference sampling.cuh:32-117).
    {
      rmsnorm_to<S>(sm, p.x, nullptr, tok, p.final_norm, sm.vec);
      const long long nb = p.vocab / 16;
      const long long b0 = (long long)wg * nb / G, b1 = (long long)(wg + 1) * nb / G;
      unsigned long long best = 0ull;
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
          const unsigned long long key = argmax_key(acc, idx);
          best = key > best ? key : best;
        }
      }
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) {
        const unsigned long long o = __shfl_xor(best, m);
        best = o > best ? o : best;
      }
      if (l == 0) sm.amax[w] = best;
      __syncthreads();
      if (tid == 0) {
        unsigned long long b = 0ull;
        for (int i = 0; i < NW; ++i) b = sm.amax[i] > b ? sm.amax[i] : b;
        if (b) __hip_atomic_fetch_max(p.amax + t, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    MK_SYNC();
  }
  if (wg == 0 && tid == 0) p.out_tokens[p.n_tokens - 1] = (int)argmax_key_index(p.amax[p.n_tokens - 1]);
#undef MK_SYNC
}

}  // namespace mk
