// Batched greedy decode of up to 16 independent sequences.
//
// One decode step of all sequences is a fixed sequence of kernels, captured
// once into a HIP graph and replayed per step:
//   embed                 x[b] = E[tok[b]]
//   per layer:  qkv       rmsnorm(x) -> fused QKV GEMM           (16-row blocks)
//               attn      QK-norm + RoPE + KV append + split attention; the last
//                         split of each (sequence, kv head) merges the partials
//               o         O GEMM + residual                       (16-row blocks)
//               gu        rmsnorm(x) -> gate/up GEMM -> SiLU(g) * u
//               down      down GEMM + residual
//   lm                    final rmsnorm -> tied LM head GEMM -> per-sequence argmax
//   tok                   argmax keys -> tokens, positions + 1
// (reference phase order /root/reference/src/megakernel.cu:132-332, per sequence).
//
// With 16 sequences every weight block is used 16 times, so the GEMMs run on
// the matrix cores: v_mfma_f32_16x16x32_bf16 with the weight tile as the A
// operand (the tile layout of mk_config.h) and the 16 sequences' activations
// as the B operand (column n = sequence n).  Activations are fp32 and enter
// the products as two bf16 parts (hi = RNE(v), lo = RNE(v - hi); relative
// error <= 2^-17), two products per tile.  Kernel boundaries order every
// hand-off, so activations are ordinary cached loads and stores; only the
// attention merge hands partials between workgroups of one launch (write-through
// stores, an agent-scope counter, agent-scope loads).
#pragma once
#include <type_traits>

#include "mk_config.h"
#include "mk_device.h"
#include "mk_host.h"

namespace mk {
namespace batch {

constexpr int BMAX = 16;       // sequences per step (MFMA columns)
constexpr int GT = 512;        // threads of the GEMM kernels (8 waves)
constexpr int GW = GT / kWave;
#ifndef MK_BATCH_AT
#define MK_BATCH_AT 256
#endif
constexpr int AT = MK_BATCH_AT;  // threads of an attention item (4 waves)
static_assert(AT >= 4 * kWave, "the attention prologue takes q0, q1, k and v on waves 0-3");
constexpr int AW = AT / kWave;
#ifndef MK_BATCH_NBW
#define MK_BATCH_NBW 2
#endif
constexpr int NBW = MK_BATCH_NBW;  // 32-position blocks per wave and attention item
constexpr int CH = 32 * AW * NBW;  // positions per attention split
constexpr int PW = 2 * 64 + 4; // partial words per item for GQA 2, D 64: o[2][64], (m, l) x 2
// K splits of the GEMM kernels (whole 32-column tiles per split)
// (measured: splitting pays only for the K = F down projection, 64 blocks of
// 88 tiles; the others lose more to the reduction than they gain)
constexpr int KS_QKV = 1, KS_O = 1, KS_GU = 1, KS_DN = 4;

// Hand-off flags of one layer in the single-kernel step (bk_step), one word
// per producer: QKV blocks, merged (sequence, kv head) attention outputs, O
// blocks, gate / up blocks, down blocks.  A producer writes the step's epoch
// into its word after its outputs are acknowledged; a consumer waits until
// every word it needs holds the epoch.  One writer per word and no atomics:
// a single counter that every producer incremented serialised the
// increments at one memory channel (5-10 us per hand-off).
enum : int { FC_QKV = 0, FC_ATT, FC_O, FC_GU, FC_DN, FC_N };
constexpr int FLAG_MAX = 256;  // producers per phase (>= F/16, QKV/16, BMAX * NKV)
// Optional timestamps of bk_step per layer and workgroup: layer start, then
// inputs ready / done of QKV, attention, O, gate/up and down (a workgroup
// without a role in a phase leaves that phase's stamps 0).
enum : int { TR_START = 0, TR_QKV_IN, TR_QKV_DONE, TR_ATT_IN, TR_ATT_DONE, TR_O_IN, TR_O_DONE, TR_GU_IN,
             TR_GU_DONE, TR_DN_IN, TR_DN_DONE, TR_N };

struct BParams {
  const u32x4* wqkv;        // per layer [QKV/16][H/32] tiles
  const u32x4* wo;          // per layer [H/16][QD/32]
  const u32x4* wg;          // per layer gate [F/16][H/32]
  const u32x4* wu;          // per layer up
  const u32x4* wd;          // per layer down [H/16][F/32]
  const u32x4* lmhead;      // [V/16][H/32]
  const u32x4* lmhead8;     // optional FP8 (e4m3) copy [V/16][H/64][64] (bk_lm<S, true>)
  const float* lm_scale;    // [V] its power-of-two row scales
  long long u_qkv, u_o, u_gu, u_dn;  // 16-byte units per layer of each matrix
  const uint16_t* norms;    // [L][NORM_STRIDE] bf16
  const uint16_t* final_norm;
  uint16_t* kv;             // K caches [B][L][NKV][s_pad][D]
  uint16_t* kvt;            // V^T caches [B][L][NKV][s_pad/32][D][32]
  long long kv_seq;         // elements per sequence in each region
  float* kscale;            // FP8 cache (null: bf16): power-of-two scale per K row and per V
  float* vscale;            //   row, [B][L][NKV][s_pad]; codes at byte index = element index
  long long sc_seq;         // scales per sequence
  int s_pad;
  // activations, per slot (x_slot .. act_slot below: L + 1 slots of x / xg /
  // ssq, L of qkv / att / act; the per-phase kernels use slot 0)
  float* x;                 // [slot][2 consumers][BMAX][H] residual streams
  uint16_t* xg;             // [slot][2 consumers][2 planes][BMAX][H] x * gain as bf16 hi / lo parts:
                            //   consumer 0 = attn_norm of the next QKV (or final_norm), 1 = ffn_norm
  float* ssq;               // [slot][2 consumers][H/16][BMAX] sums of squares of x per 16-row block
  float* qkv;               // [slot][BMAX][QKV] raw projections
  uint16_t* att;            // [slot][2][BMAX][QD] merged attention output, bf16 hi / lo parts
  uint16_t* act;            // [slot][2][BMAX][F] SiLU(g) * u, bf16 hi / lo parts
  float* part;              // [BMAX][NKV][nsplit_max][PW] attention partials
  int* cnt;                 // [BMAX][NKV] finished splits of the current layer
  float* gpart;             // split-K partial block sums of the GEMM kernels
  int* gcnt;                // [256] finished K splits per 16-row block
  u64* keys;                // [BMAX] argmax keys of the step
  int* tok;                 // [BMAX] input tokens of the step
  int* pos;                 // [BMAX] position of the step's token
  int* out;                 // [max_steps][BMAX] produced tokens
  int* step;                // step counter (row of out)
  float* dbg_logits;        // optional [BMAX][V]
  const float* inv_freq;    // [D/2]
  float* rope;              // [BMAX][2][D/2] cos / sin of the step's position per sequence
  int* flags;               // bk_step: [L][FC_N][FLAG_MAX] hand-off flags (epoch of the last write)
  int* epoch;               // step epoch: bk_embed adds one per step, never reset
  u64* trace;               // bk_step (optional): [L][TR_N][G] device wall-clock stamps per workgroup
  int* err;                 // bk_step: MK_ERR_TIMEOUT when a hand-off wait gave up
  unsigned long long timeout_ticks;  // bk_step: wall-clock ticks a hand-off wait may take
  int B, L, V, nsplit_max, max_steps;
  int prefill;              // 1: the columns are consecutive prompt tokens of one sequence whose
                            //    K / V bk_append has already stored (kv_seq = 0, shared cache)
};

// Up to PG_MAX column groups that share one pass over the weights: a prefill
// pass of up to 1,024 prompt tokens is up to 64 groups of 16 columns, each
// with its own activation buffers, tokens and positions (the decode step is
// one group).
// Every kernel takes the group as blockIdx.y; the GEMM workgroups of one
// 16-row block differ in blockIdx.y only, so they run on one XCD (grid x a
// multiple of 8) at about the same time and share the block's weights
// through that XCD's L2.
constexpr int PG_MAX = 64;
template <int N>
struct PGroupN {  // groups in the kernel argument
  static constexpr int NG = N;
  BParams p[N];
  int n;  // groups in use, 1 .. N
};
using PGroup1 = PGroupN<1>;  // the decode step
// A prefill pass: group 0's parameters; group gi's activation buffers (x, xg,
// ssq, qkv, att, act, part, cnt, gpart, gcnt, keys, rope) sit gi * gstride
// bytes after group 0's, its tokens and positions 16 gi entries after them.
struct PGroup {
  static constexpr int NG = PG_MAX;
  BParams p;
  long long gstride;
  int n, ntok;  // groups and tokens of the pass
};

template <class T>
__host__ __device__ __forceinline__ T* advance(T* q, long long bytes) {
  return reinterpret_cast<T*>(reinterpret_cast<char*>(q) + bytes);
}
// The parameters of column group gi of a pass (host and device), and of the
// workgroup's column group (blockIdx.y).
__host__ __device__ __forceinline__ BParams group_params(const PGroup& g, int gi) {
  const long long o = gi * g.gstride;
  BParams q = g.p;
  q.x = advance(q.x, o), q.xg = advance(q.xg, o), q.ssq = advance(q.ssq, o), q.qkv = advance(q.qkv, o);
  q.att = advance(q.att, o), q.act = advance(q.act, o), q.part = advance(q.part, o), q.cnt = advance(q.cnt, o);
  q.gpart = advance(q.gpart, o), q.gcnt = advance(q.gcnt, o), q.keys = advance(q.keys, o);
  q.rope = advance(q.rope, o);
  q.tok += BMAX * gi, q.pos += BMAX * gi;
  q.B = g.ntok - BMAX * gi < BMAX ? g.ntok - BMAX * gi : BMAX;
  return q;
}
__device__ __forceinline__ const BParams& group_of(const PGroup1& g) { return g.p[0]; }
__device__ __forceinline__ BParams group_of(const PGroup& g) { return group_params(g, blockIdx.y); }

// ------------------------------------------------------------ helpers
// bf16 parts of an fp32 value: hi = RNE(v), lo = RNE(v - hi).
__device__ __forceinline__ void split2(float v, uint16_t& hi, uint16_t& lo) {
  hi = f32_to_bf16(v);
  lo = f32_to_bf16(v - bf16_to_f32(hi));
}

// u32x4 holding 8 bf16 with element e (0..7) replaced by v, in registers.
__device__ __forceinline__ u32x4 with_bf16(u32x4 x, int e, uint16_t v) {
  const unsigned keep = (e & 1) ? 0x0000ffffu : 0xffff0000u;
  const unsigned put = (e & 1) ? ((unsigned)v << 16) : (unsigned)v;
  u32x4 r = x;
#pragma unroll
  for (int c = 0; c < 4; ++c) r[c] = (c == (e >> 1)) ? ((x[c] & keep) | put) : x[c];
  return r;
}

__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

// RMSNorm (reference rmsnorm.cuh:87-108) without a normalisation pass: the
// kernel that produces x also publishes x * gain as bf16 hi / lo parts (the B
// operand of the consuming product) and, per 16-row block and sequence, the
// sum of squares of its rows.  The consumer sums the H/16 partials in a fixed
// order, r_b = rsqrt(mean(x_b^2) + eps), and scales its outputs by r_b:
// W . (x * gain * r) = r * (W . (x * gain)).
// Activation slots.  The one-kernel step (bk_step) gives every layer its own
// copy of each activation buffer, so that within a launch every address is
// written once, before anything reads it: readers then use ordinary cached
// loads -- no cache can hold a stale copy, since every kernel starts with
// invalidated caches -- and only the writers' stores are write-through.  The
// per-phase kernels use slot 0 throughout (kernel boundaries order them).
// Slot s of x / xg / ssq holds, as consumer c = 0, the hidden state entering
// layer s with its attention-norm parts (s = L: the final-norm parts), and as
// c = 1 the state after layer s's O projection with its FFN-norm parts.
template <class S>
__device__ __forceinline__ float* x_slot(const BParams& p, int slot, int c) {
  return p.x + ((long long)(2 * slot + c) * BMAX) * S::H;
}
template <class S>
__device__ __forceinline__ uint16_t* xg_plane(const BParams& p, int slot, int c, int lohi) {
  return p.xg + ((long long)(4 * slot + 2 * c + lohi) * BMAX) * S::H;
}
template <class S>
__device__ __forceinline__ float* ssq_slot(const BParams& p, int slot, int c) {
  return p.ssq + (long long)(2 * slot + c) * (S::H / 16) * BMAX;
}
template <class S>
__device__ __forceinline__ float* qkv_slot(const BParams& p, int slot) {
  return p.qkv + (long long)slot * BMAX * S::QKV;
}
template <class S>
__device__ __forceinline__ uint16_t* att_slot(const BParams& p, int slot) {
  return p.att + (long long)slot * 2 * BMAX * S::QD;
}
template <class S>
__device__ __forceinline__ uint16_t* act_slot(const BParams& p, int slot) {
  return p.act + (long long)slot * 2 * BMAX * S::F;
}

// Epilogue of an x-producing 16-row block: thread t < 256 holds the new x of
// row rb * 16 + t / 16, sequence t % 16.  red: >= 256 floats of LDS.
// Stores of activations handed between workgroups: ordinary between kernels
// (SC1 false); inside the one-kernel step write-through at agent scope, and
// flagged on p.flags once acknowledged.
template <bool SC1, class T>
__device__ __forceinline__ void st_act(T* a, T v) {
  if constexpr (SC1) __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *a = v;
}

template <class S, bool SC1 = false>
__device__ __forceinline__ void publish_x(const BParams& p, int slot, int c, const uint16_t* gain, int rb, float xn,
                                          float* red) {
  const int t = ltid(), row = rb * 16 + t / 16, b = t % 16;
  if (t < 256) {
    const bool on = b < p.B;
    if (on) {
      st_act<SC1>(x_slot<S>(p, slot, c) + (long long)b * S::H + row, xn);
      uint16_t h, o;
      split2(xn * bf16_to_f32(gain[row]), h, o);
      st_act<SC1>(xg_plane<S>(p, slot, c, 0) + (long long)b * S::H + row, h);
      st_act<SC1>(xg_plane<S>(p, slot, c, 1) + (long long)b * S::H + row, o);
    }
    red[t] = on ? xn * xn : 0.f;
  }
  __syncthreads();
  if (t < BMAX) {
    float ss = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) ss += red[r * 16 + t];
    st_act<SC1>(ssq_slot<S>(p, slot, c) + (long long)rb * BMAX + t, ss);
  }
}

// r_b of slot / consumer c for b < BMAX into rr[0 .. BMAX) (read after a
// later barrier).  rr: RR_N floats of LDS; every thread of the workgroup
// calls this.  Sixteen threads per sequence each sum a run of the H/16 block
// sums (all their loads in flight together), then one thread per sequence
// adds the sixteen runs in order.
constexpr int RR_N = BMAX + 256;
template <class S>
__device__ __forceinline__ void rnorm(const BParams& p, int slot, int c, float* rr) {
  constexpr int NB = S::H / 16, PER = (NB + 15) / 16;
  const int t = ltid();
  if (t < 256) {
    const int b = t % 16, k = t / 16;
    const float* q = ssq_slot<S>(p, slot, c) + b;
    float v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) v[i] = k * PER + i < NB ? q[(k * PER + i) * BMAX] : 0.f;
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) sum += v[i];
    rr[BMAX + t] = sum;
  }
  __syncthreads();
  if (t < BMAX) {
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) ss += rr[BMAX + k * 16 + t];
    rr[t] = rsqrtf(ss / (float)S::H + kRmsEps);
  }
}

// This wave's tiles of one 16-row block (tiles kt = w, w + GW, ... of KT),
// loaded into registers: the A operands of the block product.  Issued before
// the activations are staged, so the two latencies overlap.
template <int NT>
struct ATiles {  // NT tiles of a K range; wave w holds local tiles w, w + GW, ...
  static constexpr int TW = (NT + GW - 1) / GW;
  u32x4 t[TW];
};
template <int NT>
__device__ __forceinline__ void load_tiles(ATiles<NT>& a, const u32x4* __restrict__ blk, int kt0) {
  const unsigned l = lane_id();
  const int w = wave_id();
  const auto rs = make_rsrc(blk);
#pragma unroll
  for (int j = 0; j < ATiles<NT>::TW; ++j)
    a.t[j] = w + GW * j < NT ? buf_ld_nt(rs, l * 16u, (unsigned)(kt0 + w + GW * j) * 1024u) : u32x4{0u, 0u, 0u, 0u};
}

// The 16 activation columns of this wave's tiles: the B operands.  Planes:
// element (n, k) at hi[n * ld + k], lo[n * ld + k].  Loaded on their own, so
// a block can issue its other loads (norm sums, residual) before it waits.
template <int NT>
struct BCols {
  u32x4 h[ATiles<NT>::TW], l[ATiles<NT>::TW];
};
template <int NT>
__device__ __forceinline__ void load_cols(BCols<NT>& c, const uint16_t* hi, const uint16_t* lo, int ld, int kt0) {
  const unsigned l = lane_id();
  const int w = wave_id();
  const int bo = (int)(l & 15u) * ld + 8 * (int)(l >> 4);
#pragma unroll
  for (int j = 0; j < ATiles<NT>::TW; ++j) {
    const int kt = kt0 + w + GW * j;
    if (w + GW * j < NT) {
      c.h[j] = *reinterpret_cast<const u32x4*>(hi + bo + 32 * kt);
      c.l[j] = *reinterpret_cast<const u32x4*>(lo + bo + 32 * kt);
    }
  }
}

// The tiles times the columns.  Lane (kg, n) returns rows 4 kg .. 4 kg + 3 of
// column n (this wave's share of the K sum).
template <int NT>
__device__ __forceinline__ f32x4 tiles_mma(const ATiles<NT>& a, const BCols<NT>& c) {
  const int w = wave_id();
  f32x4 a0 = f32x4{0.f, 0.f, 0.f, 0.f}, a1 = a0;
#pragma unroll
  for (int j = 0; j < ATiles<NT>::TW; ++j) {
    if (w + GW * j < NT) {
      a0 = mfma(a.t[j], c.h[j], a0);
      a1 = mfma(a.t[j], c.l[j], a1);
    }
  }
  return a0 + a1;
}

// Two blocks' tiles (gate and up) times the same columns; each result equals
// tiles_mma of that block.
template <int NT>
__device__ __forceinline__ void tiles_mma2(const ATiles<NT>& a, const ATiles<NT>& b, const BCols<NT>& c, f32x4& ra,
                                           f32x4& rb) {
  const int w = wave_id();
  f32x4 a0 = f32x4{0.f, 0.f, 0.f, 0.f}, a1 = a0, b0 = a0, b1 = a0;
#pragma unroll
  for (int j = 0; j < ATiles<NT>::TW; ++j) {
    if (w + GW * j < NT) {
      a0 = mfma(a.t[j], c.h[j], a0);
      a1 = mfma(a.t[j], c.l[j], a1);
      b0 = mfma(b.t[j], c.h[j], b0);
      b1 = mfma(b.t[j], c.l[j], b1);
    }
  }
  ra = a0 + a1;
  rb = b0 + b1;
}

// K splits of a 16-row block run on KS workgroups; each publishes its block
// sums (thread t < 256: row t / 16, column t % 16; NV values per thread) with
// write-through stores, and the workgroup that completes the block (an
// agent-scope counter) adds the KS partials in split order -- the same sum in
// every run -- and runs the epilogue.  Returns true in that workgroup, with
// v[] replaced by the totals.  `last`: one int of LDS.
template <int NV>
__device__ __forceinline__ bool splitk_finish(const BParams& p, int rb, int ks, int KS, float (&v)[NV], int* last) {
  if (KS == 1) return true;  // one workgroup per block: its sums are the totals
  const int t = ltid();
  float* buf = p.gpart + ((long long)rb * KS) * 256 * NV;
  if (t < 256) {
#pragma unroll
    for (int i = 0; i < NV; ++i)
      __hip_atomic_store(buf + ((long long)ks * NV + i) * 256 + t, v[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the partial is acknowledged before the count moves
  __syncthreads();
  if (t == 0) {
    const int done = __hip_atomic_fetch_add(p.gcnt + rb, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *last = done == KS - 1;
    if (*last) __hip_atomic_store(p.gcnt + rb, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // re-armed
  }
  __syncthreads();
  if (!*last) return false;
  if (t < 256) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      float sum = 0.f;
      for (int k = 0; k < KS; ++k)
        sum += __hip_atomic_load(buf + ((long long)k * NV + i) * 256 + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v[i] = sum;
    }
  }
  return true;
}

// Cross-wave sum of a block's partial products: red[GW][16][17] in LDS.
// Returns, for thread t < 256, the total of row t / 16, column t % 16.
__device__ __forceinline__ float block_reduce(f32x4 acc, float* red) {
  const unsigned l = lane_id();
  const int w = wave_id();
  const int n = (int)(l & 15u), kg = (int)(l >> 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) red[(w * 16 + 4 * kg + i) * 17 + n] = acc[i];
  __syncthreads();
  const int t = ltid();
  float s = 0.f;
  if (t < 256) {
#pragma unroll
    for (int ww = 0; ww < GW; ++ww) s += red[(ww * 16 + t / 16) * 17 + t % 16];
  }
  return s;
}

// ------------------------------------------------------------ kernels
// x[b] = E[tok[b]] (the tied embedding, gathered from the tile-layout LM head),
// published for layer 0's QKV.
template <class S, class G>
__global__ __launch_bounds__(256) void bk_embed(G pg) {
  __shared__ float xs[S::H];
  const BParams& p = group_of(pg);  // column group
  const int b = blockIdx.x;
  if (b >= BMAX) return;
  const int t = ltid();
  const bool on = b < p.B;
  const int t_ = on ? p.tok[b] : 0;
  const int tok = t_ < 0 ? 0 : (t_ >= p.V ? p.V - 1 : t_);  // tokens are validated on the host; never index outside
  for (int k = t; k < S::H; k += blockDim.x) {
    const int kt = k >> 5, q = (k >> 3) & 3, e = k & 7;
    const uint16_t* u = reinterpret_cast<const uint16_t*>(
        p.lmhead + ((long long)(tok >> 4) * S::KT_H + kt) * 64 + q * 16 + (tok & 15));
    const float xv = on ? bf16_to_f32(u[e]) : 0.f;
    xs[k] = xv;
    if (on) {
      x_slot<S>(p, 0, 0)[(long long)b * S::H + k] = xv;
      uint16_t h, o;
      split2(xv * bf16_to_f32(p.norms[S::NORM_ATTN + k]), h, o);
      xg_plane<S>(p, 0, 0, 0)[(long long)b * S::H + k] = h;
      xg_plane<S>(p, 0, 0, 1)[(long long)b * S::H + k] = o;
    }
  }
  __syncthreads();
  for (int rb = t; rb < S::H / 16; rb += blockDim.x) {
    float ss = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) ss += xs[rb * 16 + r] * xs[rb * 16 + r];
    ssq_slot<S>(p, 0, 0)[(long long)rb * BMAX + b] = ss;
  }
  if (t < S::D / 2) {  // RoPE angles of this step's position, shared by every layer
    float sn, cs;
    sincosf((float)(on ? p.pos[b] : 0) * p.inv_freq[t], &sn, &cs);
    p.rope[(b * 2 + 0) * (S::D / 2) + t] = cs;
    p.rope[(b * 2 + 1) * (S::D / 2) + t] = sn;
  }
  if (t == 0) p.keys[b] = 0ull;
  if (p.epoch && b == 0 && t == 0) *p.epoch += 1;  // this step's epoch for bk_step's hand-off flags
}

// Hand-off flag of producer `idx` of a phase of the one-kernel step: every
// thread's stores are acknowledged (write-through) before one thread writes
// the epoch.
__device__ __forceinline__ void fc_done(const BParams& p, int layer, int ph, int idx, int ep) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (ltid() == 0)
    __hip_atomic_store(p.flags + ((long long)layer * FC_N + ph) * FLAG_MAX + idx, ep, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until the flags of producers 0 .. n - 1 of phase ph of `layer` hold
// epoch ep: wave 0 polls them (up to FLAG_MAX / 64 words per lane, all loads
// of a round in flight together), the workgroup follows; false when the
// wait gave up (p.err is set).
__device__ __forceinline__ bool fc_wait(const BParams& p, int layer, int ph, int n, int ep) {
  int ok = 1;
  if (wave_id() == 0) {
    const auto rs = make_rsrc(p.flags + ((long long)layer * FC_N + ph) * FLAG_MAX);
    const unsigned l = lane_id();
    Spin sp;
    while (true) {
      int v[FLAG_MAX / kWave];
#pragma unroll
      for (int k = 0; k < FLAG_MAX / kWave; ++k)
        v[k] = (int)l + kWave * k < n ? (int)__builtin_amdgcn_raw_buffer_load_b32(rs, (l + kWave * k) * 4u, 0u, 16) : ep;
      bool ready = true;
#pragma unroll
      for (int k = 0; k < FLAG_MAX / kWave; ++k) ready &= v[k] == ep;
      if (__all(ready)) break;
      if (!sp.step(p.err, p.timeout_ticks)) {
        ok = 0;
        break;
      }
    }
  }
  return __syncthreads_and(ok) != 0;
}

// The GEMM phases as block functions.  FUSED (bk_step): the block's weight
// tiles are issued, then `ready()` waits for its inputs, which are read at
// agent scope, and the outputs are flagged on p.flags; otherwise (one kernel per
// phase) ready() is trivially true.  Each returns false only when ready()
// gave up.
struct NoWait {
  __device__ __forceinline__ bool operator()() const { return true; }
};

// rmsnorm(x) -> q|k|v rows of block rb for every sequence.
template <class S, bool FUSED, class Ready>
__device__ __forceinline__ bool qkv_block(const BParams& p, int layer, int ep, int rb, int ks, float* red, float* rr, int* last,
                                          const Ready& ready) {
  constexpr int NT = S::KT_H / KS_QKV;
  const int kt0 = ks * NT;
  ATiles<NT> a;
  load_tiles(a, p.wqkv + layer * p.u_qkv + (long long)rb * S::KT_H * 64, kt0);
  if (!ready()) return false;
  const int sl = FUSED ? layer : 0;
  BCols<NT> c;
  load_cols(c, xg_plane<S>(p, sl, 0, 0), xg_plane<S>(p, sl, 0, 1), S::H, kt0);
  rnorm<S>(p, sl, 0, rr);
  float v[1] = {block_reduce(tiles_mma(a, c), red)};
  if (!splitk_finish(p, rb, ks, KS_QKV, v, last)) return true;
  const int t = ltid(), row = rb * 16 + t / 16, b = t % 16;
  if (t < 256 && b < p.B) st_act<FUSED>(qkv_slot<S>(p, sl) + (long long)b * S::QKV + row, v[0] * rr[b]);
  if constexpr (FUSED) fc_done(p, layer, FC_QKV, rb, ep);
  return true;
}

// O projection + residual: x[b][row] += Wo[row] . att[b]; x published for the FFN norm.
template <class S, bool FUSED, class Ready>
__device__ __forceinline__ bool o_block(const BParams& p, int layer, int ep, int rb, int ks, float* red, int* last,
                                        const Ready& ready) {
  constexpr int NT = S::KT_Q / KS_O;
  const int kt0 = ks * NT;
  ATiles<NT> a;
  load_tiles(a, p.wo + layer * p.u_o + (long long)rb * S::KT_Q * 64, kt0);
  if (!ready()) return false;
  const int sl = FUSED ? layer : 0;
  const uint16_t* at = att_slot<S>(p, sl);
  BCols<NT> c;
  load_cols(c, at, at + BMAX * S::QD, S::QD, kt0);
  const int t = ltid(), b = t % 16;
  const float xin = t < 256 && b < p.B ? x_slot<S>(p, sl, 0)[(long long)b * S::H + rb * 16 + t / 16] : 0.f;
  float v[1] = {block_reduce(tiles_mma(a, c), red)};
  if (!splitk_finish(p, rb, ks, KS_O, v, last)) return true;
  const float xn = t < 256 && b < p.B ? xin + v[0] : 0.f;
  __syncthreads();  // red is reused
  publish_x<S, FUSED>(p, sl, 1, p.norms + (long long)layer * S::NORM_STRIDE + S::NORM_FFN, rb, xn, red);
  if constexpr (FUSED) fc_done(p, layer, FC_O, rb, ep);
  return true;
}

// rmsnorm(x) -> gate and up rows of block rb -> SiLU(g) * u parts.
template <class S, bool FUSED, class Ready>
__device__ __forceinline__ bool gu_block(const BParams& p, int layer, int ep, int rb, int ks, float* red, float* rr, int* last,
                                         const Ready& ready) {
  constexpr int NT = S::KT_H / KS_GU;
  const int kt0 = ks * NT;
  const long long off = (long long)rb * S::KT_H * 64;
  ATiles<NT> ag, au;
  load_tiles(ag, p.wg + layer * p.u_gu + off, kt0);
  load_tiles(au, p.wu + layer * p.u_gu + off, kt0);
  if (!ready()) return false;
  const int sl = FUSED ? layer : 0;
  BCols<NT> c;
  load_cols(c, xg_plane<S>(p, sl, 1, 0), xg_plane<S>(p, sl, 1, 1), S::H, kt0);
  rnorm<S>(p, sl, 1, rr);
  f32x4 pg, pu;
  tiles_mma2(ag, au, c, pg, pu);
  float v[2];
  v[0] = block_reduce(pg, red);
  __syncthreads();
  v[1] = block_reduce(pu, red);
  if (!splitk_finish(p, rb, ks, KS_GU, v, last)) return true;
  const int t = ltid(), row = rb * 16 + t / 16, b = t % 16;
  if (t < 256 && b < p.B) {
    const float g = v[0] * rr[b], u = v[1] * rr[b];
    uint16_t h, o;
    split2(g / (1.0f + __expf(-g)) * u, h, o);  // SiLU(g) * u (reference utils.cuh:59-61)
    st_act<FUSED>(act_slot<S>(p, sl) + (long long)b * S::F + row, h);
    st_act<FUSED>(act_slot<S>(p, sl) + (long long)(BMAX + b) * S::F + row, o);
  }
  if constexpr (FUSED) fc_done(p, layer, FC_GU, rb, ep);
  return true;
}

// Down projection + residual: x[b][row] += Wd[row] . act[b]; x published for
// the next layer's attention norm (the final norm after the last layer).
template <class S, bool FUSED, class Ready>
__device__ __forceinline__ bool down_block(const BParams& p, int layer, int ep, int rb, int ks, float* red, int* last,
                                           const Ready& ready) {
  static_assert(S::KT_F % KS_DN == 0, "whole tiles per K split");
  constexpr int NT = S::KT_F / KS_DN;
  const int kt0 = ks * NT;
  ATiles<NT> a;
  load_tiles(a, p.wd + layer * p.u_dn + (long long)rb * S::KT_F * 64, kt0);
  if (!ready()) return false;
  const int sl = FUSED ? layer : 0;
  const uint16_t* ac = act_slot<S>(p, sl);
  BCols<NT> c;
  load_cols(c, ac, ac + BMAX * S::F, S::F, kt0);
  const int t = ltid(), b = t % 16;
  // the residual, read by the workgroup that finishes the block (split 0 in
  // the one-kernel step, whichever split completes it otherwise)
  const float xin = (!FUSED || ks == 0) && t < 256 && b < p.B
                        ? x_slot<S>(p, sl, 1)[(long long)b * S::H + rb * 16 + t / 16]
                        : 0.f;
  float v[1] = {block_reduce(tiles_mma(a, c), red)};
  if constexpr (FUSED) {
    // K splits 1.. publish their sums as (value, tag) words; split 0 polls
    // them and adds the splits in order, as splitk_finish does
    u64* buf = reinterpret_cast<u64*>(p.gpart) + (long long)rb * KS_DN * 256;
    const unsigned tag = (unsigned)ep * 64u + (unsigned)layer;
    if (ks != 0) {
      if (t < 256) __hip_atomic_store(buf + ks * 256 + t, ((u64)tag << 32) | f32_bits(v[0]), __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
      return true;
    }
    int ok = 1;
    if (t < 256) {
      u64 wv[KS_DN - 1];
      Spin sp;
      while (true) {
        bool all = true;
#pragma unroll
        for (int k = 1; k < KS_DN; ++k) {
          wv[k - 1] = __hip_atomic_load(buf + k * 256 + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          all &= (unsigned)(wv[k - 1] >> 32) == tag;
        }
        if (all) break;
        if (!sp.step(p.err, p.timeout_ticks)) {
          ok = 0;
          break;
        }
      }
      float sum = 0.f;
      sum += v[0];
#pragma unroll
      for (int k = 1; k < KS_DN; ++k) sum += f32_from((unsigned)wv[k - 1]);
      v[0] = sum;
    }
    if (!__syncthreads_and(ok)) return false;
  } else if (!splitk_finish(p, rb, ks, KS_DN, v, last)) {
    return true;
  }
  const float xn = t < 256 && b < p.B ? xin + v[0] : 0.f;
  __syncthreads();  // red is reused
  const uint16_t* gain = layer + 1 < p.L ? p.norms + (long long)(layer + 1) * S::NORM_STRIDE + S::NORM_ATTN
                                         : p.final_norm;
  publish_x<S, FUSED>(p, FUSED ? layer + 1 : 0, 0, gain, rb, xn, red);
  if constexpr (FUSED) fc_done(p, layer, FC_DN, rb, ep);
  return true;
}

template <class S, class G>
__global__ __launch_bounds__(GT) void bk_qkv(G p, int layer) {
  __shared__ float red[GW * 16 * 17];
  __shared__ float rr[RR_N];
  __shared__ int last;
  qkv_block<S, false>(group_of(p), layer, 0, blockIdx.x / KS_QKV, blockIdx.x % KS_QKV, red, rr, &last, NoWait{});
}

template <class S, class G>
__global__ __launch_bounds__(GT) void bk_o(G p, int layer) {
  __shared__ float red[GW * 16 * 17];
  __shared__ int last;
  o_block<S, false>(group_of(p), layer, 0, blockIdx.x / KS_O, blockIdx.x % KS_O, red, &last, NoWait{});
}

template <class S, class G>
__global__ __launch_bounds__(GT) void bk_gu(G p, int layer) {
  __shared__ float red[GW * 16 * 17];
  __shared__ float rr[RR_N];
  __shared__ int last;
  gu_block<S, false>(group_of(p), layer, 0, blockIdx.x / KS_GU, blockIdx.x % KS_GU, red, rr, &last, NoWait{});
}

template <class S, class G>
__global__ __launch_bounds__(GT) void bk_down(G p, int layer) {
  __shared__ float red[GW * 16 * 17];
  __shared__ int last;
  down_block<S, false>(group_of(p), layer, 0, blockIdx.x / KS_DN, blockIdx.x % KS_DN, red, &last, NoWait{});
}

// ------------------------------------------------------------ prefill GEMMs
// A prefill pass has up to 64 column groups (1,024 tokens), so the GEMMs are
// real matrix products: the decode kernels' one-block workgroups would each
// re-read their group's activation columns (64 KB for K = 1,024) next to
// 32 KB of weights, bounded by L2 -> CU traffic.  The prefill kernels tile
// rows and column groups and stage both operands in LDS.  Per 16 x 16 tile
// the products are the decode kernels' MFMA tiles (weights as the A operand,
// the columns' bf16 hi / lo parts as two B operands), accumulated over the
// whole K by one wave, so no cross-wave reduction is needed.

// Tile shapes: MP row blocks (gate / up: block pairs of 16 gate + 16 up rows)
// x NG column groups per workgroup, K in chunks of KC tiles; each chunk's
// weight tiles and column tiles are staged in LDS once (double-buffered, the
// next chunk's loads in flight during the current chunk's products), so a
// weight byte is read from L2 once per NG groups and a column byte once per
// MP blocks.  Wave w owns WB blocks x WGR groups over the whole K; the
// epilogue runs on its accumulators.
template <int MP_, int NG_, int KC_, int WB_, int WGR_, int PD_ = 2, int NS_ = 0>
struct PTile {
  static constexpr int MP = MP_, NG = NG_, KC = KC_, WB = WB_, WGR = WGR_;
  static constexpr int PD = PD_;  // K chunks whose loads are in flight (1 or 2 register sets)
  // NS > 0: no register staging; NS LDS stages filled by direct-to-LDS loads
  // (pt_pipeline), NS - 1 chunks in flight
  static constexpr int NS = NS_;
  static_assert((MP / WB) * (NG / WGR) == GW, "every wave owns whole blocks x groups");
  static_assert(PD == 1 || PD == 2, "one or two register sets");
  static_assert(NS == 0 || NS >= 2, "two stages at least");
};

// One 16-byte load per lane straight into LDS (global_load_lds_dwordx4):
// lane l's bytes land at dst + 16 l, dst being the wave's (uniform) address,
// passed in M0.  It counts on vmcnt like any vector load and writes no
// register.  Inline assembly, so that the compiler does not add its own
// conservative wait for every such load in flight before each LDS read: the
// caller waits for exactly the loads it needs (wait_vmcnt).  M0 is declared
// clobbered (the compiler warns, M0 being reserved); the GEMM kernels that
// use this have no other M0 user (no compiler-issued LDS DMA, no indirect
// register indexing: every register array index is a compile-time constant).
__device__ __forceinline__ void lds_load16(const void* src, void* dst) {
  const unsigned m0 = __builtin_amdgcn_readfirstlane(
      (unsigned)(uintptr_t)(__attribute__((address_space(3))) void*)dst);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m0), "v"(src) : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// The K loop of a tiled GEMM over NS LDS stages filled by direct loads:
// chunk c goes to stage c % NS, issued NS - 1 chunks ahead (issue(c, stage),
// NI loads per lane).  Before multiplying chunk c a wave waits until its own
// loads of chunk c have landed (vmcnt: the later chunks' loads may stay in
// flight); the barrier after it makes every wave's share visible and retires
// the stage the next issue overwrites (multiplied in the previous iteration,
// whose LDS reads every wave has consumed before reaching the barrier).  The
// plain s_barrier: __syncthreads()' fence would wait for every load in
// flight.
template <int NS, int NC, int NI, class Issue, class Compute>
__device__ __forceinline__ void pt_pipeline(const Issue& issue, const Compute& compute) {
  static_assert(NC >= NS - 1, "the prologue fills NS - 1 stages");
#pragma unroll
  for (int c = 0; c < NS - 1; ++c) issue(c, c);
  for (int c = 0; c < NC; ++c) {
    if (c + NS - 1 <= NC) wait_vmcnt<(NS - 2) * NI>();
    else wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (c + NS - 1 < NC) issue(c + NS - 1, (c + NS - 1) % NS);
    compute(c % NS);
  }
  asm volatile("" ::: "memory");
}
// (measured per layer, us: gate / up <8,8,2,4,2> 46.5, <8,8,2,2,4> 47.3,
// <8,8,2,1,8> 50.2, <8,4,2,1,4> 67.4, <4,8,2,1,4> 71.9, <4,4,4,1,2> 61.6;
// QKV <8,2,2,2,1> 19.5, <8,2,2,1,2> 20.1, <4,4,2,1,2> 22.8, <4,2,4,1,1> 27.5,
// <4,4,4,1,2> 31.7, <8,8,2,1,8> 33.7; O <4,2,4,1,1> 20.7, <8,1,4,1,1> 20.6,
// <8,2,4,2,1> 22.1, <4,4,4,1,2> 23.7; down <4,2,4,1,1> 38.5, <8,1,4,1,1> 39.2,
// <8,2,4,2,1> 41.6, <4,4,4,1,2> 47.7, <2,4,4,1,1> 54.3.  A wave owning more
// blocks reads fewer LDS bytes per product.)
// gate / up: direct-to-LDS loads, K chunks of one tile, four stages (three
// chunks in flight): 44.0 -> 40.3 us against <8,8,2,4,2> with one register
// set (234 VGPRs)
using PTileGU = PTile<8, 8, 1, 4, 2, 1, 4>;
// gate / up of a pass of at most PT_SMALL_GROUPS groups: the 8 x 8 tile
// leaves too few workgroups (256 tokens: 44), 8 x 2 four times as many
// (measured, tok/s, 8 x 8 / 8 x 2: 128 tokens 37,869 / 44,851, 256 tokens
// 74,028 / 87,756, 512 tokens 138,672 / 154,683, 1,024 tokens 220,199 /
// 207,877)
using PTileGUs = PTile<8, 2, 2, 2, 1>;
#ifndef MK_PT_SMALL_GROUPS
#define MK_PT_SMALL_GROUPS 32
#endif
constexpr int PT_SMALL_GROUPS = MK_PT_SMALL_GROUPS;
// Direct-to-LDS loads (us per layer at 1,024 tokens): QKV three stages of
// two tiles (four, 96 KB of LDS, leave one workgroup per CU: 18.1 -> 21.1;
// chunks of four tiles 19.5); O and down 8 x 2 tiles, chunks of four tiles,
// three stages (144 KB: one workgroup per CU, 256 workgroups): O 20.9 ->
// 18.9, down 38.4 -> 32.3 (register-staged 4 x 2
// tiles before; down 4 x 2 with four direct-load stages 38.7, 8 x 2 with
// chunks of two tiles and three / four / six stages 33.2 / 33.0 / 35.1, 4 x 4
// 35.8).  Each wave owns 1 block x 2 groups in O and 2 blocks x 1 group in
// down: with 2 x 1 the epilogue's rows reach memory about twice (17.7 MB
// written per launch against 8.7 MB of output, WRITE_SIZE), with 1 x 2 once,
// at the same O time and 0.8 us more for down.
using PTileQKV = PTile<16, 2, 2, 4, 1, 2, 3>;  // 17.5 -> 16.7 us against 8 x 2 (16 x 2 with chunks of four: 18.9)
using PTileQKVs = PTile<8, 2, 2, 2, 1, 2, 3>;  // passes of at most PT_SMALL_GROUPS groups
using PTileO = PTile<8, 2, 4, 1, 2, 2, 3>;  // each wave 1 block x 2 groups (2 x 1 wrote its outputs twice)
using PTileOs = PTile<4, 2, 2, 1, 1, 2, 4>;  // passes of at most PT_SMALL_GROUPS groups (twice the workgroups)
using PTileDN = PTile<8, 2, 4, 2, 1, 1, 3>;
using PTileDNs = PTile<4, 2, 4, 1, 1, 2>;  // passes of at most PT_SMALL_GROUPS groups

template <class S, class T>
__global__ __launch_bounds__(GT) void bk_pgu_t(PGroup pg, int layer) {
  constexpr int MP = T::MP, NG = T::NG, KC = T::KC, WB = T::WB, WGR = T::WGR;
  constexpr int NT = S::KT_H, NC = NT / KC;
  constexpr int AU = 2 * MP * KC * kWave;  // u32x4 of a chunk's weight tiles
  constexpr int BU = NG * 2 * KC * kWave;  // ... of its column tiles
  constexpr int LA = AU / GT, LB = BU / GT;  // per thread
  static_assert(NT % KC == 0 && AU % GT == 0 && BU % GT == 0, "tile shape");
  constexpr int NSB = T::NS > 0 ? T::NS : 2;
  __shared__ u32x4 sa[NSB][2 * MP][KC][kWave];  // [buf][gate blocks | up blocks][tile][lane]
  __shared__ u32x4 sb[NSB][NG][2][KC][kWave];   // [buf][group][hi / lo][tile][lane]
  // workgroup i runs on XCD i % 8: tiles (r, c) numbered r * ct + c are dealt
  // to XCDs in contiguous runs, so a row tile's column tiles share an XCD's L2
  // (its 22 row tiles are no multiple of 8; with the plain grid order a
  // launch fetched 83 MB from beyond L2 for 11.5 MB of weights, and the
  // kernel took 46.3 instead of 44.0 us)
  const int ct = (int)gridDim.y, nw = (int)gridDim.x * ct, lin = (int)(blockIdx.y * gridDim.x + blockIdx.x);
  const int jt = nw % 8 == 0 ? (lin % 8) * (nw / 8) + lin / 8 : lin;
  const int rb0 = (jt / ct) * MP, g0 = (jt % ct) * NG, tid = ltid();
  const int ngr = pg.n - g0 < NG ? pg.n - g0 : NG;  // groups of this tile
  const BParams p0 = group_params(pg, g0);
  const u32x4* wgt[2] = {p0.wg + layer * p0.u_gu, p0.wu + layer * p0.u_gu};
  u32x4 ra[T::PD][LA], rbv[T::PD][LB];
  const auto load = [&](int c, u32x4(&xa)[LA], u32x4(&xb)[LB]) {
#pragma unroll
    for (int k = 0; k < LA; ++k) {
      const int i = tid + GT * k, blk = i / (KC * kWave), kt = (i / kWave) % KC, ln = i % kWave;
      xa[k] = __builtin_nontemporal_load(wgt[blk / MP] + ((long long)(rb0 + blk % MP) * NT + c * KC + kt) * 64 + ln);
    }
#pragma unroll
    for (int k = 0; k < LB; ++k) {
      const int i = tid + GT * k, gq = i / (2 * KC * kWave), pl = (i / (KC * kWave)) % 2;
      const int kt = (i / kWave) % KC, ln = i % kWave;
      xb[k] = u32x4{0u, 0u, 0u, 0u};
      if (gq < ngr)
        xb[k] = *reinterpret_cast<const u32x4*>(xg_plane<S>(group_params(pg, g0 + gq), 0, 1, pl) + (ln & 15) * S::H +
                                                 32 * (c * KC + kt) + 8 * (ln >> 4));
    }
  };
  const auto store = [&](int buf, const u32x4(&xa)[LA], const u32x4(&xb)[LB]) {
#pragma unroll
    for (int k = 0; k < LA; ++k) (&sa[buf][0][0][0])[tid + GT * k] = xa[k];
#pragma unroll
    for (int k = 0; k < LB; ++k) (&sb[buf][0][0][0][0])[tid + GT * k] = xb[k];
  };
  // direct loads: wave w moves whole 1 KB tiles w, w + 8, ... of a chunk
  const auto issue = [&](int c, int buf) {
    const int w = wave_id(), ln = (int)lane_id();
#pragma unroll
    for (int k = 0; k < LA; ++k) {
      const int t = w + GW * k, blk = t / KC, kt = t % KC;
      lds_load16(wgt[blk / MP] + ((long long)(rb0 + blk % MP) * NT + c * KC + kt) * 64 + ln, &sa[buf][blk][kt][0]);
    }
#pragma unroll
    for (int k = 0; k < LB; ++k) {
      const int t = w + GW * k, gq = t / (2 * KC), pl = (t / KC) % 2, kt = t % KC;
      const int gs = gq < ngr ? gq : 0;  // a group past the pass reads group 0 (its columns are never stored)
      lds_load16(xg_plane<S>(group_params(pg, g0 + gs), 0, 1, pl) + (ln & 15) * S::H + 32 * (c * KC + kt) +
                     8 * (ln >> 4),
                 &sb[buf][gq][pl][kt][0]);
    }
  };
  if constexpr (T::NS == 0) {
    load(0, ra[0], rbv[0]);
    store(0, ra[0], rbv[0]);
    if constexpr (T::PD == 2)
      if (NC > 1) load(1, ra[T::PD - 1], rbv[T::PD - 1]);
    __syncthreads();
  }
  const int w = wave_id(), pw = (w / (NG / WGR)) * WB, gb = (w % (NG / WGR)) * WGR;
  const unsigned l = lane_id();
  f32x4 acc[WB][WGR][2][2];  // [block][group][gate / up][hi / lo part]
#pragma unroll
  for (int r = 0; r < WB; ++r)
#pragma unroll
    for (int j = 0; j < WGR; ++j)
#pragma unroll
      for (int m = 0; m < 2; ++m) acc[r][j][m][0] = acc[r][j][m][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  const auto compute = [&](int buf) {
#pragma unroll
    for (int kt = 0; kt < KC; ++kt) {
#pragma unroll
      for (int r = 0; r < WB; ++r) {
        const u32x4 ag = sa[buf][pw + r][kt][l], au = sa[buf][MP + pw + r][kt][l];
#pragma unroll
        for (int j = 0; j < WGR; ++j) {
          const u32x4 bh = sb[buf][gb + j][0][kt][l], bl = sb[buf][gb + j][1][kt][l];
          acc[r][j][0][0] = mfma(ag, bh, acc[r][j][0][0]);
          acc[r][j][0][1] = mfma(ag, bl, acc[r][j][0][1]);
          acc[r][j][1][0] = mfma(au, bh, acc[r][j][1][0]);
          acc[r][j][1][1] = mfma(au, bl, acc[r][j][1][1]);
        }
      }
    }
  };
  if constexpr (T::NS > 0) {
    pt_pipeline<T::NS, NC, LA + LB>(issue, compute);
  } else if constexpr (T::PD == 1) {
    for (int c = 0; c < NC; ++c) {
      if (c + 1 < NC) load(c + 1, ra[0], rbv[0]);
      compute(c & 1);
      if (c + 1 < NC) store((c + 1) & 1, ra[0], rbv[0]);
      __syncthreads();
    }
  } else {
    // chunk k sits in register set k & 1, then in LDS buffer k & 1: while a
    // chunk is multiplied, the next one waits in registers and the one after
    // it is loading
    for (int c = 0; c < NC; c += 2) {
      if (c + 2 < NC) load(c + 2, ra[0], rbv[0]);
      compute(0);
      if (c + 1 < NC) store(1, ra[T::PD - 1], rbv[T::PD - 1]);
      __syncthreads();
      if (c + 1 >= NC) break;
      if (c + 3 < NC) load(c + 3, ra[T::PD - 1], rbv[T::PD - 1]);
      compute(1);
      if (c + 2 < NC) store(0, ra[0], rbv[0]);
      __syncthreads();
    }
  }
  // epilogue: lane (kg, n) holds rows 4 kg .. 4 kg + 3 of column n
  const int n = (int)(l & 15u), kg = (int)(l >> 4);
#pragma unroll
  for (int j = 0; j < WGR; ++j) {
    if (gb + j >= ngr) break;
    const BParams p = group_params(pg, g0 + gb + j);
    constexpr int NB = S::H / 16, PER = NB / 4;
    const float* q = ssq_slot<S>(p, 0, 1) + n;
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) ss += q[(kg * PER + i) * BMAX];
    ss = sum_xor32(sum_xor16(ss));
    const float rs = rsqrtf(ss / (float)S::H + kRmsEps);
    if (n < p.B) {
#pragma unroll
      for (int r = 0; r < WB; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = (rb0 + pw + r) * 16 + 4 * kg + i;
          const float g = (acc[r][j][0][0][i] + acc[r][j][0][1][i]) * rs;
          const float u = (acc[r][j][1][0][i] + acc[r][j][1][1][i]) * rs;
          uint16_t h, o;
          split2(g / (1.0f + __expf(-g)) * u, h, o);  // SiLU(g) * u (reference utils.cuh:59-61)
          act_slot<S>(p, 0)[(long long)n * S::F + row] = h;
          act_slot<S>(p, 0)[(long long)(BMAX + n) * S::F + row] = o;
        }
    }
  }
}

// QKV, O and down as LDS-tiled GEMMs, as bk_pgu_t with one weight matrix.
// Epilogues: QKV scales by the
// group's norm factor; O and down add the residual and publish x (the next
// norm's bf16 parts and per-block sums of squares) as publish_x does.
enum PtOp : int { PT_QKV = 0, PT_O = 1, PT_DN = 2 };
template <class S, int OP, class T>
__global__ __launch_bounds__(GT) void bk_ptile(PGroup pg, int layer) {
  constexpr int MP = T::MP, NG = T::NG, KC = T::KC, WB = T::WB, WGR = T::WGR;
  constexpr int K = OP == PT_QKV ? S::H : (OP == PT_O ? S::QD : S::F);
  constexpr int NT = K / 32, NC = NT / KC;
  constexpr int AU = MP * KC * kWave, BU = NG * 2 * KC * kWave;
  constexpr int LA = AU / GT, LB = BU / GT;
  static_assert(NT % KC == 0 && AU % GT == 0 && BU % GT == 0, "tile shape");
  constexpr int NSB = T::NS > 0 ? T::NS : 2;
  __shared__ u32x4 sa[NSB][MP][KC][kWave];
  __shared__ u32x4 sb[NSB][NG][2][KC][kWave];
  const int rb0 = blockIdx.x * MP, g0 = blockIdx.y * NG, tid = ltid();
  const int ngr = pg.n - g0 < NG ? pg.n - g0 : NG;
  const BParams p0 = group_params(pg, g0);
  const u32x4* wm = OP == PT_QKV ? p0.wqkv + layer * p0.u_qkv
                                 : (OP == PT_O ? p0.wo + layer * p0.u_o : p0.wd + layer * p0.u_dn);
  // column planes of group q: hi at plane(q, 0), lo at plane(q, 1), [BMAX][K]
  const auto plane = [&](const BParams& q, int pl) -> const uint16_t* {
    if constexpr (OP == PT_QKV) return xg_plane<S>(q, 0, 0, pl);
    if constexpr (OP == PT_O) return att_slot<S>(q, 0) + (long long)pl * BMAX * S::QD;
    return act_slot<S>(q, 0) + (long long)pl * BMAX * S::F;
  };
  u32x4 ra[T::PD][LA], rbv[T::PD][LB];
  const auto load = [&](int c, u32x4(&xa)[LA], u32x4(&xb)[LB]) {
#pragma unroll
    for (int k = 0; k < LA; ++k) {
      const int i = tid + GT * k, blk = i / (KC * kWave), kt = (i / kWave) % KC, ln = i % kWave;
      xa[k] = __builtin_nontemporal_load(wm + ((long long)(rb0 + blk) * NT + c * KC + kt) * 64 + ln);
    }
#pragma unroll
    for (int k = 0; k < LB; ++k) {
      const int i = tid + GT * k, gq = i / (2 * KC * kWave), pl = (i / (KC * kWave)) % 2;
      const int kt = (i / kWave) % KC, ln = i % kWave;
      xb[k] = u32x4{0u, 0u, 0u, 0u};
      if (gq < ngr)
        xb[k] = *reinterpret_cast<const u32x4*>(plane(group_params(pg, g0 + gq), pl) + (ln & 15) * K +
                                                 32 * (c * KC + kt) + 8 * (ln >> 4));
    }
  };
  const auto store = [&](int buf, const u32x4(&xa)[LA], const u32x4(&xb)[LB]) {
#pragma unroll
    for (int k = 0; k < LA; ++k) (&sa[buf][0][0][0])[tid + GT * k] = xa[k];
#pragma unroll
    for (int k = 0; k < LB; ++k) (&sb[buf][0][0][0][0])[tid + GT * k] = xb[k];
  };
  // direct loads: wave w moves whole 1 KB tiles w, w + 8, ... of a chunk
  const auto issue = [&](int c, int buf) {
    const int w = wave_id(), ln = (int)lane_id();
#pragma unroll
    for (int k = 0; k < LA; ++k) {
      const int t = w + GW * k, blk = t / KC, kt = t % KC;
      lds_load16(wm + ((long long)(rb0 + blk) * NT + c * KC + kt) * 64 + ln, &sa[buf][blk][kt][0]);
    }
#pragma unroll
    for (int k = 0; k < LB; ++k) {
      const int t = w + GW * k, gq = t / (2 * KC), pl = (t / KC) % 2, kt = t % KC;
      const int gs = gq < ngr ? gq : 0;  // a group past the pass reads group 0 (its columns are never stored)
      lds_load16(plane(group_params(pg, g0 + gs), pl) + (ln & 15) * K + 32 * (c * KC + kt) + 8 * (ln >> 4),
                 &sb[buf][gq][pl][kt][0]);
    }
  };
  if constexpr (T::NS == 0) {
    load(0, ra[0], rbv[0]);
    store(0, ra[0], rbv[0]);
    if constexpr (T::PD == 2)
      if (NC > 1) load(1, ra[T::PD - 1], rbv[T::PD - 1]);
    __syncthreads();
  }
  const int w = wave_id(), pw = (w / (NG / WGR)) * WB, gb = (w % (NG / WGR)) * WGR;
  const unsigned l = lane_id();
  f32x4 acc[WB][WGR][2];  // [block][group][hi / lo part]
#pragma unroll
  for (int r = 0; r < WB; ++r)
#pragma unroll
    for (int j = 0; j < WGR; ++j) acc[r][j][0] = acc[r][j][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  const auto compute = [&](int buf) {
#pragma unroll
    for (int kt = 0; kt < KC; ++kt) {
#pragma unroll
      for (int r = 0; r < WB; ++r) {
        const u32x4 a = sa[buf][pw + r][kt][l];
#pragma unroll
        for (int j = 0; j < WGR; ++j) {
          acc[r][j][0] = mfma(a, sb[buf][gb + j][0][kt][l], acc[r][j][0]);
          acc[r][j][1] = mfma(a, sb[buf][gb + j][1][kt][l], acc[r][j][1]);
        }
      }
    }
  };
  if constexpr (T::NS > 0) {
    pt_pipeline<T::NS, NC, LA + LB>(issue, compute);
  } else if constexpr (T::PD == 1) {
    for (int c = 0; c < NC; ++c) {
      if (c + 1 < NC) load(c + 1, ra[0], rbv[0]);
      compute(c & 1);
      if (c + 1 < NC) store((c + 1) & 1, ra[0], rbv[0]);
      __syncthreads();
    }
  } else {
    // chunk k sits in register set k & 1, then in LDS buffer k & 1: while a
    // chunk is multiplied, the next one waits in registers and the one after
    // it is loading
    for (int c = 0; c < NC; c += 2) {
      if (c + 2 < NC) load(c + 2, ra[0], rbv[0]);
      compute(0);
      if (c + 1 < NC) store(1, ra[T::PD - 1], rbv[T::PD - 1]);
      __syncthreads();
      if (c + 1 >= NC) break;
      if (c + 3 < NC) load(c + 3, ra[T::PD - 1], rbv[T::PD - 1]);
      compute(1);
      if (c + 2 < NC) store(0, ra[0], rbv[0]);
      __syncthreads();
    }
  }
  // epilogue: lane (kg, n) holds rows 4 kg .. 4 kg + 3 of column n
  const int n = (int)(l & 15u), kg = (int)(l >> 4);
#pragma unroll
  for (int j = 0; j < WGR; ++j) {
    if (gb + j >= ngr) break;
    const BParams p = group_params(pg, g0 + gb + j);
    const bool on = n < p.B;
    if constexpr (OP == PT_QKV) {
      constexpr int NB = S::H / 16, PER = NB / 4;
      const float* q = ssq_slot<S>(p, 0, 0) + n;
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < PER; ++i) ss += q[(kg * PER + i) * BMAX];
      ss = sum_xor32(sum_xor16(ss));
      const float rs = rsqrtf(ss / (float)S::H + kRmsEps);
      if (on) {
#pragma unroll
        for (int r = 0; r < WB; ++r)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            qkv_slot<S>(p, 0)[(long long)n * S::QKV + (rb0 + pw + r) * 16 + 4 * kg + i] =
                (acc[r][j][0][i] + acc[r][j][1][i]) * rs;
      }
    } else {
      // O: residual stream copy 0 in, copy 1 + the FFN norm's parts out;
      // down: copy 1 in, copy 0 + the next layer's (or the final) norm out
      constexpr int CI = OP == PT_O ? 0 : 1, CO = 1 - CI;
      const uint16_t* gain = OP == PT_O ? p.norms + (long long)layer * S::NORM_STRIDE + S::NORM_FFN
                                        : (layer + 1 < p.L ? p.norms + (long long)(layer + 1) * S::NORM_STRIDE +
                                                                 S::NORM_ATTN
                                                           : p.final_norm);
#pragma unroll
      for (int r = 0; r < WB; ++r) {
        const int rb = rb0 + pw + r;
        float sq = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = rb * 16 + 4 * kg + i;
          const long long e = (long long)n * S::H + row;
          const float xn = on ? x_slot<S>(p, 0, CI)[e] + (acc[r][j][0][i] + acc[r][j][1][i]) : 0.f;
          if (on) {
            x_slot<S>(p, 0, CO)[e] = xn;
            uint16_t h, o;
            split2(xn * bf16_to_f32(gain[row]), h, o);
            xg_plane<S>(p, 0, CO, 0)[e] = h;
            xg_plane<S>(p, 0, CO, 1)[e] = o;
          }
          sq += xn * xn;
        }
        sq = sum_xor32(sum_xor16(sq));
        if (kg == 0) ssq_slot<S>(p, 0, CO)[(long long)rb * BMAX + n] = sq;
      }
    }
  }
}

// Final rmsnorm -> tied LM head -> per-sequence argmax (reference
// sampling.cuh:32-117).  Each wave scores whole 16-row blocks; keys are
// ordered(logit) << 32 | (0xffffffff - index), combined with an atomic max, so
// the result is the largest logit and, among equal logits, the lowest index.
template <class S, bool F8 = false>
__global__ __launch_bounds__(GT) void bk_lm(BParams p, int slot) {
  // F8: the FP8 copy; a lane's 16 bytes (row l & 15, columns 64 u + 16 kg ..
  // + 15 of unit u) feed two MFMA k-steps, whose B operands take the same
  // columns of the hidden state; the row scale enters the conversion
  constexpr int LD = S::H + 8;  // padded LDS rows: the 16 sequences on different banks
  __shared__ __attribute__((aligned(16))) uint16_t hi[BMAX * LD], lo[BMAX * LD];
  __shared__ u64 best_w[GW][BMAX];
  __shared__ float rr[RR_N];
  {  // the final-norm parts published by the last layer, copied to LDS
    const uint16_t *gh = xg_plane<S>(p, slot, 0, 0), *gl = xg_plane<S>(p, slot, 0, 1);
    for (int i = threadIdx.x; i < BMAX * S::H / 8; i += GT) {
      const int b = i / (S::H / 8), k = (i % (S::H / 8)) * 8;
      *reinterpret_cast<u32x4*>(hi + b * LD + k) = *reinterpret_cast<const u32x4*>(gh + (long long)b * S::H + k);
      *reinterpret_cast<u32x4*>(lo + b * LD + k) = *reinterpret_cast<const u32x4*>(gl + (long long)b * S::H + k);
    }
    rnorm<S>(p, slot, 0, rr);
  }
  __syncthreads();
  const unsigned l = lane_id();
  const int w = wave_id();
  const int n = (int)(l & 15u), kg = (int)(l >> 4);
  const int nb = p.V / 16;
  const int bo = n * LD + 8 * kg;
  const float rn = rr[n];
  u64 best = 0ull;
  // the wave's blocks rb0, rb0 + stride, ... as a flat sequence of chunks of
  // U tiles; the next chunk's loads are issued before the current one's products
  constexpr int KT = F8 ? S::H / 64 : S::KT_H;  // 1 KiB units per 16-row block
  constexpr int U = KT < 8 ? KT : 8, CPB = KT / U;  // chunks per block
  static_assert(KT % U == 0, "whole chunks per block");
  const int rb0 = blockIdx.x * GW + w, stride = gridDim.x * GW;
  const int nblk = rb0 < nb ? (nb - 1 - rb0) / stride + 1 : 0;
  const int nch = nblk * CPB;
  u32x4 cur[U], nxt[U];
  auto load_chunk = [&](int c, u32x4* dst) {
    const int rb = rb0 + (c / CPB) * stride, k0 = (c % CPB) * U;
    const auto rs = make_rsrc((F8 ? p.lmhead8 : p.lmhead) + (long long)rb * KT * 64);
#pragma unroll
    for (int u = 0; u < U; ++u) dst[u] = buf_ld_nt(rs, l * 16u, (unsigned)(k0 + u) * 1024u);
  };
  if (nch > 0) load_chunk(0, cur);
  f32x4 a0 = f32x4{0.f, 0.f, 0.f, 0.f}, a1 = a0;
  for (int c = 0; c < nch; ++c) {
    if (c + 1 < nch) load_chunk(c + 1, nxt);
    const int k0 = (c % CPB) * U;
    if constexpr (F8) {
      const float sc = p.lm_scale[(long long)(rb0 + (c / CPB) * stride) * 16 + n];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int kt = k0 + u;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const u32x4 wb = fp8x8_to_bf16x8_scaled(half ? u32x2{cur[u][2], cur[u][3]} : u32x2{cur[u][0], cur[u][1]}, sc);
          const int col = 64 * kt + 16 * kg + 8 * half - 8 * kg;  // bo already holds 8 kg
          a0 = mfma(wb, *reinterpret_cast<const u32x4*>(hi + bo + col), a0);
          a1 = mfma(wb, *reinterpret_cast<const u32x4*>(lo + bo + col), a1);
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int kt = k0 + u;
        a0 = mfma(cur[u], *reinterpret_cast<const u32x4*>(hi + bo + 32 * kt), a0);
        a1 = mfma(cur[u], *reinterpret_cast<const u32x4*>(lo + bo + 32 * kt), a1);
      }
    }
    if (c % CPB == CPB - 1) {  // the block is complete
      const int rb = rb0 + (c / CPB) * stride;
      const f32x4 acc = (a0 + a1) * rn;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const unsigned idx = (unsigned)(rb * 16 + 4 * kg + i);
        if (p.dbg_logits && n < p.B) p.dbg_logits[(long long)n * p.V + idx] = acc[i];
        const u64 key = ((u64)f32_order_key(acc[i]) << 32) | (u64)(0xffffffffu - idx);
        best = key > best ? key : best;
      }
      a0 = a1 = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) cur[u] = nxt[u];
  }
  // lanes n, n + 16, n + 32, n + 48 hold column n
#pragma unroll
  for (int m = 16; m <= 32; m <<= 1) {
    const u64 o = __shfl_xor(best, m);
    best = o > best ? o : best;
  }
  if (kg == 0) best_w[w][n] = best;
  __syncthreads();
  const int t = threadIdx.x;
  if (t < p.B) {
    u64 b = 0ull;
#pragma unroll
    for (int ww = 0; ww < GW; ++ww) b = best_w[ww][t] > b ? best_w[ww][t] : b;
    atomicMax(reinterpret_cast<unsigned long long*>(p.keys + t), (unsigned long long)b);
  }
}

// Tokens of the step from the argmax keys; positions advance.
__global__ void bk_tok(BParams p) {
  const int b = threadIdx.x;
  const int s = *p.step;
  if (b < p.B) {
    const int tok = (int)(0xffffffffu - (unsigned)(p.keys[b] & 0xffffffffull));
    p.tok[b] = tok;
    if (s < p.max_steps) p.out[(long long)s * BMAX + b] = tok;
    p.pos[b] += 1;
  }
  __syncthreads();
  if (b == 0) *p.step = s + 1;
}

// ------------------------------------------------------------ prefill
// K / V of every column's position stored before the layer's attention reads
// the cache: in a prefill the columns are consecutive prompt tokens of ONE
// sequence (shared cache), and column b attends to the positions of columns
// < b, which no bk_attn item of the same launch may still be writing.  Same
// arithmetic as bk_attn's prologue: k = RoPE(k_norm(k)), both stored as bf16
// (reference kv_cache.cuh:58-78).  One workgroup per (column, kv head): wave
// 0 stores k, wave 1 stores v.
template <class S, bool K8, class G>
__global__ __launch_bounds__(2 * kWave) void bk_append(G pg, int layer) {
  const BParams& p = group_of(pg);  // column group
  // K8: FP8 rows (codes + the row's power-of-two scale from the wave's maximum)
  static_assert(S::D == kWave, "one lane per head dimension");
  constexpr int D = S::D, NKV = S::NKV;
  const int b = blockIdx.x / NKV, g = blockIdx.x % NKV;
  if (b >= p.B) return;
  const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
  const int pos = p.pos[b];
  const long long kbase = (long long)b * p.kv_seq + ((long long)layer * NKV + g) * (long long)p.s_pad * D;
  float v = qkv_slot<S>(p, 0)[(long long)b * S::QKV + (w == 0 ? S::QD + g * D : S::QD + S::KVD + g * D) + l];
  if (w == 0) {
    const float ss = wave_sum(v * v);
    v = v * rsqrtf(ss / (float)D + kRmsEps) *
        bf16_to_f32(p.norms[(long long)layer * S::NORM_STRIDE + S::NORM_K + l]);
    const float partner = lane_xor32(v);
    const int d = l & 31;
    const float c = p.rope[(b * 2 + 0) * (D / 2) + d], sn = p.rope[(b * 2 + 1) * (D / 2) + d];
    v = l < 32 ? v * c - partner * sn : v * c + partner * sn;
  }
  const long long at = w == 0 ? kbase + (long long)pos * D + l
                              : kbase + (long long)(pos / 32) * 32 * D + (long long)l * 32 + (pos % 32);
  if constexpr (K8) {
    const int e = e4m3_row_exp(wave_max(fabsf(v)));
    reinterpret_cast<uint8_t*>(w == 0 ? p.kv : p.kvt)[at] = (uint8_t)e4m3_encode(ldexpf(v, -e));
    if (l == 0)
      (w == 0 ? p.kscale : p.vscale)[(long long)b * p.sc_seq + ((long long)layer * NKV + g) * p.s_pad + pos] =
          ldexpf(1.f, e);
  } else {
    (w == 0 ? p.kv : p.kvt)[at] = f32_to_bf16(v);
  }
}

// ------------------------------------------------------------ attention
// One item = (sequence b, kv head g, split s) of CH positions; wave w takes
// the 32-position block 4 s + w.  Both products of a block run on the matrix
// cores exactly as the batch-1 kernel does: scores^T = K . Qb with q split into
// three bf16 parts in rows 4 j + 0..2 (j = q head of the group), and
// out^T = V^T . Pb with the softmax weights split the same way.
template <class S>
struct AttnLds {
  static constexpr int D = S::D;
  float kcs[2];  // FP8: scales of position pos's K / V rows
  __attribute__((aligned(16))) uint16_t qb[16][D];       // q parts (A operand of the scores)
  __attribute__((aligned(16))) uint16_t pb[AW][16][32];  // weight parts (A operand of the output)
  __attribute__((aligned(16))) uint16_t kcur[D], vcur[D];  // K / V of position pos
  float rc[D / 2], rsn[D / 2];
  float mw[AW][2], lw[AW][2], ow[AW][2][D];
  float cm[AT / (2 * D)][2 * D], cl[AT / (2 * D)][2 * D], co[AT / (2 * D)][2 * D];  // split-group merge
  int last;
};

// K / V registers of one item: the wave's NBW 32-position blocks (4 s + w) +
// AW * q (blocks past the item repeat a valid block).  K8: the FP8 cache
// (codes converted to bf16 in registers, exact; the K row scale enters that
// conversion, the V row scale the softmax weight).
template <class S, bool K8>
struct AttnKV {
  using Reg = typename std::conditional<K8, u32x2, u32x4>::type;
  Reg kr[NBW][2][2], vr[NBW][S::D / 16];
  float sk[K8 ? NBW : 1][2], sv[K8 ? NBW : 1][2];  // FP8: scales of the lane's score positions
};
template <class S, bool K8>
__device__ __forceinline__ void attn_kv_load(const BParams& p, int layer, bool on, int b, int g, int s, int pos,
                                             AttnKV<S, K8>& r) {
  constexpr int D = S::D, NKV = S::NKV;
  const int n = on ? pos + 1 : 0;
  const int tid = ltid() % AT, w = tid / kWave, l = tid % kWave;
  const unsigned lu = (unsigned)l;
  const long long kbase = (long long)b * p.kv_seq + ((long long)layer * NKV + g) * (long long)p.s_pad * D;
  const long long sbase = (long long)b * p.sc_seq + ((long long)layer * NKV + g) * p.s_pad;
  if (!on) {  // no item: the registers hold nothing (no value carried from an earlier item)
#pragma unroll
    for (int q = 0; q < NBW; ++q) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) r.kr[q][h][kc] = __builtin_nondeterministic_value(r.kr[q][h][kc]);
        if constexpr (K8) {
          r.sk[q][h] = __builtin_nondeterministic_value(r.sk[q][h]);
          r.sv[q][h] = __builtin_nondeterministic_value(r.sv[q][h]);
        }
      }
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) r.vr[q][dt] = __builtin_nondeterministic_value(r.vr[q][dt]);
    }
    return;
  }
#pragma unroll
  for (int q = 0; q < NBW; ++q) {
    int blk = s * AW * NBW + w + AW * q;
    blk = 32 * blk < n ? blk : s * AW * NBW;
    if constexpr (K8) {  // byte index = element index of the bf16 layout
      const auto rk = make_rsrc(reinterpret_cast<const uint8_t*>(p.kv) + kbase + (long long)blk * 32 * D);
      const auto rv = make_rsrc(reinterpret_cast<const uint8_t*>(p.kvt) + kbase + (long long)blk * 32 * D);
      const auto rks = make_rsrc(p.kscale + sbase + (long long)blk * 32);
      const auto rvs = make_rsrc(p.vscale + sbase + (long long)blk * 32);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
          r.kr[q][h][kc] =
              __builtin_amdgcn_raw_buffer_load_b64(rk, (16u * h + (lu & 15u)) * D + 32u * kc + 8u * (lu >> 4), 0u, 2);
        r.sk[q][h] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rks, (16u * h + (lu & 15u)) * 4u, 0u, 2));
        r.sv[q][h] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rvs, (16u * h + (lu & 15u)) * 4u, 0u, 2));
      }
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt)
        r.vr[q][dt] = __builtin_amdgcn_raw_buffer_load_b64(rv, (16u * dt + (lu & 15u)) * 32u + 8u * (lu >> 4), 0u, 2);
    } else {
      const auto rk = make_rsrc(p.kv + kbase + (long long)blk * 32 * D);
      const auto rv = make_rsrc(p.kvt + kbase + (long long)blk * 32 * D);
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
          r.kr[q][h][kc] = __builtin_amdgcn_raw_buffer_load_b128(
              rk, ((16u * h + (lu & 15u)) * D + 32u * kc + 8u * (lu >> 4)) * 2u, 0u, 2);
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt)
        r.vr[q][dt] =
            __builtin_amdgcn_raw_buffer_load_b128(rv, ((16u * dt + (lu & 15u)) * 32u + 8u * (lu >> 4)) * 2u, 0u, 2);
    }
  }
}

// The item's code for AT threads (local thread threadIdx.x % AT).
// FUSED: inside bk_step, where the two AT-thread halves of a workgroup run
// two items and share every barrier: `on` false (a half without an item)
// passes the barriers only; the item reads its layer's qkv slot and writes
// its layer's att slot (write-through), flagged on p.flags.  Otherwise (bk_attn) one
// item per workgroup, always on.
// ready(): as for the GEMM blocks, between the K / V loads and the first read
// of q / k / v; the return is false only when it gave up.
template <class S, bool K8, bool FUSED, class Ready>
__device__ __forceinline__ bool attn_item(const BParams& p, int layer, int ep, AttnLds<S>& sm, bool on, int b, int g,
                                          int s, int nsplit, int pos, AttnKV<S, K8>& kv, const Ready& ready) {
  static_assert(S::GQA == 2 && S::D == 64, "batched attention is built for 2 q heads of 64 per kv head");
  constexpr int D = S::D, NKV = S::NKV;
  // K / V of the item's blocks are in kv (attn_kv_load, issued before)
  const int n = on ? pos + 1 : 0;
  const int tid = ltid() % AT, w = tid / kWave, l = tid % kWave;
  const int c16 = l & 15, rg = l >> 4;
  const long long kbase = (long long)b * p.kv_seq + ((long long)layer * NKV + g) * (long long)p.s_pad * D;
  const long long sbase = (long long)b * p.sc_seq + ((long long)layer * NKV + g) * p.s_pad;
  auto& kr = kv.kr;
  auto& vr = kv.vr;
  auto& sk = kv.sk;
  auto& sv = kv.sv;
  for (int i = tid; i < 16 * D; i += AT) (&sm.qb[0][0])[i] = 0;
  for (int i = tid; i < AW * 16 * 32; i += AT) (&sm.pb[0][0][0])[i] = 0;
  if (on && tid < D / 2) {
    sm.rc[tid] = p.rope[(b * 2 + 0) * (D / 2) + tid];
    sm.rsn[tid] = p.rope[(b * 2 + 1) * (D / 2) + tid];
  }
  if (!ready()) return false;
  __syncthreads();
  // 1. q heads (waves 0, 1), k (wave 2), v (wave 3) of position pos: QK-norm
  //    (reference rmsnorm.cuh:57-84) and RoPE rotate-half (attention.cuh:22-44)
  const int sl = FUSED ? layer : 0;
  const float* src = qkv_slot<S>(p, sl) + (long long)b * S::QKV +
                     (w < 2 ? (g * 2 + w) * D : (w == 2 ? S::QD + g * D : S::QD + S::KVD + g * D));
  const float v0 = on ? src[l] : 0.f;
  float v = v0;
  const bool own = on && !p.prefill && pos >= s * CH && pos < (s + 1) * CH;
  if (on && w < 3) {
    const float ss = wave_sum(v * v);
    const uint16_t* gn = p.norms + (long long)layer * S::NORM_STRIDE + (w < 2 ? S::NORM_Q : S::NORM_K);
    v = v * rsqrtf(ss / (float)D + kRmsEps) * bf16_to_f32(gn[l]);
    const float partner = lane_xor32(v);
    const int d = l & 31;
    v = l < 32 ? v * sm.rc[d] - partner * sm.rsn[d] : v * sm.rc[d] + partner * sm.rsn[d];
    if (w < 2) {
      uint16_t h, m, o;
      split_bf16(v, h, m, o);
      sm.qb[4 * w + 0][l] = h;
      sm.qb[4 * w + 1][l] = m;
      sm.qb[4 * w + 2][l] = o;
    } else if constexpr (K8) {  // FP8 append: the row's power-of-two scale from the wave's max
      const int e = e4m3_row_exp(wave_max(fabsf(v)));
      const uint8_t code = (uint8_t)e4m3_encode(ldexpf(v, -e));
      reinterpret_cast<uint8_t*>(sm.kcur)[l] = code;
      if (l == 0) sm.kcs[0] = ldexpf(1.f, e);
      if (own) {
        reinterpret_cast<uint8_t*>(p.kv)[kbase + (long long)pos * D + l] = code;
        if (l == 0) p.kscale[sbase + pos] = ldexpf(1.f, e);
      }
    } else {
      const uint16_t kb = f32_to_bf16(v);
      sm.kcur[l] = kb;
      if (own) p.kv[kbase + (long long)pos * D + l] = kb;  // KV append (reference kv_cache.cuh:58-78)
    }
  } else if (on && w == 3) {
    if constexpr (K8) {
      const int e = e4m3_row_exp(wave_max(fabsf(v)));
      const uint8_t code = (uint8_t)e4m3_encode(ldexpf(v, -e));
      reinterpret_cast<uint8_t*>(sm.vcur)[l] = code;
      if (l == 0) sm.kcs[1] = ldexpf(1.f, e);
      if (own) {
        reinterpret_cast<uint8_t*>(p.kvt)[kbase + (long long)(pos / 32) * 32 * D + (long long)l * 32 + (pos % 32)] = code;
        if (l == 0) p.vscale[sbase + pos] = ldexpf(1.f, e);
      }
    } else {
      const uint16_t vb = f32_to_bf16(v);
      sm.vcur[l] = vb;
      if (own) p.kvt[kbase + (long long)(pos / 32) * 32 * D + (long long)l * 32 + (pos % 32)] = vb;
    }
  }
  __syncthreads();
  // 2. the wave's blocks: online softmax over them on the matrix cores
  const float scale = 1.0f / sqrtf((float)D);
  float m = -INFINITY, lsum = 0.f;
  f32x4 acc[D / 16];
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < NBW; ++q) {
    const int t0 = 32 * (s * AW * NBW + w + AW * q);
    if (t0 >= n) break;  // uniform over the wave (every block of an item that is off)
    // position pos takes K / V from LDS (this item appended them; in a
    // prefill bk_append stored them before this kernel)
    if (!p.prefill && pos >= t0 && pos < t0 + 32) {
      const int rp = pos - t0;
      if constexpr (K8) {
        if (c16 == (rp & 15)) {  // register arrays take compile-time indices only
          const uint8_t* kc8 = reinterpret_cast<const uint8_t*>(sm.kcur);
#pragma unroll
          for (int kc = 0; kc < 2; ++kc) {
            const u32x2 kv = *reinterpret_cast<const u32x2*>(&kc8[32 * kc + 8 * rg]);
            if (rp >> 4) kr[q][1][kc] = kv;
            else kr[q][0][kc] = kv;
          }
          if (rp >> 4) sk[q][1] = sm.kcs[0], sv[q][1] = sm.kcs[1];
          else sk[q][0] = sm.kcs[0], sv[q][0] = sm.kcs[1];
        }
        if (rg == (rp >> 3)) {
          const uint8_t* vc8 = reinterpret_cast<const uint8_t*>(sm.vcur);
#pragma unroll
          for (int dt = 0; dt < D / 16; ++dt) vr[q][dt] = set_u8(vr[q][dt], rp & 7, vc8[16 * dt + c16]);
        }
      } else {
        if (c16 == (rp & 15)) {  // register arrays take compile-time indices only
#pragma unroll
          for (int kc = 0; kc < 2; ++kc) {
            const u32x4 kv = *reinterpret_cast<const u32x4*>(&sm.kcur[32 * kc + 8 * rg]);
            if (rp >> 4) kr[q][1][kc] = kv;
            else kr[q][0][kc] = kv;
          }
        }
        if (rg == (rp >> 3)) {
#pragma unroll
          for (int dt = 0; dt < D / 16; ++dt) vr[q][dt] = with_bf16(vr[q][dt], rp & 7, sm.vcur[16 * dt + c16]);
        }
      }
    }
    float sc[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      f32x4 d4 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {  // q read from LDS per block: registers for a fifth workgroup per CU
        u32x4 kb;
        if constexpr (K8) kb = fp8x8_to_bf16x8_scaled(kr[q][h][kc], sk[q][h]);
        else kb = kr[q][h][kc];
        d4 = mfma(*reinterpret_cast<const u32x4*>(&sm.qb[c16][32 * kc + 8 * rg]), kb, d4);
      }
      const int t = t0 + 16 * h + c16;
      sc[h] = t < n ? ((d4[0] + d4[1]) + d4[2]) * scale : -INFINITY;
    }
    const float mn = fmaxf(m, group_max<16>(fmaxf(sc[0], sc[1])));  // finite: position t0 < n is valid
    const float alpha = __expf(m - mn);
    m = mn;
    float ps = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      sc[h] = __expf(sc[h] - m);
      ps += sc[h];
    }
    lsum = lsum * alpha + group_sum<16>(ps);
    if (rg < 2) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const Split3 a = split3(K8 ? sc[h] * sv[q][h] : sc[h]);
        sm.pb[w][4 * rg + 0][16 * h + c16] = (uint16_t)(a.hi >> 16);
        sm.pb[w][4 * rg + 1][16 * h + c16] = (uint16_t)(a.mid >> 16);
        sm.pb[w][4 * rg + 2][16 * h + c16] = (uint16_t)(a.lo >> 16);
      }
    }
    asm volatile("" ::: "memory");  // LDS operations of one wave complete in order
    const u32x4 pa = *reinterpret_cast<const u32x4*>(&sm.pb[w][c16][8 * rg]);
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[dt][i] *= alpha;
      if constexpr (K8) acc[dt] = mfma(pa, fp8x8_to_bf16x8_scaled(vr[q][dt], 1.0f), acc[dt]);
      else acc[dt] = mfma(pa, vr[q][dt], acc[dt]);
    }
  }
  // 3. combine the waves into the item's partial
  if (rg < 2) {
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) sm.ow[w][rg][16 * dt + c16] = (acc[dt][0] + acc[dt][1]) + acc[dt][2];
    if (c16 == 0) {
      sm.mw[w][rg] = m;
      sm.lw[w][rg] = lsum;
    }
  }
  __syncthreads();
  float* part = p.part + (((long long)b * NKV + g) * p.nsplit_max + s) * PW;
  if (on && tid < 2 * D) {
    const int h = tid / D, d = tid % D;
    float M = sm.mw[0][h];
#pragma unroll
    for (int i = 1; i < AW; ++i) M = fmaxf(M, sm.mw[i][h]);
    float o = 0.f, L = 0.f;
#pragma unroll
    for (int i = 0; i < AW; ++i) {
      const float f = __expf(sm.mw[i][h] - M);
      o = fmaf(f, sm.ow[i][h][d], o);
      L = fmaf(f, sm.lw[i][h], L);
    }
    __hip_atomic_store(part + tid, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (d == 0) {
      __hip_atomic_store(part + 2 * D + 2 * h, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(part + 2 * D + 2 * h + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // 4. the last split of (b, g) to finish merges: the partial stores above are
  //    acknowledged (write-through) before the counter moves
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    bool last = false;
    if (on) {
      int* c = p.cnt + b * NKV + g;
      const int done = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = done == nsplit - 1;
      if (last) __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // re-armed for the next layer
    }
    sm.last = last;
  }
  __syncthreads();
  const bool merge = sm.last;
  if (!FUSED && !merge) return true;  // one item per workgroup: nothing else shares its barriers
  // 5. the merge: thread (split group sg, output hd) reads output hd of every
  //    SG-th split, MG splits per load round (all loads of a round issued
  //    before any is used: one round trip, not one per split); the SG groups
  //    are then combined in LDS
  {
    constexpr int SG = AT / (2 * D), MG = 8;
    const int hd = tid % (2 * D), sg = tid / (2 * D), h = hd / D;
    const float* base = p.part + ((long long)b * NKV + g) * p.nsplit_max * PW;
    float M = -INFINITY, o = 0.f, L = 0.f;
    const int ns = merge ? nsplit : 0;
    for (int r0 = 0; r0 < ns; r0 += SG * MG) {
      float mv[MG], lv[MG], ov[MG];
#pragma unroll
      for (int u = 0; u < MG; ++u) {
        const int i = r0 + sg + SG * u;
        const float* pi = base + (long long)(i < ns ? i : 0) * PW;
        mv[u] = __hip_atomic_load(pi + 2 * D + 2 * h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        lv[u] = __hip_atomic_load(pi + 2 * D + 2 * h + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ov[u] = __hip_atomic_load(pi + hd, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      float Mb = M;
#pragma unroll
      for (int u = 0; u < MG; ++u) Mb = r0 + sg + SG * u < ns ? fmaxf(Mb, mv[u]) : Mb;
      const float sc = M == -INFINITY ? 0.f : __expf(M - Mb);  // o, L are 0 while M is -inf
      o *= sc, L *= sc;
#pragma unroll
      for (int u = 0; u < MG; ++u) {
        const bool on_ = r0 + sg + SG * u < ns;  // select: skipped words hold anything
        const float f = __expf(mv[u] - Mb);
        o = on_ ? fmaf(f, ov[u], o) : o;
        L = on_ ? fmaf(f, lv[u], L) : L;
      }
      M = Mb;
    }
    sm.cm[sg][hd] = M, sm.cl[sg][hd] = L, sm.co[sg][hd] = o;
    __syncthreads();
    if (merge && tid < 2 * D) {
      float Mx = sm.cm[0][tid];  // group 0 holds split 0
#pragma unroll
      for (int k = 1; k < SG; ++k) Mx = fmaxf(Mx, sm.cm[k][tid]);
      float oo = 0.f, ll = 0.f;
#pragma unroll
      for (int k = 0; k < SG; ++k) {
        const float f = sm.cm[k][tid] == -INFINITY ? 0.f : __expf(sm.cm[k][tid] - Mx);
        oo = fmaf(f, sm.co[k][tid], oo);
        ll = fmaf(f, sm.cl[k][tid], ll);
      }
      uint16_t hi, lo;
      split2(oo / ll, hi, lo);
      const long long k = (long long)b * S::QD + g * 2 * D + tid;
      st_act<FUSED>(att_slot<S>(p, sl) + k, hi);
      st_act<FUSED>(att_slot<S>(p, sl) + (long long)BMAX * S::QD + k, lo);
    }
  }
  if constexpr (FUSED) {  // the merged output is acknowledged before it is counted
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (merge && tid == 0)
      __hip_atomic_store(p.flags + ((long long)layer * FC_N + FC_ATT) * FLAG_MAX + b * NKV + g, ep, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  return true;
}

// Five 256-thread items per CU (<= 102 registers per lane): the 16-sequence
// step at KV 512-4096 has ~1,100 items; with four per CU the last ~10 % ran
// as a second, latency-bound residency wave.
constexpr int ATTN_WAVES_PER_EU = AT == 256 ? 5 : 2;
template <class S, bool K8, class G>
__global__ __launch_bounds__(AT) __attribute__((amdgpu_waves_per_eu(ATTN_WAVES_PER_EU, ATTN_WAVES_PER_EU))) void bk_attn(
    G pg, int layer) {
  __shared__ AttnLds<S> sm;
  const BParams& p = group_of(pg);  // column group
  // workgroup i runs on XCD i % 8: every split of one (sequence, kv head)
  // pair gets the same XCD, so the merging split reads its partials there; a
  // pair's splits are consecutive slots of its XCD (split-major numbering,
  // split 0 of every pair first, measured 3 % slower for the batched decode)
  static_assert((BMAX * S::NKV) % 8 == 0, "whole (sequence, kv head) pairs per XCD");
  const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
  const int bg = (slot / p.nsplit_max) * 8 + xcd, s = slot % p.nsplit_max;
  const int b = bg / S::NKV, g = bg % S::NKV;
  if (b >= p.B) return;
  const int pos = p.pos[b];
  const int nsplit = (pos + 1 + CH - 1) / CH;
  if (s >= nsplit) return;
  AttnKV<S, K8> kv;
  attn_kv_load<S, K8>(p, layer, true, b, g, s, pos, kv);
  attn_item<S, K8, false>(p, layer, 0, sm, true, b, g, s, nsplit, pos, kv, NoWait{});
}

// ------------------------------------------------------------ prefill attention
// One workgroup of PC_AW waves per (kv head g, column group): the group's
// <= 16 tokens x 2 q heads = 32 queries (query q: token q / 2, head 2 g + q % 2)
// as two 16-column tiles; wave w takes the 32-position K / V blocks w, w +
// PC_AW, ... of the causal prefix [0, the group's last position] with an
// online softmax per query, and the waves' states are combined at the end.
// Products (v_mfma_f32_16x16x32_bf16):
//   scores^T (16 positions x 16 queries) = K (A operand: the cache rows as
//     loaded) . Q^T (B operand: q in NPART bf16 parts, one product each);
//   out^T (16 dims x 16 queries) += V^T (A operand: the transposed cache, the
//     block's positions in the order the scores leave them in a lane) . P^T
//     (B operand: the softmax weights in NPART parts, built in registers).
// A lane holds 4 positions x 1 query of each 16-position score tile: the
// block max takes two cross-lane steps, the row sums stay per lane until the
// end, and the weights never pass through LDS.  NPART 3: q and the weights
// split exactly (hi + mid + lo by truncation); 2: hi + lo (RNE), relative
// error <= 2^-17.
// (measured per layer at 1,024 tokens, us: 8 waves 22.6 against 4 waves
// 20.9; three K / V register sets 23.2 against two 20.6; two parts 20.8
// against three 21.6; a timing probe limited to one block per workgroup
// 9.0, so about half is the prologue, the merge and the launch; the earlier
// kernel with q
// as the A operand -- 4 queries per 16-row tile, the weights through LDS --
// 34.0.)
#ifndef MK_PATTN_NPART
#define MK_PATTN_NPART 3
#endif
constexpr int PC_AW = 4;         // waves of a workgroup
constexpr int PC_NQ = 2 * BMAX;  // queries of a workgroup (a column group x 2 q heads)
template <class S, bool K8>
struct PcKV {  // one block's K / V operands of a lane, as loaded (K8: FP8 codes, converted at use)
  using Reg = typename std::conditional<K8, u32x2, u32x4>::type;
  Reg k[2][2];  // [16-position half][32-dim chunk]
  Reg v[S::D / 16];  // [16-dim tile]: positions (4 gq .. 4 gq + 3, 16 + 4 gq .. 16 + 4 gq + 3)
  f32x4 sk[2], sv[2];  // K8: row scales of the lane's score positions t0 + 16 h + 4 gq + i
};
// bf16 operand of a loaded register: FP8 codes converted exactly (scale 1)
__device__ __forceinline__ u32x4 pc_op(u32x4 r) { return r; }
__device__ __forceinline__ u32x4 pc_op(u32x2 r) { return fp8x8_to_bf16x8_scaled(r, 1.0f); }
template <class S, bool K8>
__device__ __forceinline__ void pc_load(const BParams& p, __amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv,
                                        long long sbase, int t0, unsigned c16, unsigned gq, PcKV<S, K8>& r) {
  constexpr int D = S::D;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      const unsigned e = ((unsigned)t0 + 16u * h + c16) * D + 32u * kc + 8u * gq;
      if constexpr (K8)
        r.k[h][kc] = __builtin_amdgcn_raw_buffer_load_b64(rk, e, 0u, 2);
      else
        r.k[h][kc] = __builtin_amdgcn_raw_buffer_load_b128(rk, e * 2u, 0u, 2);
    }
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) {
    const unsigned e = (unsigned)t0 * D + (16u * dt + c16) * 32u + 4u * gq;
    if constexpr (K8) {
      r.v[dt] = u32x2{__builtin_amdgcn_raw_buffer_load_b32(rv, e, 0u, 2),
                      __builtin_amdgcn_raw_buffer_load_b32(rv, e + 16u, 0u, 2)};
    } else {
      const u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(rv, e * 2u, 0u, 2);
      const u32x2 b = __builtin_amdgcn_raw_buffer_load_b64(rv, (e + 16u) * 2u, 0u, 2);
      r.v[dt] = u32x4{a[0], a[1], b[0], b[1]};
    }
  }
  if constexpr (K8) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      r.sk[h] = *reinterpret_cast<const f32x4*>(p.kscale + sbase + t0 + 16 * h + 4 * (int)gq);
      r.sv[h] = *reinterpret_cast<const f32x4*>(p.vscale + sbase + t0 + 16 * h + 4 * (int)gq);
    }
  }
}
// 8 fp32 values -> NPART bf16x8 parts (3: exact truncation split; 2: RNE hi + lo)
template <int NPART>
__device__ __forceinline__ void pc_parts(const float (&x)[8], u32x4 (&o)[NPART]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (NPART == 3) {
      const Split3 a = split3(x[2 * e]), b = split3(x[2 * e + 1]);
      o[0][e] = pack_hi16(a.hi, b.hi);
      o[1][e] = pack_hi16(a.mid, b.mid);
      o[2][e] = pack_hi16(a.lo, b.lo);
    } else {
      uint32_t hi, lo;
      bf16_hilo2(x[2 * e], x[2 * e + 1], hi, lo);
      o[0][e] = hi;
      o[1][e] = lo;
    }
  }
}
template <class S, bool K8, int NPART = MK_PATTN_NPART>
__global__ __launch_bounds__(PC_AW * kWave) void bk_pattn(PGroup pg, int layer) {
  static_assert(S::GQA == 2 && S::D == 64, "2 q heads of 64 per kv head");
  static_assert(NPART == 2 || NPART == 3, "two or three bf16 parts");
  constexpr int D = S::D, NKV = S::NKV, AWc = PC_AW, NT = PC_AW * kWave, QT = PC_NQ / 16;
  constexpr int QP = D + 8;  // padded q row (elements)
  // q is multiplied by log2(e) / sqrt(D) before it is split, so a score is
  // already the exponent of 2 of its softmax weight
  constexpr float kLog2Scale = 1.4426950408889634f / 8.0f;
  static_assert(D == 64, "1 / sqrt(D) = 1 / 8");
  __shared__ __attribute__((aligned(16))) uint16_t qs[NPART][PC_NQ][QP];
  __shared__ float ow[AWc][PC_NQ][D + 4];  // padded rows: the lanes of one store hit distinct banks
  __shared__ float mw[AWc][PC_NQ], lw[AWc][PC_NQ];
  // the longest prefixes (the last groups) first
  const BParams p = group_params(pg, pg.n - 1 - (int)blockIdx.y);
  const int g = blockIdx.x, tid = ltid(), w = wave_id(), l = (int)lane_id();
  const unsigned c16 = (unsigned)l & 15u, gq = (unsigned)l >> 4;
  const long long kbase = ((long long)layer * NKV + g) * (long long)p.s_pad * D;
  const long long sbase = ((long long)layer * NKV + g) * p.s_pad;
  const auto rk = K8 ? make_rsrc(reinterpret_cast<const uint8_t*>(p.kv) + kbase) : make_rsrc(p.kv + kbase);
  const auto rv = K8 ? make_rsrc(reinterpret_cast<const uint8_t*>(p.kvt) + kbase) : make_rsrc(p.kvt + kbase);
  // the wave's first block is loading during the prologue, issued before the
  // group's position is read (block w lies inside the cache whatever the
  // prefix; unused when the prefix is shorter)
  PcKV<S, K8> cur, nxt;
  if (32 * w + 32 <= p.s_pad) pc_load<S, K8>(p, rk, rv, sbase, 32 * w, c16, gq, cur);
  __builtin_amdgcn_sched_barrier(0);
  const int p0 = p.pos[0], pmax = p0 + p.B - 1, nblk = pmax / 32 + 1;
  // 1. q of the 32 queries (wave w: queries NQW w .. NQW w + NQW - 1; lane =
  //    dimension): QK-norm (reference rmsnorm.cuh:57-84) and RoPE
  //    rotate-half (attention.cuh:22-44), as bk_attn's prologue; every
  //    query's loads are issued before the first is used
  {
    constexpr int NQW = PC_NQ / AWc;
    const uint16_t* gn = p.norms + (long long)layer * S::NORM_STRIDE + S::NORM_Q;
    const float gain = bf16_to_f32(gn[l]);
    const int d = l & 31;
    float qv[NQW], qc[NQW], qn[NQW];
#pragma unroll
    for (int k = 0; k < NQW; ++k) {
      const int q = NQW * w + k, col = q >> 1, j = q & 1;
      const bool on = col < p.B;
      qv[k] = on ? qkv_slot<S>(p, 0)[(long long)col * S::QKV + (g * 2 + j) * D + l] : 0.f;
      qc[k] = on ? p.rope[(col * 2 + 0) * (D / 2) + d] : 0.f;
      qn[k] = on ? p.rope[(col * 2 + 1) * (D / 2) + d] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < NQW; ++k) {
      const int q = NQW * w + k, col = q >> 1;
      const bool on = col < p.B;
      float v = qv[k];
      const float ss = wave_sum(v * v);
      v = on ? v * rsqrtf(ss / (float)D + kRmsEps) * gain : 0.f;
      const float partner = lane_xor32(v);
      const float cs = qc[k], sn = qn[k];
      v = l < 32 ? v * cs - partner * sn : v * cs + partner * sn;
      v *= kLog2Scale;  // scores in log2 units, softmax scale included
      if constexpr (NPART == 3) {
        uint16_t h, m, o;
        split_bf16(v, h, m, o);
        qs[0][q][l] = h, qs[1][q][l] = m, qs[2][q][l] = o;
      } else {
        uint32_t h, o;
        bf16_hilo2(v, 0.f, h, o);
        qs[0][q][l] = (uint16_t)h, qs[1][q][l] = (uint16_t)o;
      }
    }
  }
  __syncthreads();
  // the q parts as B operands, held for the whole loop
  u32x4 qb[QT][NPART][2];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int pt = 0; pt < NPART; ++pt)
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
        qb[qt][pt][kc] = *reinterpret_cast<const u32x4*>(&qs[pt][16 * qt + c16][32 * kc + 8 * gq]);
  // 2. the wave's blocks
  float m[QT], ls[QT];
  int qpos[QT];
  f32x4 acc[QT][D / 16];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m[qt] = -INFINITY, ls[qt] = 0.f;
    const int col = (16 * qt + (int)c16) >> 1;
    qpos[qt] = col < p.B ? p0 + col : -1;  // -1: no token (every score masked)
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) acc[qt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // the first position of a tile's queries when all its 8 tokens exist, else
  // -1: a block that ends at or before it is visible to every query of the
  // tile (no mask)
  int qmin[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) qmin[qt] = 8 * qt + 7 < p.B ? p0 + 8 * qt : -1;
  // one query tile's products and online-softmax step on a block (r: its K /
  // V operands); MASK: the causal mask and the guards of a query that has no
  // visible position yet
  const auto step = [&](auto mask_c, int qt, int t0, const PcKV<S, K8>& r) __attribute__((always_inline)) {
    constexpr bool MASK = decltype(mask_c)::value;
    float sc[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      f32x4 d4 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
#pragma unroll
        for (int pt = 0; pt < NPART; ++pt) d4 = mfma(pc_op(r.k[h][kc]), qb[qt][pt][kc], d4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // K8: the K row scale (a power of two) multiplies the exact product
        const float x = K8 ? d4[i] * r.sk[h][i] : d4[i];
        sc[h][i] = MASK && t0 + 16 * h + 4 * (int)gq + i > qpos[qt] ? -INFINITY : x;
      }
    }
    float bm = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
                     fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
    bm = max_xor32(max_xor16(bm));
    const float mo = m[qt], mn = fmaxf(mo, bm);
    m[qt] = mn;
    float pw[8], ps = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // a query none of whose positions so far is visible keeps m = -inf
        // and weight 0 (no -inf - -inf)
        const float e = MASK && mn == -INFINITY ? 0.f : exp2f(sc[h][i] - mn);
        ps += e;
        pw[4 * h + i] = K8 ? e * r.sv[h][i] : e;  // the V row scale enters the weight
      }
    // the running state is rescaled only when some query's maximum grew (the
    // factor is exactly 1 otherwise).  The branch is taken by the whole wave:
    // a query still without a visible position (mn = mo = -inf) keeps factor
    // 1, not exp2(-inf - -inf)
    if (__builtin_amdgcn_ballot_w64(mn != mo)) {
      const float alpha = MASK && mn == -INFINITY ? 1.f : exp2f(mo - mn);
      ls[qt] *= alpha;
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[qt][dt][i] *= alpha;
    }
    ls[qt] += ps;
    u32x4 pb[NPART];
    pc_parts<NPART>(pw, pb);
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
      for (int pt = 0; pt < NPART; ++pt) acc[qt][dt] = mfma(pc_op(r.v[dt]), pb[pt], acc[qt][dt]);
  };
  const auto block = [&](int t0, const PcKV<S, K8>& r) __attribute__((always_inline)) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      if (t0 + 31 <= qmin[qt]) step(std::false_type{}, qt, t0, r);
      else step(std::true_type{}, qt, t0, r);
    }
  };
  // two register sets in turn (no copy between them: a copy would wait for
  // the next block's loads before the current block's products).  Every
  // iteration issues both sets' loads (past the prefix they repeat its last
  // block, unused), so that each product waits for exactly its own block's
  // loads: with a conditional issue the compiler's waits, merged over both
  // paths, also waited for the block after.
  // The scheduling barriers keep the loads where they are: the scheduler
  // otherwise sinks them to their first use.
  for (int kb = w; kb < nblk; kb += 2 * AWc) {
    pc_load<S, K8>(p, rk, rv, sbase, 32 * min(kb + AWc, nblk - 1), c16, gq, nxt);
    __builtin_amdgcn_sched_barrier(0);
    block(32 * kb, cur);
    if (kb + AWc >= nblk) break;
    pc_load<S, K8>(p, rk, rv, sbase, 32 * min(kb + 2 * AWc, nblk - 1), c16, gq, cur);
    __builtin_amdgcn_sched_barrier(0);
    block(32 * (kb + AWc), nxt);
  }
  // 3. combine the waves and write the output as bf16 hi / lo parts
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int q = 16 * qt + (int)c16;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) ow[w][q][16 * dt + 4 * gq + i] = acc[qt][dt][i];
    const float lt = sum_xor32(sum_xor16(ls[qt]));
    if (gq == 0) {
      mw[w][q] = m[qt];
      lw[w][q] = lt;
    }
  }
  __syncthreads();
  {
    const int d = tid % D;
#pragma unroll
    for (int k = 0; k < PC_NQ / (NT / D); ++k) {
      const int q = tid / D + (NT / D) * k, col = q >> 1, j = q & 1;
      if (col >= p.B) continue;
      float M = mw[0][q];
#pragma unroll
      for (int i = 1; i < AWc; ++i) M = fmaxf(M, mw[i][q]);
      float o = 0.f, L = 0.f;
#pragma unroll
      for (int i = 0; i < AWc; ++i) {
        const float f = mw[i][q] == -INFINITY ? 0.f : exp2f(mw[i][q] - M);
        o = fmaf(f, ow[i][q][d], o);
        L = fmaf(f, lw[i][q], L);
      }
      uint16_t hi, lo;
      split2(o / L, hi, lo);
      const long long k0 = (long long)col * S::QD + (g * 2 + j) * D + d;
      att_slot<S>(p, 0)[k0] = hi;
      att_slot<S>(p, 0)[(long long)BMAX * S::QD + k0] = lo;
    }
  }
}

// ------------------------------------------------------------ one-kernel step
// Workgroups of bk_step per CU (waves per SIMD = 2 x that): two, so twice the
// attention items run at once (<= 128 registers per lane).
#ifndef MK_STEP_WG_PER_CU
#define MK_STEP_WG_PER_CU 2
#endif
constexpr int STEP_WG_PER_CU = MK_STEP_WG_PER_CU;
constexpr int STEP_WAVES_PER_EU = 2 * STEP_WG_PER_CU;
// Every layer of a decode step in one persistent kernel: STEP_WG_PER_CU
// workgroups of GT threads per CU (all resident; the host checks the
// occupancy), each running
// its share of every phase of a layer in phase order and handing off through
// p.flags (one word per producer, the step's epoch once its outputs are out):
//   QKV block rb            on workgroup rb            waits: down of layer - 1 (H/16 blocks)
//   attention item pairs    pair j on workgroup (j + QKV/16) % G
//                                                      waits: every QKV block
//     (the two AT-thread halves of a workgroup run items 2j and 2j + 1)
//   O block rb              on workgroup (G - H/16 + rb) % G (G > H/16)
//                                                      waits: every (sequence, kv head) merged
//   gate/up block rb        on workgroup rb             waits: every O block
//   down piece (rb, ks)     on workgroup 4 rb + ks      waits: every gate/up block
//     (split 0 then waits for splits 1-3 of its block, whose sums carry a tag)
// Each block issues its weight loads before it waits, and every workgroup
// without a QKV block the K / V loads of its first attention pair at the
// layer start, so the loads overlap the hand-offs; every wait is for a phase that precedes it in the order
// above, and no phase waits for a later one, so the persistent grid cannot
// deadlock.  The arithmetic is that of the per-phase kernels (same block
// functions, same summation order): the logits are bit-identical.
template <class S, bool K8 = false>
__global__ __launch_bounds__(GT) __attribute__((amdgpu_waves_per_eu(STEP_WAVES_PER_EU, STEP_WAVES_PER_EU))) void bk_step(
    PGroup1 pg) {
  const BParams& p = pg.p[0];  // one group
  static_assert(GT == 2 * AT, "two attention items per workgroup");
  __shared__ float red[GW * 16 * 17];
  __shared__ float rr[RR_N];
  __shared__ int last;
  __shared__ AttnLds<S> att[2];
  __shared__ int icum[BMAX + 1], ins[BMAX], ipos[BMAX];
  const int G = gridDim.x, wg = blockIdx.x;
  if (threadIdx.x == 0) {  // attention items of the step: sequence b has NKV * nsplit_b, in (b, g, s) order
    int c = 0;
    for (int b = 0; b < BMAX; ++b) {
      const int pos = b < p.B ? p.pos[b] : 0;
      const int ns = b < p.B ? (pos + 1 + CH - 1) / CH : 0;
      icum[b] = c;
      ins[b] = ns;
      ipos[b] = pos;
      c += S::NKV * ns;
    }
    icum[BMAX] = c;
  }
  __syncthreads();
  const int n_items = icum[BMAX];
  const int ep = *p.epoch;  // this step's epoch (bk_embed advanced it)
  u64* const tr = p.trace;
  int layer = 0;
  auto stamp = [&](int ev) {
    if (tr && ltid() == 0) tr[((long long)layer * TR_N + ev) * G + wg] = wall_clock64();
  };
  // a wait followed by its "inputs ready" stamp
  auto waited = [&](bool ok, int ev) {
    stamp(ev);
    return ok;
  };
  // pair j on workgroup (j + QKV blocks) % G: the workgroups without a QKV
  // block take the first pairs; every workgroup issues the K / V loads of its
  // first pair at the layer start (they only read the cache)
  const int j0 = (wg - S::RB_QKV % G + G) % G;
  struct Item {
    bool on;
    int b, g, s, ns;
  };
  auto item_of = [&](int j) {
    const int i = 2 * j + ltid() / AT;
    Item it;
    it.on = i < n_items;
    int b = 0;
    while (b + 1 < BMAX && icum[b + 1] <= i) ++b;
    const int r = it.on ? i - icum[b] : 0;
    it.ns = ins[b] > 0 ? ins[b] : 1;
    it.b = b, it.g = r / it.ns, it.s = r % it.ns;
    return it;
  };
  for (; layer < p.L; ++layer) {
    stamp(TR_START);
    bool qkv_in = false;  // this layer's QKV flags already seen by this workgroup
    auto qkv_ready = [&] {
      if (qkv_in) return true;
      qkv_in = waited(fc_wait(p, layer, FC_QKV, S::RB_QKV, ep), TR_ATT_IN);
      return qkv_in;
    };
    int jn = j0;  // the next attention pair of this workgroup
    if (wg >= S::RB_QKV && 2 * j0 < n_items) {
      // no QKV block: the first pair's K / V loads are issued at the layer
      // start and overlap the QKV phase (a workgroup with a QKV block issues
      // them after it, in the loop below: both at once do not fit the registers)
      const Item it = item_of(j0);
      AttnKV<S, K8> kv;
      attn_kv_load<S, K8>(p, layer, it.on, it.b, it.g, it.s, ipos[it.b], kv);
      if (!attn_item<S, K8, true>(p, layer, ep, att[ltid() / AT], it.on, it.b, it.g, it.s, it.ns, ipos[it.b], kv,
                                  qkv_ready))
        return;
      stamp(TR_ATT_DONE);
      jn += G;
    } else {
      for (int rb = wg; rb < S::RB_QKV; rb += G) {
        if (!qkv_block<S, true>(p, layer, ep, rb, 0, red, rr, &last, [&] {
              return waited(layer == 0 || fc_wait(p, layer - 1, FC_DN, S::RB_H, ep), TR_QKV_IN);
            }))
          return;
        stamp(TR_QKV_DONE);
      }
    }
    for (int j = jn; 2 * j < n_items; j += G) {
      const Item it = item_of(j);
      AttnKV<S, K8> kv;
      attn_kv_load<S, K8>(p, layer, it.on, it.b, it.g, it.s, ipos[it.b], kv);
      if (!attn_item<S, K8, true>(p, layer, ep, att[ltid() / AT], it.on, it.b, it.g, it.s, it.ns, ipos[it.b], kv,
                                  qkv_ready))
        return;
      stamp(TR_ATT_DONE);
    }
    const int o_off = G > S::RB_H ? G - S::RB_H : 0;  // O on the last workgroups (fewest attention pairs)
    for (int rb = 0; rb < S::RB_H; ++rb)
      if ((rb + o_off) % G == wg) {
        if (!o_block<S, true>(p, layer, ep, rb, 0, red, &last,
                              [&] { return waited(fc_wait(p, layer, FC_ATT, p.B * S::NKV, ep), TR_O_IN); }))
          return;
        stamp(TR_O_DONE);
      }
    for (int rb = wg; rb < S::RB_F; rb += G) {
      if (!gu_block<S, true>(p, layer, ep, rb, 0, red, rr, &last,
                             [&] { return waited(fc_wait(p, layer, FC_O, S::RB_H, ep), TR_GU_IN); }))
        return;
      stamp(TR_GU_DONE);
    }
    // a workgroup with several down pieces runs its split-0 pieces (which
    // wait for the other splits of their block) after the others
    for (int pass = 0; pass < 2; ++pass)
      for (int k = wg; k < S::RB_H * KS_DN; k += G) {
        if ((k % KS_DN == 0) != (pass == 1)) continue;
        if (!down_block<S, true>(p, layer, ep, k / KS_DN, k % KS_DN, red, &last,
                                 [&] { return waited(fc_wait(p, layer, FC_GU, S::RB_F, ep), TR_DN_IN); }))
          return;
        stamp(TR_DN_DONE);
      }
  }
}

}  // namespace batch
}  // namespace mk
