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
// Synchronisation: there is no grid barrier.  Each phase instance has a
// global number (its tag); every activation word carries the tag of the phase
// that wrote it, and a consumer waits for exactly the words it reads (tagged
// dataflow, see mk_device.h).  Every residual element has exactly one writer
// per phase (the owner of its 16-row block), so there is no read-modify-write
// race on x (unlike megakernel.cu:243-245,288-290), and per-token tags make the
// reference's never-re-armed KV flag problem (barriers.cuh:112-134)
// impossible.  Buffers are single-buffered: every write of a buffer depends
// (through the phase chain) on every read of its previous contents.
//
// Streaming: weights do not depend on activations, so each workgroup issues
// the loads of its NEXT phase's weight slice (and, one phase ahead of the
// attention, its K/V slice) into registers right after its current inputs
// arrive, and computes the current phase from registers loaded one phase
// earlier.  The wait for the next inputs therefore overlaps the HBM transfer.
#pragma once
#include <type_traits>

#include "mk_config.h"
#include "mk_device.h"

namespace mk {

constexpr int NT = 512;               // threads per workgroup (8 waves)
constexpr int NW = NT / kWave;
#ifndef MK_KV_BLOCKS
#define MK_KV_BLOCKS 2
#endif
// 32-position K/V blocks a wave holds in registers (prefetched a layer ahead).
// Two per wave halves the attention splits (and so the partials every O
// workgroup merges) against one, at the cost of a longer block step.
constexpr int KVB = MK_KV_BLOCKS;
// Cache policy of the LM-head stream (buffer-load aux bits): plain loads on
// 80 % of it and non-temporal loads on the rest measured fastest (part of the
// plain-loaded share is served from the memory-side cache across tokens).
#ifndef MK_LMHEAD_AUX
#define MK_LMHEAD_AUX 0
#endif
#ifndef MK_LMHEAD_KEEP_PCT
#define MK_LMHEAD_KEEP_PCT 80
#endif

constexpr int NSPLIT_CAP = 32;        // max attention splits per kv head
constexpr int IDX_BITS = 18;          // argmax words: 14-bit tag (TAG14) and an 18-bit vocabulary index
constexpr unsigned IDX_MAX = (1u << IDX_BITS) - 1;

struct Params {
  const u32x4* layers;        // packed per-layer weights (L * U_LAYER units)
  const uint16_t* norms;      // [L][NORM_STRIDE] bf16 gains
  const uint16_t* final_norm; // [H] bf16
  const u32x4* lmhead;        // packed tied embedding [V/16][KT_H][64]
  const u32x4* lmhead8;       // optional FP8 (e4m3) copy of the LM head [V/16][H/64][64]
  const float* lm_scale;      // [V] power-of-two row scales of lmhead8
  const float* lm_err;        // [V] error bounds of the FP8 rows: set = screened LM head (class kernel)
  float* kscale;              // FP8 KV cache (MODE bit 3): power-of-two scale of each K row
  float* vscale;              //   and V row, [L][NKV][s_pad]; the codes replace the bf16 values
                              //   at byte index = element index of kv / kvt
  uint16_t* kv;               // K cache [L][NKV][s_pad][D] bf16
  uint16_t* kvt;              // V cache, transposed blocks [L][NKV][s_pad/32][D][32] bf16
  const u32x2* layers8;       // optional FP8 (e4m3) layer weights, the same blocks at one byte per weight
  const float* lscale;        //   and their power-of-two row scales [L][SROWS_LAYER] (class kernel, MODE bit 16)
  u64* x;                     // [H/2] residual stream (packed pairs: rows 2i, 2i + 1 in word i)
  u64* qkv;                   // [QKV] projections of the current layer (tagged)
  u64* part;                  // [nsplit_max + 1][NKV][part_words] attention partials (packed
                              //   pairs): unnormalised output, then (max, sum) per q head; the
                              //   last row holds the merged partial of a long context
  u64* act;                   // [F/2] silu(gate)*up (packed pairs)
  u64* amax;                  // [2][G] per-workgroup argmax words (token parity)
  int* out_tokens;            // [n_tokens]
  int* err;                   // error word
  float* dbg_layers;          // optional [(L+1)][H]: embedding, then x after each layer
  float* dbg_logits;          // optional [V]
  u64* trace;                 // optional [(5L+1)][2][G] wall-clock ready/done per phase,
                              // then [EVT_N][G] events of layer trace_layer
  int trace_layer;
  const float* inv_freq;      // [D/2] RoPE inverse frequencies
  u64 timeout_ticks;
  unsigned tag_base;          // tag of the first phase of this launch
  int n_layers, vocab, max_seq, s_pad;
  int pos0, n_tokens, first_token;
  int nsplit_max, chunk_min;
  int merge_min;              // above this many splits the last split of a kv head merges them
  int trace_token;
  const int* roles;           // class kernel: [G][ROLE_INTS] role rows (null for the spread kernel)
  int pace_pct;               // class kernel: prefetch pacing, percent of the default spacing (0: bursts)
};

// Wave-share buffers of the block products, one per block a phase computes
// (a phase's product ends without a barrier after its reads, so the next
// phase's product must not overwrite the shares being summed).
enum RedBuf : int { RED_Q = 0, RED_O0, RED_O1, RED_G, RED_U, RED_D, RED_N };
// LM-head rows of one workgroup the screened LM head holds bounds for (the
// host uses the bf16 head when a workgroup would have more)
constexpr int LM_ROWS_MAX = 1024;

template <class S>
struct Smem {
  // GEMV input vectors, one per phase type (a phase's GEMV ends without a
  // barrier, so the next phase must not overwrite the vector it reads)
  // (the four layer GEMV inputs hold split-bf16 pairs, mk_device.h xs_put)
  float vec_q[S::H];                  // QKV: x * attn_norm gain
  float vec_o[S::QD];                 // O: attention output
  float vec_g[S::H];                  // gate/up: x * ffn_norm gain
  float vec_d[S::F];                  // down: SiLU(gate) * up
  float vec_l[S::H];                  // LM head: x * final_norm gain (fp32)
  float xres_o[32], xres_d[16];       // residual rows of this workgroup's O block(s) / down block
  __attribute__((aligned(16))) float ssw[3][NW];  // RMSNorm sum-of-squares partials (QKV, gate/up, LM head)
  float red[RED_N][NW * 16];          // block products: each wave's share of the 16 row sums (blk_mma)
  __attribute__((aligned(16))) uint16_t qb[16][S::D];  // attention: q parts, score A operand
  __attribute__((aligned(16))) uint16_t pb[NW][16][32 * KVB];  // attention: weight parts, output A operand
  u32x4 kvcur[2][S::D / 8];           // bf16 (FP8 cache: e4m3 codes) K/V of the current position
  float kvcs[2];                      // FP8 cache: scales of the current K / V rows
  __attribute__((aligned(16))) float pv[NW][S::GQA * S::D];  // attention: per-wave unnormalised outputs
  float mw[S::GQA][NW], lw[S::GQA][NW];  // attention: per-wave max / sum per q head
  float rc[S::D / 2], rs[S::D / 2];   // RoPE cos / sin of this token
  u64 amax[NW];
  float mrg[4][NT];                   // long-context split merge: (max, sum, out0, out1) per thread
  float lmu[LM_ROWS_MAX];             // screened LM head: upper bounds of this workgroup's row logits
  float lmw[NW];                      // screened LM head: per-wave partials
  int lmc[LM_ROWS_MAX];               // screened LM head: this workgroup's rows to rescore
  int lmn;                            //   and their count
};

// Element `col` of row `row` of a packed [R][K] matrix (K = 32 * KT).

// Workgroup-wide "did any thread give up waiting".  A failure aborts the
// launch, so the flag is only ever set after its initial clear: one LDS word
// serves every wait, and the check is a plain barrier plus one LDS read (the
// device library's __syncthreads_or is a full work-group reduction, about
// ten times slower).
__shared__ int wg_abort;
__device__ __forceinline__ bool block_failed(int failed) {
  if (failed) wg_abort = 1;
  __syncthreads();
  // an LDS read (ds_read): a volatile access compiles to a flat load, which
  // also waits for every outstanding global load and store of the wave
  return __hip_atomic_load(&wg_abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0;
}
// The abort flag after a barrier that follows every thread's last chance to
// set it.
__device__ __forceinline__ bool block_aborted() {
  return __hip_atomic_load(&wg_abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0;
}

// The wave that runs the one-wave epilogues and publishes a block's results.
// Stores and loads retire in issue order (one vmcnt counter on gfx9-class
// CUs), so a wave that polls right after its own write-through publish waits
// for that store's acknowledgement in its first round; the waits that can
// follow a publish of the same workgroup directly (act -> down after gate/up)
// poll with the other waves.
constexpr int PUB_WAVE = NW - 1;

// Poll a set of tagged words until they are ready, then consume them:
// issue(w) loads every word of one round into w (all loads before any test:
// one round trip per round), ready(w) tests it, consume(w) uses the round
// that passed.  Returns false when the wait was abandoned.
template <int N, class Issue, class Ready, class Consume>
__device__ __forceinline__ bool poll_rounds(const Params& p, Issue issue, Ready ready, Consume consume) {
  Spin sp;
  u64 w[N];
  while (true) {
    issue(w);
    if (ready(w)) {
      consume(w);
      return true;
    }
    if (!sp.step(p.err, p.timeout_ticks)) return false;
  }
}

// Phase trace of one token (profiling only).  Timestamps go to an LDS buffer
// and are written out once at the end of the traced token, so recording them
// adds no global stores (and no store waits) inside the phases being timed.
constexpr int TRACE_MAX_LAYERS = 48;
// Poll-level events of the traced layer, per wait site: when wave 0 of a
// consumer entered the wait, when each of its waves left its poll loop and
// how many rounds wave 0 polled (EVP_PER slots per site after the EVT events).
enum PollSite : int { PS_QKV = 0, PS_ATT, PS_O, PS_GU, PS_DN, PS_N };
constexpr int EV_ROLE = 16;  // the workgroup's role class (class kernel), one slot
constexpr int EVP_BASE = 17, EVP_PER = NW + 2;
constexpr int EVT_N = EVP_BASE + PS_N * EVP_PER;
constexpr int TRACE_LDS = (5 * TRACE_MAX_LAYERS + 1) * 2 + EVT_N;
__shared__ u64 trace_lds[TRACE_LDS];

__device__ __forceinline__ bool tracing(const Params& p, int t) { return p.trace && t == p.trace_token; }


__device__ __forceinline__ void trace_mark(const Params& p, int t, int slot, int which, int wave = 0) {
  if (tracing(p, t) && ltid() == wave * kWave) trace_lds[slot * 2 + which] = wall_clock64();
}

// Fine-grained events of one layer of the traced token.
enum Evt : int {
  EV_ATT_READY = 0, EV_ATT_ROPE, EV_ATT_SOFTMAX, EV_ATT_STORED,
  EV_ATT_PARTIAL, EV_ATT_GATHERED, EV_O_READY, EV_O_STORED,
  EV_QKV_STORED, EV_GU_STORED, EV_DN_STORED, EV_DN_READY,
  EV_ATT_REDUCED, EV_ATT_COMBINED, EV_MERGE_SCALED, EV_MERGE_DONE
};
#ifndef MK_TRACE_EVENTS
#define MK_TRACE_EVENTS 0  // fine-grained events of one layer (investigation builds only)
#endif
__device__ __forceinline__ void evt(const Params& p, int t, int layer, int e) {
  if (MK_TRACE_EVENTS && tracing(p, t) && layer == p.trace_layer && ltid() == 0)
    trace_lds[(5 * p.n_layers + 1) * 2 + e] = wall_clock64();
}

// A wait site of the traced token and layer (site < 0: not recorded).
struct EvPoll {
  int t = -1, layer = -1, site = -1;
};
__device__ __forceinline__ EvPoll ev_at(int t, int layer, int site) {
  EvPoll e;
  if (MK_TRACE_EVENTS) e.t = t, e.layer = layer, e.site = site;
  return e;
}
__device__ __forceinline__ bool ev_on(const Params& p, const EvPoll& e) {
  return MK_TRACE_EVENTS && e.site >= 0 && tracing(p, e.t) && e.layer == p.trace_layer;
}
// wave 0 enters the wait (thread 0)
__device__ __forceinline__ void evp_enter(const Params& p, const EvPoll& e) {
  if (ev_on(p, e) && ltid() == 0)
    trace_lds[(5 * p.n_layers + 1) * 2 + EVP_BASE + e.site * EVP_PER] = wall_clock64();
}
// a wave leaves its poll loop (its lane 0); thread 0 also records its rounds
__device__ __forceinline__ void evp_exit(const Params& p, const EvPoll& e, unsigned rounds) {
  if (!ev_on(p, e)) return;
  const int base = (5 * p.n_layers + 1) * 2 + EVP_BASE + e.site * EVP_PER;
  if ((ltid() & (kWave - 1)) == 0) trace_lds[base + 1 + wave_id()] = wall_clock64();
  if (ltid() == 0) trace_lds[base + 1 + NW] = rounds;
}

// Clear before the traced token; write out after it ([entry][G] layout).
// role: the workgroup's role class + 1 (0: none recorded).
__device__ __forceinline__ void trace_begin(const Params& p, int t, int role = -1) {
  if (!tracing(p, t)) return;
  for (int i = ltid(); i < TRACE_LDS; i += NT) trace_lds[i] = 0ull;
  __syncthreads();
  if (ltid() == 0) trace_lds[(5 * p.n_layers + 1) * 2 + EV_ROLE] = (u64)(role + 1);
}
__device__ __forceinline__ void trace_end(const Params& p, int t) {
  if (!tracing(p, t)) return;
  __syncthreads();
  const int n = (5 * p.n_layers + 1) * 2 + EVT_N;
  for (int i = ltid(); i < n; i += NT) p.trace[(long long)i * gridDim.x + blockIdx.x] = trace_lds[i];
}

// ------------------------------------------------------------------ GEMV
// One packed 16-row block in the tile layout (mk_config.h): wave w holds the
// 1 KiB units (16 x 32 tiles) w KC .. w KC + KC - 1, lane l of unit kt row
// l & 15, columns 32 kt + 8 (l >> 4) .. +7.
template <int KC>
struct Blk {
  u32x4 w[KC];
};

// The same block with FP8 (e4m3) weights: a tile is 512 bytes, lane l holds
// the 8 codes of row l & 15, columns 32 kt + 8 (l >> 4) .. +7; s is the
// power-of-two scale of row l >> 2 (the row lane l finishes in the epilogue).
template <int KC>
struct Blk8 {
  u32x2 w[KC];
  float s;
};
template <int KC, bool W8>
using BlkW = typename std::conditional<W8, Blk8<KC>, Blk<KC>>::type;

// A operand of one tile: the bf16 weights, or the FP8 codes converted to bf16
// (exact: every e4m3 value is a bf16 value).
__device__ __forceinline__ u32x4 a_tile(u32x4 w) { return w; }
__device__ __forceinline__ u32x4 a_tile(u32x2 w) { return fp8x8_to_bf16x8_scaled(w, 1.0f); }
template <int KC>
__device__ __forceinline__ float row_scale(const Blk<KC>&) { return 1.0f; }
template <int KC>
__device__ __forceinline__ float row_scale(const Blk8<KC>& b) { return b.s; }

template <int KC>
__device__ __forceinline__ void blk_load(Blk<KC>& b, const u32x4* __restrict__ block) {
  const int w = wave_id();
  const unsigned lb = lane_id() * 16u;
  const auto rs = make_rsrc(block);
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) b.w[kc] = buf_ld_nt(rs, lb, (unsigned)(w * KC + kc) * 1024u);
}

// A prefetch register set that this workgroup does not load in this phase
// gets an unspecified value: every path to its next use then defines it, so
// the compiler does not keep the previous phase's contents alive around the
// layer loop (loads and uses sit under the same runtime condition, which it
// cannot see).
template <int KC>
__device__ __forceinline__ void blk_forget(Blk<KC>& b) {
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) b.w[kc] = __builtin_nondeterministic_value(b.w[kc]);
}
template <int KC>
__device__ __forceinline__ void blk_forget(Blk8<KC>& b) {
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) b.w[kc] = __builtin_nondeterministic_value(b.w[kc]);
  b.s = __builtin_nondeterministic_value(b.s);
}

// Block product on the matrix cores (tile-layout blocks, mk_config.h: wave w
// holds tiles w KC .. w KC + KC - 1, i.e. columns 32 w KC .. 32 (w + 1) KC - 1
// of all 16 rows, lane l row l & 15 and columns 32 kt + 8 (l >> 4) .. +7 --
// the A operand of v_mfma_f32_16x16x32_bf16).  The B operand's column 0 holds
// the hi parts and column 1 the lo parts of the input (split-bf16 staging in
// LDS, xs_put); the other 14 columns are never loaded: a D column depends only
// on its own B column, and only columns 0 and 1 are read.  Lanes 0, 16, 32,
// 48 then hold rows 4 (l >> 4) .. +3 of both columns (lanes l and l + 1), and
// write their hi + lo sums -- the wave's share of the 16 row sums -- to
// red[wave][16].  No barrier: the row sums are read after one (red_row4).
//
// NB blocks against the same input share the B loads; each block's chain of
// KC products runs as two interleaved accumulators (even / odd k-steps), so
// the matrix core has independent products in flight.
template <int KC>
__device__ __forceinline__ void mma_b_load(u32x4 (&bx)[KC], const float* vec) {
  const unsigned l = lane_id();
  const uint32_t* xs = reinterpret_cast<const uint32_t*>(vec) + (wave_id() * KC * 4 + (int)(l >> 4)) * 8 + (int)(l & 1u) * 4;
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) asm volatile("" : "=v"(bx[kc]));  // columns 2..15: left as they are
  if ((l & 14u) == 0u) {  // B columns 0 and 1
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) bx[kc] = *reinterpret_cast<const u32x4*>(xs + kc * 32);
  }
}
__device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}
__device__ __forceinline__ void mma_share_out(f32x4 a0, f32x4 a1, float* red) {
  const unsigned l = lane_id();
  f32x4 s;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float v = a0[i] + a1[i];
    s[i] = v + dpp_sel<DPP_XOR1>(v);  // column 0 + column 1
  }
  if ((l & 15u) == 0u) *reinterpret_cast<f32x4*>(red + wave_id() * 16 + 4 * (int)(l >> 4)) = s;
}
template <int KC, template <int> class B>
__device__ __forceinline__ void blk_mma(const B<KC>& b, const float* vec, float* red) {
  u32x4 bx[KC];
  mma_b_load<KC>(bx, vec);
  f32x4 e = f32x4{0.f, 0.f, 0.f, 0.f}, o = e;
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    if (kc & 1) o = mma(a_tile(b.w[kc]), bx[kc], o);
    else e = mma(a_tile(b.w[kc]), bx[kc], e);
  }
  mma_share_out(e, o, red);
}
template <int KC, template <int> class B>
__device__ __forceinline__ void blk_mma2(const B<KC>& b0, const B<KC>& b1, const float* vec, float* red0,
                                         float* red1) {
  u32x4 bx[KC];
  mma_b_load<KC>(bx, vec);
  f32x4 e0 = f32x4{0.f, 0.f, 0.f, 0.f}, o0 = e0, e1 = e0, o1 = e0;
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    if (kc & 1) {
      o0 = mma(a_tile(b0.w[kc]), bx[kc], o0);
      o1 = mma(a_tile(b1.w[kc]), bx[kc], o1);
    } else {
      e0 = mma(a_tile(b0.w[kc]), bx[kc], e0);
      e1 = mma(a_tile(b1.w[kc]), bx[kc], e1);
    }
  }
  mma_share_out(e0, o0, red0);
  mma_share_out(e1, o1, red1);
}

// Row sums of a block product, in one wave (after the barrier that follows
// blk_mma): lane l adds the shares of waves 2 (l & 3) and 2 (l & 3) + 1 of row
// l >> 2, then the 4 lanes of the row exchange partials (DPP), so all four end
// with the same total, summed in a fixed order.
__device__ __forceinline__ float red_row4(const float* red, unsigned l) {
  const int r = (int)(l >> 2), w = 2 * (int)(l & 3u);
  float v = red[w * 16 + r] + red[(w + 1) * 16 + r];
  v += dpp_sel<DPP_XOR1>(v);
  v += dpp_sel<DPP_XOR2>(v);
  return v;
}
// Value of lane l + 4 (row r + 1 of red_row4's layout, inside a row of 16 lanes).
constexpr int DPP_ROW_SHL4 = 0x104;

// Row t of a block from the NW wave shares in red, summed in wave order (one
// thread per row; off the decode path).
__device__ __forceinline__ float red_sum(const float* red, int t) {
  float y = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) y += red[w * 16 + t];
  return y;
}

// SiLU(g) * u (reference utils.cuh:57-61, x / (1 + exp(-x)); the hardware
// reciprocal, relative error ~1 ulp, in place of the division).
__device__ __forceinline__ float silu_mul(float g, float u) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

// RMSNorm scale rsqrt(mean(x^2) + eps) from the NW wave partials of the sum
// of squares (a fixed summation tree, so every caller gets identical bits).
static_assert(NW == 8, "norm_scale sums eight wave partials");
__device__ __forceinline__ float norm_scale(const float* ssw, float inv_h) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(ssw), b = *reinterpret_cast<const f32x4*>(ssw + 4);
  const float tot = ((a[0] + a[1]) + (a[2] + a[3])) + ((b[0] + b[1]) + (b[2] + b[3]));
  return __builtin_amdgcn_rsqf(fmaf(tot, inv_h, kRmsEps));
}

// Epilogues, one barrier each, run by wave PUB_WAVE (lane l: row l >> 2).
// With ssw set, the rows are also scaled by norm_scale(ssw, inv_h): the
// wave partials of the input's sum of squares are read with the block shares,
// so the norm costs the critical path no LDS round trip of its own.
// QKV block: the 16 rows times `scale`, full tagged words.  NORM (ssw set):
// the norm scale is taken here; its LDS reads issue with the shares' reads
// (one round trip, not two).
template <bool NORM = false>
__device__ __forceinline__ bool store_block(const float* red, u64* dst16, float scale, unsigned tag,
                                            const float* ssw = nullptr, float inv_h = 0.f) {
  __syncthreads();
  const bool ok = !block_aborted();  // read with the shares (one LDS round trip)
  if (wave_id() == PUB_WAVE) {
    const unsigned l = lane_id();
    const float sh = red_row4(red, l);
    const float s = NORM ? scale * norm_scale(ssw, inv_h) : scale;
    const float y = sh * s;
    if (ok && (l & 3u) == 0u) ll_put(dst16 + (l >> 2), ll_pack(y, tag));
  }
  return ok;
}

// Gate/up pair: SiLU(g r) * (u r) of the 16 rows (gate shares in rg, up
// shares in ru), published as 8 packed-pair words.  NORM: r = norm_scale(ssw).
template <bool NORM = false>
__device__ __forceinline__ bool store_block_gu(const float* rg, const float* ru, u64* dst8, float r, unsigned t4,
                                               float sg = 1.0f, float su = 1.0f, const float* ssw = nullptr,
                                               float inv_h = 0.f) {
  __syncthreads();
  const bool ok = !block_aborted();  // read with the shares (one LDS round trip)
  if (wave_id() == PUB_WAVE) {
    const unsigned l = lane_id();
    const float g = red_row4(rg, l), u = red_row4(ru, l);
    const float rr = NORM ? norm_scale(ssw, inv_h) : r;
    const float a = silu_mul(g * (rr * sg), u * (rr * su));
    const float b = dpp_sel<DPP_ROW_SHL4>(a);  // the next row
    if (ok && (l & 7u) == 0u) ll_put(dst8 + (l >> 3), pk_pack(a, b, t4));
  }
  return ok;
}

// Element of the tile-layout LM head / embedding (row, col).
template <int KT>
__device__ __forceinline__ float packed_elem(const u32x4* base, int row, int col) {
  const int kt = col >> 5, q = (col >> 3) & 3, e = col & 7;
  const uint16_t* u = reinterpret_cast<const uint16_t*>(
      base + ((long long)(row >> 4) * KT + kt) * 64 + q * 16 + (row & 15));
  return bf16_to_f32(u[e]);
}

// RMSNorm (reference rmsnorm.cuh:87-108) is folded into the GEMVs that consume
// it: the input vector is stored as x * gain, and the row results are scaled
// by r = rsqrt(mean(x^2) + eps).  Each thread owns the element quads
// 4q .. 4q + 3, q = tid + k*NT (one 16-byte load of two packed x words).
template <class S>
struct NormIn {
  static constexpr int NQ = S::H / 4;              // element quads of x
  static constexpr int PQ = (NQ + NT - 1) / NT;    // quads per thread
  float g[4 * PQ];
};

template <class S>
__device__ __forceinline__ void gains_forget(NormIn<S>& n) {
#pragma unroll
  for (int k = 0; k < 4 * NormIn<S>::PQ; ++k) n.g[k] = __builtin_nondeterministic_value(n.g[k]);
}

// The gains of this thread's elements, loaded before the phase's wait.
template <class S>
__device__ __forceinline__ void gains_load(NormIn<S>& n, const uint16_t* gain) {
  constexpr int NQ = NormIn<S>::NQ;
  const int t_ = ltid();
  const uint32_t* g2 = reinterpret_cast<const uint32_t*>(gain);
#pragma unroll
  for (int k = 0; k < NormIn<S>::PQ; ++k) {  // unconditional loads: no wait until the gains are used
    const int q = t_ + k * NT < NQ ? t_ + k * NT : NQ - 1;
    const uint32_t a = g2[2 * q], b = g2[2 * q + 1];
    n.g[4 * k] = bf16_to_f32((uint16_t)a), n.g[4 * k + 1] = bf16_to_f32((uint16_t)(a >> 16));
    n.g[4 * k + 2] = bf16_to_f32((uint16_t)b), n.g[4 * k + 3] = bf16_to_f32((uint16_t)(b >> 16));
  }
}

// Block-wide sum of squares from per-thread partials -> r (unless r is null:
// the epilogue then takes norm_scale(ssw) itself).  ssw: NW floats used only
// by this call site (so no wave can overwrite a slot another wave of a
// previous call still reads).
__device__ __forceinline__ bool norm_finish(float ss, float* ssw, int failed, float h, float* r) {
  const int t_ = ltid();
  ss = wave_sum(ss);
  if (t_ % kWave == 0) ssw[t_ / kWave] = ss;
  if (block_failed(failed)) return false;
  if (r) *r = norm_scale(ssw, 1.0f / h);
  return true;
}

// Four values v (elements 4q .. 4q + 3) times their gains into the GEMV input
// dst: split-bf16 pairs for a layer GEMV, fp32 for the LM head.
template <bool SPLIT>
__device__ __forceinline__ void put_quad(float* dst, int q, const float (&v)[4], const float* g) {
  if constexpr (SPLIT) {
    xs_put_quad(reinterpret_cast<uint32_t*>(dst), 4 * q, v[0] * g[0], v[1] * g[1], v[2] * g[2], v[3] * g[3]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[4 * q + e] = v[e] * g[e];
  }
}

// Wait for the packed-pair H-vector x of tag `tag` (one bulk round of 16-byte
// loads), store x * gain to dst and the wave partials of its sum of squares
// to ssw, and return the RMSNorm scale of x in r (r null: left to the
// epilogue, norm_scale(ssw)).  Only the threads that own element quads poll
// (whole waves); the others go straight to the barrier.
template <class S, bool SPLIT = true>
__device__ __forceinline__ bool fetch_norm(const Params& p, const u64* src, unsigned tag, const NormIn<S>& n,
                                           float* dst, float* ssw, float* r, EvPoll ev = EvPoll()) {
  constexpr int PQ = NormIn<S>::PQ, NQ = NormIn<S>::NQ;
  const int tid = ltid();
  const unsigned t4 = tag4(tag);
  const auto rs = make_rsrc(src);
  int failed = 0;
  float ss = 0.f;
  __syncthreads();  // every wave is done with the LDS of its previous phase
  evp_enter(p, ev);
  if (tid < NQ) {
    u32x4 wv[PQ];
    Spin sp;
    while (true) {
      asm volatile("" ::: "memory");
      // every load is issued before any is tested (one round trip per poll
      // round); quads past the vector re-read its last quad
#pragma unroll
      for (int k = 0; k < PQ; ++k) {
        const int q = tid + k * NT;
        wv[k] = pk_get2(rs, (unsigned)(q < NQ ? q : NQ - 1) * 16u);
      }
      bool ready = true;
#pragma unroll
      for (int k = 0; k < PQ; ++k) ready &= tid + k * NT >= NQ || pk2_ready(wv[k], t4);
      if (ready) break;
      if (!sp.step(p.err, p.timeout_ticks)) {
        failed = 1;
        break;
      }
    }
    evp_exit(p, ev, sp.n + 1);
#pragma unroll
    for (int k = 0; k < PQ; ++k) {
      const int q = tid + k * NT;
      if (q < NQ) {
        const float v[4] = {pkv(wv[k].x), pkv(wv[k].y), pkv(wv[k].z), pkv(wv[k].w)};
#pragma unroll
        for (int e = 0; e < 4; ++e) ss = fmaf(v[e], v[e], ss);
        put_quad<SPLIT>(dst, q, v, n.g + 4 * k);
      }
    }
  }
  return norm_finish(ss, ssw, failed, (float)S::H, r);
}

// Barrier-free form of fetch_norm for the layer GEMVs (class kernel): wave w
// waits for the QW = H / (4 NW) element quads that are its own block
// products' input columns (lanes 0 .. QW - 1, one 16-byte load each), stages
// them and its wave partial of the sum of squares (ssw[w], read by the
// epilogue after its barrier); no barrier before the products (LDS
// operations of one wave complete in order).  Every LDS word it writes was
// last read in this workgroup's previous phase of the same type, before that
// phase's epilogue published the rows the awaited x depends on.  An
// abandoned wait sets the abort flag (read by the epilogue).
template <class S>
struct NormInW {
  float g[4];
};
template <class S>
__device__ __forceinline__ void gains_load_w(NormInW<S>& n, const uint16_t* gain) {
  constexpr int QW = S::H / 4 / NW;
  const int l = (int)lane_id(), q = wave_id() * QW + (l < QW ? l : QW - 1);
  const uint32_t* g2 = reinterpret_cast<const uint32_t*>(gain);
  const uint32_t a = g2[2 * q], b = g2[2 * q + 1];
  n.g[0] = bf16_to_f32((uint16_t)a), n.g[1] = bf16_to_f32((uint16_t)(a >> 16));
  n.g[2] = bf16_to_f32((uint16_t)b), n.g[3] = bf16_to_f32((uint16_t)(b >> 16));
}
template <class S>
__device__ __forceinline__ void fetch_norm_nb(const Params& p, const u64* src, unsigned tag, const NormInW<S>& n,
                                              float* dst, float* ssw, EvPoll ev = EvPoll()) {
  constexpr int QW = S::H / 4 / NW;
  static_assert(S::H % (4 * NW) == 0 && QW <= kWave, "a wave's input quads fit its lanes");
  const int w = wave_id(), l = (int)lane_id();
  const unsigned t4 = tag4(tag);
  const auto rs = make_rsrc(src);
  int failed = 0;
  float ss = 0.f;
  evp_enter(p, ev);
  if (l < QW) {
    const int q = w * QW + l;
    u32x4 wv;
    Spin sp;
    while (true) {
      asm volatile("" ::: "memory");
      wv = pk_get2(rs, (unsigned)q * 16u);
      if (pk2_ready(wv, t4)) break;
      if (!sp.step(p.err, p.timeout_ticks)) {
        failed = 1;
        break;
      }
    }
    evp_exit(p, ev, sp.n + 1);
    const float v[4] = {pkv(wv.x), pkv(wv.y), pkv(wv.z), pkv(wv.w)};
#pragma unroll
    for (int e = 0; e < 4; ++e) ss = fmaf(v[e], v[e], ss);
    put_quad<true>(dst, q, v, n.g);
  }
  ss = wave_sum(ss);
  if (l == 0) ssw[w] = ss;
  if (failed) wg_abort = 1;
  asm volatile("" ::: "memory");  // staging stores before the wave's B-operand reads
}
// Layer 0: wave w gathers its input quads of the embedding row of `tok`.
template <class S>
__device__ __forceinline__ void embed_norm_nb(const Params& p, int tok, const NormInW<S>& n, float* dst, float* ssw) {
  constexpr int QW = S::H / 4 / NW;
  const int w = wave_id(), l = (int)lane_id();
  float ss = 0.f;
  if (l < QW) {
    const int q = w * QW + l;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = packed_elem<S::KT_H>(p.lmhead, tok, 4 * q + e);
      ss = fmaf(v[e], v[e], ss);
    }
    put_quad<true>(dst, q, v, n.g);
  }
  ss = wave_sum(ss);
  if (l == 0) ssw[w] = ss;
  asm volatile("" ::: "memory");
}


// Wait for a packed-pair vector of 2*NPK values (NPK words, 4-bit tag t4) and,
// unless xblk < 0, the 16 residual rows of block xblk of x (8 packed words,
// tag xt4, threads 0..7), in one bulk round of 8-byte loads (hot lines that
// many workgroups poll: 16-byte loads made these rounds slower, not faster).
// (Leaving the publishing wave out of this poll, so that its own store's
// acknowledgement cannot hold up a round, measured no faster: 2,927 vs 2,934.)
template <int NPK>
__device__ __forceinline__ bool fetch_pk(const Params& p, const u64* src, unsigned t4, const u64* x, int xblk,
                                          unsigned xt4, float* dst, float* xres, EvPoll ev = EvPoll()) {
  constexpr int NPT = NT;  // polling threads
  constexpr int PER = (NPK + NPT - 1) / NPT;
  const int tid = ltid();
  const bool want_x = xblk >= 0 && tid < 8;
  int failed = 0;
  __syncthreads();
  evp_enter(p, ev);
  if (tid < NPT) {
    u64 wv[PER], wx = 0ull;
    Spin sp;
    while (true) {
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const int i = tid + k * NPT;
        wv[k] = ll_get(const_cast<u64*>(src) + (i < NPK ? i : NPK - 1));
      }
      if (want_x) wx = ll_get(const_cast<u64*>(x) + xblk * 8 + tid);
      bool ready = !want_x || pk_ready(wx, xt4);
#pragma unroll
      for (int k = 0; k < PER; ++k) ready &= tid + k * NPT >= NPK || pk_ready(wv[k], t4);
      if (ready) break;
      if (!sp.step(p.err, p.timeout_ticks)) {
        failed = 1;
        break;
      }
    }
    evp_exit(p, ev, sp.n + 1);
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int i = tid + k * NPT;
      if (i < NPK) xs_put_pair(reinterpret_cast<uint32_t*>(dst), 2 * i, pk_lo(wv[k]), pk_hi(wv[k]));
    }
    if (want_x) xres[2 * tid] = pk_lo(wx), xres[2 * tid + 1] = pk_hi(wx);
  }
  return !block_failed(failed);
}


// Wait for the 16 rows of block blk of x (8 packed words, tag t4) into xres.
__device__ __forceinline__ bool fetch_xrows(const Params& p, const u64* x, int blk, unsigned t4, float* xres) {
  const int tid = ltid();
  const auto rx = make_rsrc(x);
  int failed = 0;
  __syncthreads();  // every wave is done with the LDS of its previous phase
  if (tid < 4) {
    Spin sp;
    u32x4 w;
    while (true) {
      asm volatile("" ::: "memory");
      w = pk_get2(rx, (unsigned)(blk * 8 + 2 * tid) * 8u);
      if (pk2_ready(w, t4)) break;
      if (!sp.step(p.err, p.timeout_ticks)) {
        failed = 1;
        break;
      }
    }
    xres[4 * tid] = pkv(w.x), xres[4 * tid + 1] = pkv(w.y);
    xres[4 * tid + 2] = pkv(w.z), xres[4 * tid + 3] = pkv(w.w);
  }
  return !block_failed(failed);
}

// Layer 0: the embedding row of `tok` (gathered from the tied LM head).
template <class S>
__device__ __forceinline__ void embed_norm(const Params& p, int tok, const NormIn<S>& n, float* dst, float* ssw,
                                           float* r) {
  constexpr int NQ = NormIn<S>::NQ;
  const int tid = ltid();
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NormIn<S>::PQ; ++k) {
    const int q = tid + k * NT;
    if (q < NQ) {
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = packed_elem<S::KT_H>(p.lmhead, tok, 4 * q + e);
        ss = fmaf(v[e], v[e], ss);
      }
      put_quad<true>(dst, q, v, n.g + 4 * k);
    }
  }
  (void)norm_finish(ss, ssw, 0, (float)S::H, r);
}

// A workgroup with no role in the token's last layer reaches the LM head
// without having consumed x since the previous token, so a packed x word a
// multiple of 15 phases older than the awaited one could pass the 4-bit tag
// check.  Such a workgroup first waits for the last layer's QKV output (one
// word, full 32-bit tag, tag tl - 5): that phase read the whole x at the
// previous layer's down tag, so every x word is then at most 5 phases older
// than the LM head's.
__device__ __forceinline__ bool wait_last_qkv(const Params& p, unsigned tl) {
  int failed = 0;
  if (ltid() == 0) {
    Spin sp;
    while (ll_tag(ll_get(p.qkv)) != tl - (unsigned)PHASES_PER_LAYER)
      if (!sp.step(p.err, p.timeout_ticks)) {
        failed = 1;
        break;
      }
  }
  return !block_failed(failed);
}

// O block blk (shares in red) plus its residual rows xres, or the embedding
// row at layer 0, -> the block's 8 x words (packed pairs, tag of the phase).
// One wave (red_row4 layout).
template <class S>
__device__ __forceinline__ void o_rows(const Params& p, const float* red, const float* xres, int blk, int layer,
                                       int tok, unsigned tag, float rs = 1.0f, bool ok = true) {
  const unsigned l = lane_id();
  const int r = (int)(l >> 2);
  const float xo = layer == 0 ? packed_elem<S::KT_H>(p.lmhead, tok, blk * 16 + r) : xres[r];
  const float a = xo + red_row4(red, l) * rs;
  const float b = dpp_sel<DPP_ROW_SHL4>(a);  // the next row
  if (ok && (l & 7u) == 0u) ll_put(p.x + blk * 8 + (l >> 3), pk_pack(a, b, tag4(tag)));
}

// Down block blk (shares in red[RED_D]) plus the residual rows xres_d -> the
// block's 8 x words; dbg (layer dumps) unless null.  One wave.
template <class S>
__device__ __forceinline__ void down_rows(const Params& p, Smem<S>& sm, int blk, float* dbg, int layer,
                                          unsigned tag, float rs = 1.0f) {
  const unsigned l = lane_id();
  const int r = (int)(l >> 2);
  const float a = sm.xres_d[r] + red_row4(sm.red[RED_D], l) * rs;
  if (dbg && (l & 3u) == 0u) dbg[(long long)(layer + 1) * S::H + blk * 16 + r] = a;
  const float b = dpp_sel<DPP_ROW_SHL4>(a);
  if ((l & 7u) == 0u) ll_put(p.x + blk * 8 + (l >> 3), pk_pack(a, b, tag4(tag)));
}

// Work item i of a phase runs on workgroup (i + off) mod G.
__device__ __forceinline__ int first_item(int wg, int off, int G) { return (wg + G - (off % G)) % G; }

// ------------------------------------------------------------ attention
// KV cache on the device (the C ABI's set/get convert from/to the reference's
// [L][2][NKV][S][D] layout):
//   K:  [L][NKV][S_pad][D] bf16, row-major per position;
//   V^T: [L][NKV][S_pad/32][D][32] bf16, 32-position blocks with each dim's
//        32 values contiguous.
// Both products of a 32-position block run on the matrix cores
// (v_mfma_f32_16x16x32_bf16: D[m][n] = sum_k A[m][k] B[k][n]; lane l holds
// A[l & 15][8 (l >> 4) + e], B[8 (l >> 4) + e][l & 15] and
// D[4 (l >> 4) + i][l & 15]):
//   scores[r][pos] = Qb[r][:] . K[pos][:]   (B = K^T: a lane's 8 dims of one cached row)
//   out[r][dim]    = Pb[r][:] . V[:][dim]   (B = V:   a lane's 8 positions of one V^T row)
// Row r = 4 j + part carries q head j (resp. its softmax weights) split into
// three bf16 parts hi + mid + lo, which reproduces fp32 activations.  Lanes
// 16 j .. 16 j + 15 therefore hold head j's three part rows (i = 0..2), sum
// them in-register and own 16 positions (resp. dims) of head j each.
// A work item (kv head g, split s) covers whole 32-position blocks
// [t0, t1); wave w takes the item's blocks w, w + NW, ...
template <class S, bool K8 = false>
struct KV {
  static constexpr int KC = S::D / 32;  // k-steps of the score product
  static constexpr int DT = S::D / 16;  // dim tiles of the output product
  // 8 values per lane and operand: bf16 (u32x4) or, for an FP8 cache, e4m3 codes (u32x2)
  using Reg = typename std::conditional<K8, u32x2, u32x4>::type;
  Reg k[KVB][2][KC];  // K of the wave's blocks: [block][16-position half][k-step]
  Reg v[KVB][DT];     // V^T of the blocks: [block][dim tile]
  float sk[K8 ? KVB : 1][2], sv[K8 ? KVB : 1][2];  // FP8: scales of the lane's score positions
  uint16_t gn[S::D / kWave];  // QK-norm gain(s) of this lane's dim(s) for its wave's head
};

// Words of one item's published partial: GQA * D / 2 packed pairs of the
// unnormalised output, then one packed (max, sum) pair per q head, padded to
// whole 128-byte lines (no line is shared by two items).
template <class S>
constexpr int part_words() { return (S::GQA * S::D / 2 + S::GQA + 15) / 16 * 16; }

// u32x4 holding 8 bf16 with element e (0..7) replaced by v (register-only).
__device__ __forceinline__ u32x4 set_bf16(u32x4 x, int e, uint16_t v) {
  const unsigned lo_mask = (e & 1) ? 0x0000ffffu : 0xffff0000u;
  const unsigned put = (e & 1) ? ((unsigned)v << 16) : (unsigned)v;
  u32x4 r = x;
#pragma unroll
  for (int c = 0; c < 4; ++c) r[c] = (c == (e >> 1)) ? ((x[c] & lo_mask) | put) : x[c];
  return r;
}

__device__ __forceinline__ long long kt_base(const Params& p, int layer, int g, int nkv, int d) {
  return ((long long)layer * nkv + g) * (long long)p.s_pad * d;
}

// KV cache loads use agent-scope (sc1) reads: positions appended by another
// workgroup in an earlier token must not be served from a stale L2 line.
__device__ __forceinline__ u32x4 buf_ld_kv(__amdgpu_buffer_rsrc_t rs, unsigned voff) {
  return __builtin_amdgcn_raw_buffer_load_b128(rs, voff, 0u, 16 | 2);
}

// Loads this wave's KVB blocks of an item starting at block index `bi`
// (item blocks bi, bi + NW, ...; blocks past the item's nb repeat a valid
// block and are masked by the caller).
template <class S, bool K8>
__device__ __forceinline__ void kv_load(KV<S, K8>& r, const Params& p, int layer, int g, int b0, int nb, int bi) {
  constexpr int D = S::D;
  const unsigned l = lane_id();
  const long long base = kt_base(p, layer, g, S::NKV, D);
#pragma unroll
  for (int q = 0; q < KVB; ++q) {
    const int bq = bi + q * NW;
    const int blk = b0 + (bq < nb ? bq : 0);
    if constexpr (K8) {  // byte index = element index of the bf16 layout
      const auto rk = make_rsrc(reinterpret_cast<const uint8_t*>(p.kv) + base + (long long)blk * 32 * D);
      const auto rv = make_rsrc(reinterpret_cast<const uint8_t*>(p.kvt) + base + (long long)blk * 32 * D);
      const long long sb = ((long long)layer * S::NKV + g) * p.s_pad + (long long)blk * 32;
      const auto rks = make_rsrc(p.kscale + sb);
      const auto rvs = make_rsrc(p.vscale + sb);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int kc = 0; kc < KV<S, K8>::KC; ++kc)
          r.k[q][h][kc] = __builtin_amdgcn_raw_buffer_load_b64(
              rk, (16u * h + (l & 15u)) * D + 32u * kc + 8u * (l >> 4), 0u, 16 | 2);
        r.sk[q][h] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rks, (16u * h + (l & 15u)) * 4u, 0u, 16 | 2));
        r.sv[q][h] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rvs, (16u * h + (l & 15u)) * 4u, 0u, 16 | 2));
      }
#pragma unroll
      for (int dt = 0; dt < KV<S, K8>::DT; ++dt)
        r.v[q][dt] = __builtin_amdgcn_raw_buffer_load_b64(rv, (16u * dt + (l & 15u)) * 32u + 8u * (l >> 4), 0u, 16 | 2);
    } else {
      const auto rk = make_rsrc(p.kv + base + (long long)blk * 32 * D);
      const auto rv = make_rsrc(p.kvt + base + (long long)blk * 32 * D);
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int kc = 0; kc < KV<S, K8>::KC; ++kc)
          r.k[q][h][kc] = buf_ld_kv(rk, ((16u * h + (l & 15u)) * D + 32u * kc + 8u * (l >> 4)) * 2u);
#pragma unroll
      for (int dt = 0; dt < KV<S, K8>::DT; ++dt)
        r.v[q][dt] = buf_ld_kv(rv, ((16u * dt + (l & 15u)) * 32u + 8u * (l >> 4)) * 2u);
    }
  }
}

template <class S, bool K8>
__device__ __forceinline__ void kv_forget(KV<S, K8>& r) {
#pragma unroll
  for (int q = 0; q < KVB; ++q) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int kc = 0; kc < KV<S, K8>::KC; ++kc) r.k[q][h][kc] = __builtin_nondeterministic_value(r.k[q][h][kc]);
#pragma unroll
    for (int dt = 0; dt < KV<S, K8>::DT; ++dt) r.v[q][dt] = __builtin_nondeterministic_value(r.v[q][dt]);
  }
  if constexpr (K8) {
#pragma unroll
    for (int q = 0; q < KVB; ++q)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        r.sk[q][h] = __builtin_nondeterministic_value(r.sk[q][h]);
        r.sv[q][h] = __builtin_nondeterministic_value(r.sv[q][h]);
      }
  }
#pragma unroll
  for (int c = 0; c < S::D / kWave; ++c) r.gn[c] = __builtin_nondeterministic_value(r.gn[c]);
}

// QK-norm gains of this lane's dims: waves 0..GQA-1 normalise q heads, wave
// GQA the k head.
template <class S, bool K8>
__device__ __forceinline__ void gain_load_qk(KV<S, K8>& r, const Params& p, int layer) {
  const int t_ = ltid(), w = t_ / kWave, l = t_ % kWave;
  const uint16_t* g = p.norms + (long long)layer * S::NORM_STRIDE + (w < S::GQA ? S::NORM_Q : S::NORM_K);
#pragma unroll
  for (int c = 0; c < S::D / kWave; ++c) r.gn[c] = g[l + c * kWave];
}

// The split of the n = pos + 1 cached positions among items: nsplit splits of
// whole 32-position blocks, as even as possible (every split non-empty).
// nsplit never decreases as the position grows, so a consumer of split slot
// s < nsplit only ever finds this layer's word or an older one with another
// tag there.
__host__ __device__ __forceinline__ int split_count(int n, int chunk_min, int nsplit_max) {
  const int nbt = (n + 31) / 32;
  int ns = (n + chunk_min - 1) / chunk_min;
  ns = ns < 1 ? 1 : ns;
  ns = ns > nsplit_max ? nsplit_max : ns;
  return ns > nbt ? nbt : ns;
}
// Positions [t0, t1) of split s of ns.
__device__ __forceinline__ void split_range(int n, int ns, int s, int* t0, int* t1) {
  const int nbt = (n + 31) / 32;
  *t0 = 32 * (s * nbt / ns);
  *t1 = min(n, 32 * ((s + 1) * nbt / ns));
}

// The attention item of work index `it` for n cached positions: kv head g,
// split s of nsplit, positions [t0, t1).
struct Item {
  bool on;
  int g, s, t0, t1, nsplit;
};
__device__ __forceinline__ Item att_item(int it, int n, int nkv, int chunk_min, int nsplit_max) {
  Item r;
  r.nsplit = split_count(n, chunk_min, nsplit_max);
  r.on = it < nkv * r.nsplit;
  r.g = r.on ? it / r.nsplit : 0;
  r.s = r.on ? it % r.nsplit : 0;
  split_range(n, r.nsplit, r.s, &r.t0, &r.t1);
  return r;
}

// Stage 1 of an attention item: wait for q, k and v of kv head g (wave
// w < GQA: q head g GQA + w; wave GQA: k; wave GQA + 1: v; lane l holds dims
// l + 64 c), then per-head RMSNorm (reference rmsnorm.cuh:57-84) and RoPE
// rotate-half (attention.cuh:22-44) in registers:
//   q waves write the three bf16 parts of q as the score product's A rows;
//   the k / v waves put bf16 K / V of `pos` in LDS (for the block holding pos)
//   and, in the split that owns pos, append them to the cache (reference
//   kv_cache.cuh:58-78; write-through agent-scope stores, read by later
//   tokens on any XCD).
// FP8 cache append of one K or V row (D values, DPL per lane of one wave):
// the power-of-two scale from the wave's absolute maximum, the e4m3 codes
// (dim d at byte dst[d * stride]) and the scale, written through to the
// device-coherent level; the codes and the scale also go to LDS for this
// token's own attention.
template <int DPL>
__device__ __forceinline__ void kv_append_fp8(const float* val, uint8_t* dst, int stride, float* scale_dst,
                                              uint8_t* lds_codes, float* lds_scale, bool append) {
  const int l = (int)lane_id();
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < DPL; ++c) amax = fmaxf(amax, fabsf(val[c]));
  const int e = e4m3_row_exp(wave_max(amax));
#pragma unroll
  for (int c = 0; c < DPL; ++c) {
    const uint8_t code = (uint8_t)e4m3_encode(ldexpf(val[c], -e));
    lds_codes[l + c * kWave] = code;
    if (append)
      __hip_atomic_store(dst + (long long)(l + c * kWave) * stride, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (l == 0) {
    *lds_scale = ldexpf(1.f, e);
    if (append) __hip_atomic_store(scale_dst, ldexpf(1.f, e), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <class S, int MODE>
__device__ __forceinline__ bool attention_prologue(const Params& p, Smem<S>& sm, const KV<S, (MODE & 8) != 0>& kvr,
                                                   int layer,
                                                   int pos, int g, bool own, unsigned tg, int tt) {
  constexpr int D = S::D, GQA = S::GQA, DPL = D / kWave;
  const int w = wave_id();
  const int l = (int)lane_id();
  int failed = 0;
  float v[DPL];
#pragma unroll
  for (int c = 0; c < DPL; ++c) v[c] = 0.f;
  __syncthreads();  // every wave is done with the LDS of its previous phase
  const EvPoll ev = ev_at(tt, layer, PS_ATT);
  evp_enter(p, ev);
  if (w < GQA + 2) {
    u64* src = p.qkv + (w < GQA ? (g * GQA + w) * D : (w == GQA ? S::QD + g * D : S::QD + S::KVD + g * D));
    Spin sp;
    while (true) {
      u64 wv[DPL];
      bool ready = true;
#pragma unroll
      for (int c = 0; c < DPL; ++c) {
        wv[c] = ll_get(src + l + kWave * c);
        ready &= ll_tag(wv[c]) == tg;
      }
      if (ready) {
#pragma unroll
        for (int c = 0; c < DPL; ++c) v[c] = ll_val(wv[c]);
        break;
      }
      if (!sp.step(p.err, p.timeout_ticks)) {
        failed = 1;
        break;
      }
    }
    evp_exit(p, ev, sp.n + 1);
  }
  if constexpr ((MODE & 2) != 0) trace_mark(p, tt, PHASES_PER_LAYER * layer + 1, 0);
  evt(p, tt, layer, EV_ATT_READY);
  const bool append = own && __ballot(failed) == 0ull;  // never append values of a failed wait
  const long long base = kt_base(p, layer, g, S::NKV, D);
  if (w <= GQA) {
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < DPL; ++c) ss = fmaf(v[c], v[c], ss);
    ss = wave_sum(ss);
    const float r = rsqrtf(ss / (float)D + kRmsEps);
#pragma unroll
    for (int c = 0; c < DPL; ++c) v[c] = v[c] * r * bf16_to_f32(kvr.gn[c]);
    float o[DPL];
    if constexpr (DPL == 1) {  // partner of dim l is l ^ 32, in another lane
      const float partner = lane_xor32(v[0]);
      const int d = l & 31;
      o[0] = l < 32 ? v[0] * sm.rc[d] - partner * sm.rs[d] : v[0] * sm.rc[d] + partner * sm.rs[d];
    } else {  // D = 128: dims l and l + 64 pair up in the same lane
      o[0] = v[0] * sm.rc[l] - v[1] * sm.rs[l];
      o[1] = v[1] * sm.rc[l] + v[0] * sm.rs[l];
    }
    if (w < GQA) {
#pragma unroll
      for (int c = 0; c < DPL; ++c) {
        uint16_t hi, mid, lo;
        split_bf16(o[c], hi, mid, lo);
        sm.qb[4 * w + 0][l + c * kWave] = hi;
        sm.qb[4 * w + 1][l + c * kWave] = mid;
        sm.qb[4 * w + 2][l + c * kWave] = lo;
      }
    } else if constexpr ((MODE & 8) != 0) {
      kv_append_fp8<DPL>(o, reinterpret_cast<uint8_t*>(p.kv) + base + (long long)pos * D, 1,
                         p.kscale + ((long long)layer * S::NKV + g) * p.s_pad + pos,
                         reinterpret_cast<uint8_t*>(sm.kvcur[0]), &sm.kvcs[0], append);
    } else {
      uint16_t* krow = p.kv + base + (long long)pos * D;
#pragma unroll
      for (int c = 0; c < DPL; ++c) {
        const uint16_t kb = f32_to_bf16(o[c]);
        reinterpret_cast<uint16_t*>(sm.kvcur[0])[l + c * kWave] = kb;
        if (append) __hip_atomic_store(krow + l + c * kWave, kb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  } else if (w == GQA + 1) {
    if constexpr ((MODE & 8) != 0) {
      kv_append_fp8<DPL>(v, reinterpret_cast<uint8_t*>(p.kvt) + base + (long long)(pos / 32) * 32 * D + (pos % 32), 32,
                         p.vscale + ((long long)layer * S::NKV + g) * p.s_pad + pos,
                         reinterpret_cast<uint8_t*>(sm.kvcur[1]), &sm.kvcs[1], append);
    } else {
      uint16_t* vt = p.kvt + base + (long long)(pos / 32) * 32 * D + (pos % 32);
#pragma unroll
      for (int c = 0; c < DPL; ++c) {
        const uint16_t vb = f32_to_bf16(v[c]);
        reinterpret_cast<uint16_t*>(sm.kvcur[1])[l + c * kWave] = vb;
        if (append)
          __hip_atomic_store(vt + (long long)(l + c * kWave) * 32, vb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  return !block_failed(failed);
}

template <class S>
__device__ bool attention_merge(const Params& p, Smem<S>& sm, int g, int nsplit, unsigned tg);

// One attention item (kv head g, split s of nsplit over positions [t0, t1)):
// per-wave online softmax over the wave's blocks on the matrix cores, the NW
// waves combined in LDS, and the item's partial -- unnormalised output and
// (max, sum) per q head -- published as packed pairs for the O phase, which
// merges the splits (MODE bit 0: beyond merge_min splits the first split's
// workgroup merges them; without it that code is not compiled in).  K / V of
// the wave's first blocks are already in kvr.
template <class S, int MODE>
__device__ bool attention_compute(const Params& p, Smem<S>& sm, KV<S, (MODE & 8) != 0>& kvr, int layer, int pos,
                                  int g, int s, int nsplit, int t0, int t1, unsigned tg, int tt) {
  constexpr bool K8 = (MODE & 8) != 0;
  constexpr int D = S::D, GQA = S::GQA, KC = KV<S, K8>::KC, DT = KV<S, K8>::DT;
  static_assert(GQA <= 4, "q heads of a group fit the 16 MFMA rows (4 per head)");
  if (!attention_prologue<S, MODE>(p, sm, kvr, layer, pos, g, t0 <= pos && pos < t1, tg, tt)) return false;
  evt(p, tt, layer, EV_ATT_ROPE);
  const int tid = ltid(), w = tid / kWave;
  const float scale = 1.0f / sqrtf((float)D);
  const unsigned lu = lane_id();
  const int c16 = (int)(lu & 15u), rg = (int)(lu >> 4);  // MFMA column / row group (= head)
  u32x4 qa[KC];  // A operand of the score product
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) qa[kc] = *reinterpret_cast<const u32x4*>(&sm.qb[c16][32 * kc + 8 * rg]);
  float m = -INFINITY, lsum = 0.f;  // of head rg (meaningful for rg < GQA)
  f32x4 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int b0 = t0 / 32, nb = (t1 - t0 + 31) / 32;
  // groups of KVB blocks (w + NW * (KVB * gi + q)); the first group was
  // prefetched, later ones (long contexts) are loaded here
  for (int bi = w; bi < nb; bi += KVB * NW) {
    if (bi != w) kv_load<S>(kvr, p, layer, g, b0, nb, bi);
    // the block holding pos takes K / V of pos from LDS
#pragma unroll
    for (int q = 0; q < KVB; ++q) {
      const int bp = 32 * (b0 + bi + q * NW);
      if (bi + q * NW < nb && bp <= pos && pos < bp + 32) {
        const int rp = pos - bp;
        if constexpr (K8) {
          if (c16 == (rp & 15)) {
            const u32x2* kc8 = reinterpret_cast<const u32x2*>(sm.kvcur[0]);
#pragma unroll
            for (int kc = 0; kc < KC; ++kc)
              if (rp >> 4) kvr.k[q][1][kc] = kc8[4 * kc + rg];
              else kvr.k[q][0][kc] = kc8[4 * kc + rg];
            if (rp >> 4) kvr.sk[q][1] = sm.kvcs[0], kvr.sv[q][1] = sm.kvcs[1];
            else kvr.sk[q][0] = sm.kvcs[0], kvr.sv[q][0] = sm.kvcs[1];
          }
          if (rg == (rp >> 3)) {
            const uint8_t* vc = reinterpret_cast<const uint8_t*>(sm.kvcur[1]);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) kvr.v[q][dt] = set_u8(kvr.v[q][dt], rp & 7, vc[16 * dt + c16]);
          }
        } else {
          if (c16 == (rp & 15)) {
#pragma unroll
            for (int kc = 0; kc < KC; ++kc)
              if (rp >> 4) kvr.k[q][1][kc] = sm.kvcur[0][4 * kc + rg];
              else kvr.k[q][0][kc] = sm.kvcur[0][4 * kc + rg];
          }
          if (rg == (rp >> 3)) {
            const uint16_t* vc = reinterpret_cast<const uint16_t*>(sm.kvcur[1]);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) kvr.v[q][dt] = set_bf16(kvr.v[q][dt], rp & 7, vc[16 * dt + c16]);
          }
        }
      }
    }
    // scores: lane (rg, c16) gets head rg at positions 32 (b0 + bi + q NW) + 16 h + c16
    float sc[KVB][2];
    float bmax = -INFINITY;
#pragma unroll
    for (int q = 0; q < KVB; ++q)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        f32x4 d4 = f32x4{0.f, 0.f, 0.f, 0.f};
        // a block past the item (the wave has fewer blocks than KVB) is all
        // -inf below: its products are skipped (a wave-uniform branch)
        if (bi + q * NW < nb) {
#pragma unroll
          for (int kc = 0; kc < KC; ++kc) {
            u32x4 kb;  // FP8: a lane's 8 values share one position, so its K scale enters here
            if constexpr (K8) kb = fp8x8_to_bf16x8_scaled(kvr.k[q][h][kc], kvr.sk[q][h]);
            else kb = kvr.k[q][h][kc];
            d4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, qa[kc]),
                                                        __builtin_bit_cast(bf16x8, kb), d4, 0, 0, 0);
          }
        }
        const float v = (d4[0] + d4[1]) + d4[2];
        const int t = 32 * (b0 + bi + q * NW) + 16 * h + c16;
        sc[q][h] = (bi + q * NW < nb && t < t1) ? v * scale : -INFINITY;
        bmax = fmaxf(bmax, sc[q][h]);
      }
    bmax = group_max<16>(bmax);
    const float mn = fmaxf(m, bmax);  // finite: block bi has a valid position
    const float alpha = __expf(m - mn);
    m = mn;
    float bsum = 0.f;
#pragma unroll
    for (int q = 0; q < KVB; ++q)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        sc[q][h] = __expf(sc[q][h] - mn);
        bsum += sc[q][h];
      }
    lsum = lsum * alpha + group_sum<16>(bsum);
    // weights -> the output product's A rows via LDS (rows 4 rg .. 4 rg + 2;
    // LDS operations of one wave complete in order; the other rows stay 0)
    if (rg < GQA) {
#pragma unroll
      for (int q = 0; q < KVB; ++q)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          // FP8 cache: the V row's scale enters with the weight (the sum above stays unscaled)
          const Split3 a = split3(K8 ? sc[q][h] * kvr.sv[q][h] : sc[q][h]);
          const int o = 32 * q + 16 * h + c16;
          sm.pb[w][4 * rg + 0][o] = (uint16_t)(a.hi >> 16);
          sm.pb[w][4 * rg + 1][o] = (uint16_t)(a.mid >> 16);
          sm.pb[w][4 * rg + 2][o] = (uint16_t)(a.lo >> 16);
        }
    }
    asm volatile("" ::: "memory");
    u32x4 pa[KVB];
#pragma unroll
    for (int q = 0; q < KVB; ++q) pa[q] = *reinterpret_cast<const u32x4*>(&sm.pb[w][c16][32 * q + 8 * rg]);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[dt][i] *= alpha;
#pragma unroll
      for (int q = 0; q < KVB; ++q) {
        if (bi + q * NW < nb) {  // a skipped block has weight 0: no product
          u32x4 vb;
          if constexpr (K8) vb = fp8x8_to_bf16x8_scaled(kvr.v[q][dt], 1.0f);  // V scales ride on the weights
          else vb = kvr.v[q][dt];
          acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, pa[q]),
                                                           __builtin_bit_cast(bf16x8, vb), acc[dt], 0, 0, 0);
        }
      }
    }
  }
  evt(p, tt, layer, EV_ATT_SOFTMAX);
  // per-wave partials -> LDS (lane (rg, c16): head rg, dims 16 dt + c16)
  if (rg < GQA) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) sm.pv[w][rg * D + 16 * dt + c16] = (acc[dt][0] + acc[dt][1]) + acc[dt][2];
    if (c16 == 0) {
      sm.mw[rg][w] = m;
      sm.lw[rg][w] = lsum;
    }
  }
  __syncthreads();
  evt(p, tt, layer, EV_ATT_REDUCED);
  // The item's partial over its NW waves: one output pair (two dims of one
  // head) per lane of the first NPAIR / 64 waves, so each of those waves
  // publishes whole 128-byte lines.  A wave without positions has max -inf
  // and weight exp(-inf) = 0; the item's max is finite.
  constexpr int NPAIR = GQA * D / 2;
  static_assert(NPAIR <= NT, "pairs of a group fit the workgroup");
  if (tid < NPAIR) {
    const int pi = tid, j = (2 * pi) / D;
    float mv[NW], lv[NW];
    float2 pv[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      mv[i] = sm.mw[j][i];
      lv[i] = sm.lw[j][i];
      pv[i] = *reinterpret_cast<const float2*>(&sm.pv[i][2 * pi]);
    }
    float M = mv[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) M = fmaxf(M, mv[i]);
    float o0 = 0.f, o1 = 0.f, ls = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      const float f = __expf(mv[i] - M);
      o0 = fmaf(f, pv[i].x, o0);
      o1 = fmaf(f, pv[i].y, o1);
      ls = fmaf(f, lv[i], ls);
    }
    const unsigned t4 = tag4(tg + 1u);
    u64* dst = p.part + ((long long)s * S::NKV + g) * part_words<S>();
    ll_put(dst + pi, pk_pack(o0, o1, t4));
    if ((2 * pi) % D == 0) ll_put(dst + NPAIR + j, pk_pack(M, ls, t4));
  }
  evt(p, tt, layer, EV_ATT_PARTIAL);
  if constexpr ((MODE & 1) != 0) {
    if (nsplit > p.merge_min && s == 0) return attention_merge<S>(p, sm, g, nsplit, tg);
  }
  return true;
}

// Long contexts: many splits per kv head would make every O workgroup read
// and merge all of them (hot lines, several rounds), so the workgroup of
// split 0 of head g waits for the head's other partials, merges them once and
// publishes one merged partial (the row after the splits) for the O phase.
// Each thread reads its output pair from every SGN-th split in one load
// round; the SGN split groups are combined in LDS.  Same log-sum-exp merge as
// the O phase's.
template <class S>
__device__ bool attention_merge(const Params& p, Smem<S>& sm, int g, int nsplit, unsigned tg) {
  constexpr int NPAIR = S::GQA * S::D / 2, WP = part_words<S>();
  constexpr int SGN = NT / NPAIR, PER = NSPLIT_CAP / SGN;
  static_assert(NT % NPAIR == 0 && NSPLIT_CAP % SGN == 0, "split groups tile the workgroup");
  const int tid = ltid();
  const unsigned t4 = tag4(tg + 1u);
  const int pi = tid % NPAIR, sg = tid / NPAIR, j = (2 * pi) / S::D;
  int failed = 0;
  float M = -INFINITY, o0 = 0.f, o1 = 0.f, L = 0.f;
  const bool ok = poll_rounds<2 * PER>(
      p,
      [&](u64(&w)[2 * PER]) {  // splits past nsplit re-read split 0
#pragma unroll
        for (int u = 0; u < PER; ++u) {
          const int sp = sg + u * SGN < nsplit ? sg + u * SGN : 0;
          const u64* src = p.part + ((long long)sp * S::NKV + g) * WP;
          w[2 * u] = ll_get(const_cast<u64*>(src) + pi);
          w[2 * u + 1] = ll_get(const_cast<u64*>(src) + NPAIR + j);
        }
      },
      [&](const u64(&w)[2 * PER]) {
        bool ready = true;
#pragma unroll
        for (int u = 0; u < PER; ++u) ready &= pk_ready(w[2 * u], t4) && pk_ready(w[2 * u + 1], t4);
        return ready;
      },
      [&](const u64(&w)[2 * PER]) {
#pragma unroll
        for (int u = 0; u < PER; ++u) M = sg + u * SGN < nsplit ? fmaxf(M, pk_lo(w[2 * u + 1])) : M;
#pragma unroll
        for (int u = 0; u < PER; ++u) {
          const bool on = sg + u * SGN < nsplit;
          const float f = __expf(pk_lo(w[2 * u + 1]) - M);
          o0 = on ? fmaf(f, pk_lo(w[2 * u]), o0) : o0;
          o1 = on ? fmaf(f, pk_hi(w[2 * u]), o1) : o1;
          L = on ? fmaf(f, pk_hi(w[2 * u + 1]), L) : L;
        }
      });
  if (!ok) failed = 1;
  sm.mrg[0][tid] = M, sm.mrg[1][tid] = L, sm.mrg[2][tid] = o0, sm.mrg[3][tid] = o1;
  __syncthreads();
  if (tid < NPAIR) {
    float Mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < SGN; ++k) Mx = fmaxf(Mx, sm.mrg[0][tid + k * NPAIR]);  // group 0 always has split 0
    float a0 = 0.f, a1 = 0.f, ls = 0.f;
#pragma unroll
    for (int k = 0; k < SGN; ++k) {
      const int i = tid + k * NPAIR;
      const float f = sm.mrg[0][i] == -INFINITY ? 0.f : __expf(sm.mrg[0][i] - Mx);
      a0 = fmaf(f, sm.mrg[2][i], a0);
      a1 = fmaf(f, sm.mrg[3][i], a1);
      ls = fmaf(f, sm.mrg[1][i], ls);
    }
    u64* dst = p.part + ((long long)p.nsplit_max * S::NKV + g) * WP;
    ll_put(dst + pi, pk_pack(a0, a1, t4));
    if ((2 * pi) % S::D == 0) ll_put(dst + NPAIR + j, pk_pack(Mx, ls, t4));
  }
  return !block_failed(failed);
}

// O phase input: wait for the partials of the nsplit splits of every kv head
// and merge them (log-sum-exp, reference attention.cuh:96-140 computes the
// same softmax in one pass) into dst[QD], in batches of SB splits with a
// running max; plus, unless xb0 < 0, the 16 residual rows of x block xb0
// (threads 0..7) and, unless xb1 < 0, of block xb1 (threads 8..15).  Thread t
// owns output pairs t + k NT (8-byte loads, as fetch_pk).  A batch's slots
// past nsplit are skipped by wave-uniform branches; fetch_attn picks SB from
// the split count, so the registers and the merge arithmetic of a round are
// those of the splits that exist (the merge sits between the last poll round
// and the O products, on the critical path).
template <class S, int SB>
__device__ __forceinline__ int fetch_attn_core(const Params& p, const u64* part, int nsplit, unsigned t4, const u64* x,
                                               int xb0, int xb1, unsigned xt4, float* dst, float* xres, EvPoll ev) {
  constexpr int NPG = S::GQA * S::D / 2;
  constexpr int WP = part_words<S>();
  constexpr int PPT = (S::QD / 2 + NT - 1) / NT;
  const int tid = ltid();
  const bool want_x0 = xb0 >= 0 && (tid < 8 || (tid < 16 && xb1 >= 0));
  int failed = 0;
  float M[PPT], L[PPT], o0[PPT], o1[PPT];
#pragma unroll
  for (int k = 0; k < PPT; ++k) M[k] = -INFINITY, L[k] = 0.f, o0[k] = 0.f, o1[k] = 0.f;
  evp_enter(p, ev);
  unsigned rounds = 0;
  for (int s0 = 0; s0 < nsplit && !failed; s0 += SB) {
    u64 wa[PPT][SB], wm[PPT][SB], wx = 0ull;
    const bool want_x = s0 == 0 && want_x0;
    Spin sp;
    while (true) {
#pragma unroll
      for (int k = 0; k < PPT; ++k) {
        const int pi = tid + k * NT < S::QD / 2 ? tid + k * NT : 0;
        const int g = pi / NPG, pg = pi % NPG, j = (2 * pg) / S::D;
#pragma unroll
        for (int u = 0; u < SB; ++u) {
          wa[k][u] = wm[k][u] = 0ull;
          if (s0 + u < nsplit) {
            u64* src = const_cast<u64*>(part) + ((long long)(s0 + u) * S::NKV + g) * WP;
            wa[k][u] = ll_get(src + pg);
            wm[k][u] = ll_get(src + NPG + j);
          }
        }
      }
      if (want_x) wx = ll_get(const_cast<u64*>(x) + (tid < 8 ? xb0 : xb1) * 8 + (tid & 7));
      bool ready = !want_x || pk_ready(wx, xt4);
#pragma unroll
      for (int k = 0; k < PPT; ++k)
#pragma unroll
        for (int u = 0; u < SB; ++u)
          ready &= tid + k * NT >= S::QD / 2 || s0 + u >= nsplit ||
                   (pk_ready(wa[k][u], t4) && pk_ready(wm[k][u], t4));
      if (ready) break;
      if (!sp.step(p.err, p.timeout_ticks)) {
        failed = 1;
        break;
      }
    }
    rounds += sp.n + 1;
    if (want_x) xres[2 * tid] = pk_lo(wx), xres[2 * tid + 1] = pk_hi(wx);
    const int nb = nsplit - s0 < SB ? nsplit - s0 : SB;  // splits in this batch (wave-uniform)
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      float Mb = M[k];
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        if (u >= nb) break;
        Mb = fmaxf(Mb, pk_lo(wm[k][u]));
      }
      const float r = __expf(M[k] - Mb);
      o0[k] *= r, o1[k] *= r, L[k] *= r;
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        if (u >= nb) break;
        const float f = __expf(pk_lo(wm[k][u]) - Mb);
        o0[k] = fmaf(f, pk_lo(wa[k][u]), o0[k]);
        o1[k] = fmaf(f, pk_hi(wa[k][u]), o1[k]);
        L[k] = fmaf(f, pk_hi(wm[k][u]), L[k]);
      }
      M[k] = Mb;
    }
  }
#pragma unroll
  for (int k = 0; k < PPT; ++k) {
    const int pi = tid + k * NT;
    if (pi < S::QD / 2) {
      const float il = __builtin_amdgcn_rcpf(L[k]);  // one reciprocal (~1 ulp) for both outputs
      xs_put_pair(reinterpret_cast<uint32_t*>(dst), 2 * pi, o0[k] * il, o1[k] * il);
    }
  }
  evp_exit(p, ev, rounds);
  return failed;
}

// Batch size by split count: 2, 3 or 4 splits in one batch (the class
// kernel's contexts up to 2,048 positions), batches of 4 up to 8 splits, of 8
// beyond (the spread kernel's long contexts).
template <class S>
__device__ __forceinline__ int fetch_attn_any(const Params& p, const u64* part, int nsplit, unsigned t4, const u64* x,
                                              int xb0, int xb1, unsigned xt4, float* dst, float* xres, EvPoll ev) {
  if (nsplit <= 2) return fetch_attn_core<S, 2>(p, part, nsplit, t4, x, xb0, xb1, xt4, dst, xres, ev);
  if (nsplit == 3) return fetch_attn_core<S, 3>(p, part, nsplit, t4, x, xb0, xb1, xt4, dst, xres, ev);
  if (nsplit <= 8) return fetch_attn_core<S, 4>(p, part, nsplit, t4, x, xb0, xb1, xt4, dst, xres, ev);
  return fetch_attn_core<S, 8>(p, part, nsplit, t4, x, xb0, xb1, xt4, dst, xres, ev);
}

// Workgroup-synchronous form (spread kernel): a barrier before (every wave is
// done with the LDS of its previous phase) and after (the staged input is
// complete; false when a wait was abandoned).
template <class S>
__device__ __forceinline__ bool fetch_attn(const Params& p, const u64* part, int nsplit, unsigned t4, const u64* x,
                                            int xb0, int xb1, unsigned xt4, float* dst, float* xres,
                                            EvPoll ev = EvPoll()) {
  __syncthreads();
  return !block_failed(fetch_attn_any<S>(p, part, nsplit, t4, x, xb0, xb1, xt4, dst, xres, ev));
}

// Barrier-free form (class kernel).  When the pairs are as many as the
// threads (BASELINE: QD / 2 = 512), thread t stages pair t, so wave w stages
// exactly the QD / NW input columns its own block products read (LDS
// operations of one wave complete in order): no barrier before the products.
// No barrier before the wait either: every LDS word this phase writes (its
// staged input, block shares, residual rows) was last read in this
// workgroup's previous O phase, before that phase's epilogue stored the x
// rows that this phase's partials depend on.  A wait abandoned by any thread
// sets the workgroup's abort flag; the caller reads it after its epilogue
// barrier (block_aborted).
template <class S>
__device__ __forceinline__ void fetch_attn_nb(const Params& p, const u64* part, int nsplit, unsigned t4, const u64* x,
                                              int xb0, int xb1, unsigned xt4, float* dst, float* xres,
                                              EvPoll ev = EvPoll()) {
  if (fetch_attn_any<S>(p, part, nsplit, t4, x, xb0, xb1, xt4, dst, xres, ev)) wg_abort = 1;
  if constexpr (S::QD / 2 != NT) __syncthreads();  // a wave's pairs are not its own input columns
  else asm volatile("" ::: "memory");              // staging stores before the wave's B-operand reads
}

// argmax over the G per-workgroup words of a token (tag t14): the token id.
__device__ __forceinline__ bool token_from_slots(const Params& p, u64* slots, unsigned t14, u64* red, int* tok) {
  const int G = gridDim.x, tid = ltid(), w = tid / kWave, l = tid % kWave;
  int failed = 0;
  u64 best = 0;
  for (int i = tid; i < G && !failed; i += NT) {
    Spin sp;
    u64 v;
    while (((v = ll_get(slots + i)) & TAG14) != t14)
      if (!sp.step(p.err, p.timeout_ticks)) {
        failed = 1;
        break;
      }
    best = v > best ? v : best;
  }
  if (block_failed(failed)) return false;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const u64 o = __shfl_xor(best, m);
    best = o > best ? o : best;
  }
  if (l == 0) red[w] = best;
  __syncthreads();
  best = red[0];
  for (int i = 1; i < NW; ++i) best = red[i] > best ? red[i] : best;
  __syncthreads();
  const unsigned idx = IDX_MAX - (unsigned)((best >> 14) & IDX_MAX);
  *tok = idx < (unsigned)p.vocab ? (int)idx : 0;
  return true;
}

// ------------------------------------------------------------------ kernel
// MODE bit 0 (LC): the launch's contexts reach more than merge_min attention
// splits per kv head (long-context merge and deferred K/V prefetch compiled
// in); bit 1 (DBG): per-phase timestamps and the validation outputs
// (dbg_layers, dbg_logits) compiled in; bit 2 (F8): the LM head streams the
// FP8 copy (lmhead8, lm_scale) instead of the bf16 tiles; bit 3 (K8): the KV
// cache holds e4m3 codes with a power-of-two scale per row (kscale, vscale).
// The host picks the instantiation per launch; the plain one carries none
// (fewer live scalar values).
template <class S, int MODE>
__global__ __launch_bounds__(NT) void decode_kernel(Params p) {
  constexpr bool LC = (MODE & 1) != 0, DBG = (MODE & 2) != 0, F8 = (MODE & 4) != 0, K8 = (MODE & 8) != 0;
  __shared__ Smem<S> sm;
  if (threadIdx.x == 0) wg_abort = 0;
  for (int i = threadIdx.x; i < 16 * S::D; i += NT) (&sm.qb[0][0])[i] = 0;  // unused columns stay 0
  for (int i = threadIdx.x; i < NW * 16 * 32 * KVB; i += NT) (&sm.pb[0][0][0])[i] = 0;
  __syncthreads();
  const int G = gridDim.x, wg = blockIdx.x, tid = threadIdx.x;
  const int w = tid / kWave, l = tid % kWave;
  const int L = p.n_layers;
  const unsigned per_token = (unsigned)(PHASES_PER_LAYER * L + 1);
  // Phase -> workgroup offsets spread the per-layer byte load across CUs:
  // with 256 CUs, down (88 KiB) on 0..63, QKV (32 KiB) on 64..191, gate/up
  // (64 KiB) on 64..239, O (32 KiB) on 192..255, attention from 0 upwards.
  const int off_qkv = G / 4, off_gu = G / 4, off_o = (3 * G) / 4, off_down = 0, off_att = 0;
  const int it_qkv = first_item(wg, off_qkv, G), it_o = first_item(wg, off_o, G);
  const int it_gu = first_item(wg, off_gu, G), it_dn = first_item(wg, off_down, G);
  const int it_att = first_item(wg, off_att, G);

  Blk<S::KC_H> rq;      // QKV block
  KV<S, K8> rkv;        // attention K/V sub-chunk
  Blk<S::KC_Q> ro;      // O block
  Blk<S::KC_H> rg, ru;  // gate / up blocks
  Blk<S::KC_F> rd;      // down block
  NormIn<S> gq, gf;     // attn_norm / ffn_norm gains of this thread's elements

  int tok = p.first_token;
  for (int t = 0; t < p.n_tokens; ++t) {
    if constexpr (DBG) trace_begin(p, t);
    const int pos = p.pos0 + t;
    const unsigned tb = p.tag_base + (unsigned)t * per_token;  // tag of this token's first phase
    if (it_qkv < S::RB_QKV) {
      blk_load(rq, p.layers + S::OFF_QKV + (long long)it_qkv * S::KT_H * 64);
      gains_load(gq, p.norms + S::NORM_ATTN);
    } else {
      blk_forget(rq);
      gains_forget(gq);
    }
    if (t > 0) {
      if (!token_from_slots(p, p.amax + ((t - 1) & 1) * G, tag14(tb - 1u), sm.amax, &tok)) return;
      if (wg == 0 && tid == 0) p.out_tokens[t - 1] = tok;
    }
    if (tid < S::D / 2) {
      float sn, cs;
      sincosf((float)pos * p.inv_freq[tid], &sn, &cs);
      sm.rc[tid] = cs;
      sm.rs[tid] = sn;
    }
    if (DBG && p.dbg_layers && wg == 0)
      for (int i = tid; i < S::H; i += NT) p.dbg_layers[i] = packed_elem<S::KT_H>(p.lmhead, tok, i);
    __syncthreads();
    // attention split: nsplit <= nsplit_max items per kv head, none empty;
    // this token's item and the next token's (whose layer-0 K/V this
    // workgroup prefetches during the last layer)
    const int n = pos + 1;
    const Item cur = att_item(it_att, n, S::NKV, p.chunk_min, p.nsplit_max);
    const Item nxt = att_item(it_att, n + 1, S::NKV, p.chunk_min, p.nsplit_max);
    const int nsplit = cur.nsplit;
    const bool has_att = cur.on;
    // some phase of every layer (the LM head's x poll relies on it, wait_last_qkv)
    const bool layer_role =
        has_att || it_qkv < S::RB_QKV || it_o < S::RB_H || it_gu < S::RB_F || it_dn < S::RB_H;
    const int kv_at = !LC || nsplit <= p.merge_min
                          ? 2
                          : (it_gu < S::RB_F ? 4 : (it_dn < S::RB_H ? 5 : (it_o < S::RB_H ? 3 : 2)));
    if (t == 0) {
      if (has_att) {
        kv_load<S>(rkv, p, 0, cur.g, cur.t0 / 32, (cur.t1 - cur.t0 + 31) / 32, wave_id());
        gain_load_qk<S>(rkv, p, 0);
      } else {
        kv_forget<S>(rkv);
      }
    }

    for (int layer = 0; layer < L; ++layer) {
      const int tid = ltid();
      const u32x4* wl = p.layers + (long long)layer * S::U_LAYER;
      const uint16_t* nrm = p.norms + (long long)layer * S::NORM_STRIDE;
      const unsigned tg = tb + (unsigned)(PHASES_PER_LAYER * layer);  // tag of P1 of this layer
      const unsigned tg_x = tg - 1u;  // tag of the x rows this layer starts from (layer > 0)
      const int slot = PHASES_PER_LAYER * layer;
      // Each phase issues the next phase's prefetch before its own wait:
      // loads complete in order, so the wait absorbs the prefetch, and no
      // product ever waits behind loads issued after its own block.
      // ---------------- P1: QKV
      if (it_qkv < S::RB_QKV) {
        float r;
        if (layer > 0) {
          if (!fetch_norm<S>(p, p.x, tg_x, gq, sm.vec_q, sm.ssw[0], &r)) return;
        } else {
          embed_norm<S>(p, tok, gq, sm.vec_q, sm.ssw[0], &r);
        }
        if constexpr (DBG) trace_mark(p, t, slot + 0, 0);
        {  // the prefetched block
          blk_mma(rq, sm.vec_q, sm.red[RED_Q]);
          store_block(sm.red[RED_Q], p.qkv + it_qkv * 16, r, tg);
          evt(p, t, layer, EV_QKV_STORED);
        }
        for (int rb = it_qkv + G; rb < S::RB_QKV; rb += G) {  // grids smaller than the block count
          blk_load(rq, wl + S::OFF_QKV + (long long)rb * S::KT_H * 64);
          __syncthreads();  // the previous block's shares are summed
          blk_mma(rq, sm.vec_q, sm.red[RED_Q]);
          store_block(sm.red[RED_Q], p.qkv + rb * 16, r, tg);
        }
        if constexpr (DBG) trace_mark(p, t, slot + 0, 1);
      }
      // ---------------- P2: attention partials (prefetch: O)
      if (it_o < S::RB_H) blk_load(ro, wl + S::OFF_O + (long long)it_o * S::KT_Q * 64);
      else blk_forget(ro);
      if (has_att) {
        if (!attention_compute<S, MODE>(p, sm, rkv, layer, pos, cur.g, cur.s, nsplit, cur.t0, cur.t1, tg, t)) return;
        evt(p, t, layer, EV_ATT_STORED);
        if constexpr (DBG) trace_mark(p, t, slot + 1, 1);
      }
      // K/V of this workgroup's next item (next layer, or the next token's
      // layer 0), a whole layer ahead.  Loads complete in order, so a poll
      // issued after the prefetch waits for it: with few splits the prefetch
      // is small and goes right after attention; with many (long contexts,
      // every workgroup prefetching) it goes after this workgroup's last
      // item of the layer (kv_at: 2 attention, 3 O, 4 gate/up, 5 down).
      auto prefetch_kv = [&]() {
        const bool last = layer + 1 == L;
        const Item ni = last ? nxt : cur;
        if (ni.on && (!last || t + 1 < p.n_tokens)) {
          kv_load<S>(rkv, p, last ? 0 : layer + 1, ni.g, ni.t0 / 32, (ni.t1 - ni.t0 + 31) / 32, wave_id());
          gain_load_qk<S>(rkv, p, last ? 0 : layer + 1);
        } else {
          kv_forget<S>(rkv);
        }
      };
      if constexpr (LC) {
        if (kv_at != 2) kv_forget<S>(rkv);
      }
      if (kv_at == 2) prefetch_kv();
      // ---------------- P3: O projection + residual (prefetch: gate/up + ffn gains)
      if (it_gu < S::RB_F) {
        const u32x4* gp = wl + S::OFF_GU + (long long)(2 * it_gu) * S::KT_H * 64;
        blk_load(rg, gp);
        blk_load(ru, gp + S::KT_H * 64);
        gains_load(gf, nrm + S::NORM_FFN);
      } else {
        blk_forget(rg);
        blk_forget(ru);
        gains_forget(gf);
      }
      if (it_o < S::RB_H) {
        // a long context's splits arrive merged (one row after the splits)
        const bool merged = LC && nsplit > p.merge_min;
        if (!fetch_attn<S>(p, merged ? p.part + (long long)p.nsplit_max * S::NKV * part_words<S>() : p.part,
                           merged ? 1 : nsplit, tag4(tg + 1u), p.x, layer > 0 ? it_o : -1, -1, tag4(tg_x), sm.vec_o,
                           sm.xres_o))
          return;
        if constexpr (DBG) trace_mark(p, t, slot + 2, 0);
        evt(p, t, layer, EV_O_READY);
        blk_mma(ro, sm.vec_o, sm.red[RED_O0]);
        __syncthreads();
        if (wave_id() == PUB_WAVE) o_rows<S>(p, sm.red[RED_O0], sm.xres_o, it_o, layer, tok, tg + 2u);
        evt(p, t, layer, EV_O_STORED);
        if constexpr (DBG) trace_mark(p, t, slot + 2, 1);
      }
      for (int rb = it_o + G; rb < S::RB_H; rb += G) {  // grids smaller than the block count
        blk_load(ro, wl + S::OFF_O + (long long)rb * S::KT_Q * 64);
        if (layer > 0 && !fetch_xrows(p, p.x, rb, tag4(tg_x), sm.xres_o)) return;
        __syncthreads();  // the previous block's shares are summed
        blk_mma(ro, sm.vec_o, sm.red[RED_O0]);
        __syncthreads();
        if (wave_id() == PUB_WAVE) o_rows<S>(p, sm.red[RED_O0], sm.xres_o, rb, layer, tok, tg + 2u);
      }
      if (kv_at == 3) prefetch_kv();
      // ---------------- P4: gate/up + SiLU (prefetch: down)
      if (it_dn < S::RB_H) blk_load(rd, wl + S::OFF_DOWN + (long long)it_dn * S::KT_F * 64);
      else blk_forget(rd);
      if (it_gu < S::RB_F) {
        float r;
        if (!fetch_norm<S>(p, p.x, tg + 2u, gf, sm.vec_g, sm.ssw[1], &r)) return;
        if constexpr (DBG) trace_mark(p, t, slot + 3, 0);
        {  // the prefetched block pair
          blk_mma2(rg, ru, sm.vec_g, sm.red[RED_G], sm.red[RED_U]);
          store_block_gu(sm.red[RED_G], sm.red[RED_U], p.act + it_gu * 8, r, tag4(tg + 3u));
          evt(p, t, layer, EV_GU_STORED);
        }
        for (int pr = it_gu + G; pr < S::RB_F; pr += G) {  // grids smaller than the block count
          const u32x4* gp = wl + S::OFF_GU + (long long)(2 * pr) * S::KT_H * 64;
          blk_load(rg, gp);
          blk_load(ru, gp + S::KT_H * 64);
          __syncthreads();  // the previous pair's shares are summed
          blk_mma2(rg, ru, sm.vec_g, sm.red[RED_G], sm.red[RED_U]);
          store_block_gu(sm.red[RED_G], sm.red[RED_U], p.act + pr * 8, r, tag4(tg + 3u));
        }
        if constexpr (DBG) trace_mark(p, t, slot + 3, 1);
      }
      // ---------------- P5: down projection + residual (prefetch: next QKV + attn gains)
      if (layer + 1 < L && it_qkv < S::RB_QKV) {
        blk_load(rq, wl + S::U_LAYER + S::OFF_QKV + (long long)it_qkv * S::KT_H * 64);
        gains_load(gq, nrm + S::NORM_STRIDE + S::NORM_ATTN);
      } else {
        blk_forget(rq);
        gains_forget(gq);
      }
      if (kv_at == 4) prefetch_kv();
      if (it_dn < S::RB_H) {
        if (!fetch_pk<S::F / 2>(p, p.act, tag4(tg + 3u), p.x, it_dn, tag4(tg + 2u), sm.vec_d, sm.xres_d)) return;
        if constexpr (DBG) trace_mark(p, t, slot + 4, 0);
        evt(p, t, layer, EV_DN_READY);
        blk_mma(rd, sm.vec_d, sm.red[RED_D]);
        __syncthreads();
        if (wave_id() == PUB_WAVE) down_rows<S>(p, sm, it_dn, DBG ? p.dbg_layers : nullptr, layer, tg + 4u);
        evt(p, t, layer, EV_DN_STORED);
        if constexpr (DBG) trace_mark(p, t, slot + 4, 1);
      }
      for (int rb = it_dn + G; rb < S::RB_H; rb += G) {  // grids smaller than the block count
        blk_load(rd, wl + S::OFF_DOWN + (long long)rb * S::KT_F * 64);
        if (!fetch_xrows(p, p.x, rb, tag4(tg + 2u), sm.xres_d)) return;
        __syncthreads();  // the previous block's shares are summed
        blk_mma(rd, sm.vec_d, sm.red[RED_D]);
        __syncthreads();
        if (wave_id() == PUB_WAVE) down_rows<S>(p, sm, rb, DBG ? p.dbg_layers : nullptr, layer, tg + 4u);
      }
      if (kv_at == 5) prefetch_kv();
    }
    // ---------------- final norm + tied LM head + per-workgroup argmax
    // (reference sampling.cuh:32-117)
    {
      const int tid = ltid(), w = tid / kWave, l = tid % kWave;
      const unsigned tl = tb + (unsigned)(PHASES_PER_LAYER * L);
      NormIn<S> gfin;
      gains_load(gfin, p.final_norm);
      float rn;
      if (!layer_role && !wait_last_qkv(p, tl)) return;
      if (!fetch_norm<S, false>(p, p.x, tl - 1u, gfin, sm.vec_l, sm.ssw[2], &rn)) return;
      if constexpr (DBG) trace_mark(p, t, PHASES_PER_LAYER * L, 0);
      const long long nb = p.vocab / 16;
      const long long b0 = (long long)wg * nb / G, b1 = (long long)(wg + 1) * nb / G;
      u64 best = 0ull;
      const int wv_ = wave_id();
      for (long long b = b0 + wv_; b < b1; b += NW) {
        // re-derived per block so the LDS reads of the hidden vector are not
        // hoisted out of the block loop (256 floats per lane would not fit)
        const unsigned lo = lane_id();
        // a 16-row block is KT 1 KiB units of 64 lanes x 16 bytes: lane
        // (q, r) holds row r, columns q*E .. q*E+E-1 of each 4E-column unit
        // (E = 8 bf16 or 16 FP8 values)
        constexpr int E = F8 ? 16 : 8, KT = S::H / (4 * E);
        const float* hv = sm.vec_l + (lo >> 4) * E;
        const auto rs = make_rsrc((F8 ? p.lmhead8 : p.lmhead) + b * KT * 64);  // wave-uniform block base
        float acc = 0.f;
        constexpr int U = 16;
        // the first MK_LMHEAD_KEEP_PCT % of each workgroup's blocks are loaded
        // with the plain policy (kept by the memory-side cache across tokens),
        // the rest non-temporally
        const bool keep = (b - b0) * 100 < (b1 - b0) * MK_LMHEAD_KEEP_PCT;
#pragma unroll 1
        for (int k0 = 0; k0 < KT; k0 += U) {
          u32x4 wv[U];
          if (keep) {
#pragma unroll
            for (int u = 0; u < U; ++u)
              if (k0 + u < KT) wv[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, lo * 16u, (unsigned)(k0 + u) * 1024u, MK_LMHEAD_AUX);
          } else {
#pragma unroll
            for (int u = 0; u < U; ++u)
              if (k0 + u < KT) wv[u] = buf_ld_nt(rs, lo * 16u, (unsigned)(k0 + u) * 1024u);
          }
#pragma unroll
          for (int u = 0; u < U; ++u) {
            if (k0 + u < KT) {
              if constexpr (F8)
                acc = dot16_fp8(wv[u], hv + (k0 + u) * 64, acc);
              else
                acc = dot8(wv[u], hv + (k0 + u) * 32, acc);
            }
          }
        }
        acc = stride_sum<16>(acc) * rn;
        if constexpr (F8) acc *= p.lm_scale[b * 16 + (l & 15)];
        if (l < 16) {
          const unsigned idx = (unsigned)(b * 16 + l);
          if (DBG && p.dbg_logits) p.dbg_logits[idx] = acc;
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
      if constexpr (DBG) trace_mark(p, t, PHASES_PER_LAYER * L, 1);
      __syncthreads();
    }
    if constexpr (DBG) trace_end(p, t);
  }
  if (wg == 0) {  // the last token's id
    const int t = p.n_tokens;
    int last = 0;
    if (!token_from_slots(p, p.amax + ((t - 1) & 1) * G, tag14(p.tag_base + (unsigned)t * per_token - 1u),
                          sm.amax, &last))
      return;
    if (tid == 0) p.out_tokens[t - 1] = last;
  }
}

}  // namespace mk
