// Class-specialised persistent decode kernel for gfx950.
//
// Same phases, tags, hand-off words and arithmetic as decode_kernel
// (mk_kernel.h; reference phase order /root/reference/src/megakernel.cu:132-332),
// but every workgroup has a fixed ROLE CLASS for the whole launch -- the set
// of phases it computes -- and runs a layer loop that contains only those
// phases.  Two things follow:
//
// * Prefetch never sits in front of a poll.  Loads return in order on CDNA and
//   a CU that streams HBM slows its own hand-off loads about 2.5x (other CUs
//   streaming do not), so each workgroup issues the next weights of a role
//   right after it has computed and published that role, and the next wait of
//   the workgroup comes at least one phase later:
//     A    attention (P2)            next K/V after attention (the default
//                                    where the O blocks fit elsewhere)
//     ATT  attention (P2) + O (P3)   next K/V and next O after O
//     QG   QKV (P1) + gate/up (P4)   gate/up after QKV, next QKV after gate/up
//     DG   gate/up (P4) + down (P5)  next gate/up and next down after down
//     DO   O (P3) + down (P5)        next O and next down after down
//     O    one or two O blocks (P3)  next O after O
//   plus single-role classes (Q, G, D) for shapes whose block counts leave a
//   role without a partner, and IDLE workgroups that only join the LM head.
// * Registers: a class keeps only its own prefetch sets live across the
//   layer, and the kernel's register count is the maximum over the classes,
//   not the sum.
//
// XCD-aware placement: workgroup w runs on XCD w % 8, so the QKV blocks of kv
// head g and the attention items of head g sit on the same XCD and the
// qkv -> attention hand-off stays inside one L2.
//
// The host builds the role table (one row per workgroup) for the number of
// attention items of a launch; launches with more items than attention
// workgroups can hold, or with the long-context merge, use decode_kernel.
#pragma once
#include "mk_kernel.h"

namespace mk {

// Gains of the layer GEMV inputs in the per-wave staging layout (fetch_norm_nb).
template <class S>
using GIn = NormInW<S>;

enum RoleClass : int { CLS_IDLE = 0, CLS_ATT, CLS_QG, CLS_DG, CLS_DO, CLS_O, CLS_Q, CLS_G, CLS_D, CLS_A, CLS_N };
// Role row: class, then item indices (-1: none).  att: kv head att % NKV,
// split att / NKV.
enum RoleField : int { RF_CLS = 0, RF_Q, RF_G, RF_O0, RF_O1, RF_D, RF_ATT, RF_PAD, ROLE_INTS };

// Attention item (kv head g, split s) for n cached positions.
__device__ __forceinline__ Item att_item_gs(int g, int s, int n, int chunk_min, int nsplit_max) {
  Item r;
  r.nsplit = split_count(n, chunk_min, nsplit_max);
  r.on = s < r.nsplit;
  r.g = g;
  r.s = r.on ? s : 0;
  split_range(n, r.nsplit, r.s, &r.t0, &r.t1);
  return r;
}

// Start of token t: the previous token's id from the argmax slots (only the
// classes that read the embedding need it, and workgroup 0, which records
// it), this token's RoPE table (attention only), the embedding row of the
// validation output.
template <class S, int MODE>
__device__ __forceinline__ bool cls_token_start(const Params& p, Smem<S>& sm, int t, unsigned tb, bool need_tok,
                                                bool rope, int* tok) {
  const int G = gridDim.x, wg = blockIdx.x, tid = ltid();
  if (t > 0 && (need_tok || wg == 0)) {
    if (!token_from_slots(p, p.amax + ((t - 1) & 1) * G, tag14(tb - 1u), sm.amax, tok)) return false;
    if (wg == 0 && tid == 0) p.out_tokens[t - 1] = *tok;
  }
  if (rope && tid < S::D / 2) {
    float sn, cs;
    sincosf((float)(p.pos0 + t) * p.inv_freq[tid], &sn, &cs);
    sm.rc[tid] = cs;
    sm.rs[tid] = sn;
  }
  if (((MODE & 2) != 0) && p.dbg_layers && wg == 0)
    for (int i = tid; i < S::H; i += NT) p.dbg_layers[i] = packed_elem<S::KT_H>(p.lmhead, *tok, i);
  __syncthreads();
  return true;
}

// Final RMSNorm + this workgroup's share of the tied LM head + its argmax word
// (reference sampling.cuh:32-117), as in decode_kernel.  after_poll() issues
// the workgroup's prefetch for the next token's layer 0 once the LM head's
// rows have been scored and its argmax word published: issued before the
// LM head's wait it would delay that wait, issued before the scoring it would
// delay this workgroup's share of the LM-head stream.
// LM head warm start: a workgroup's first LM-head weights do not depend on
// the final x, so each wave loads the first LM_U units of its first block
// into registers right after the workgroup's last-layer role (the registers
// of the next layer's weights are free then); the LM head's first step then
// starts from registers instead of a cold HBM round trip.
constexpr int LM_U = 16;  // 1 KiB units in flight per wave in the LM-head loop
struct LmWarm {
  u32x4 w[LM_U];
};
template <class S, int MODE>
__device__ __forceinline__ void lm_warm_load(const Params& p, LmWarm& lw) {
  constexpr bool F8 = (MODE & 4) != 0;
  constexpr int E = F8 ? 16 : 8, KT = S::H / (4 * E);
  const int G = gridDim.x, wg = blockIdx.x;
  const long long nb = p.vocab / 16;
  const long long b0 = (long long)wg * nb / G, b1 = (long long)(wg + 1) * nb / G, b = b0 + wave_id();
  if (b >= b1) return;
  const auto rs = make_rsrc((F8 ? p.lmhead8 : p.lmhead) + b * KT * 64);
  const unsigned lo = lane_id();
#pragma unroll
  for (int u = 0; u < LM_U; ++u)
    if (u < KT) lw.w[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, lo * 16u, (unsigned)u * 1024u, MK_LMHEAD_AUX);
}

// ||h|| of the LM head's input (sm.vec_l, x * final_norm gain, in LDS).
template <class S>
__device__ __forceinline__ float lm_hnorm(Smem<S>& sm) {
  const int tid = ltid();
  float ss = 0.f;
  for (int i = tid; i < S::H; i += NT) ss = fmaf(sm.vec_l[i], sm.vec_l[i], ss);
  ss = wave_sum(ss);
  if (lane_id() == 0) sm.lmw[wave_id()] = ss;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < NW; ++i) t += sm.lmw[i];
  __syncthreads();
  return sqrtf(t) * (1.0f + 0x1p-12f);  // rounded up: part of the bound
}

// Screening threshold: the largest lower bound over all workgroups.  Each
// workgroup publishes its own in the second half of p.amax as one word: the
// ordered value in the high half and the LM-head phase's full 32-bit tag in
// the low half (only screened launches write these words, so a short tag
// could alias after a run of other launches; a full tag never repeats), and
// reads every workgroup's.
template <class S>
__device__ __forceinline__ bool lm_threshold(const Params& p, Smem<S>& sm, int t, unsigned tl, float lowmax,
                                             float* thr) {
  const int G = gridDim.x, wg = blockIdx.x, tid = ltid(), w = wave_id(), l = (int)lane_id();
  u64* slots = p.amax + 2 * G + (t & 1) * G;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) lowmax = fmaxf(lowmax, __shfl_xor(lowmax, m));
  if (l == 0) sm.lmw[w] = lowmax;
  __syncthreads();
  if (tid == 0) {
    float v = sm.lmw[0];
    for (int i = 1; i < NW; ++i) v = fmaxf(v, sm.lmw[i]);
    ll_put(slots + wg, ((u64)f32_order_key(v) << 32) | (u64)tl);
  }
  int failed = 0;
  u64 best = 0ull;
  for (int i = tid; i < G && !failed; i += NT) {
    Spin sp;
    u64 v;
    while ((unsigned)(v = ll_get(slots + i)) != tl)
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
  if (l == 0) sm.amax[w] = best;
  __syncthreads();
  best = sm.amax[0];
  for (int i = 1; i < NW; ++i) best = sm.amax[i] > best ? sm.amax[i] : best;
  __syncthreads();
  const uint32_t k = (uint32_t)(best >> 32);
  *thr = __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);  // inverse of f32_order_key
  return true;
}

template <class S, int MODE, class AfterPoll>
__device__ __forceinline__ bool cls_lm_head(const Params& p, Smem<S>& sm, int t, unsigned tb, AfterPoll after_poll,
                                            const LmWarm& lw, bool idle = false) {
  constexpr bool DBG = (MODE & 2) != 0, F8 = (MODE & 4) != 0;
  const int G = gridDim.x, wg = blockIdx.x;
  const int tid = ltid(), w = tid / kWave, l = tid % kWave;
  const unsigned tl = tb + (unsigned)(PHASES_PER_LAYER * p.n_layers);
  NormIn<S> gfin;
  gains_load(gfin, p.final_norm);
  float rn;
  if (idle && !wait_last_qkv(p, tl)) return false;  // no role in the last layer
  if (!fetch_norm<S, false>(p, p.x, tl - 1u, gfin, sm.vec_l, sm.ssw[2], &rn)) return false;
  if constexpr (DBG) trace_mark(p, t, PHASES_PER_LAYER * p.n_layers, 0);
  const long long nb = p.vocab / 16;
  const long long b0 = (long long)wg * nb / G, b1 = (long long)(wg + 1) * nb / G;
  u64 best = 0ull;
  const int wv_ = wave_id();
  // screened (FP8 copy + p.lm_err): the FP8 pass keeps, per row, the upper
  // bound u = l8 + e of the bf16 logit (e = rn ||h|| B_r) and the largest
  // lower bound l8 - e; the rows that can still hold the argmax are scored
  // again from the bf16 tiles below
  const bool screen = F8 && p.lm_err != nullptr;
  float eh = 0.f, lowmax = -INFINITY;
  if (screen) eh = rn * lm_hnorm<S>(sm) * (1.0f + 0x1p-12f);
  for (long long b = b0 + wv_; b < b1; b += NW) {
    const unsigned lo = lane_id();
    constexpr int E = F8 ? 16 : 8, KT = S::H / (4 * E);
    const float* hv = sm.vec_l + (lo >> 4) * E;
    const auto rs = make_rsrc((F8 ? p.lmhead8 : p.lmhead) + b * KT * 64);
    float acc = 0.f;
    constexpr int U = LM_U;
    const bool keep = (b - b0) * 100 < (b1 - b0) * MK_LMHEAD_KEEP_PCT;
#pragma unroll 1
    for (int k0 = 0; k0 < KT; k0 += U) {
      u32x4 wv[U];
      if (b == b0 + wv_ && k0 == 0) {  // loaded by lm_warm_load
#pragma unroll
        for (int u = 0; u < U; ++u) wv[u] = lw.w[u];
      } else if (keep) {
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (k0 + u < KT)
            wv[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, lo * 16u, (unsigned)(k0 + u) * 1024u, MK_LMHEAD_AUX);
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
      if (screen) {
        const float e = eh * p.lm_err[idx];
        sm.lmu[idx - b0 * 16] = acc + e;
        lowmax = fmaxf(lowmax, acc - e);
      } else {
        if (DBG && p.dbg_logits) p.dbg_logits[idx] = acc;
        const u64 key = ((u64)f32_order_key(acc) << 32) | ((u64)(IDX_MAX - idx) << 14);
        best = key > best ? key : best;
      }
    }
  }
  if (screen) {
    float thr;
    if (!lm_threshold<S>(p, sm, t, tl, lowmax, &thr)) return false;
    // rescoring: every row whose bound reaches the threshold is scored from
    // the bf16 tiles with the bf16 head's arithmetic -- lane (q, s) of a wave
    // takes column group q of its row s from every unit (the lane that holds
    // them in the row's block), the same dot8 chain over the same units and
    // the same lane sum as the bf16 head's block scoring, so the logit is
    // bit-identical; every row that can be the argmax is among them (its bf16
    // logit >= thr > every skipped row's upper bound), so the argmax equals
    // the bf16 head's.  Sixteen rows per wave at a time.
    if (tid == 0) sm.lmn = 0;
    __syncthreads();
    for (long long b = b0 + wv_; b < b1; b += NW)
      if (l < 16 && sm.lmu[b * 16 + l - b0 * 16] >= thr) sm.lmc[atomicAdd(&sm.lmn, 1)] = (int)(b * 16 + l);
    __syncthreads();
    const int nc = sm.lmn;
    const unsigned lo = lane_id();
    const float* hv = sm.vec_l + (lo >> 4) * 8;
    constexpr int KTB = S::KT_H;
    for (int c0 = wv_ * 16; c0 < nc; c0 += NW * 16) {
      const int j = c0 + (int)(lo & 15u);
      const int row = sm.lmc[j < nc ? j : c0];
      const u32x4* base = p.lmhead + (long long)(row >> 4) * KTB * 64 + (lo >> 4) * 16 + (row & 15);
      float acc = 0.f;
#pragma unroll 1
      for (int k0 = 0; k0 < KTB; k0 += LM_U) {
        u32x4 wv[LM_U];
#pragma unroll
        for (int u = 0; u < LM_U; ++u)
          if (k0 + u < KTB) wv[u] = __builtin_nontemporal_load(base + (k0 + u) * 64);
#pragma unroll
        for (int u = 0; u < LM_U; ++u)
          if (k0 + u < KTB) acc = dot8(wv[u], hv + (k0 + u) * 32, acc);
      }
      acc = stride_sum<16>(acc) * rn;
      if (lo < 16u && j < nc) {
        const u64 key = ((u64)f32_order_key(acc) << 32) | ((u64)(IDX_MAX - (unsigned)row) << 14);
        best = key > best ? key : best;
      }
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
    u64 bb = 0ull;
    for (int i = 0; i < NW; ++i) bb = sm.amax[i] > bb ? sm.amax[i] : bb;
    ll_put(p.amax + (t & 1) * G + wg, bb | (u64)tag14(tl));
  }
  if constexpr (DBG) trace_mark(p, t, PHASES_PER_LAYER * p.n_layers, 1);
  __syncthreads();
  if (t + 1 < p.n_tokens) after_poll();
  return true;
}

// ----------------------------------------------------------- phase bodies
// P1: QKV block q of layer `layer` from the prefetched rq (inputs: x of the
// previous layer, or the embedding row at layer 0).
template <class S, int MODE, class BH>
__device__ __forceinline__ bool cls_qkv(const Params& p, Smem<S>& sm, const BH& rq, const GIn<S>& gq,
                                        int t, int layer, int q, int tok, unsigned tg) {
  if (layer > 0) {
    fetch_norm_nb<S>(p, p.x, tg - 1u, gq, sm.vec_q, sm.ssw[0], ev_at(t, layer, PS_QKV));
  } else {
    embed_norm_nb<S>(p, tok, gq, sm.vec_q, sm.ssw[0]);
  }
  if constexpr ((MODE & 2) != 0) trace_mark(p, t, PHASES_PER_LAYER * layer + 0, 0);
  blk_mma(rq, sm.vec_q, sm.red[RED_Q]);
  const bool ok = store_block<true>(sm.red[RED_Q], p.qkv + q * 16, row_scale(rq), tg, sm.ssw[0], 1.0f / S::H);
  if constexpr ((MODE & 2) != 0) trace_mark(p, t, PHASES_PER_LAYER * layer + 0, 1, PUB_WAVE);
  return ok;
}

// P4: gate/up pair g + SiLU from the prefetched rg / ru (input: x after O).
template <class S, int MODE, class BH>
__device__ __forceinline__ bool cls_gu(const Params& p, Smem<S>& sm, const BH& rg, const BH& ru,
                                       const GIn<S>& gf, int t, int layer, int g, unsigned tg) {
  fetch_norm_nb<S>(p, p.x, tg + 2u, gf, sm.vec_g, sm.ssw[1], ev_at(t, layer, PS_GU));
  if constexpr ((MODE & 2) != 0) trace_mark(p, t, PHASES_PER_LAYER * layer + 3, 0);
  blk_mma2(rg, ru, sm.vec_g, sm.red[RED_G], sm.red[RED_U]);
  const bool ok = store_block_gu<true>(sm.red[RED_G], sm.red[RED_U], p.act + g * 8, 0.f, tag4(tg + 3u), row_scale(rg),
                                       row_scale(ru), sm.ssw[1], 1.0f / S::H);
  if constexpr ((MODE & 2) != 0) trace_mark(p, t, PHASES_PER_LAYER * layer + 3, 1, PUB_WAVE);
  return ok;
}

// P5: down block d + residual from the prefetched rd (inputs: act and this
// block's rows of x after O).
template <class S, int MODE, class BF>
__device__ __forceinline__ bool cls_down(const Params& p, Smem<S>& sm, const BF& rd, int t, int layer, int d,
                                         unsigned tg) {
  if (!fetch_pk<S::F / 2>(p, p.act, tag4(tg + 3u), p.x, d, tag4(tg + 2u), sm.vec_d, sm.xres_d,
                          ev_at(t, layer, PS_DN)))
    return false;
  if constexpr ((MODE & 2) != 0) trace_mark(p, t, PHASES_PER_LAYER * layer + 4, 0);
  blk_mma(rd, sm.vec_d, sm.red[RED_D]);
  __syncthreads();
  if (wave_id() == PUB_WAVE)
    down_rows<S>(p, sm, d, (MODE & 2) != 0 ? p.dbg_layers : nullptr, layer, tg + 4u, row_scale(rd));
  if constexpr ((MODE & 2) != 0) trace_mark(p, t, PHASES_PER_LAYER * layer + 4, 1, PUB_WAVE);
  return true;
}

// P3: O blocks o0 (and o1 >= 0) + residual (inputs: every kv head's split
// partials, merged here, and the blocks' rows of x, or the embedding row at
// layer 0).  (Merging a head's splits first in its split-0 workgroup, on the
// head's XCD, so that O reads one word per thread: O hand-off 2.06 -> 0.90 us
// but attention 1.72 -> 3.38 us, 2,808 vs 2,979 tok/s.)
template <class S, int MODE, class BQ>
__device__ __forceinline__ bool cls_o(const Params& p, Smem<S>& sm, const BQ& ro0, const BQ& ro1,
                                      int t, int layer, int o0, int o1, int nsplit, int tok, unsigned tg) {
  const unsigned tg_x = tg - 1u;
  fetch_attn_nb<S>(p, p.part, nsplit, tag4(tg + 1u), p.x, layer > 0 ? o0 : -1, o1, tag4(tg_x), sm.vec_o,
                   sm.xres_o, ev_at(t, layer, PS_O));
  if constexpr ((MODE & 2) != 0) trace_mark(p, t, PHASES_PER_LAYER * layer + 2, 0);
  if (o1 >= 0) blk_mma2(ro0, ro1, sm.vec_o, sm.red[RED_O0], sm.red[RED_O1]);
  else blk_mma(ro0, sm.vec_o, sm.red[RED_O0]);
  __syncthreads();
  // the abort flag is read with the block shares (one LDS round trip); rows
  // of an abandoned wait are not published
  const bool ok = !block_aborted();
  // wave PUB_WAVE: block o0, the wave before it: block o1
  const int w_ = wave_id();
  if (w_ == PUB_WAVE) o_rows<S>(p, sm.red[RED_O0], sm.xres_o, o0, layer, tok, tg + 2u, row_scale(ro0), ok);
  else if (w_ == PUB_WAVE - 1 && o1 >= 0)
    o_rows<S>(p, sm.red[RED_O1], sm.xres_o + 16, o1, layer, tok, tg + 2u, row_scale(ro1), ok);
  if constexpr ((MODE & 2) != 0) trace_mark(p, t, PHASES_PER_LAYER * layer + 2, 1, PUB_WAVE);
  return ok;
}

// Prefetch pacing.  A class's next weights are loaded while the workgroup is
// idle between its roles; issued as one burst, the bursts of a whole class
// (up to ~9 MB from 64-128 CUs at once) queue in the memory system in front of
// the cross-XCD hand-off loads of the phase that runs meanwhile.  So each
// wave issues one 1 KiB load per step and sleeps between steps, spreading a
// class's bytes over most of its idle window.  Spacing per step (units of
// s_sleep 1, 64 clocks) by class and window, scaled by p.pace_pct.  The
// spacings follow the layer period: they were set for an 11.7 us layer and
// taken to 70 % when the layer fell to ~10 us (3,127 -> 3,166 tok/s; 130 % of
// the old values lost 8 %, 0 % -- bursts -- 3 %).
enum PaceSlot : int { PACE_QG_GU = 0, PACE_QG_Q, PACE_DG, PACE_DO, PACE_O, PACE_ATT, PACE_N };
__device__ __forceinline__ int pace_units(const Params& p, int slot) {
  constexpr int base[PACE_N] = {9, 8, 8, 6, 13, 10};
  return base[slot] * p.pace_pct / 100;
}
__device__ __forceinline__ void pace_step(int units) {
  asm volatile("" ::: "memory");  // the loads before stay before, the loads after stay after
  for (int i = 0; i < units; ++i) __builtin_amdgcn_s_sleep(1);
  asm volatile("" ::: "memory");
}

template <int KC>
__device__ __forceinline__ void blk_load_paced(Blk<KC>& b, const u32x4* __restrict__ block, int units) {
  const int w = wave_id();
  const unsigned lb = lane_id() * 16u;
  const auto rs = make_rsrc(block);
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    b.w[kc] = buf_ld_nt(rs, lb, (unsigned)(w * KC + kc) * 1024u);
    if (units) pace_step(units);
  }
}

// FP8 variant: 512-byte tiles, 8 bytes per lane, and the row scale of the
// lane's epilogue row.
template <int KC>
__device__ __forceinline__ void blk_load_paced(Blk8<KC>& b, const u32x2* __restrict__ block,
                                               const float* __restrict__ scales16, int units) {
  const int w = wave_id();
  const unsigned lb = lane_id() * 8u;
  const auto rs = make_rsrc(block);
  b.s = scales16[lane_id() >> 2];
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    b.w[kc] = __builtin_amdgcn_raw_buffer_load_b64(rs, lb, (unsigned)(w * KC + kc) * 512u, 2);
    if (units) pace_step(units);
  }
}
// Block at unit offset u of the layer weights (the same offset in both
// formats), scale rows from srow (FP8).
template <int KC>
__device__ __forceinline__ void blk_load_at(Blk<KC>& b, const Params& p, long long u, long long srow, int units) {
  (void)srow;
  blk_load_paced(b, p.layers + u, units);
}
template <int KC>
__device__ __forceinline__ void blk_load_at(Blk8<KC>& b, const Params& p, long long u, long long srow, int units) {
  blk_load_paced(b, p.layers8 + u, p.lscale + srow, units);
}

// Weight block loads of one layer.
template <class S, class BH>
__device__ __forceinline__ void ld_qkv(BH& rq, GIn<S>& gq, const Params& p, int layer, int q, int units = 0) {
  gains_load_w(gq, p.norms + (long long)layer * S::NORM_STRIDE + S::NORM_ATTN);
  blk_load_at(rq, p, (long long)layer * S::U_LAYER + S::OFF_QKV + (long long)q * S::KT_H * 64,
              (long long)layer * S::SROWS_LAYER + S::SROW_QKV + q * 16, units);
}
template <class S, class BH>
__device__ __forceinline__ void ld_gu(BH& rg, BH& ru, GIn<S>& gf, const Params& p, int layer, int g,
                                      int units = 0) {
  const long long u = (long long)layer * S::U_LAYER + S::OFF_GU + (long long)(2 * g) * S::KT_H * 64;
  const long long sr = (long long)layer * S::SROWS_LAYER + S::SROW_GU + (2 * g) * 16;
  gains_load_w(gf, p.norms + (long long)layer * S::NORM_STRIDE + S::NORM_FFN);
  blk_load_at(rg, p, u, sr, units);
  blk_load_at(ru, p, u + S::KT_H * 64, sr + 16, units);
}
template <class S, class BQ>
__device__ __forceinline__ void ld_o(BQ& ro, const Params& p, int layer, int o, int units = 0) {
  blk_load_at(ro, p, (long long)layer * S::U_LAYER + S::OFF_O + (long long)o * S::KT_Q * 64,
              (long long)layer * S::SROWS_LAYER + S::SROW_O + o * 16, units);
}
template <class S, class BF>
__device__ __forceinline__ void ld_down(BF& rd, const Params& p, int layer, int d, int units = 0) {
  blk_load_at(rd, p, (long long)layer * S::U_LAYER + S::OFF_DOWN + (long long)d * S::KT_F * 64,
              (long long)layer * S::SROWS_LAYER + S::SROW_DOWN + d * 16, units);
}

// K / V of an attention item's first blocks (kv_load) with a pause after each
// of a wave's loads.
template <class S, bool K8>
__device__ __forceinline__ void kv_load_paced(KV<S, K8>& r, const Params& p, int layer, int g, int b0, int nb,
                                              int units) {
  if (!units) {
    kv_load<S>(r, p, layer, g, b0, nb, wave_id());
    return;
  }
  // one block of the wave's KVB per step (its K and V^T loads together)
  constexpr int D = S::D;
  const unsigned l = lane_id();
  const long long base = kt_base(p, layer, g, S::NKV, D);
  const int bi = wave_id();
#pragma unroll
  for (int q = 0; q < KVB; ++q) {
    const int bq = bi + q * NW;
    const int blk = b0 + (bq < nb ? bq : 0);
    if constexpr (K8) {
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
    pace_step(units);
  }
}

// -------------------------------------------------------------- classes
// The weights a class prefetches at the end of a layer are those of the next
// layer; the next token's layer-0 weights are prefetched inside the LM head,
// after its input has arrived.
__device__ __forceinline__ bool has_next(const Params& p, int t, int layer) { return layer + 1 < p.n_layers; }
__device__ __forceinline__ int next_layer(const Params& p, int layer) { return layer + 1; }

template <class S, int MODE, bool HAS_O = true>
__device__ __forceinline__ void run_att(const Params& p, Smem<S>& sm, const int* role) {
  constexpr bool W8 = (MODE & 16) != 0;  // FP8 layer weights
  constexpr bool K8 = (MODE & 8) != 0;
  const int a = role[RF_ATT], o0 = HAS_O ? role[RF_O0] : -1;
  const int g = a % S::NKV, s = a / S::NKV;
  KV<S, K8> rkv;
  BlkW<S::KC_Q, W8> ro;
  int tok = p.first_token;
  {
    const Item it = att_item_gs(g, s, p.pos0 + 1, p.chunk_min, p.nsplit_max);
    if (it.on) {
      kv_load<S>(rkv, p, 0, g, it.t0 / 32, (it.t1 - it.t0 + 31) / 32, wave_id());
      gain_load_qk<S>(rkv, p, 0);
    }
    if (o0 >= 0) ld_o<S>(ro, p, 0, o0);
  }
  const unsigned per_token = (unsigned)(PHASES_PER_LAYER * p.n_layers + 1);
  for (int t = 0; t < p.n_tokens; ++t) {
    if constexpr ((MODE & 2) != 0) trace_begin(p, t, role ? role[RF_CLS] : CLS_IDLE);
    const unsigned tb = p.tag_base + (unsigned)t * per_token;
    if (!cls_token_start<S, MODE>(p, sm, t, tb, o0 >= 0, true, &tok)) return;
    const int pos = p.pos0 + t;
    const Item cur = att_item_gs(g, s, pos + 1, p.chunk_min, p.nsplit_max);
    const Item nxt = att_item_gs(g, s, pos + 2, p.chunk_min, p.nsplit_max);
    for (int layer = 0; layer < p.n_layers; ++layer) {
      const unsigned tg = tb + (unsigned)(PHASES_PER_LAYER * layer);
      if (cur.on) {
        if (!attention_compute<S, MODE>(p, sm, rkv, layer, pos, g, cur.s, cur.nsplit, cur.t0, cur.t1, tg, t)) return;
        if constexpr ((MODE & 2) != 0) trace_mark(p, t, PHASES_PER_LAYER * layer + 1, 1);
      }
      // O right after attention (no load in between); the next layer's K/V
      // and O block after it
      if (o0 >= 0 && !cls_o<S, MODE>(p, sm, ro, ro, t, layer, o0, -1, cur.nsplit, tok, tg)) return;
      if (has_next(p, t, layer)) {
        if (o0 >= 0) ld_o<S>(ro, p, layer + 1, o0, pace_units(p, PACE_ATT));
        if (cur.on) {
          gain_load_qk<S>(rkv, p, layer + 1);
          kv_load_paced<S>(rkv, p, layer + 1, g, cur.t0 / 32, (cur.t1 - cur.t0 + 31) / 32, pace_units(p, PACE_ATT));
        }
      }
    }
    LmWarm lw;
    lm_warm_load<S, MODE>(p, lw);
    if (!cls_lm_head<S, MODE>(p, sm, t, tb, [&]() {
          if (o0 >= 0) ld_o<S>(ro, p, 0, o0);
          if (nxt.on) {
            kv_load<S>(rkv, p, 0, g, nxt.t0 / 32, (nxt.t1 - nxt.t0 + 31) / 32, wave_id());
            gain_load_qk<S>(rkv, p, 0);
          }
        }, lw))
      return;
    if constexpr ((MODE & 2) != 0) trace_end(p, t);
  }
}

// QKV + gate/up (Q: QKV only, G: gate/up only).
template <class S, int MODE, bool HAS_Q, bool HAS_G>
__device__ __forceinline__ void run_qg(const Params& p, Smem<S>& sm, const int* role) {
  constexpr bool W8 = (MODE & 16) != 0;  // FP8 layer weights
  const int q = role[RF_Q], gi = role[RF_G];
  BlkW<S::KC_H, W8> rq, rg, ru;
  GIn<S> gq, gf;
  if constexpr (HAS_Q) ld_qkv<S>(rq, gq, p, 0, q);
  if constexpr (!HAS_Q && HAS_G) ld_gu<S>(rg, ru, gf, p, 0, gi);
  int tok = p.first_token;
  const unsigned per_token = (unsigned)(PHASES_PER_LAYER * p.n_layers + 1);
  for (int t = 0; t < p.n_tokens; ++t) {
    if constexpr ((MODE & 2) != 0) trace_begin(p, t, role ? role[RF_CLS] : CLS_IDLE);
    const unsigned tb = p.tag_base + (unsigned)t * per_token;
    if (!cls_token_start<S, MODE>(p, sm, t, tb, HAS_Q, false, &tok)) return;
    for (int layer = 0; layer < p.n_layers; ++layer) {
      const unsigned tg = tb + (unsigned)(PHASES_PER_LAYER * layer);
      if constexpr (HAS_Q) {
        if (!cls_qkv<S, MODE>(p, sm, rq, gq, t, layer, q, tok, tg)) return;
        if constexpr (HAS_G) ld_gu<S>(rg, ru, gf, p, layer, gi, pace_units(p, PACE_QG_GU));
        else if (has_next(p, t, layer)) ld_qkv<S>(rq, gq, p, next_layer(p, layer), q, pace_units(p, PACE_QG_Q));
      }
      if constexpr (HAS_G) {
        if (!cls_gu<S, MODE>(p, sm, rg, ru, gf, t, layer, gi, tg)) return;
        if (has_next(p, t, layer)) {
          if constexpr (HAS_Q) ld_qkv<S>(rq, gq, p, next_layer(p, layer), q, pace_units(p, PACE_QG_Q));
          else ld_gu<S>(rg, ru, gf, p, next_layer(p, layer), gi, pace_units(p, PACE_QG_GU));
        }
      }
    }
    LmWarm lw;
    lm_warm_load<S, MODE>(p, lw);
    if (!cls_lm_head<S, MODE>(p, sm, t, tb, [&]() {
          if constexpr (HAS_Q) ld_qkv<S>(rq, gq, p, 0, q);
          else ld_gu<S>(rg, ru, gf, p, 0, gi);
        }, lw))
      return;
    if constexpr ((MODE & 2) != 0) trace_end(p, t);
  }
}

// down + a partner role: gate/up (DG), O (DO) or none (D).  The partner's
// next weights are loaded together with the next down block, after down.
template <class S, int MODE, int PARTNER>
__device__ __forceinline__ void run_down(const Params& p, Smem<S>& sm, const int* role) {
  constexpr bool W8 = (MODE & 16) != 0;  // FP8 layer weights
  const int d = role[RF_D], gi = role[RF_G], o0 = role[RF_O0];
  BlkW<S::KC_F, W8> rd;
  BlkW<S::KC_H, W8> rg, ru;
  GIn<S> gf;
  BlkW<S::KC_Q, W8> ro;
  if constexpr (PARTNER == CLS_DG) ld_gu<S>(rg, ru, gf, p, 0, gi);
  if constexpr (PARTNER == CLS_DO) ld_o<S>(ro, p, 0, o0);
  ld_down<S>(rd, p, 0, d);
  int tok = p.first_token;
  const unsigned per_token = (unsigned)(PHASES_PER_LAYER * p.n_layers + 1);
  for (int t = 0; t < p.n_tokens; ++t) {
    if constexpr ((MODE & 2) != 0) trace_begin(p, t, role ? role[RF_CLS] : CLS_IDLE);
    const unsigned tb = p.tag_base + (unsigned)t * per_token;
    if (!cls_token_start<S, MODE>(p, sm, t, tb, PARTNER == CLS_DO, false, &tok)) return;
    const int nsplit = split_count(p.pos0 + t + 1, p.chunk_min, p.nsplit_max);
    for (int layer = 0; layer < p.n_layers; ++layer) {
      const unsigned tg = tb + (unsigned)(PHASES_PER_LAYER * layer);
      if constexpr (PARTNER == CLS_DO) {
        if (!cls_o<S, MODE>(p, sm, ro, ro, t, layer, o0, -1, nsplit, tok, tg)) return;
      }
      if constexpr (PARTNER == CLS_DG) {
        if (!cls_gu<S, MODE>(p, sm, rg, ru, gf, t, layer, gi, tg)) return;
      }
      if (!cls_down<S, MODE>(p, sm, rd, t, layer, d, tg)) return;
      if (has_next(p, t, layer)) {
        const int nl = next_layer(p, layer);
        const int u = pace_units(p, PARTNER == CLS_DO ? PACE_DO : PACE_DG);
        if constexpr (PARTNER == CLS_DG) ld_gu<S>(rg, ru, gf, p, nl, gi, u);
        if constexpr (PARTNER == CLS_DO) ld_o<S>(ro, p, nl, o0, u);
        ld_down<S>(rd, p, nl, d, u);
      }
    }
    LmWarm lw;
    lm_warm_load<S, MODE>(p, lw);
    if (!cls_lm_head<S, MODE>(p, sm, t, tb, [&]() {
          if constexpr (PARTNER == CLS_DG) ld_gu<S>(rg, ru, gf, p, 0, gi);
          if constexpr (PARTNER == CLS_DO) ld_o<S>(ro, p, 0, o0);
          ld_down<S>(rd, p, 0, d);
        }, lw))
      return;
    if constexpr ((MODE & 2) != 0) trace_end(p, t);
  }
}

// One or two O blocks.
template <class S, int MODE>
__device__ __forceinline__ void run_o(const Params& p, Smem<S>& sm, const int* role) {
  constexpr bool W8 = (MODE & 16) != 0;  // FP8 layer weights
  const int o0 = role[RF_O0], o1 = role[RF_O1];
  BlkW<S::KC_Q, W8> ra, rb;
  ld_o<S>(ra, p, 0, o0);
  if (o1 >= 0) ld_o<S>(rb, p, 0, o1);
  int tok = p.first_token;
  const unsigned per_token = (unsigned)(PHASES_PER_LAYER * p.n_layers + 1);
  for (int t = 0; t < p.n_tokens; ++t) {
    if constexpr ((MODE & 2) != 0) trace_begin(p, t, role ? role[RF_CLS] : CLS_IDLE);
    const unsigned tb = p.tag_base + (unsigned)t * per_token;
    if (!cls_token_start<S, MODE>(p, sm, t, tb, true, false, &tok)) return;
    const int nsplit = split_count(p.pos0 + t + 1, p.chunk_min, p.nsplit_max);
    for (int layer = 0; layer < p.n_layers; ++layer) {
      const unsigned tg = tb + (unsigned)(PHASES_PER_LAYER * layer);
      if (!cls_o<S, MODE>(p, sm, ra, rb, t, layer, o0, o1, nsplit, tok, tg)) return;
      if (has_next(p, t, layer)) {
        ld_o<S>(ra, p, next_layer(p, layer), o0, pace_units(p, PACE_O));
        if (o1 >= 0) ld_o<S>(rb, p, next_layer(p, layer), o1, pace_units(p, PACE_O));
      }
    }
    LmWarm lw;
    lm_warm_load<S, MODE>(p, lw);
    if (!cls_lm_head<S, MODE>(p, sm, t, tb, [&]() {
          ld_o<S>(ra, p, 0, o0);
          if (o1 >= 0) ld_o<S>(rb, p, 0, o1);
        }, lw))
      return;
    if constexpr ((MODE & 2) != 0) trace_end(p, t);
  }
}

template <class S, int MODE>
__device__ __forceinline__ void run_idle(const Params& p, Smem<S>& sm) {
  int tok = p.first_token;
  const unsigned per_token = (unsigned)(PHASES_PER_LAYER * p.n_layers + 1);
  for (int t = 0; t < p.n_tokens; ++t) {
    if constexpr ((MODE & 2) != 0) trace_begin(p, t, CLS_IDLE);
    const unsigned tb = p.tag_base + (unsigned)t * per_token;
    if (!cls_token_start<S, MODE>(p, sm, t, tb, false, false, &tok)) return;
    LmWarm lw;
    lm_warm_load<S, MODE>(p, lw);
    if (!cls_lm_head<S, MODE>(p, sm, t, tb, []() {}, lw, true)) return;
    if constexpr ((MODE & 2) != 0) trace_end(p, t);
  }
}

// MODE bits as decode_kernel's, without bit 0 (no long-context merge here).
template <class S, int MODE>
__global__ __launch_bounds__(NT) void decode_cls_kernel(Params p) {
  static_assert((MODE & 1) == 0, "the class kernel has no long-context merge");
  __shared__ Smem<S> sm;
  if (threadIdx.x == 0) wg_abort = 0;
  for (int i = threadIdx.x; i < 16 * S::D; i += NT) (&sm.qb[0][0])[i] = 0;  // unused columns stay 0
  for (int i = threadIdx.x; i < NW * 16 * 32 * KVB; i += NT) (&sm.pb[0][0][0])[i] = 0;
  __syncthreads();
  const int* role = p.roles + blockIdx.x * ROLE_INTS;
  switch (role[RF_CLS]) {
    case CLS_ATT: run_att<S, MODE>(p, sm, role); break;
    case CLS_A: run_att<S, MODE, false>(p, sm, role); break;
    case CLS_QG: run_qg<S, MODE, true, true>(p, sm, role); break;
    case CLS_Q: run_qg<S, MODE, true, false>(p, sm, role); break;
    case CLS_G: run_qg<S, MODE, false, true>(p, sm, role); break;
    case CLS_DG: run_down<S, MODE, CLS_DG>(p, sm, role); break;
    case CLS_DO: run_down<S, MODE, CLS_DO>(p, sm, role); break;
    case CLS_D: run_down<S, MODE, CLS_D>(p, sm, role); break;
    case CLS_O: run_o<S, MODE>(p, sm, role); break;
    default: run_idle<S, MODE>(p, sm); break;
  }
  if (blockIdx.x == 0) {  // the last token's id
    const int t = p.n_tokens;
    int last = 0;
    if (!token_from_slots(p, p.amax + ((t - 1) & 1) * gridDim.x,
                          tag14(p.tag_base + (unsigned)t * (unsigned)(PHASES_PER_LAYER * p.n_layers + 1) - 1u),
                          sm.amax, &last))
      return;
    if (threadIdx.x == 0) p.out_tokens[t - 1] = last;
  }
}

}  // namespace mk
