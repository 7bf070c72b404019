// Batched-decode handle of megakernel.so (16 independent
// sequences, per-sequence KV lengths, greedy decode).  Additive extension of
// the reference ABI; the kernels are in mk_batch.h.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "mk_batch.h"
#include "mk_config.h"
#include "mk_host.h"

#include "../../include/megakernel.h"

namespace mk {
namespace batch {

struct BHandle {
  int device = 0, preset = 0, B = 0, L = 0, V = 0, S = 0, s_pad = 0, nsplit_max = 0, max_steps = 0;
  int H = 0, QD = 0, KVD = 0, QKV = 0, F = 0, D = 0, NKV = 0, norm_stride = 0, G = 0;
  hipStream_t stream = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  float last_ms = 0.f;
  BParams p{};
  // prefill: the prompt's tokens and positions (max_seq entries each), and
  // the token / step outputs of its last chunk (kept apart from the decode's)
  int *pf_tok = nullptr, *pf_pos = nullptr, *pf_out = nullptr, *pf_step = nullptr;
  std::vector<void*> owned;
  float *kscale = nullptr, *vscale = nullptr;  // FP8 cache scales, allocated on first use
  u32x4* lmhead8 = nullptr;                     // FP8 LM head copy, built on first use
  float* lm_scale = nullptr;
  int (*launch_step)(BHandle*, const BParams&) = nullptr;
  int step_variant = MK_BATCH_STEP_PER_PHASE;  // one kernel per phase and layer, or the layers in bk_step
  bool persistent_ok = false;                  // bk_step fits one workgroup on every CU
  int (*launch_prefill)(BHandle*, const PGroup&, const BParams&, bool) = nullptr;
  // prefill column groups: one block of activation buffers per group (slot 0
  // sizes), pf_gstride bytes apart, grown as prompts need more groups
  char* pf_slab = nullptr;
  int pf_groups = 0;
  long long pf_gstride = 0;
};

static void free_all(BHandle* h) {
  if (h->exec) (void)hipGraphExecDestroy(h->exec);
  if (h->graph) (void)hipGraphDestroy(h->graph);
  for (void* q : h->owned) (void)hipFree(q);
  if (h->ev0) (void)hipEventDestroy(h->ev0);
  if (h->ev1) (void)hipEventDestroy(h->ev1);
  if (h->stream) (void)hipStreamDestroy(h->stream);
}

template <class T>
static int alloc(BHandle* h, T** ptr, size_t bytes, bool zero = true) {
  void* q = nullptr;
  HIPCHK(hipMalloc(&q, bytes), -1);
  h->owned.push_back(q);
  if (zero) HIPCHK(hipMemsetAsync(q, 0, bytes, h->stream), -1);
  *ptr = static_cast<T*>(q);
  return 0;
}

// Row-major bf16 W[R][K] (at base + off) -> tile layout, blocks rb -> rb.
static int repack_tiles(BHandle* h, const char* base, long long off, int R, int K, u32x4* dst) {
  if (off < 0 || (off & 15)) {
    set_err("weight offset %lld is negative or not 16-byte aligned", off);
    return -1;
  }
  const long long units = (long long)R * K / 8;
  const int threads = 256;
  const int blocks = (int)((units + threads - 1) / threads < 65536 ? (units + threads - 1) / threads : 65536);
  hipLaunchKernelGGL(repack_kernel, dim3(blocks), dim3(threads), 0, h->stream,
                     reinterpret_cast<const u32x4*>(base + off), R, K, dst, 1, 0);
  HIPCHK(hipGetLastError(), -1);
  return 0;
}

// One decode step of every sequence: the kernels of mk_batch.h in order --
// one kernel per phase and layer (default), or the layers as one persistent
// bk_step.
template <class S>
static int launch_step(BHandle* h, const BParams& p) {
  const int L = h->L;
  PGroup1 g{};  // one column group
  g.p[0] = p;
  g.n = 1;
  hipLaunchKernelGGL((bk_embed<S, PGroup1>), dim3(BMAX), dim3(256), 0, h->stream, g);
  // the final-norm parts: slot L of the persistent step, slot 0 of the per-phase kernels
  const int lm_slot = h->step_variant == MK_BATCH_STEP_PERSISTENT ? L : 0;
  if (h->step_variant == MK_BATCH_STEP_PERSISTENT) {
    if (p.kscale)
      hipLaunchKernelGGL((bk_step<S, true>), dim3(h->G * STEP_WG_PER_CU), dim3(GT), 0, h->stream, g);
    else
      hipLaunchKernelGGL((bk_step<S, false>), dim3(h->G * STEP_WG_PER_CU), dim3(GT), 0, h->stream, g);
  }
  for (int l = 0; l < (h->step_variant == MK_BATCH_STEP_PERSISTENT ? 0 : L); ++l) {
    hipLaunchKernelGGL((bk_qkv<S, PGroup1>), dim3(S::QKV / 16 * KS_QKV), dim3(GT), 0, h->stream, g, l);
    if (p.kscale)
      hipLaunchKernelGGL((bk_attn<S, true, PGroup1>), dim3(BMAX * S::NKV * h->nsplit_max), dim3(AT), 0, h->stream, g,
                         l);
    else
      hipLaunchKernelGGL((bk_attn<S, false, PGroup1>), dim3(BMAX * S::NKV * h->nsplit_max), dim3(AT), 0, h->stream,
                         g, l);
    hipLaunchKernelGGL((bk_o<S, PGroup1>), dim3(S::H / 16 * KS_O), dim3(GT), 0, h->stream, g, l);
    hipLaunchKernelGGL((bk_gu<S, PGroup1>), dim3(S::F / 16 * KS_GU), dim3(GT), 0, h->stream, g, l);
    hipLaunchKernelGGL((bk_down<S, PGroup1>), dim3(S::H / 16 * KS_DN), dim3(GT), 0, h->stream, g, l);
  }
  if (p.lmhead8)
    hipLaunchKernelGGL((bk_lm<S, true>), dim3(h->G), dim3(GT), 0, h->stream, p, lm_slot);
  else
    hipLaunchKernelGGL((bk_lm<S, false>), dim3(h->G), dim3(GT), 0, h->stream, p, lm_slot);
  hipLaunchKernelGGL(bk_tok, dim3(1), dim3(BMAX), 0, h->stream, p);
  HIPCHK(hipGetLastError(), -1);
  return 0;
}

// One prefill pass: up to PG_MAX column groups of <= 16 consecutive prompt
// tokens of one sequence (up to 1,024 tokens per pass over the weights): the
// decode step's kernels with bk_append storing every column's K / V before
// each layer's attention; the LM head and the token only for the prompt's
// last pass, on its last group (the one holding the prompt's last token).
// pl: the parameters of the pass's last group (the LM head's input when last).
template <class S>
static int launch_prefill(BHandle* h, const PGroup& g, const BParams& pl, bool last) {
  const int L = h->L, ng = g.n;
  const auto rows = [ng](int cg) { return (ng + cg - 1) / cg; };  // GEMM workgroup rows: cg groups each
  const BParams& p = g.p;
  hipLaunchKernelGGL((bk_embed<S, PGroup>), dim3(BMAX, ng), dim3(256), 0, h->stream, g);
  for (int l = 0; l < L; ++l) {
    if (ng > PT_SMALL_GROUPS)
      hipLaunchKernelGGL((bk_ptile<S, PT_QKV, PTileQKV>), dim3(S::QKV / 16 / PTileQKV::MP, rows(PTileQKV::NG)),
                         dim3(GT), 0, h->stream, g, l);
    else
      hipLaunchKernelGGL((bk_ptile<S, PT_QKV, PTileQKVs>), dim3(S::QKV / 16 / PTileQKVs::MP, rows(PTileQKVs::NG)),
                         dim3(GT), 0, h->stream, g, l);
    if (p.kscale) {
      hipLaunchKernelGGL((bk_append<S, true, PGroup>), dim3(BMAX * S::NKV, ng), dim3(2 * kWave), 0, h->stream, g,
                         l);
      hipLaunchKernelGGL((bk_pattn<S, true>), dim3(S::NKV, ng), dim3(PC_AW * kWave), 0, h->stream, g, l);
    } else {
      hipLaunchKernelGGL((bk_append<S, false, PGroup>), dim3(BMAX * S::NKV, ng), dim3(2 * kWave), 0, h->stream, g,
                         l);
      hipLaunchKernelGGL((bk_pattn<S, false>), dim3(S::NKV, ng), dim3(PC_AW * kWave), 0, h->stream, g, l);
    }
    if (ng > PT_SMALL_GROUPS)
      hipLaunchKernelGGL((bk_ptile<S, PT_O, PTileO>), dim3(S::H / 16 / PTileO::MP, rows(PTileO::NG)), dim3(GT), 0,
                         h->stream, g, l);
    else
      hipLaunchKernelGGL((bk_ptile<S, PT_O, PTileOs>), dim3(S::H / 16 / PTileOs::MP, rows(PTileOs::NG)), dim3(GT), 0,
                         h->stream, g, l);
    if (ng > PT_SMALL_GROUPS)
      hipLaunchKernelGGL((bk_pgu_t<S, PTileGU>), dim3(S::F / 16 / PTileGU::MP, rows(PTileGU::NG)), dim3(GT), 0,
                         h->stream, g, l);
    else
      hipLaunchKernelGGL((bk_pgu_t<S, PTileGUs>), dim3(S::F / 16 / PTileGUs::MP, rows(PTileGUs::NG)), dim3(GT), 0,
                         h->stream, g, l);
    if (ng > PT_SMALL_GROUPS)
      hipLaunchKernelGGL((bk_ptile<S, PT_DN, PTileDN>), dim3(S::H / 16 / PTileDN::MP, rows(PTileDN::NG)), dim3(GT), 0,
                         h->stream, g, l);
    else
      hipLaunchKernelGGL((bk_ptile<S, PT_DN, PTileDNs>), dim3(S::H / 16 / PTileDNs::MP, rows(PTileDNs::NG)), dim3(GT),
                         0, h->stream, g, l);
  }
  if (last) {
    if (pl.lmhead8)
      hipLaunchKernelGGL((bk_lm<S, true>), dim3(h->G), dim3(GT), 0, h->stream, pl, 0);
    else
      hipLaunchKernelGGL((bk_lm<S, false>), dim3(h->G), dim3(GT), 0, h->stream, pl, 0);
    hipLaunchKernelGGL(bk_tok, dim3(1), dim3(BMAX), 0, h->stream, pl);
  }
  HIPCHK(hipGetLastError(), -1);
  return 0;
}
// QKV, O and down grids of whole XCD rounds: a row tile's column-group
// workgroups share an XCD and its L2 (gate / up has 44 row tiles: its tiles'
// groups spread over XCDs)
static_assert((ShapeBaseline::QKV / 16 / PTileQKV::MP) % 8 == 0 && (ShapeBaseline::H / 16 / PTileO::MP) % 8 == 0 &&
                  (ShapeBaseline::H / 16 / PTileDN::MP) % 8 == 0,
              "prefill GEMM grids of whole XCD rounds");

template <class S>
static bool persistent_fits() {
  int a = 0, b = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&a, bk_step<S, false>, GT, 0) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, bk_step<S, true>, GT, 0) != hipSuccess)
    return false;
  return a >= STEP_WG_PER_CU && b >= STEP_WG_PER_CU;
}

template <class S>
static void set_shape(BHandle* h) {
  h->H = S::H, h->QD = S::QD, h->KVD = S::KVD, h->QKV = S::QKV, h->F = S::F, h->D = S::D, h->NKV = S::NKV;
  h->norm_stride = S::NORM_STRIDE;
  h->launch_step = launch_step<S>;
  h->launch_prefill = launch_prefill<S>;
  h->persistent_ok = persistent_fits<S>();
}

// ext_kv / ext_kvt: bind to an external single-sequence cache (a prefill
// context of a batch-1 handle) instead of allocating BMAX caches.
static int init_state(BHandle* h, const char* base, const long long* off, int n_off, uint16_t* ext_kv = nullptr,
                      uint16_t* ext_kvt = nullptr) {
  if (n_off < 13 || (n_off - 2) % 11 != 0) {
    set_err("num_offsets=%d is not 2 + 11*layers", n_off);
    return -1;
  }
  h->L = (n_off - 2) / 11;
  if (h->V <= 0 || h->V % 16) {
    set_err("vocab %d must be a positive multiple of 16", h->V);
    return -1;
  }
  HIPCHK(hipGetDevice(&h->device), -1);
  HIPCHK(hipDeviceGetAttribute(&h->G, hipDeviceAttributeMultiprocessorCount, h->device), -1);
  HIPCHK(hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking), -1);
  HIPCHK(hipEventCreate(&h->ev0), -1);
  HIPCHK(hipEventCreate(&h->ev1), -1);
  BParams& p = h->p;
  const int L = h->L;
  p.u_qkv = (long long)h->QKV * h->H / 8;
  p.u_o = (long long)h->H * h->QD / 8;
  p.u_gu = (long long)h->F * h->H / 8;
  p.u_dn = (long long)h->H * h->F / 8;
  u32x4 *wqkv, *wo, *wg, *wu, *wd, *lm;
  if (alloc(h, &wqkv, p.u_qkv * 16 * L, false) || alloc(h, &wo, p.u_o * 16 * L, false) ||
      alloc(h, &wg, p.u_gu * 16 * L, false) || alloc(h, &wu, p.u_gu * 16 * L, false) ||
      alloc(h, &wd, p.u_dn * 16 * L, false) || alloc(h, &lm, (size_t)h->V * h->H * 2, false))
    return -1;
  uint16_t *norms, *fnorm;
  if (alloc(h, &norms, (size_t)h->norm_stride * 2 * L) || alloc(h, &fnorm, (size_t)h->H * 2)) return -1;
  // weights: tile layout for every matrix (offset order: reference megakernel.cu:518-532)
  if (repack_tiles(h, base, off[0], h->V, h->H, lm)) return -1;
  HIPCHK(hipMemcpyAsync(fnorm, base + off[1], (size_t)h->H * 2, hipMemcpyDeviceToDevice, h->stream), -1);
  const int NORM_ATTN = 0, NORM_Q = h->H, NORM_K = h->H + h->D, NORM_FFN = h->H + 2 * h->D;
  for (int i = 0; i < L; ++i) {
    const long long* o = off + 2 + 11 * i;
    uint16_t* nl = norms + (long long)i * h->norm_stride;
    HIPCHK(hipMemcpyAsync(nl + NORM_ATTN, base + o[0], (size_t)h->H * 2, hipMemcpyDeviceToDevice, h->stream), -1);
    HIPCHK(hipMemcpyAsync(nl + NORM_Q, base + o[4], (size_t)h->D * 2, hipMemcpyDeviceToDevice, h->stream), -1);
    HIPCHK(hipMemcpyAsync(nl + NORM_K, base + o[5], (size_t)h->D * 2, hipMemcpyDeviceToDevice, h->stream), -1);
    HIPCHK(hipMemcpyAsync(nl + NORM_FFN, base + o[7], (size_t)h->H * 2, hipMemcpyDeviceToDevice, h->stream), -1);
    u32x4* q = wqkv + i * p.u_qkv;
    if (repack_tiles(h, base, o[1], h->QD, h->H, q) ||
        repack_tiles(h, base, o[2], h->KVD, h->H, q + (long long)h->QD * h->H / 8) ||
        repack_tiles(h, base, o[3], h->KVD, h->H, q + (long long)(h->QD + h->KVD) * h->H / 8) ||
        repack_tiles(h, base, o[6], h->H, h->QD, wo + i * p.u_o) ||
        repack_tiles(h, base, o[8], h->F, h->H, wg + i * p.u_gu) ||
        repack_tiles(h, base, o[9], h->F, h->H, wu + i * p.u_gu) ||
        repack_tiles(h, base, o[10], h->H, h->F, wd + i * p.u_dn))
      return -1;
  }
  p.wqkv = wqkv, p.wo = wo, p.wg = wg, p.wu = wu, p.wd = wd, p.lmhead = lm;
  p.norms = norms, p.final_norm = fnorm;
  // KV caches: K then V^T regions, one slice per sequence
  h->s_pad = (h->S + 31) / 32 * 32;
  p.s_pad = h->s_pad;
  p.kv_seq = (long long)L * h->NKV * h->s_pad * h->D;
  p.sc_seq = (long long)L * h->NKV * h->s_pad;
  p.kscale = p.vscale = nullptr;
  if (ext_kv) {
    p.kv = ext_kv;
    p.kvt = ext_kvt;
  } else {
    uint16_t* kv;
    if (alloc(h, &kv, (size_t)2 * BMAX * p.kv_seq * 2)) return -1;
    p.kv = kv;
    p.kvt = kv + (long long)BMAX * p.kv_seq;
  }
  h->nsplit_max = (h->S + CH - 1) / CH;
  p.nsplit_max = h->nsplit_max;
  h->max_steps = 1 << 16;
  p.max_steps = h->max_steps;
  // activation slots (x_slot .. act_slot in mk_batch.h): L + 1 of x / xg / ssq,
  // L of qkv / att / act (the per-phase kernels use slot 0)
  const size_t xs = (size_t)L + 1, ls = (size_t)L;
  if (alloc(h, &p.x, xs * 2 * BMAX * h->H * 4) || alloc(h, &p.qkv, ls * BMAX * h->QKV * 4) ||
      alloc(h, &p.xg, xs * 4 * BMAX * h->H * 2) || alloc(h, &p.ssq, xs * 2 * (h->H / 16) * BMAX * 4) ||
      alloc(h, &p.att, ls * 2 * BMAX * h->QD * 2) || alloc(h, &p.act, ls * 2 * BMAX * h->F * 2) ||
      alloc(h, &p.part, (size_t)BMAX * h->NKV * h->nsplit_max * PW * 4) ||
      alloc(h, &p.cnt, (size_t)BMAX * h->NKV * 4) || alloc(h, &p.keys, (size_t)BMAX * 8) ||
      alloc(h, &p.rope, (size_t)BMAX * h->D * 4) ||
      alloc(h, &p.gcnt, (size_t)(h->F / 16 > h->QKV / 16 ? h->F / 16 : h->QKV / 16) * 4) ||
      alloc(h, &p.gpart, (size_t)((h->F / 16) * KS_GU * 2 > (h->QKV / 16) * KS_QKV ? (h->F / 16) * KS_GU * 2
                                                                                    : (h->QKV / 16) * KS_QKV) *
                             256 * 4 + (size_t)(h->H / 16) * (KS_O > KS_DN ? KS_O : KS_DN) * 256 * 4) ||
      alloc(h, &p.tok, (size_t)BMAX * 4) || alloc(h, &p.pos, (size_t)BMAX * 4) ||
      alloc(h, &p.out, (size_t)h->max_steps * BMAX * 4) || alloc(h, &p.step, 64) ||
      alloc(h, &p.dbg_logits, (size_t)BMAX * h->V * 4) || alloc(h, &h->pf_tok, (size_t)h->S * 4) ||
      alloc(h, &h->pf_pos, (size_t)h->S * 4) || alloc(h, &h->pf_out, (size_t)BMAX * 4) ||
      alloc(h, &h->pf_step, 64) || alloc(h, &p.flags, (size_t)L * FC_N * FLAG_MAX * 4) ||
      alloc(h, &p.epoch, 64) || alloc(h, &p.err, 256))
    return -1;
  int wall_khz = 0;
  HIPCHK(hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, h->device), -1);
  p.timeout_ticks = (unsigned long long)(wall_khz > 0 ? wall_khz : 100000) * 10000ull;  // 10 s per hand-off wait
  std::vector<float> invf(h->D / 2);
  for (int i = 0; i < h->D / 2; ++i) invf[i] = 1.0f / powf((float)kRopeTheta, (float)(2 * i) / (float)h->D);
  float* inv;
  if (alloc(h, &inv, invf.size() * 4, false)) return -1;
  HIPCHK(hipMemcpyAsync(inv, invf.data(), invf.size() * 4, hipMemcpyHostToDevice, h->stream), -1);
  p.inv_freq = inv;
  p.B = h->B, p.L = L, p.V = h->V;
  if (L >= 64) h->persistent_ok = false;  // the persistent step's split-K tags hold the layer in 6 bits
  p.prefill = 0;
  HIPCHK(hipStreamSynchronize(h->stream), -1);
  return 0;
}

static BHandle* create(int preset, int vocab, int n_seq, int max_seq) {
  if (n_seq < 1 || n_seq > BMAX) {
    set_err("n_seq %d outside [1, %d]", n_seq, BMAX);
    return nullptr;
  }
  if (max_seq < 1) {
    set_err("max_seq must be positive");
    return nullptr;
  }
  BHandle* h = new (std::nothrow) BHandle();
  if (!h) {
    set_err("out of host memory");
    return nullptr;
  }
  h->preset = preset, h->V = vocab, h->B = n_seq, h->S = max_seq;
  switch (preset) {
    case PRESET_BASELINE: set_shape<ShapeBaseline>(h); break;
    case PRESET_TINY: set_shape<ShapeTiny>(h); break;
    default:
      set_err("batched decode supports the BASELINE and TINY presets (head_dim 64, 2 q heads per kv head)");
      delete h;
      return nullptr;
  }
  return h;
}

static int check_positions(BHandle* h, int steps) {
  std::vector<int> pos(BMAX);
  HIPCHK(hipMemcpy(pos.data(), h->p.pos, BMAX * 4, hipMemcpyDeviceToHost), -1);
  for (int b = 0; b < h->B; ++b)
    if (pos[b] + steps > h->S) {
      set_err("sequence %d: position %d + %d steps exceeds KV capacity %d", b, pos[b], steps, h->S);
      return -1;
    }
  return 0;
}

static int set_tokens(BHandle* h, const int* tokens) {
  std::vector<int> t(BMAX, 0);
  for (int b = 0; b < h->B; ++b) {
    if (tokens[b] < 0 || tokens[b] >= h->V) {
      set_err("sequence %d: token id %d outside [0, %d)", b, tokens[b], h->V);
      return -1;
    }
    t[b] = tokens[b];
  }
  HIPCHK(hipMemcpyAsync(h->p.tok, t.data(), BMAX * 4, hipMemcpyHostToDevice, h->stream), -1);
  HIPCHK(hipMemsetAsync(h->p.step, 0, 4, h->stream), -1);
  return 0;
}

// A hand-off wait of the persistent step that gave up (MK_ERR_TIMEOUT in
// p.err): the error is reported and the step's counters are cleared, so the
// handle can run again.
static int check_step_error(BHandle* h) {
  int err = 0;
  HIPCHK(hipMemcpy(&err, h->p.err, 4, hipMemcpyDeviceToHost), -1);
  if (err == 0) return 0;
  HIPCHK(hipMemset(h->p.err, 0, 4), -1);
  HIPCHK(hipMemset(h->p.cnt, 0, (size_t)BMAX * h->NKV * 4), -1);
  HIPCHK(hipMemset(h->p.gcnt, 0, (size_t)(h->F / 16 > h->QKV / 16 ? h->F / 16 : h->QKV / 16) * 4), -1);
  set_err("batched decode step aborted: a hand-off wait timed out");
  return -1;
}

// The step graph: the same kernels with the same arguments every step (the
// step's inputs live in device memory), captured once.
static int ensure_graph(BHandle* h) {
  if (h->exec) return 0;
  BParams p = h->p;
  p.dbg_logits = nullptr;
  HIPCHK(hipStreamBeginCapture(h->stream, hipStreamCaptureModeThreadLocal), -1);
  const int rc = h->launch_step(h, p);
  hipGraph_t g = nullptr;
  const hipError_t e = hipStreamEndCapture(h->stream, &g);
  if (rc || e != hipSuccess) {
    if (g) (void)hipGraphDestroy(g);
    if (!rc) set_err("graph capture failed: %s", hipGetErrorString(e));
    return -1;
  }
  h->graph = g;
  HIPCHK(hipGraphInstantiate(&h->exec, g, nullptr, nullptr, 0), -1);
  return 0;
}

static int run_steps(BHandle* h, const int* first, int n, int* out) {
  if (n <= 0 || n > h->max_steps) {
    set_err("step count %d outside [1, %d]", n, h->max_steps);
    return -1;
  }
  if (check_positions(h, n) || set_tokens(h, first) || ensure_graph(h)) return -1;
  HIPCHK(hipEventRecord(h->ev0, h->stream), -1);
  for (int i = 0; i < n; ++i) HIPCHK(hipGraphLaunch(h->exec, h->stream), -1);
  HIPCHK(hipEventRecord(h->ev1, h->stream), -1);
  HIPCHK(hipStreamSynchronize(h->stream), -1);
  HIPCHK(hipEventElapsedTime(&h->last_ms, h->ev0, h->ev1), -1);
  if (check_step_error(h)) return -1;
  if (out) {
    std::vector<int> all((size_t)n * BMAX);
    HIPCHK(hipMemcpy(all.data(), h->p.out, all.size() * 4, hipMemcpyDeviceToHost), -1);
    for (int i = 0; i < n; ++i)
      for (int b = 0; b < h->B; ++b) out[(size_t)i * h->B + b] = all[(size_t)i * BMAX + b];
  }
  return 0;
}

// The activation buffers of prefill column groups (group 0's at the slab's
// start, group gi's gi * pf_gstride bytes later): offsets inside one group's
// block, in BParams order x, xg, ssq, qkv, att, act, part, cnt, gpart, gcnt,
// keys, rope.
static long long group_layout(const BHandle* h, long long off[12]) {
  // the prefill kernels keep no attention partials or split-K sums (their
  // attention merges in registers, their GEMMs run the whole K): part, cnt,
  // gpart and gcnt get one line each
  const long long sz[12] = {(long long)2 * BMAX * h->H * 4,
                            (long long)4 * BMAX * h->H * 2,
                            (long long)2 * (h->H / 16) * BMAX * 4,
                            (long long)BMAX * h->QKV * 4,
                            (long long)2 * BMAX * h->QD * 2,
                            (long long)2 * BMAX * h->F * 2,
                            256,
                            256,
                            256,
                            256,
                            (long long)BMAX * 8,
                            (long long)BMAX * h->D * 4};
  long long o = 0;
  for (int i = 0; i < 12; ++i) {
    off[i] = o;
    o += (sz[i] + 255) / 256 * 256;
  }
  return o;
}

// A slab of ng groups' buffers, cleared; a larger prompt replaces it with a
// larger one.
static int ensure_groups(BHandle* h, int ng) {
  if (h->pf_groups >= ng) return 0;
  long long off[12];
  const long long stride = group_layout(h, off);
  if (h->pf_slab) {
    HIPCHK(hipStreamSynchronize(h->stream), -1);
    for (size_t i = 0; i < h->owned.size(); ++i)
      if (h->owned[i] == h->pf_slab) {
        h->owned.erase(h->owned.begin() + (long)i);
        break;
      }
    HIPCHK(hipFree(h->pf_slab), -1);
    h->pf_slab = nullptr, h->pf_groups = 0;
  }
  if (alloc(h, &h->pf_slab, (size_t)stride * ng)) return -1;
  HIPCHK(hipStreamSynchronize(h->stream), -1);
  h->pf_groups = ng, h->pf_gstride = stride;
  return 0;
}

// n prompt tokens at positions pos0 .. of sequence seq's cache: passes of up
// to PG_MAX * 16 tokens (column groups of 16), each one pass over the weights
// with the tokens as MFMA columns.
static int prefill_passes(BHandle* h, int seq, const int* tokens, int n, int pos0, int* next_token, float* logits) {
  if (n < 1) {
    set_err("prefill: n = %d < 1", n);
    return -1;
  }
  if (pos0 < 0 || (long long)pos0 + n > h->S) {
    set_err("prefill: sequence %d position %d + %d tokens exceeds KV capacity %d", seq, pos0, n, h->S);
    return -1;
  }
  std::vector<int> t(n), q(n);
  for (int i = 0; i < n; ++i) {
    if (tokens[i] < 0 || tokens[i] >= h->V) {
      set_err("prefill: token %d = %d outside [0, %d)", i, tokens[i], h->V);
      return -1;
    }
    t[i] = tokens[i];
    q[i] = pos0 + i;
  }
  HIPCHK(hipMemcpyAsync(h->pf_tok, t.data(), (size_t)n * 4, hipMemcpyHostToDevice, h->stream), -1);
  HIPCHK(hipMemcpyAsync(h->pf_pos, q.data(), (size_t)n * 4, hipMemcpyHostToDevice, h->stream), -1);
  HIPCHK(hipMemsetAsync(h->pf_step, 0, 4, h->stream), -1);
  HIPCHK(hipEventRecord(h->ev0, h->stream), -1);
  const int ngt = (n + BMAX - 1) / BMAX, passes = (ngt + PG_MAX - 1) / PG_MAX;
  if (ensure_groups(h, ngt < PG_MAX ? ngt : PG_MAX)) return -1;
  long long off[12];
  group_layout(h, off);
  char* slab = h->pf_slab;
  for (int ps = 0; ps < passes; ++ps) {
    const int c0 = ps * PG_MAX * BMAX, ntok = n - c0 < PG_MAX * BMAX ? n - c0 : PG_MAX * BMAX;
    PGroup g{};
    BParams& pp = g.p;  // group 0 of the pass
    pp = h->p;
    pp.x = reinterpret_cast<float*>(slab + off[0]), pp.xg = reinterpret_cast<uint16_t*>(slab + off[1]);
    pp.ssq = reinterpret_cast<float*>(slab + off[2]), pp.qkv = reinterpret_cast<float*>(slab + off[3]);
    pp.att = reinterpret_cast<uint16_t*>(slab + off[4]), pp.act = reinterpret_cast<uint16_t*>(slab + off[5]);
    pp.part = reinterpret_cast<float*>(slab + off[6]), pp.cnt = reinterpret_cast<int*>(slab + off[7]);
    pp.gpart = reinterpret_cast<float*>(slab + off[8]), pp.gcnt = reinterpret_cast<int*>(slab + off[9]);
    pp.keys = reinterpret_cast<u64*>(slab + off[10]), pp.rope = reinterpret_cast<float*>(slab + off[11]);
    // every column writes and reads this sequence's cache (FP8: byte index =
    // element index, so the sequence starts at byte seq * kv_seq)
    if (h->p.kscale) {
      pp.kv = reinterpret_cast<uint16_t*>(reinterpret_cast<uint8_t*>(h->p.kv) + seq * h->p.kv_seq);
      pp.kvt = reinterpret_cast<uint16_t*>(reinterpret_cast<uint8_t*>(h->p.kvt) + seq * h->p.kv_seq);
      pp.kscale = h->p.kscale + seq * h->p.sc_seq;
      pp.vscale = h->p.vscale + seq * h->p.sc_seq;
    } else {
      pp.kv = h->p.kv + seq * h->p.kv_seq;
      pp.kvt = h->p.kvt + seq * h->p.kv_seq;
    }
    pp.kv_seq = 0;
    pp.sc_seq = 0;
    pp.prefill = 1;
    pp.tok = h->pf_tok + c0;
    pp.pos = h->pf_pos + c0;
    pp.out = h->pf_out;
    pp.step = h->pf_step;
    pp.dbg_logits = nullptr;
    g.gstride = h->pf_gstride;
    g.n = (ntok + BMAX - 1) / BMAX;
    g.ntok = ntok;
    pp.B = ntok < BMAX ? ntok : BMAX;
    const bool last = ps == passes - 1;
    BParams pl = group_params(g, g.n - 1);
    pl.dbg_logits = last && logits ? h->p.dbg_logits : nullptr;
    if (h->launch_prefill(h, g, pl, last)) return -1;
  }
  HIPCHK(hipEventRecord(h->ev1, h->stream), -1);
  HIPCHK(hipStreamSynchronize(h->stream), -1);
  HIPCHK(hipEventElapsedTime(&h->last_ms, h->ev0, h->ev1), -1);
  const int lastcol = (n - 1) % BMAX;
  if (next_token) HIPCHK(hipMemcpy(next_token, h->pf_out + lastcol, 4, hipMemcpyDeviceToHost), -1);
  if (logits)
    HIPCHK(hipMemcpy(logits, h->p.dbg_logits + (size_t)lastcol * h->V, (size_t)h->V * 4, hipMemcpyDeviceToHost), -1);
  return 0;
}

// Prefill of sequence seq of a batch handle at its position, which advances by n.
static int run_prefill(BHandle* h, int seq, const int* tokens, int n, int* next_token, float* logits) {
  if (seq < 0 || seq >= h->B || n < 1) {
    set_err("prefill: sequence %d outside [0, %d) or n = %d < 1", seq, h->B, n);
    return -1;
  }
  int pos0 = 0;
  HIPCHK(hipMemcpy(&pos0, h->p.pos + seq, 4, hipMemcpyDeviceToHost), -1);
  if (prefill_passes(h, seq, tokens, n, pos0, next_token, logits)) return -1;
  const int pend = pos0 + n;
  HIPCHK(hipMemcpy(h->p.pos + seq, &pend, 4, hipMemcpyHostToDevice), -1);
  return 0;
}

BHandle* create_prefill_context(int preset, int vocab, int max_seq, const char* d_weights, const long long* offsets,
                                int num_offsets, uint16_t* kv, uint16_t* kvt) {
  if (!d_weights || !offsets || !kv || !kvt) {
    set_err("prefill context: null weights, offsets or cache");
    return nullptr;
  }
  BHandle* h = create(preset, vocab, 1, max_seq);
  if (!h) return nullptr;
  if (init_state(h, d_weights, offsets, num_offsets, kv, kvt)) {
    free_all(h);
    delete h;
    return nullptr;
  }
  return h;
}

int prefill_context_run(BHandle* h, const int* tokens, int n, int pos0, int* next_token, float* logits,
                        float* kscale, float* vscale) {
  h->p.kscale = kscale;  // the bound cache's FP8 row scales, or null for a bf16 cache
  h->p.vscale = vscale;
  return prefill_passes(h, 0, tokens, n, pos0, next_token, logits);
}

float prefill_context_ms(BHandle* h) { return h->last_ms; }

void destroy_prefill_context(BHandle* h) {
  if (!h) return;
  (void)hipStreamSynchronize(h->stream);
  free_all(h);
  delete h;
}

}  // namespace batch
}  // namespace mk

using mk::batch::BHandle;

extern "C" {

void* megakernel_batch_init(void* d_weights, const long long* offsets, int num_offsets, int preset, int vocab,
                            int n_seq, int max_seq) {
  if (!d_weights || !offsets) {
    mk::set_err("null weights or offsets");
    return nullptr;
  }
  BHandle* h = mk::batch::create(preset, vocab, n_seq, max_seq);
  if (!h) return nullptr;
  if (mk::batch::init_state(h, static_cast<const char*>(d_weights), offsets, num_offsets)) {
    mk::batch::free_all(h);
    delete h;
    return nullptr;
  }
  return h;
}

void megakernel_batch_free(void* handle) {
  BHandle* h = static_cast<BHandle*>(handle);
  if (!h) return;
  (void)hipStreamSynchronize(h->stream);
  mk::batch::free_all(h);
  delete h;
}

int megakernel_batch_set_pos(void* handle, int seq, int pos) {
  BHandle* h = static_cast<BHandle*>(handle);
  if (!h || seq < 0 || seq >= h->B || pos < 0 || pos > h->S) {
    mk::set_err("invalid handle, sequence %d or position %d", seq, pos);
    return -1;
  }
  HIPCHK(hipMemcpy(h->p.pos + seq, &pos, 4, hipMemcpyHostToDevice), -1);
  return 0;
}

int megakernel_batch_get_pos(void* handle, int* pos) {
  BHandle* h = static_cast<BHandle*>(handle);
  if (!h || !pos) {
    mk::set_err("invalid arguments");
    return -1;
  }
  HIPCHK(hipMemcpy(pos, h->p.pos, (size_t)h->B * 4, hipMemcpyDeviceToHost), -1);
  return 0;
}

int megakernel_batch_fill_kv_synthetic(void* handle, int seq, int len, unsigned long long seed, float std) {
  BHandle* h = static_cast<BHandle*>(handle);
  if (!h || seq < 0 || seq >= h->B || len < 0 || len > h->S) {
    mk::set_err("invalid fill arguments (sequence %d, len %d)", seq, len);
    return -1;
  }
  if (len > 0 && h->p.kscale) {  // FP8 cache: the bf16 values in the reference layout, then quantised rows
    const float c = (float)(std * sqrt(3.0) / 65536.0);
    void* stage = nullptr;
    HIPCHK(hipMalloc(&stage, (size_t)2 * h->L * h->NKV * (size_t)len * h->D * 2), -1);
    hipLaunchKernelGGL(mk::synth_kv_ref_kernel, dim3(4096), dim3(256), 0, h->stream, static_cast<uint16_t*>(stage),
                       h->L, h->NKV, h->D, len, seed, c);
    hipLaunchKernelGGL(mk::kv_quant_kernel, dim3(2048), dim3(256), 0, h->stream, static_cast<const uint16_t*>(stage),
                       reinterpret_cast<uint8_t*>(h->p.kv) + seq * h->p.kv_seq,
                       reinterpret_cast<uint8_t*>(h->p.kvt) + seq * h->p.kv_seq, h->p.kscale + seq * h->p.sc_seq,
                       h->p.vscale + seq * h->p.sc_seq, h->L, h->NKV, h->s_pad, h->D, len);
    const hipError_t e = hipGetLastError() == hipSuccess ? hipStreamSynchronize(h->stream) : hipErrorLaunchFailure;
    (void)hipFree(stage);
    if (e != hipSuccess) {
      mk::set_err("FP8 KV fill failed: %s", hipGetErrorString(e));
      return -1;
    }
  } else if (len > 0) {
    const float c = (float)(std * sqrt(3.0) / 65536.0);
    hipLaunchKernelGGL(mk::synth_kv_kernel, dim3(4096), dim3(256), 0, h->stream, h->p.kv + seq * h->p.kv_seq,
                       h->p.kvt + seq * h->p.kv_seq, h->L, h->NKV, h->s_pad, h->D, len, seed, c);
    HIPCHK(hipGetLastError(), -1);
    HIPCHK(hipStreamSynchronize(h->stream), -1);
  }
  return megakernel_batch_set_pos(handle, seq, len);
}

static int batch_kv_transfer(BHandle* h, int seq, void* host_kv, int len, int to_cache) {
  const size_t bytes = (size_t)2 * h->L * h->NKV * (size_t)len * h->D * 2;
  void* stage = nullptr;
  HIPCHK(hipMalloc(&stage, bytes), -1);
  int rc = -1;
  do {
    if (to_cache && hipMemcpy(stage, host_kv, bytes, hipMemcpyHostToDevice) != hipSuccess) {
      mk::set_err("KV upload failed");
      break;
    }
    // FP8: byte index = element index, so sequence seq starts at byte seq * kv_seq
    uint8_t* k8 = reinterpret_cast<uint8_t*>(h->p.kv) + seq * h->p.kv_seq;
    uint8_t* v8 = reinterpret_cast<uint8_t*>(h->p.kvt) + seq * h->p.kv_seq;
    if (h->p.kscale && to_cache)
      hipLaunchKernelGGL(mk::kv_quant_kernel, dim3(2048), dim3(256), 0, h->stream, static_cast<const uint16_t*>(stage),
                         k8, v8, h->p.kscale + seq * h->p.sc_seq, h->p.vscale + seq * h->p.sc_seq, h->L, h->NKV,
                         h->s_pad, h->D, len);
    else if (h->p.kscale)
      hipLaunchKernelGGL(mk::kv_dequant_kernel, dim3(2048), dim3(256), 0, h->stream, static_cast<uint16_t*>(stage),
                         k8, v8, h->p.kscale + seq * h->p.sc_seq, h->p.vscale + seq * h->p.sc_seq, h->L, h->NKV,
                         h->s_pad, h->D, len);
    else
      hipLaunchKernelGGL(mk::kv_convert_kernel, dim3(2048), dim3(256), 0, h->stream, static_cast<uint16_t*>(stage),
                         h->p.kv + seq * h->p.kv_seq, h->p.kvt + seq * h->p.kv_seq, h->L, h->NKV, h->s_pad, h->D,
                         len, to_cache);
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

int megakernel_batch_set_kv(void* handle, int seq, const void* host_kv, int len) {
  BHandle* h = static_cast<BHandle*>(handle);
  if (!h || !host_kv || seq < 0 || seq >= h->B || len < 0 || len > h->S) {
    mk::set_err("invalid set_kv arguments (sequence %d, len %d)", seq, len);
    return -1;
  }
  if (len > 0 && batch_kv_transfer(h, seq, const_cast<void*>(host_kv), len, 1)) return -1;
  return megakernel_batch_set_pos(handle, seq, len);
}

int megakernel_batch_get_kv(void* handle, int seq, void* host_kv, int len) {
  BHandle* h = static_cast<BHandle*>(handle);
  if (!h || !host_kv || seq < 0 || seq >= h->B || len < 0 || len > h->S) {
    mk::set_err("invalid get_kv arguments (sequence %d, len %d)", seq, len);
    return -1;
  }
  return len > 0 ? batch_kv_transfer(h, seq, host_kv, len, 0) : 0;
}

int megakernel_decode_batch(void* handle, const int* tokens_in, int* tokens_out) {
  BHandle* h = static_cast<BHandle*>(handle);
  if (!h || !tokens_in) {
    mk::set_err("null handle or tokens");
    return -1;
  }
  return mk::batch::run_steps(h, tokens_in, 1, tokens_out);
}

int megakernel_generate_batch(void* handle, const int* first_tokens, int n_steps, int* tokens_out) {
  BHandle* h = static_cast<BHandle*>(handle);
  if (!h || !first_tokens) {
    mk::set_err("null handle or tokens");
    return -1;
  }
  return mk::batch::run_steps(h, first_tokens, n_steps, tokens_out);
}

int megakernel_batch_debug_logits(void* handle, const int* tokens_in, int* tokens_out, float* logits) {
  BHandle* h = static_cast<BHandle*>(handle);
  if (!h || !tokens_in || !logits) {
    mk::set_err("null handle, tokens or logits");
    return -1;
  }
  if (mk::batch::check_positions(h, 1) || mk::batch::set_tokens(h, tokens_in)) return -1;
  if (h->launch_step(h, h->p)) return -1;  // eager launches, logits written
  HIPCHK(hipStreamSynchronize(h->stream), -1);
  if (mk::batch::check_step_error(h)) return -1;
  HIPCHK(hipMemcpy(logits, h->p.dbg_logits, (size_t)h->B * h->V * 4, hipMemcpyDeviceToHost), -1);
  if (tokens_out) {
    std::vector<int> t(mk::batch::BMAX);
    HIPCHK(hipMemcpy(t.data(), h->p.out, mk::batch::BMAX * 4, hipMemcpyDeviceToHost), -1);
    for (int b = 0; b < h->B; ++b) tokens_out[b] = t[b];
  }
  return 0;
}

int megakernel_batch_prefill(void* handle, int seq, const int* tokens, int n, int* next_token, float* logits) {
  BHandle* h = static_cast<BHandle*>(handle);
  if (!h || !tokens) {
    mk::set_err("null handle or tokens");
    return -1;
  }
  return mk::batch::run_prefill(h, seq, tokens, n, next_token, logits);
}

int megakernel_batch_set_kv_fp8(void* handle, int enable) {
  BHandle* h = static_cast<BHandle*>(handle);
  if (!h) {
    mk::set_err("null handle");
    return -1;
  }
  const size_t sb = (size_t)mk::batch::BMAX * h->p.sc_seq * 4;
  if (enable && !h->kscale) {
    if (mk::batch::alloc(h, &h->kscale, sb) || mk::batch::alloc(h, &h->vscale, sb)) return -1;
  }
  h->p.kscale = enable ? h->kscale : nullptr;
  h->p.vscale = enable ? h->vscale : nullptr;
  // empty caches in the new format, every sequence at position 0, and a step
  // graph captured again with the matching attention kernel
  HIPCHK(hipMemsetAsync(h->p.kv, 0, (size_t)mk::batch::BMAX * h->p.kv_seq * 2, h->stream), -1);
  HIPCHK(hipMemsetAsync(h->p.kvt, 0, (size_t)mk::batch::BMAX * h->p.kv_seq * 2, h->stream), -1);
  if (h->kscale) {
    HIPCHK(hipMemsetAsync(h->kscale, 0, sb, h->stream), -1);
    HIPCHK(hipMemsetAsync(h->vscale, 0, sb, h->stream), -1);
  }
  HIPCHK(hipMemsetAsync(h->p.pos, 0, mk::batch::BMAX * 4, h->stream), -1);
  HIPCHK(hipStreamSynchronize(h->stream), -1);
  if (h->exec) (void)hipGraphExecDestroy(h->exec);
  if (h->graph) (void)hipGraphDestroy(h->graph);
  h->exec = nullptr;
  h->graph = nullptr;
  return 0;
}

int megakernel_batch_set_lmhead_fp8(void* handle, int enable) {
  BHandle* h = static_cast<BHandle*>(handle);
  if (!h) {
    mk::set_err("null handle");
    return -1;
  }
  if (enable && !h->lmhead8) {
    if (h->V % 16 || h->H % 64) {
      mk::set_err("FP8 LM head needs vocab %% 16 == 0 and hidden %% 64 == 0");
      return -1;
    }
    if (mk::batch::alloc(h, &h->lmhead8, (size_t)h->V * h->H, false) ||
        mk::batch::alloc(h, &h->lm_scale, (size_t)h->V * 4, false))
      return -1;
    hipLaunchKernelGGL(mk::lmhead_fp8_kernel, dim3(h->V / 16), dim3(256), 0, h->stream, h->p.lmhead, h->H,
                       reinterpret_cast<unsigned char*>(h->lmhead8), h->lm_scale, nullptr);
    HIPCHK(hipGetLastError(), -1);
    HIPCHK(hipStreamSynchronize(h->stream), -1);
  }
  h->p.lmhead8 = enable ? h->lmhead8 : nullptr;
  h->p.lm_scale = enable ? h->lm_scale : nullptr;
  if (h->exec) (void)hipGraphExecDestroy(h->exec);  // captured again with the matching LM head
  if (h->graph) (void)hipGraphDestroy(h->graph);
  h->exec = nullptr;
  h->graph = nullptr;
  return 0;
}

int megakernel_batch_trace_step(void* handle, const int* tokens_in, unsigned long long* stamps, long long n_stamps) {
  BHandle* h = static_cast<BHandle*>(handle);
  if (!h || !tokens_in || !stamps || h->step_variant != MK_BATCH_STEP_PERSISTENT) {
    mk::set_err("null handle / tokens / output, or the persistent step is not selected");
    return -1;
  }
  const int G = h->G * mk::batch::STEP_WG_PER_CU;
  const long long need = (long long)h->L * mk::batch::TR_N * G;
  if (n_stamps < need) {
    mk::set_err("trace needs %lld stamps, got %lld", need, n_stamps);
    return -1;
  }
  if (mk::batch::check_positions(h, 1) || mk::batch::set_tokens(h, tokens_in)) return -1;
  unsigned long long* dev = nullptr;
  HIPCHK(hipMalloc(&dev, (size_t)need * 8), -1);
  int rc = -1;
  do {
    if (hipMemsetAsync(dev, 0, (size_t)need * 8, h->stream) != hipSuccess) break;
    mk::batch::BParams p = h->p;
    p.trace = dev;
    if (h->launch_step(h, p) || hipStreamSynchronize(h->stream) != hipSuccess) break;
    if (mk::batch::check_step_error(h)) break;
    if (hipMemcpy(stamps, dev, (size_t)need * 8, hipMemcpyDeviceToHost) != hipSuccess) break;
    rc = G;
  } while (0);
  (void)hipFree(dev);
  if (rc < 0) mk::set_err("batched trace step failed");
  return rc;
}

int megakernel_batch_set_step_kernel(void* handle, int variant) {
  BHandle* h = static_cast<BHandle*>(handle);
  if (!h || (variant != MK_BATCH_STEP_PERSISTENT && variant != MK_BATCH_STEP_PER_PHASE)) {
    mk::set_err("null handle or unknown step variant %d", variant);
    return -1;
  }
  if (variant == MK_BATCH_STEP_PERSISTENT && !h->persistent_ok) {
    mk::set_err("the persistent batched step does not fit one workgroup per CU on this device");
    return -1;
  }
  if (variant != h->step_variant) {
    h->step_variant = variant;
    if (h->exec) (void)hipGraphExecDestroy(h->exec);  // captured again with the chosen kernels
    if (h->graph) (void)hipGraphDestroy(h->graph);
    h->exec = nullptr;
    h->graph = nullptr;
  }
  return 0;
}

float megakernel_batch_last_ms(void* handle) {
  BHandle* h = static_cast<BHandle*>(handle);
  return h ? h->last_ms : -1.f;
}

}  // extern "C"
