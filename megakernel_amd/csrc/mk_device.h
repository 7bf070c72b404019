// Device-side helpers for the gfx950 megakernel: bf16 handling, wave64
// reductions, the counter-based generator and the grid synchronisation.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mk_protocol.h"

namespace mk {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ------------------------------------------------------------------ bf16
__device__ __forceinline__ float bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Round-to-nearest-even fp32 -> bf16 bits (finite inputs; NaN stays NaN-ish).
__host__ __device__ __forceinline__ uint16_t f32_to_bf16(float f) {
#ifdef __HIP_DEVICE_COMPILE__
  uint32_t b = __float_as_uint(f);
#else
  uint32_t b;
  __builtin_memcpy(&b, &f, 4);
#endif
  b += 0x7fffu + ((b >> 16) & 1u);
  return (uint16_t)(b >> 16);
}

// 8 bf16 (one 16-byte unit) dotted with 8 fp32 values.
// x = hi + mid + lo, three bf16 parts taken by truncation: hi holds the top
// 8 significant bits of x, mid the next 8 of the (exact) remainder, lo the
// rest, which has at most 8 significant bits -- so the split is exact (up to
// underflow) and bf16 x bf16 products on the matrix cores, exact in fp32,
// reproduce an fp32 operand.  Results are the raw 32-bit patterns whose upper
// halves are the bf16 parts.
struct Split3 {
  unsigned hi, mid, lo;
};
__device__ __forceinline__ Split3 split3(float v) {
  const unsigned u = __float_as_uint(v);
  const float r1 = v - __uint_as_float(u & 0xffff0000u);
  const unsigned u1 = __float_as_uint(r1);
  const float r2 = r1 - __uint_as_float(u1 & 0xffff0000u);
  return Split3{u, u1, __float_as_uint(r2)};
}
// upper halves of a (low 16 bits of the result) and b (high 16 bits)
__device__ __forceinline__ unsigned pack_hi16(unsigned a, unsigned b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }
__device__ __forceinline__ void split_bf16(float v, uint16_t& hi, uint16_t& mid, uint16_t& lo) {
  const Split3 t = split3(v);
  hi = (uint16_t)(t.hi >> 16);
  mid = (uint16_t)(t.mid >> 16);
  lo = (uint16_t)(t.lo >> 16);
}

__device__ __forceinline__ float dot8(u32x4 w, const float* h, float acc) {
  acc = fmaf(bf16_lo(w.x), h[0], acc);
  acc = fmaf(bf16_hi(w.x), h[1], acc);
  acc = fmaf(bf16_lo(w.y), h[2], acc);
  acc = fmaf(bf16_hi(w.y), h[3], acc);
  acc = fmaf(bf16_lo(w.z), h[4], acc);
  acc = fmaf(bf16_hi(w.z), h[5], acc);
  acc = fmaf(bf16_lo(w.w), h[6], acc);
  acc = fmaf(bf16_hi(w.w), h[7], acc);
  return acc;
}

// Split-bf16 GEMV input vectors.  A layer GEMV's input x lives in LDS as two
// bf16 parts, x = hi + lo with hi = RNE(x) and lo = RNE(x - hi) (x - hi is
// exact; relative error of the pair <= 2^-17), the B operand's columns 0 and
// 1 of the block product (mk_kernel.h blk_mma).  Layout: 8 columns per
// 32-byte group, the group's 4 dwords of hi pairs (columns 2i, 2i+1 in the
// low / high half) then its 4 of lo pairs -- one 16-byte load per part and
// 8 columns, and the same 4-byte slot count as an fp32 vector.
// Split-bf16 parts of two values by the hardware conversion (gfx950
// v_cvt_pk_bf16_f32, round to nearest even): hi holds RNE(a) in its low half
// and RNE(b) in its high half, lo the same for a - hi(a), b - hi(b) (exact
// differences).  Three conversions' worth of work in two instructions plus
// the differences, where the bit-twiddled RNE took about ten per value.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void bf16_hilo2(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
  const float ha = __uint_as_float(hi << 16), hb = __uint_as_float(hi & 0xffff0000u);
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a - ha, b - hb}, bf16x2_t));
}
__device__ __forceinline__ void xs_put(uint32_t* xs, int e, float v) {
  uint16_t* h = reinterpret_cast<uint16_t*>(xs);
  const int g = e >> 3, j = e & 7;
  uint32_t hi, lo;
  bf16_hilo2(v, 0.f, hi, lo);
  h[(g * 8 + (j >> 1)) * 2 + (j & 1)] = (uint16_t)hi;
  h[(g * 8 + 4 + (j >> 1)) * 2 + (j & 1)] = (uint16_t)lo;
}
// columns e, e + 1 (e even): one dword of each part
__device__ __forceinline__ void xs_put_pair(uint32_t* xs, int e, float a, float b) {
  const int g = e >> 3, i = (e & 7) >> 1;
  uint32_t hi, lo;
  bf16_hilo2(a, b, hi, lo);
  xs[g * 8 + i] = hi;
  xs[g * 8 + 4 + i] = lo;
}
// columns e .. e + 3 (e a multiple of 4): two dwords of each part, one 8-byte
// LDS store per part
__device__ __forceinline__ void xs_put_quad(uint32_t* xs, int e, float a, float b, float c, float d) {
  const int g = e >> 3, i = (e & 7) >> 1;
  uint32_t h0, l0, h1, l1;
  bf16_hilo2(a, b, h0, l0);
  bf16_hilo2(c, d, h1, l1);
  *reinterpret_cast<u32x2*>(xs + g * 8 + i) = u32x2{h0, h1};
  *reinterpret_cast<u32x2*>(xs + g * 8 + 4 + i) = u32x2{l0, l1};
}
// 16 FP8 (OCP e4m3) weights against 16 fp32 inputs: the hardware converts two
// bytes per instruction (bytes 0-1 / 2-3 of each dword, in order).
__device__ __forceinline__ float dot16_fp8(u32x4 w, const float* h, float acc) {
  const unsigned d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)d[i], false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)d[i], true);
    acc = fmaf(lo[0], h[4 * i + 0], acc);
    acc = fmaf(lo[1], h[4 * i + 1], acc);
    acc = fmaf(hi[0], h[4 * i + 2], acc);
    acc = fmaf(hi[1], h[4 * i + 3], acc);
  }
  return acc;
}

// 8 FP8 (OCP e4m3) values -> 8 bf16 in the same order, each multiplied by a
// power of two s.  Exact: an e4m3 value has 4 significant bits.  One
// instruction per two values (gfx950 v_cvt_scalef32_pk_bf16_fp8).
__device__ __forceinline__ u32x4 fp8x8_to_bf16x8_scaled(u32x2 r, float s) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  u32x4 o;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    o[2 * i] = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r[i], s, false));
    o[2 * i + 1] = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r[i], s, true));
  }
  return o;
}

// u32x2 holding 8 bytes with byte e (0..7) replaced by v (register-only).
__device__ __forceinline__ u32x2 set_u8(u32x2 x, int e, unsigned v) {
  const unsigned sh = 8u * (unsigned)(e & 3);
  u32x2 r = x;
#pragma unroll
  for (int c = 0; c < 2; ++c) r[c] = (c == (e >> 2)) ? ((x[c] & ~(0xffu << sh)) | (v << sh)) : x[c];
  return r;
}

// Power-of-two scale exponent of a row with absolute maximum amax: the
// smallest e with amax <= 448 * 2^e (0 for an all-zero row).
__device__ __forceinline__ int e4m3_row_exp(float amax) {
  if (!(amax > 0.f)) return 0;
  int e = ilogbf(amax) - 8;  // 448 = 1.75 * 2^8
  if (amax > ldexpf(448.f, e)) ++e;
  return e;
}

// OCP e4m3 (bias 7, largest finite 448, no infinities) of x, |x| <= 448,
// rounded to nearest, ties to even.  Subnormals are m * 2^-9 (m < 8).
__device__ __forceinline__ unsigned e4m3_encode(float x) {
  const unsigned s = signbit(x) ? 0x80u : 0u;
  const float a = fabsf(x);
  unsigned c;
  if (a < 0.015625f) {
    c = (unsigned)rintf(a * 512.0f);  // 0..8; 8 is the smallest normal
  } else {
    const int e = ilogbf(a);
    c = (unsigned)((e + 7) << 3) + (unsigned)rintf(ldexpf(a, 3 - e)) - 8u;
  }
  return s | (c > 0x7eu ? 0x7eu : c);
}

__device__ __forceinline__ u32x4 ld_nt(const u32x4* p) { return __builtin_nontemporal_load(p); }

// Raw buffer loads: a wave-uniform base in a buffer descriptor (SGPRs), a
// 32-bit per-lane byte offset (one VGPR shared by every load of a stream) and
// a wave-uniform byte offset (SGPR).  Streamed loads then carry no per-load
// 64-bit address registers.  Dword 3 selects 32-bit raw data for gfx9-class
// descriptors; out-of-range offsets (>= num_records) read as zero.
// The base must be wave-uniform; it is passed through readfirstlane so the
// descriptor is built in SGPRs (otherwise each load becomes a waterfall loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
  const unsigned long long a = reinterpret_cast<unsigned long long>(base);
  const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)a);
  const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(a >> 32));
  void* ub = reinterpret_cast<void*>(((unsigned long long)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(ub, (short)0, 0x7fffffff, 0x00020000);
}
// Non-temporal 16-byte load at base + voff + soff.
__device__ __forceinline__ u32x4 buf_ld_nt(__amdgpu_buffer_rsrc_t rs, unsigned voff, unsigned soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 2);
}

// Returns v unchanged but opaque to the optimiser.  Values derived from it
// cannot be hoisted above this point, which keeps loop-invariant per-lane
// addresses of later phases from being held in registers across the whole
// persistent loop (they are cheap to recompute, expensive to keep live).
__device__ __forceinline__ int opaque_v(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// The thread index, opaque to the optimiser (see opaque_v): every helper that
// derives per-lane addresses reads it through here, so those addresses are
// recomputed where they are used instead of living in registers across the
// whole persistent loop.
__device__ __forceinline__ int ltid() { return opaque_v((int)threadIdx.x); }

// Wave index as a wave-uniform (scalar) value and the lane index.  Loads are
// written as  uniform_base + (unsigned)lane_offset  so the compiler can use the
// SGPR-base + 32-bit VGPR-offset form: prefetched loads then need no per-load
// 64-bit address registers, which would otherwise alias the destinations of
// loads still in flight and force a wait before the next load is issued.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave); }
__device__ __forceinline__ unsigned lane_id() { return (unsigned)opaque_v((int)threadIdx.x) & (kWave - 1u); }

// ------------------------------------------------------------ reductions
// Cross-lane steps use DPP lane selects (folded into the ALU op) inside a row
// of 16 lanes and the gfx950 permlane swaps across rows, so no step goes
// through LDS.  Every pattern pairs each lane with exactly one partner, and
// both partners add the same two values, so all lanes of a group end with
// identical bits.
template <int CTRL>
__device__ __forceinline__ float dpp_sel(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}
constexpr int DPP_XOR1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141; // lane i <-> 7 - i within 8
constexpr int DPP_MIRROR = 0x140;      // lane i <-> 15 - i within 16
constexpr int DPP_ROR8 = 0x128;        // lane i <- (i + 8) mod 16, i.e. i ^ 8

// x of lane l ^ 16 / l ^ 32 (v_permlane16_swap / v_permlane32_swap with both
// operands x: the first result holds the even-row / low-half copy, the second
// the odd-row / high-half copy).
__device__ __forceinline__ float lane_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(((int)lane_id() & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(((int)lane_id() & 32) ? r[0] : r[1]);
}
// x + x(l ^ 16), x + x(l ^ 32): the two swap results are the pair in row order.
__device__ __forceinline__ float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Sum over aligned groups of N = 1, 2, 4, 8 or 16 consecutive lanes (result
// in all of them).
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "group of 1, 2, 4, 8 or 16 lanes");
  if constexpr (N >= 2) v += dpp_sel<DPP_XOR1>(v);
  if constexpr (N >= 4) v += dpp_sel<DPP_XOR2>(v);
  if constexpr (N >= 8) v += dpp_sel<DPP_HALF_MIRROR>(v);  // quads are uniform: pairs quad 0 with quad 1
  if constexpr (N == 16) v += dpp_sel<DPP_MIRROR>(v);      // pairs the two 8-lane halves
  return v;
}
template <int N>
__device__ __forceinline__ float group_max(float v) {
  static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "group of 1, 2, 4, 8 or 16 lanes");
  if constexpr (N >= 2) v = fmaxf(v, dpp_sel<DPP_XOR1>(v));
  if constexpr (N >= 4) v = fmaxf(v, dpp_sel<DPP_XOR2>(v));
  if constexpr (N >= 8) v = fmaxf(v, dpp_sel<DPP_HALF_MIRROR>(v));
  if constexpr (N == 16) v = fmaxf(v, dpp_sel<DPP_MIRROR>(v));
  return v;
}

// Sum over the lanes l, l ^ S, ... with the same l mod S (S = 8 or 16): the
// per-lane reduction of S-lane-strided partials.
template <int S>
__device__ __forceinline__ float stride_sum(float v) {
  static_assert(S == 8 || S == 16, "stride 8 or 16");
  if constexpr (S == 8) v += dpp_sel<DPP_ROR8>(v);
  return sum_xor32(sum_xor16(v));
}

__device__ __forceinline__ float wave_sum(float v) { return sum_xor32(sum_xor16(group_sum<16>(v))); }
__device__ __forceinline__ float wave_max(float v) { return max_xor32(max_xor16(group_max<16>(v))); }

// Block-wide sum/max.  `red` is LDS scratch of >= NW floats.  Every thread
// combines the per-wave values in the same order, so all get identical bits.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int t_ = ltid(), w = t_ / kWave, l = t_ % kWave;
  if (l == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NW; ++i) s += red[i];
  __syncthreads();
  return s;
}
template <int NW>
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int t_ = ltid(), w = t_ / kWave, l = t_ % kWave;
  if (l == 0) red[w] = v;
  __syncthreads();
  float s = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) s = fmaxf(s, red[i]);
  __syncthreads();
  return s;
}

// Monotone map of fp32 onto uint32 (larger float -> larger key).
__device__ __forceinline__ uint32_t f32_order_key(float f) {
  uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
// Argmax key: value in the high word, ~index in the low word, so an unsigned
// 64-bit max picks the largest value and, among equal values, the lowest index
// (torch.argmax semantics).
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
  return ((unsigned long long)f32_order_key(v) << 32) | (unsigned long long)(0xffffffffu - idx);
}
__device__ __forceinline__ uint32_t argmax_key_index(unsigned long long k) {
  return 0xffffffffu - (uint32_t)(k & 0xffffffffull);
}

// -------------------------------------------------------- synthetic data
// Counter-based generator; the CPU restatement is oracle/synth.py.
constexpr unsigned long long kGold = 0x9E3779B97F4A7C15ull;
__host__ __device__ __forceinline__ unsigned long long mix64(unsigned long long z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__host__ __device__ __forceinline__ unsigned long long sm_h(unsigned long long k, unsigned long long i) {
  return mix64(k + (i + 1ull) * kGold);
}
// One value of the Irwin-Hall(4) stream: float32(S - 131070) * c [+ 1].
__device__ __forceinline__ uint16_t synth_bf16(unsigned long long key, unsigned long long i, float c,
                                               int add_one) {
  unsigned long long r = sm_h(key, i);
  int s = (int)(r & 0xffff) + (int)((r >> 16) & 0xffff) + (int)((r >> 32) & 0xffff) + (int)(r >> 48);
  float f = __fmul_rn((float)(s - 131070), c);
  if (add_one) f = __fadd_rn(1.0f, f);
  return f32_to_bf16(f);
}

// ------------------------------------------------ tagged dataflow words
// Workgroups never meet at a barrier.  Every value one workgroup hands to
// another is a single 64-bit word  (tag << 32) | fp32 bits, written with ONE
// agent-scope relaxed atomic store (global_store_dwordx2 sc1 on gfx950: write
// through to the device coherence point) and read with agent-scope relaxed
// atomic loads (sc1: miss the non-coherent per-XCD caches).  The tag is the
// global number of the phase that produced the value, so a consumer spins on
// exactly the words it needs until every tag equals the producing phase's
// number.  Because value and tag travel in one single-copy-atomic word, no
// release/acquire fence (L2 write-back / invalidate) and no read-modify-write
// is needed: a word with the right tag carries the right value.  Waits are
// bounded: on timeout the error word is set and every workgroup unwinds.
// (encodings and tag arithmetic: mk_protocol.h)
enum : int { MK_OK = 0, MK_ERR_TIMEOUT = 1 };

__device__ __forceinline__ void ll_put(u64* p, u64 w) {
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 ll_get(u64* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// Two adjacent packed-pair words (16-byte aligned, byte offset off in the
// buffer rs) in one 16-byte load with agent scope (sc1, as ll_get): a poll
// round needs half the load instructions of 8-byte loads.  Every 32-bit half
// carries its own tag, so a half that predates its word's last write never
// passes for current, however the load is split.  Poll loops put an asm
// memory clobber at the top of each round so the load is re-issued.
__device__ __forceinline__ u32x4 pk_get2(__amdgpu_buffer_rsrc_t rs, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0u, 16);
}
// Value of one 32-bit half, and whether all four halves carry tag t4.
__device__ __forceinline__ float pkv(unsigned h) { return __uint_as_float(h & ~15u); }
__device__ __forceinline__ bool pk2_ready(u32x4 q, unsigned t4) {
  return (q.x & 15u) == t4 && (q.y & 15u) == t4 && (q.z & 15u) == t4 && (q.w & 15u) == t4;
}

// Bounded spinning of one thread.  step() returns false when the wait must be
// abandoned (this thread timed out, or another workgroup already failed).
// Pause between poll rounds (s_sleep units of 64 clocks).  No pause measured
// fastest: 1 / 4 / 12 units gave 2,893 / 2,811 / 2,662 tok/s at ctx 1024, and
// 0 is 0.3 % above 1 -- a hand-off is bound by its detection latency, not by
// the L2 bandwidth the polls take.
#ifndef MK_SPIN_SLEEP
#define MK_SPIN_SLEEP 0
#endif
struct Spin {
  u64 t0 = 0;
  unsigned n = 0;
  __device__ __forceinline__ bool step(int* err, u64 timeout_ticks) {
    if (n == 0) t0 = wall_clock64();
    ++n;
    __builtin_amdgcn_s_sleep(MK_SPIN_SLEEP);
    if ((n & 1023u) == 0) {
      if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != MK_OK) return false;
      if (wall_clock64() - t0 > timeout_ticks) {
        __hip_atomic_store(err, (int)MK_ERR_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
      }
    }
    return true;
  }
};

}  // namespace mk
