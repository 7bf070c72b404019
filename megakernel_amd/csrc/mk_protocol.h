// Tag arithmetic and word encodings of the decode kernel's dataflow.  Plain
// C++ shared by the device code (hipcc) and the CPU model of the protocol
// (tests/protocol/dataflow_model.cpp, g++), so both run the same arithmetic.
//
// A tagged word carries a value and the global number of the phase that
// produced it (tag_base + 5 * layer + phase, the LM head being phase 5 * L of
// a token); a consumer spins on exactly the words it needs until every tag
// equals the producing phase's number.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define MK_HD __host__ __device__ __forceinline__
#else
#define MK_HD inline
#endif

namespace mk {

typedef unsigned long long u64;

constexpr int PHASES_PER_LAYER = 5;  // QKV, attention, O, gate/up, down
constexpr unsigned TAG14 = 0x3FFF;   // argmax words carry a 14-bit tag, never 0

MK_HD unsigned f32_bits(float v) { return __builtin_bit_cast(unsigned, v); }
MK_HD float f32_from(unsigned b) { return __builtin_bit_cast(float, b); }

// Full word: fp32 value in the low half, 32-bit tag in the high half.
MK_HD u64 ll_pack(float v, unsigned tag) { return ((u64)tag << 32) | (u64)f32_bits(v); }
MK_HD unsigned ll_tag(u64 w) { return (unsigned)(w >> 32); }
MK_HD float ll_val(u64 w) { return f32_from((unsigned)w); }

// Packed pair: two values in one word, each rounded to a 19-bit mantissa
// (relative error <= 2^-20) with a 4-bit tag in its low bits, so a large
// vector needs half the words and a reader checks each 32-bit half on its
// own.  The 4-bit tag (1..15, never 0) is the full tag mod 15 + 1: a reader
// can only mistake a stale word for current if the word's last write is a
// multiple of 15 phases older than the awaited one.  The protocol keeps that
// gap below 15 phases for every reader: every word is rewritten at least once
// a layer (5 phases, 6 across a token boundary), every reader of a buffer
// read it in the previous layer or waits first on a phase that did (the LM
// head of a workgroup with no layer role), and the host clears the words (tag
// 0) wherever a reconfiguration could break that.
MK_HD unsigned tag4(unsigned tag) { return tag % 15u + 1u; }
MK_HD unsigned tag14(unsigned tag) { return tag % 16383u + 1u; }
MK_HD unsigned pk_half(float v, unsigned t4) { return ((f32_bits(v) + 8u) & ~15u) | t4; }
MK_HD u64 pk_pack(float a, float b, unsigned t4) { return ((u64)pk_half(b, t4) << 32) | pk_half(a, t4); }
MK_HD bool pk_ready(u64 w, unsigned t4) {
  return ((unsigned)w & 15u) == t4 && ((unsigned)(w >> 32) & 15u) == t4;
}
MK_HD float pk_lo(u64 w) { return f32_from((unsigned)w & ~15u); }
MK_HD float pk_hi(u64 w) { return f32_from((unsigned)(w >> 32) & ~15u); }

}  // namespace mk
