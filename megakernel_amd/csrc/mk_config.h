// Model shape presets and the on-device packed weight layout.
//
// Shapes: the BASELINE preset is the one BASELINE.json quotes (head_dim 64,
// SwiGLU 2816); QWEN3_06B is the reference's src/config.cuh:13-22 (head_dim
// 128, 3072); TINY is a small shape used by fast parity tests.  Layer count,
// vocabulary and KV capacity are runtime values.
#pragma once
#include <stdint.h>

namespace mk {

enum Preset : int { PRESET_BASELINE = 0, PRESET_QWEN3_06B = 1, PRESET_TINY = 2 };

constexpr float kRmsEps = 1e-6f;     // reference src/config.cuh:22
constexpr double kRopeTheta = 1e6;   // reference src/config.cuh:21

template <int H_, int NQ_, int NKV_, int D_, int F_>
struct Shape {
  static constexpr int H = H_, NQ = NQ_, NKV = NKV_, D = D_, F = F_;
  static constexpr int QD = NQ * D;          // q rows / O-proj input width
  static constexpr int KVD = NKV * D;
  static constexpr int QKV = QD + 2 * KVD;   // fused q|k|v rows
  static constexpr int GQA = NQ / NKV;       // q heads per kv head
  // Packed weights are stored as 16-row x 32-column tiles (see below).
  static constexpr int KT_H = H / 32;        // 1 KiB units per 16 rows of a K = H matrix
  static constexpr int KT_Q = QD / 32;       // ... of the O projection (K = QD)
  static constexpr int KT_F = F / 32;        // ... of the down projection (K = F)
  static constexpr int KC_H = H / 256;       // 256-column chunks of a K = H row
  static constexpr int KC_Q = QD / 256;
  static constexpr int KC_F = F / 256;
  static constexpr int RB_QKV = QKV / 16;    // 16-row blocks of the fused QKV
  static constexpr int RB_H = H / 16;        // 16-row blocks of O / down outputs
  static constexpr int RB_F = F / 16;        // 16-row blocks of gate (and of up)
  // Packed per-layer sizes in 16-byte units (one tile = 64 units = 1 KiB).
  static constexpr long long U_QKV = (long long)RB_QKV * KT_H * 64;
  static constexpr long long U_O = (long long)RB_H * KT_Q * 64;
  static constexpr long long U_GU = (long long)RB_F * 2 * KT_H * 64;
  static constexpr long long U_DOWN = (long long)RB_H * KT_F * 64;
  static constexpr long long OFF_QKV = 0;
  static constexpr long long OFF_O = U_QKV;
  static constexpr long long OFF_GU = U_QKV + U_O;
  static constexpr long long OFF_DOWN = U_QKV + U_O + U_GU;
  static constexpr long long U_LAYER = U_QKV + U_O + U_GU + U_DOWN;
  // FP8 layer weights (opt-in): the same blocks with one e4m3 byte per weight
  // (a tile is 512 bytes: the offsets above in 8-byte units), and one fp32
  // power-of-two scale per packed row: QKV rows | O rows | gate/up rows in
  // their interleaved block order | down rows.
  static constexpr int SROW_QKV = 0, SROW_O = QKV, SROW_GU = QKV + H, SROW_DOWN = QKV + H + 2 * F;
  static constexpr int SROWS_LAYER = QKV + 2 * H + 2 * F;
  // Per-layer norm gains, bf16: attn_norm[H] | q_norm[D] | k_norm[D] | ffn_norm[H]
  static constexpr int NORM_ATTN = 0, NORM_Q = H, NORM_K = H + D, NORM_FFN = H + 2 * D;
  static constexpr int NORM_STRIDE = 2 * H + 2 * D;

  static_assert(H % 256 == 0 && QD % 256 == 0 && F % 256 == 0, "K dims must be multiples of 256");
  static_assert(QKV % 16 == 0 && F % 16 == 0 && H % 16 == 0, "row dims must be multiples of 16");
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static_assert(NQ % NKV == 0, "GQA");
};

using ShapeBaseline = Shape<1024, 16, 8, 64, 2816>;
using ShapeQwen3 = Shape<1024, 16, 8, 128, 3072>;
using ShapeTiny = Shape<256, 4, 2, 64, 512>;

// ---------------------------------------------------------------------------
// Packed weight layout ("tile"): a row-major bf16 matrix W[R][K] (R % 16 ==
// 0, K % 32 == 0) is cut into 16-row blocks of 16*K*2 bytes, block rb's bytes
// contiguous, so a workgroup streams one block with wave-wide 1 KiB loads.
// Inside block rb, 1 KiB unit kt holds the 16 x 32 tile at columns 32kt: lane
// l holds W[16rb + (l & 15)][32kt + 8(l >> 4) + e], e = 0..7 -- the A operand
// of v_mfma_f32_16x16x32_bf16.  Layer GEMVs (K % 256 == 0) give wave w of the
// owning workgroup the units w K/256 .. (w + 1) K/256 - 1 (a K slice of all 16
// rows); the LM head's waves reduce whole blocks.
//
// Per layer: fused QKV (q rows, then k rows, then v rows) | O | gate/up with
// blocks interleaved (gate block p at 2p, up block p at 2p+1) | down.
// ---------------------------------------------------------------------------

}  // namespace mk
