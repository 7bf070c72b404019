"""Model shapes and byte accounting of the decode hot path.

Shapes: BASELINE (head_dim 64, SwiGLU 2816) and QWEN3_06B (the
reference's src/config.cuh:13-22: head_dim 128, 3072).  Layer count and vocab
are runtime values of the library; the per-layer dims select a compiled preset.
"""
from __future__ import annotations

from dataclasses import dataclass, replace

from . import _lib

LAYER_KEYS = ("attn_norm", "w_q", "w_k", "w_v", "q_norm", "k_norm",
              "w_o", "ffn_norm", "w_gate", "w_up", "w_down")

HBM_PEAK_GBPS = 8000.0  # MI355X published HBM3E peak
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X published dense bf16 matrix peak


@dataclass(frozen=True)
class ModelShape:
    hidden: int
    n_q_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    n_layers: int
    vocab: int
    preset: int

    def with_(self, **kw) -> "ModelShape":
        return replace(self, **kw)

    # ---- byte accounting (algorithmic bytes: weights once + KV read + KV write per token) ----
    @property
    def layer_weight_bytes(self) -> int:
        q, kv = self.n_q_heads * self.head_dim, self.n_kv_heads * self.head_dim
        mats = (q + 2 * kv) * self.hidden + self.hidden * q + 3 * self.ffn * self.hidden
        norms = 2 * self.hidden + 2 * self.head_dim
        return 2 * (mats + norms)

    @property
    def weight_bytes(self) -> int:
        """Bytes of weights streamed per token: all layers + tied LM head + final norm."""
        return self.n_layers * self.layer_weight_bytes + 2 * self.vocab * self.hidden + 2 * self.hidden

    @property
    def kv_bytes_per_pos(self) -> int:
        return 2 * self.n_layers * self.n_kv_heads * self.head_dim * 2

    def token_bytes(self, pos: int) -> int:
        """Algorithmic HBM bytes of one decode step at position pos: weights,
        KV read for positions 0..pos, KV write of position pos."""
        return self.weight_bytes + self.kv_bytes_per_pos * (pos + 2)

    def token_flops(self, pos: int) -> int:
        q, kv = self.n_q_heads * self.head_dim, self.n_kv_heads * self.head_dim
        macs = self.n_layers * ((q + 2 * kv) * self.hidden + self.hidden * q + 3 * self.ffn * self.hidden)
        macs += self.vocab * self.hidden
        attn = self.n_layers * self.n_q_heads * (pos + 1) * self.head_dim * 2
        return 2 * (macs + attn)


BASELINE = ModelShape(1024, 16, 8, 64, 2816, 28, 151936, _lib.PRESET_BASELINE)
QWEN3_06B = ModelShape(1024, 16, 8, 128, 3072, 28, 151936, _lib.PRESET_QWEN3_06B)
TINY = ModelShape(256, 4, 2, 64, 512, 2, 1024, _lib.PRESET_TINY)
