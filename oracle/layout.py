"""The reference's flat weight-file layout, restated for the oracle.

TEST INFRASTRUCTURE.  Follows /root/reference/host/weight_loader.py:141-192
(``save_flat_binary``: embedding, final_norm, then per layer the 11 tensors in
the order below, all bf16 row-major [out, in]) and the 310-entry offset array
order built by /root/reference/host/bridge.py:86-93 and consumed by
/root/reference/src/megakernel.cu:551-570.

Shapes follow /root/reference/src/config.cuh:115-134 with ``w_o`` stored as
[hidden, q_dim] (the reference's ``validate_shapes`` at weight_loader.py:128
has that one transposed; the kernel and HF both use [hidden, q_dim]).
"""
from __future__ import annotations

from dataclasses import dataclass

LAYER_KEYS = ("attn_norm", "w_q", "w_k", "w_v", "q_norm", "k_norm",
              "w_o", "ffn_norm", "w_gate", "w_up", "w_down")

MATRIX_KEYS = ("w_q", "w_k", "w_v", "w_o", "w_gate", "w_up", "w_down")


@dataclass(frozen=True)
class Shape:
    hidden: int
    n_q_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    n_layers: int
    vocab: int
    eps: float = 1e-6
    theta: float = 1e6

    @property
    def q_dim(self) -> int:
        return self.n_q_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim


# BASELINE.json shapes (head_dim 64, SwiGLU 2816) and the reference's
# config.cuh shapes (head_dim 128, 3072).
BASELINE = Shape(1024, 16, 8, 64, 2816, 28, 151936)
QWEN3_06B = Shape(1024, 16, 8, 128, 3072, 28, 151936)


def tensor_shape(s: Shape, key: str) -> tuple[int, ...]:
    return {
        "embedding": (s.vocab, s.hidden),
        "final_norm": (s.hidden,),
        "attn_norm": (s.hidden,),
        "w_q": (s.q_dim, s.hidden),
        "w_k": (s.kv_dim, s.hidden),
        "w_v": (s.kv_dim, s.hidden),
        "q_norm": (s.head_dim,),
        "k_norm": (s.head_dim,),
        "w_o": (s.hidden, s.q_dim),
        "ffn_norm": (s.hidden,),
        "w_gate": (s.ffn, s.hidden),
        "w_up": (s.ffn, s.hidden),
        "w_down": (s.hidden, s.ffn),
    }[key]


def ordered_names(s: Shape) -> list[str]:
    names = ["embedding", "final_norm"]
    for i in range(s.n_layers):
        names += [f"layer.{i}.{k}" for k in LAYER_KEYS]
    return names


def base_key(name: str) -> str:
    return name.split(".")[-1]


def offsets(s: Shape) -> dict[str, int]:
    """Byte offsets of the packed file, in file order (no padding)."""
    out, cur = {}, 0
    for n in ordered_names(s):
        out[n] = cur
        numel = 1
        for d in tensor_shape(s, base_key(n)):
            numel *= d
        cur += 2 * numel
    out["__total__"] = cur
    return out


def tensor_id(name: str) -> int:
    """Synthetic-stream id of a tensor (its index in the reference order)."""
    if name == "embedding":
        return 0
    if name == "final_norm":
        return 1
    _, layer, key = name.split(".")
    return 2 + 11 * int(layer) + LAYER_KEYS.index(key)
