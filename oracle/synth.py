"""Counter-based synthetic data generator (numpy restatement, CPU).

TEST INFRASTRUCTURE: the HIP library computes the same values on the device
(``megakernel_synth_fill``); tests check the two are bit-identical.

Definition (identical in both implementations):

  GOLD        = 0x9E3779B97F4A7C15
  mix64(z)    = splitmix64 finaliser (Vigna):
                z ^= z >> 30; z *= 0xBF58476D1CE4E5B9;
                z ^= z >> 27; z *= 0x94D049BB133111EB; z ^= z >> 31
  h(k, i)     = mix64(k + (i + 1) * GOLD)   (the (i+1)-th splitmix64 output
                                             of a generator seeded with k)
  key(seed,t) = h(seed, t)                  one stream per tensor id t
  value(i)    = bf16_rne( float32(S_i - 131070) * c )   [+ 1.0f, see below]
                S_i = sum of the four 16-bit fields of h(key, i)
                c   = float32(std * sqrt(3) / 65536)   (computed in double)

S_i is an Irwin-Hall(4) sum of discrete uniforms, mean 131070 and standard
deviation 65536/sqrt(3), so value(i) ~ approx N(0, std^2) (bounded at
+-3.46 std).  Every step is exact integer arithmetic or one IEEE fp32 operation,
so CPU and GPU produce the same bits.  Norm gains use
``bf16_rne(1.0f + float32(S_i - 131070) * c)`` (two separately rounded fp32
ops, never fused).

Tensor ids follow the reference's flat layout order
(/root/reference/host/weight_loader.py:141-192): 0 = embedding,
1 = final_norm, 2 + 11*layer + j for the j-th per-layer tensor in the order
attn_norm, w_q, w_k, w_v, q_norm, k_norm, w_o, ffn_norm, w_gate, w_up, w_down.
KV prefill uses id KV_ID_BASE + 2*layer + (0 for K, 1 for V) with element
index ((t * n_kv_heads) + g) * head_dim + d, so a position's values do not
depend on how many positions are generated.
"""
from __future__ import annotations

import math

import numpy as np

GOLD = 0x9E3779B97F4A7C15
MASK64 = (1 << 64) - 1
KV_ID_BASE = 0x40000000
PROMPT_ID = 0x7F000000


def mix64_int(z: int) -> int:
    z &= MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def h_int(k: int, i: int) -> int:
    """(i+1)-th output of splitmix64 seeded with k (pure Python ints)."""
    return mix64_int((k + (i + 1) * GOLD) & MASK64)


def stream_key(seed: int, tensor_id: int) -> int:
    return h_int(seed, tensor_id)


def h_vec(key: int, start: int, count: int) -> np.ndarray:
    """h(key, i) for i in [start, start+count) as uint64 (vectorised)."""
    with np.errstate(over="ignore"):
        i = np.arange(start + 1, start + 1 + count, dtype=np.uint64)
        z = np.uint64(key) + i * np.uint64(GOLD)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def scale_const(std: float) -> np.float32:
    return np.float32(std * math.sqrt(3.0) / 65536.0)


def f32_to_bf16_bits(f: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 (inputs here are finite)."""
    b = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32)
    lsb = (b >> np.uint32(16)) & np.uint32(1)
    with np.errstate(over="ignore"):
        r = (b + np.uint32(0x7FFF) + lsb) >> np.uint32(16)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_f32(key: int, start: int, count: int, std: float, add_one: bool = False) -> np.ndarray:
    r = h_vec(key, start, count)
    m = np.uint64(0xFFFF)
    s = (r & m) + ((r >> np.uint64(16)) & m) + ((r >> np.uint64(32)) & m) + (r >> np.uint64(48))
    z = (s.astype(np.int64) - 131070).astype(np.float32)  # exact: |S-131070| < 2^18
    f = z * scale_const(std)                                # one fp32 multiply (RNE)
    if add_one:
        f = np.float32(1.0) + f                             # separately rounded fp32 add
    return f


def normal_bf16_bits(key: int, count: int, std: float, add_one: bool = False,
                     start: int = 0, chunk: int = 1 << 24) -> np.ndarray:
    out = np.empty(count, dtype=np.uint16)
    for s in range(0, count, chunk):
        n = min(chunk, count - s)
        out[s:s + n] = f32_to_bf16_bits(normal_f32(key, start + s, n, std, add_one))
    return out


def prompt_tokens(seed: int, n: int, vocab: int) -> list[int]:
    key = stream_key(seed, PROMPT_ID)
    return [h_int(key, j) % vocab for j in range(n)]


def kv_prefill_bits(seed: int, layer: int, kv: int, n_pos: int, n_kv_heads: int,
                    head_dim: int, std: float = 1.0) -> np.ndarray:
    """Synthetic prefilled K (kv=0) or V (kv=1) for one layer as bf16 bits in
    the canonical [n_kv_heads][n_pos][head_dim] layout."""
    key = stream_key(seed, KV_ID_BASE + 2 * layer + kv)
    flat = normal_bf16_bits(key, n_pos * n_kv_heads * head_dim, std)  # [t][g][d]
    return flat.reshape(n_pos, n_kv_heads, head_dim).transpose(1, 0, 2).copy()
