"""fp32-activation PyTorch oracle of one Qwen3 decode step (CPU).

TEST INFRASTRUCTURE.  Restates the reference kernel's per-token computation
(/root/reference/src/megakernel.cu:132-332) with the numerics policy the
reference documents (megakernel.cu:17-37, gemv.cuh:17,30-32, kv_cache.cuh:72,76):
bf16 weights, fp32 activations, fp32 accumulation, fp32 residual stream, K/V
stored in the cache as bf16 after QK-norm + RoPE, fp32 softmax.  The reference
kernel's data races (every block re-adding the residual, megakernel.cu:243-245,
288-290; the never re-armed KV flag, barriers.cuh:112-134) are NOT reproduced:
this is the mathematical forward.

Op-by-op sources:
  rmsnorm        rmsnorm.cuh:87-108   y = x * rsqrt(mean(x^2) + eps) * w
  qk_norm        rmsnorm.cuh:57-84    per-head rmsnorm over head_dim
  rope           attention.cuh:22-44  rotate-half pairs (i, i+D/2); angles as HF
                                      computes them (fp32 inv_freq * fp32 pos)
  kv append      kv_cache.cuh:58-78   bf16(k), bf16(v) at position pos
  attention      attention.cuh:100-167 GQA (kv head = q head // (NQ/NKV)),
                                      scale 1/sqrt(D), seq_len = pos + 1
  silu * up      gemv.cuh:212-279, utils.cuh:59-61
  lm head argmax sampling.cuh:32-117  tied embedding; lowest index wins ties
                                      (torch.argmax semantics; the reference
                                      leaves ties unspecified)
"""
from __future__ import annotations

import numpy as np
import torch

from . import layout, synth
from .layout import Shape


# ---------------------------------------------------------------- single ops
def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    x = x.float()
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w.float()


def inv_freq(head_dim: int, theta: float) -> torch.Tensor:
    """HF Qwen3RotaryEmbedding.compute_default_rope_parameters (fp32)."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))


def rope_cos_sin(pos: int, head_dim: int, theta: float):
    freqs = inv_freq(head_dim, theta) * torch.tensor(float(pos), dtype=torch.float32)
    emb = torch.cat((freqs, freqs))
    return emb.cos(), emb.sin()


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def rope(x: torch.Tensor, pos: int, theta: float) -> torch.Tensor:
    """x: [..., D] fp32."""
    cos, sin = rope_cos_sin(pos, x.shape[-1], theta)
    return x * cos + rotate_half(x) * sin


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """q: [NQ, D] fp32; k, v: [NKV, S, D] fp32.  Returns [NQ, D]."""
    nq, d = q.shape
    rep = nq // k.shape[0]
    kk = k.repeat_interleave(rep, dim=0)
    vv = v.repeat_interleave(rep, dim=0)
    scores = torch.einsum("hd,hsd->hs", q, kk) * (1.0 / float(np.sqrt(d)))
    p = torch.softmax(scores, dim=-1, dtype=torch.float32)
    return torch.einsum("hs,hsd->hd", p, vv)


def silu_mul(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    return torch.nn.functional.silu(g) * u


def bf16_round(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).float()


def argmax_first(logits: torch.Tensor) -> int:
    return int(torch.argmax(logits).item())


# ------------------------------------------------------------ model weights
def synthetic_bits(shape: Shape, seed: int, std: float = 0.02,
                   gain_std: float = 0.0) -> dict[str, np.ndarray]:
    """All tensors of the model as bf16 bit arrays (uint16), by name."""
    out = {}
    for name in layout.ordered_names(shape):
        key = layout.base_key(name)
        dims = layout.tensor_shape(shape, key)
        n = int(np.prod(dims))
        sk = synth.stream_key(seed, layout.tensor_id(name))
        if key.endswith("norm"):
            bits = synth.normal_bf16_bits(sk, n, gain_std, add_one=True)
        else:
            bits = synth.normal_bf16_bits(sk, n, std)
        out[name] = bits.reshape(dims)
    return out


def pack_flat(shape: Shape, bits: dict[str, np.ndarray]) -> tuple[np.ndarray, dict[str, int]]:
    """Flat weights.bin image (uint8) and its offsets, reference order."""
    offs = layout.offsets(shape)
    buf = np.empty(offs["__total__"], dtype=np.uint8)
    for name in layout.ordered_names(shape):
        b = np.ascontiguousarray(bits[name]).view(np.uint8).reshape(-1)
        buf[offs[name]:offs[name] + b.size] = b
    return buf, {k: v for k, v in offs.items() if k != "__total__"}


def unpack_flat(shape: Shape, buf: np.ndarray, offs: dict[str, int]) -> dict[str, np.ndarray]:
    out = {}
    for name in layout.ordered_names(shape):
        dims = layout.tensor_shape(shape, layout.base_key(name))
        n = int(np.prod(dims))
        o = offs[name]
        out[name] = buf[o:o + 2 * n].view(np.uint16).reshape(dims)
    return out


def bits_to_torch(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


# -------------------------------------------------------------- the forward
class Qwen3Oracle:
    """One-token-at-a-time greedy decode with a bf16 KV cache.

    ``step(token)`` consumes ``token`` at position ``self.pos`` and returns the
    next token (argmax of fp32 logits); ``pos`` advances by one, mirroring
    ``megakernel_decode`` (/root/reference/src/megakernel.cu:377-413).
    """

    def __init__(self, shape: Shape, bits: dict[str, np.ndarray], max_seq: int,
                 matmul_dtype: torch.dtype = torch.float32,
                 kv_dtype: torch.dtype = torch.bfloat16, kv_fp8: bool = False):
        self.s = shape
        self.max_seq = max_seq
        f = lambda n: bits_to_torch(bits[n]).to(matmul_dtype)  # noqa: E731
        g = lambda n: bits_to_torch(bits[n]).float()           # noqa: E731
        self.embed = f("embedding")
        self.lm_head = self.embed  # tied; use_fp8_lm_head() swaps in the FP8 copy
        self.final_norm = g("final_norm")
        self.layers = []
        for i in range(shape.n_layers):
            p = f"layer.{i}."
            self.layers.append(dict(
                attn_norm=g(p + "attn_norm"), q_norm=g(p + "q_norm"), k_norm=g(p + "k_norm"),
                ffn_norm=g(p + "ffn_norm"),
                w_q=f(p + "w_q"), w_k=f(p + "w_k"), w_v=f(p + "w_v"), w_o=f(p + "w_o"),
                w_gate=f(p + "w_gate"), w_up=f(p + "w_up"), w_down=f(p + "w_down")))
        # kv_dtype=bfloat16 is the reference policy; float32 exists only to
        # compare with an fp32-cache forward (the HF golden fixtures).
        # kv_fp8: the cache holds the exact dequantised FP8 rows (oracle/fp8.py,
        # one power-of-two scale per (layer, kv head, position) row of K and V).
        self.kv_fp8 = kv_fp8
        self.k_cache = torch.zeros(shape.n_layers, shape.n_kv_heads, max_seq, shape.head_dim,
                                   dtype=torch.float32 if kv_fp8 else kv_dtype)
        self.v_cache = torch.zeros_like(self.k_cache)
        self.pos = 0

    def use_fp8_lm_head(self) -> tuple[np.ndarray, np.ndarray]:
        """Logits from the FP8 (e4m3, power-of-two row scales) copy of the tied
        table, dequantised exactly (oracle/fp8.py); the embedding gather keeps
        the bf16 table.  Returns (codes, scales)."""
        from . import fp8
        codes, scales = fp8.quantize_rows(self.embed.float().numpy())
        self.lm_head = torch.from_numpy(fp8.dequantize_rows(codes, scales)).to(self.embed.dtype)
        return codes, scales

    def use_fp8_layers(self) -> list[dict[str, tuple[np.ndarray, np.ndarray]]]:
        """Every layer matrix replaced by its FP8 copy (e4m3, power-of-two row
        scales, oracle/fp8.py), dequantised exactly; norm gains stay.  Returns
        per layer {name: (codes, scales)} with "qkv" the fused q | k | v rows."""
        from . import fp8
        out = []
        for w in self.layers:
            d = {}
            for n in ("w_q", "w_k", "w_v", "w_o", "w_gate", "w_up", "w_down"):
                codes, scales = fp8.quantize_rows(w[n].float().numpy())
                w[n] = torch.from_numpy(fp8.dequantize_rows(codes, scales)).to(w[n].dtype)
                d[n[2:]] = (codes, scales)
            d["qkv"] = tuple(np.concatenate([d[k][i] for k in ("q", "k", "v")]) for i in range(2))
            out.append(d)
        return out

    def reset(self) -> None:
        self.k_cache.zero_()
        self.v_cache.zero_()
        self.pos = 0

    def set_kv(self, k_bits: np.ndarray, v_bits: np.ndarray) -> None:
        """k_bits, v_bits: bf16 bits [L][NKV][len][D] (canonical layout)."""
        n = k_bits.shape[2]
        self.k_cache[:, :, :n] = self._kv_rows(bits_to_torch(k_bits).float())
        self.v_cache[:, :, :n] = self._kv_rows(bits_to_torch(v_bits).float())
        self.pos = n

    def _kv_rows(self, t: torch.Tensor) -> torch.Tensor:
        """What the cache stores of K / V rows t[..., D]: the values (cast to
        the cache dtype), or with kv_fp8 the dequantised e4m3 rows."""
        if not self.kv_fp8:
            return t.to(self.k_cache.dtype)
        from . import fp8
        rows = t.reshape(-1, t.shape[-1]).numpy()
        return torch.from_numpy(fp8.dequantize_rows(*fp8.quantize_rows(rows))).reshape(t.shape)

    @staticmethod
    def _mv(w: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        return (w @ x.to(w.dtype)).float()

    @torch.no_grad()
    def step(self, token: int, capture: bool = False) -> dict:
        s, pos = self.s, self.pos
        if pos >= self.max_seq:
            raise ValueError("KV cache full")
        D = s.head_dim
        x = self.embed[token].float()
        layers_out = [x.clone()] if capture else None
        for li, w in enumerate(self.layers):
            h = rmsnorm(x, w["attn_norm"], s.eps)
            q = self._mv(w["w_q"], h).view(s.n_q_heads, D)
            k = self._mv(w["w_k"], h).view(s.n_kv_heads, D)
            v = self._mv(w["w_v"], h).view(s.n_kv_heads, D)
            q = rmsnorm(q, w["q_norm"], s.eps)
            k = rmsnorm(k, w["k_norm"], s.eps)
            q = rope(q, pos, s.theta)
            k = rope(k, pos, s.theta)
            self.k_cache[li, :, pos] = self._kv_rows(k)
            self.v_cache[li, :, pos] = self._kv_rows(v)
            kc = self.k_cache[li, :, :pos + 1].float()
            vc = self.v_cache[li, :, :pos + 1].float()
            o = attention(q, kc, vc).reshape(-1)
            x = x + self._mv(w["w_o"], o)
            h2 = rmsnorm(x, w["ffn_norm"], s.eps)
            a = silu_mul(self._mv(w["w_gate"], h2), self._mv(w["w_up"], h2))
            x = x + self._mv(w["w_down"], a)
            if capture:
                layers_out.append(x.clone())
        hf = rmsnorm(x, self.final_norm, s.eps)
        logits = self._mv(self.lm_head, hf)
        nxt = argmax_first(logits)
        self.pos += 1
        out = {"token": nxt}
        if capture:
            out["logits"] = logits
            out["layers"] = torch.stack(layers_out)
        return out

    def generate(self, first_token: int, n: int) -> list[int]:
        toks, t = [], first_token
        for _ in range(n):
            t = self.step(t)["token"]
            toks.append(t)
        return toks


def top2_margin(logits: torch.Tensor) -> float:
    v = torch.topk(logits, 2).values
    return float(v[0] - v[1])
