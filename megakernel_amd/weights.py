"""The flat weight format and the synthetic model of the benchmark configs.

Format: the reference's ``weights.bin`` + ``weights_offsets.json``
(/root/reference/host/weight_loader.py:141-206): bf16 tensors back to back,
keyed ``embedding``, ``final_norm``, ``layer.{i}.{attn_norm,w_q,w_k,w_v,q_norm,
k_norm,w_o,ffn_norm,w_gate,w_up,w_down}``; the C ABI takes the offsets in that
order (/root/reference/host/bridge.py:86-93).

Synthetic weights are produced on the device by the library's counter-based
generator (``megakernel_synth_fill``), so a 972 MB model appears in HBM in
milliseconds with no host staging.  The generator's definition (and a CPU
restatement used by the tests) is documented in include/megakernel.h.
"""
from __future__ import annotations

import ctypes
import json
import math
from dataclasses import dataclass

import numpy as np

from . import _lib
from .config import LAYER_KEYS, ModelShape


@dataclass
class FlatLayout:
    shape: ModelShape
    offsets: dict[str, int]
    total_bytes: int

    def ordered_offsets(self) -> list[int]:
        out = [self.offsets["embedding"], self.offsets["final_norm"]]
        for i in range(self.shape.n_layers):
            out += [self.offsets[f"layer.{i}.{k}"] for k in LAYER_KEYS]
        return out

    def c_offsets(self):
        arr = self.ordered_offsets()
        return (ctypes.c_longlong * len(arr))(*arr)


def tensor_dims(s: ModelShape, key: str) -> tuple[int, ...]:
    q, kv = s.n_q_heads * s.head_dim, s.n_kv_heads * s.head_dim
    return {"embedding": (s.vocab, s.hidden), "final_norm": (s.hidden,),
            "attn_norm": (s.hidden,), "w_q": (q, s.hidden), "w_k": (kv, s.hidden),
            "w_v": (kv, s.hidden), "q_norm": (s.head_dim,), "k_norm": (s.head_dim,),
            "w_o": (s.hidden, q), "ffn_norm": (s.hidden,), "w_gate": (s.ffn, s.hidden),
            "w_up": (s.ffn, s.hidden), "w_down": (s.hidden, s.ffn)}[key]


def names(s: ModelShape) -> list[str]:
    out = ["embedding", "final_norm"]
    for i in range(s.n_layers):
        out += [f"layer.{i}.{k}" for k in LAYER_KEYS]
    return out


def flat_layout(s: ModelShape) -> FlatLayout:
    offs, cur = {}, 0
    for n in names(s):
        offs[n] = cur
        cur += 2 * math.prod(tensor_dims(s, n.split(".")[-1]))
    return FlatLayout(s, offs, cur)


def stream_id(name: str) -> int:
    if name == "embedding":
        return 0
    if name == "final_norm":
        return 1
    _, layer, key = name.split(".")
    return 2 + 11 * int(layer) + LAYER_KEYS.index(key)


def save_flat(path: str, buf: np.ndarray, layout: FlatLayout) -> str:
    """Write weights.bin + weights_offsets.json (reference weight_loader.py:195-206)."""
    buf.tofile(path)
    offs_path = path.replace(".bin", "_offsets.json")
    with open(offs_path, "w") as f:
        json.dump(layout.offsets, f, indent=2)
    return offs_path


def load_offsets(offsets_path: str) -> dict[str, int]:
    with open(offsets_path) as f:
        return {k: int(v) for k, v in json.load(f).items()}


def infer_shape(offs: dict[str, int]) -> ModelShape:
    """The compiled preset (with layer count and vocabulary) whose contiguous
    weights.bin these offsets describe exactly -- the file the reference's
    weight loader writes (/root/reference/host/weight_loader.py:141-192).
    Raises ValueError when no preset matches (the library's megakernel_init
    applies the same rule)."""
    from . import config as _cfg
    n_layers = 0
    while f"layer.{n_layers}.attn_norm" in offs:
        n_layers += 1
    if n_layers == 0 or "embedding" not in offs or "final_norm" not in offs:
        raise ValueError("offsets lack embedding / final_norm / layer tensors")
    for preset in (_cfg.BASELINE, _cfg.QWEN3_06B, _cfg.TINY):
        emb = offs["final_norm"] - offs["embedding"]
        if emb <= 0 or emb % (2 * preset.hidden):
            continue
        cand = preset.with_(n_layers=n_layers, vocab=emb // (2 * preset.hidden))
        if _contiguous(cand, offs):
            return cand
    raise ValueError("offsets do not describe a contiguous weights.bin of a compiled preset "
                     "(BASELINE, QWEN3_06B, TINY); pass shape= explicitly")


def _contiguous(s: ModelShape, offs: dict[str, int]) -> bool:
    order = ordered_from_dict(s, offs)
    want = flat_layout(s).ordered_offsets()
    return all(a - order[0] == b for a, b in zip(order, want))


def ordered_from_dict(s: ModelShape, offs: dict[str, int]) -> list[int]:
    out = [offs["embedding"], offs["final_norm"]]
    for i in range(s.n_layers):
        out += [offs[f"layer.{i}.{k}"] for k in LAYER_KEYS]
    return out


class DeviceWeights:
    """A synthetic flat weight image generated directly in device memory."""

    def __init__(self, shape: ModelShape, seed: int, std: float = 0.02, gain_std: float = 0.0,
                 lib_path: str | None = None):
        self.lib = _lib.load(lib_path)
        self.shape = shape
        self.layout = flat_layout(shape)
        self.ptr = self.lib.megakernel_device_alloc(self.layout.total_bytes)
        if not self.ptr:
            raise _lib.MegakernelError(_lib.last_error(self.lib))
        c_w = float(np.float32(std * math.sqrt(3.0) / 65536.0))
        c_g = float(np.float32(gain_std * math.sqrt(3.0) / 65536.0))
        for n in names(shape):
            key = n.split(".")[-1]
            numel = math.prod(tensor_dims(shape, key))
            sk = self.lib.megakernel_synth_key(seed, stream_id(n))
            is_norm = key.endswith("norm")
            _lib.check(self.lib, self.lib.megakernel_synth_fill(
                ctypes.c_void_p(self.ptr + self.layout.offsets[n]), numel, sk,
                c_g if is_norm else c_w, 1 if is_norm else 0), f"synth_fill {n}")

    def to_host(self) -> np.ndarray:
        buf = np.empty(self.layout.total_bytes, dtype=np.uint8)
        _lib.check(self.lib, self.lib.megakernel_memcpy(
            buf.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(self.ptr), buf.nbytes, _lib.D2H),
            "memcpy D2H")
        return buf

    def free(self) -> None:
        if self.ptr:
            self.lib.megakernel_device_free(ctypes.c_void_p(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ------------------------------------------------------------------ real weights
# HF Qwen3 state-dict key of each flat tensor (reference host/weight_loader.py:62-110).
_HF_KEYS = {
    "attn_norm": "input_layernorm.weight", "w_q": "self_attn.q_proj.weight",
    "w_k": "self_attn.k_proj.weight", "w_v": "self_attn.v_proj.weight",
    "q_norm": "self_attn.q_norm.weight", "k_norm": "self_attn.k_norm.weight",
    "w_o": "self_attn.o_proj.weight", "ffn_norm": "post_attention_layernorm.weight",
    "w_gate": "mlp.gate_proj.weight", "w_up": "mlp.up_proj.weight", "w_down": "mlp.down_proj.weight",
}


def shape_from_hf_config(cfg: dict) -> ModelShape:
    """ModelShape of a Qwen3 config.json (the preset is chosen by head_dim /
    intermediate size; other shapes are rejected by the library at init)."""
    from . import config as _cfg
    hidden, nq, nkv = cfg["hidden_size"], cfg["num_attention_heads"], cfg["num_key_value_heads"]
    d = cfg.get("head_dim", hidden // nq)
    shape = ModelShape(hidden, nq, nkv, d, cfg["intermediate_size"], cfg["num_hidden_layers"],
                       cfg["vocab_size"], _lib.PRESET_BASELINE)
    for preset in (_cfg.BASELINE, _cfg.QWEN3_06B, _cfg.TINY):
        if (preset.hidden, preset.n_q_heads, preset.n_kv_heads, preset.head_dim, preset.ffn) == \
                (hidden, nq, nkv, d, cfg["intermediate_size"]):
            return preset.with_(n_layers=shape.n_layers, vocab=shape.vocab)
    raise ValueError(f"no compiled preset for hidden {hidden}, heads {nq}/{nkv}, head_dim {d}, "
                     f"ffn {cfg['intermediate_size']}")


def flat_from_state(state: dict, shape: ModelShape) -> np.ndarray:
    """The flat bf16 image (uint8 bytes, reference order) of an HF Qwen3 state
    dict of torch tensors.  The tied embedding is the LM head, as in the
    reference kernel; a separate lm_head.weight is ignored."""
    import torch
    layout = flat_layout(shape)
    buf = np.zeros(layout.total_bytes, dtype=np.uint8)

    def put(name: str, key: str):
        t = state[key]
        want = tensor_dims(shape, name.split(".")[-1])
        if tuple(t.shape) != want:
            raise ValueError(f"{key}: shape {tuple(t.shape)}, expected {want}")
        raw = t.detach().to(torch.bfloat16).contiguous().view(torch.int16).cpu().numpy().view(np.uint8).reshape(-1)
        off = layout.offsets[name]
        buf[off:off + raw.size] = raw

    put("embedding", "model.embed_tokens.weight")
    put("final_norm", "model.norm.weight")
    for i in range(shape.n_layers):
        for k, hk in _HF_KEYS.items():
            put(f"layer.{i}.{k}", f"model.layers.{i}.{hk}")
    return buf


def convert_safetensors(model_dir: str, output_path: str) -> tuple[str, ModelShape]:
    """Convert a local HF Qwen3 checkpoint directory (config.json +
    *.safetensors; no download) to weights.bin + weights_offsets.json
    (reference host/weight_loader.py:141-206).  Returns (offsets path, shape)."""
    import glob
    import os

    from safetensors.torch import load_file
    with open(os.path.join(model_dir, "config.json")) as f:
        shape = shape_from_hf_config(json.load(f))
    state = {}
    for fn in sorted(glob.glob(os.path.join(model_dir, "*.safetensors"))):
        state.update(load_file(fn))
    if not state:
        raise FileNotFoundError(f"no .safetensors files in {model_dir}")
    buf = flat_from_state(state, shape)
    return save_flat(output_path, buf, flat_layout(shape)), shape
