"""Batched greedy decode of up to 16 independent sequences
over the library's batch handle (``megakernel_batch_*``, ``megakernel_decode_batch``).

The reference decodes one sequence per engine (/root/reference/host/bridge.py:70-261);
``BatchEngine`` is the additive counterpart for several sequences sharing one
weight stream: every step consumes one token per sequence at that sequence's
own position and returns one greedy token per sequence.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .config import BASELINE, ModelShape

# prompt tokens per weight pass of a prefill: 64 column groups of 16
PREFILL_PASS_TOKENS = 1024


class BatchEngine:
    def __init__(self, device_weights, n_seq: int, max_seq: int, shape: ModelShape = BASELINE,
                 lib_path: str | None = None):
        self.shape = shape
        self.n_seq = n_seq
        self.max_seq = max_seq
        self.lib = _lib.load(lib_path)
        arr = device_weights.layout.c_offsets()
        self._handle = self.lib.megakernel_batch_init(
            ctypes.c_void_p(device_weights.ptr), arr, len(arr), shape.preset, shape.vocab, n_seq, max_seq)
        if not self._handle:
            raise _lib.MegakernelError(f"megakernel_batch_init failed: {_lib.last_error(self.lib)}")

    def _ints(self, vals) -> ctypes.Array:
        vals = [int(v) for v in vals]
        if len(vals) != self.n_seq:
            raise ValueError(f"expected {self.n_seq} values, got {len(vals)}")
        return (ctypes.c_int * self.n_seq)(*vals)

    # ------------------------------------------------------------ state
    def positions(self) -> list[int]:
        out = (ctypes.c_int * self.n_seq)()
        _lib.check(self.lib, self.lib.megakernel_batch_get_pos(self._handle, out), "batch_get_pos")
        return list(out)

    def set_pos(self, seq: int, pos: int):
        _lib.check(self.lib, self.lib.megakernel_batch_set_pos(self._handle, seq, pos), "batch_set_pos")

    def set_kv_fp8(self, enable: bool = True):
        """FP8 (e4m3, power-of-two row scales) KV caches for every sequence;
        the caches are emptied and every position reset to 0."""
        _lib.check(self.lib, self.lib.megakernel_batch_set_kv_fp8(self._handle, int(bool(enable))), "batch_set_kv_fp8")

    def set_lmhead_fp8(self, enable: bool = True):
        """Stream the FP8 (e4m3, power-of-two row scales) copy of the LM head."""
        _lib.check(self.lib, self.lib.megakernel_batch_set_lmhead_fp8(self._handle, int(bool(enable))),
                   "batch_set_lmhead_fp8")

    def set_step_kernel(self, variant: int):
        """_lib.BATCH_STEP_PER_PHASE (one kernel per phase and layer, the
        default) or _lib.BATCH_STEP_PERSISTENT (every layer in one persistent
        kernel); identical results."""
        _lib.check(self.lib, self.lib.megakernel_batch_set_step_kernel(self._handle, int(variant)),
                   "batch_set_step_kernel")

    TRACE_EVENTS = ("start", "qkv_in", "qkv_done", "att_in", "att_done", "o_in", "o_done", "gu_in", "gu_done",
                    "down_in", "down_done")

    def trace_step(self, tokens, max_workgroups: int = 1024) -> np.ndarray:
        """One persistent step with device wall-clock stamps (100 MHz):
        uint64 [layers][len(TRACE_EVENTS)][workgroups], 0 where a workgroup
        has no role in a phase."""
        n = self.shape.n_layers * len(self.TRACE_EVENTS) * max_workgroups
        buf = (ctypes.c_ulonglong * n)()
        g = _lib.check(self.lib, self.lib.megakernel_batch_trace_step(self._handle, self._ints(tokens), buf, n),
                       "batch_trace_step")
        a = np.frombuffer(buf, dtype=np.uint64)[: self.shape.n_layers * len(self.TRACE_EVENTS) * g]
        return a.reshape(self.shape.n_layers, len(self.TRACE_EVENTS), g).copy()

    def fill_kv_synthetic(self, seq: int, length: int, seed: int, std: float = 1.0):
        _lib.check(self.lib, self.lib.megakernel_batch_fill_kv_synthetic(self._handle, seq, length, seed, std),
                   "batch_fill_kv_synthetic")

    def set_kv(self, seq: int, kv_bits: np.ndarray):
        """kv_bits: uint16 [L][2][NKV][len][D] (bf16 bits), the single-sequence set_kv layout."""
        kv_bits = np.ascontiguousarray(kv_bits, dtype=np.uint16)
        _lib.check(self.lib, self.lib.megakernel_batch_set_kv(
            self._handle, seq, kv_bits.ctypes.data_as(ctypes.c_void_p), kv_bits.shape[3]), "batch_set_kv")

    def get_kv(self, seq: int, length: int) -> np.ndarray:
        s = self.shape
        out = np.empty((s.n_layers, 2, s.n_kv_heads, length, s.head_dim), dtype=np.uint16)
        _lib.check(self.lib, self.lib.megakernel_batch_get_kv(
            self._handle, seq, out.ctypes.data_as(ctypes.c_void_p), length), "batch_get_kv")
        return out

    # ------------------------------------------------------------ decode
    def decode(self, tokens) -> list[int]:
        """One greedy step of every sequence."""
        out = (ctypes.c_int * self.n_seq)()
        _lib.check(self.lib, self.lib.megakernel_decode_batch(self._handle, self._ints(tokens), out),
                   "decode_batch")
        return list(out)

    def generate(self, first_tokens, n_steps: int) -> np.ndarray:
        """n_steps greedy steps; returns int32 [n_steps][n_seq]."""
        out = (ctypes.c_int * (n_steps * self.n_seq))()
        _lib.check(self.lib, self.lib.megakernel_generate_batch(self._handle, self._ints(first_tokens), n_steps, out),
                   "generate_batch")
        return np.frombuffer(out, dtype=np.int32).reshape(n_steps, self.n_seq).copy()

    def debug_logits(self, tokens):
        """One step returning (next tokens, fp32 logits [n_seq][vocab])."""
        out = (ctypes.c_int * self.n_seq)()
        logits = np.empty((self.n_seq, self.shape.vocab), dtype=np.float32)
        _lib.check(self.lib, self.lib.megakernel_batch_debug_logits(
            self._handle, self._ints(tokens), out, logits.ctypes.data_as(_lib.P_float)), "batch_debug_logits")
        return list(out), logits

    def prefill(self, seq: int, tokens, with_logits: bool = False):
        """Consume a prompt for sequence seq at its position (passes of
        PREFILL_PASS_TOKENS tokens, one weight pass each); returns the greedy
        next token, and its fp32 logits [vocab] when with_logits."""
        toks = [int(t) for t in tokens]
        arr = (ctypes.c_int * max(1, len(toks)))(*toks)
        nxt = ctypes.c_int(-1)
        logits = np.empty(self.shape.vocab, dtype=np.float32) if with_logits else None
        _lib.check(self.lib, self.lib.megakernel_batch_prefill(
            self._handle, seq, arr, len(toks), ctypes.byref(nxt),
            logits.ctypes.data_as(_lib.P_float) if with_logits else None), "batch_prefill")
        return (nxt.value, logits) if with_logits else nxt.value

    @property
    def last_ms(self) -> float:
        return float(self.lib.megakernel_batch_last_ms(self._handle))

    def close(self):
        if getattr(self, "_handle", None):
            self.lib.megakernel_batch_free(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
