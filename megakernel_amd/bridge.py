"""Python bridge: ``MegakernelEngine`` over megakernel.so via ctypes.

Mirrors /root/reference/host/bridge.py (same class name, constructor
arguments and methods: reset, decode_token, generate, benchmark,
benchmark_sweep, close) with three deliberate differences:

* no torch in the product path: weights are read with numpy and uploaded by
  the library (``megakernel_init_from_host``);
* ``generate`` prefills the prompt once (the reference prefills it twice,
  bridge.py:136-163) -- with ``prefill=True``, up to 1,024 prompt tokens per
  weight pass on the matrix cores instead of one decode step per token -- and can
  decode all new tokens in one resident launch;
* throughput accounting counts KV bytes as well as weight bytes, from the
  model shape instead of a fixed 926e6 constant (bridge.py:229).

Errors raise ``MegakernelError`` with the library's message.
"""
from __future__ import annotations

import ctypes
import time

import numpy as np

from . import _lib
from .config import HBM_PEAK_GBPS, ModelShape
from .weights import infer_shape, load_offsets, ordered_from_dict


class MegakernelEngine:
    """Python wrapper around the megakernel shared library."""

    def __init__(self, weights_path=None, offsets_path=None, lib_path=None, tokenizer=None,
                 shape: ModelShape | None = None, max_seq: int | None = None,
                 device_weights=None, prefill: bool = False):
        self.tokenizer = tokenizer
        # shape: given, that of device_weights, or inferred from the offsets
        # file (the reference's bridge passes no shape)
        if shape is None and device_weights is not None:
            shape = device_weights.shape
        self.shape = shape
        self.lib = _lib.load(lib_path)
        self.max_seq = max_seq or 33024
        self._prefill = False
        if device_weights is not None:
            self._init_from_device(device_weights)
        else:
            self._load_weights(weights_path, offsets_path)
        if prefill:
            self.attach_prefill(device_weights)

    # ------------------------------------------------------------ set-up
    def _load_weights(self, weights_path, offsets_path):
        offs = load_offsets(offsets_path)
        if self.shape is None:
            try:
                self.shape = infer_shape(offs)
            except ValueError as e:
                raise _lib.MegakernelError(str(e)) from None
        order = ordered_from_dict(self.shape, offs)
        data = np.fromfile(weights_path, dtype=np.uint8)
        arr = (ctypes.c_longlong * len(order))(*order)
        self._handle = self.lib.megakernel_init_from_host(
            data.ctypes.data_as(ctypes.c_void_p), data.nbytes, arr, len(order),
            self.shape.preset, self.shape.vocab, self.max_seq)
        if not self._handle:
            raise _lib.MegakernelError(f"megakernel_init failed: {_lib.last_error(self.lib)}")

    def _init_from_device(self, dw):
        arr = dw.layout.c_offsets()
        self._handle = self.lib.megakernel_init_ex(
            ctypes.c_void_p(dw.ptr), arr, len(arr), self.shape.preset, self.shape.vocab, self.max_seq)
        if not self._handle:
            raise _lib.MegakernelError(f"megakernel_init failed: {_lib.last_error(self.lib)}")

    # ---------------------------------------------------- reference methods
    def reset(self):
        """Reset KV cache and position for a new generation."""
        self.lib.megakernel_reset(self._handle)

    def decode_token(self, token_id):
        """Run one forward pass: input token -> next token."""
        return _lib.check(self.lib, self.lib.megakernel_decode(self._handle, int(token_id)), "decode")

    @property
    def pos(self) -> int:
        return self.lib.megakernel_get_pos(self._handle)

    def decode_many(self, first_token: int, n: int) -> list[int]:
        """n greedy steps in one resident launch (megakernel_generate)."""
        out = (ctypes.c_int * n)()
        _lib.check(self.lib, self.lib.megakernel_generate(self._handle, int(first_token), n, out), "generate")
        return list(out)

    def attach_prefill(self, device_weights=None):
        """Build the prefill context (matrix-core weight copy bound to this
        handle's KV cache): from device_weights, or from the library's own
        upload when the engine was loaded from a weights file."""
        if self._prefill:
            return
        if device_weights is not None:
            arr = device_weights.layout.c_offsets()
            rc = self.lib.megakernel_prefill_attach(self._handle, ctypes.c_void_p(device_weights.ptr), arr, len(arr))
        else:
            rc = self.lib.megakernel_prefill_attach(self._handle, None, None, 0)
        _lib.check(self.lib, rc, "prefill_attach")
        self._prefill = True

    def prefill(self, token_ids) -> int:
        """Consume prompt tokens at the current position, up to 1,024 per
        weight pass; returns the greedy next token."""
        ids = [int(t) for t in token_ids]
        arr = (ctypes.c_int * max(1, len(ids)))(*ids)
        nxt = ctypes.c_int(-1)
        _lib.check(self.lib, self.lib.megakernel_prefill(self._handle, arr, len(ids), ctypes.byref(nxt)), "prefill")
        return nxt.value

    def generate_ids(self, prompt_ids, max_tokens=100, eos_id=None, one_launch=True, on_token=None):
        """Greedy continuation of token ids (reference host/bridge.py:118-192):
        the prompt is consumed (with the prefill context in one call, else
        token by token), then up to max_tokens tokens are generated, the EOS
        token included when it comes.  on_token(id) is called for each
        generated token as it is produced (token by token then).  Returns
        (generated_ids, tok/s of the generation loop)."""
        if not prompt_ids:
            raise ValueError("empty prompt")
        self.reset()
        if self._prefill:
            nxt = self.prefill(prompt_ids)
        else:
            for tok in prompt_ids[:-1]:
                self.decode_token(tok)
            nxt = self.decode_token(prompt_ids[-1])
        self.lib.megakernel_sync()
        start = time.perf_counter()
        generated = [nxt]
        if on_token is not None:
            on_token(nxt)
        if one_launch and eos_id is None and on_token is None and max_tokens > 1:
            generated += self.decode_many(nxt, max_tokens - 1)
        else:
            while len(generated) < max_tokens and nxt != eos_id:
                nxt = self.decode_token(nxt)
                generated.append(nxt)
                if on_token is not None:
                    on_token(nxt)
        self.lib.megakernel_sync()
        elapsed = time.perf_counter() - start
        if eos_id is not None and eos_id in generated:
            generated = generated[:generated.index(eos_id) + 1]
        return generated, (len(generated) - 1) / elapsed if elapsed > 0 and len(generated) > 1 else 0.0

    def generate(self, prompt, max_tokens=100, print_stream=False):
        """Generate text from a prompt (reference host/bridge.py:118-192): encode,
        consume the prompt, greedy decode until EOS or max_tokens (the EOS token
        included), print each token as it comes when print_stream.  Returns
        (prompt + generated text with special tokens skipped, tok/s).  Needs a
        tokenizer (``megakernel_amd.tokenizer``: a local checkpoint's
        tokenizer.json, or ByteTokenizer for synthetic models)."""
        if self.tokenizer is None:
            raise ValueError("generate(prompt) needs a tokenizer; use generate_ids for token ids")
        ids = list(self.tokenizer.encode(prompt))
        eos = getattr(self.tokenizer, "eos_token_id", None)
        stream = (lambda t: print(self.tokenizer.decode([t]), end="", flush=True)) if print_stream else None
        gen, tps = self.generate_ids(ids, max_tokens, eos_id=eos, one_launch=eos is None, on_token=stream)
        if print_stream:
            print()
        return self.tokenizer.decode(ids + gen, skip_special_tokens=True), tps

    def benchmark(self, num_tokens=50, prompt_token=1):
        """Raw per-call decode throughput (one launch + host sync per token)."""
        self.reset()
        token = prompt_token
        for _ in range(5):
            token = self.decode_token(token)
        self.reset()
        self.lib.megakernel_sync()
        token = prompt_token
        start = time.perf_counter()
        for _ in range(num_tokens):
            token = self.decode_token(token)
        self.lib.megakernel_sync()
        return num_tokens / (time.perf_counter() - start)

    def benchmark_sweep(self, positions=None, bench_tokens=20, seed=1):
        """Throughput at several context positions (KV prefilled synthetically
        instead of decoding pos tokens one by one).  Returns a list of dicts."""
        positions = positions or [1, 10, 50, 100, 500, 1000, 2000]
        results = []
        for pos in positions:
            self.fill_kv_synthetic(pos, seed)
            self.decode_many(1, bench_tokens)  # warm-up at this position
            self.fill_kv_synthetic(pos, seed)
            ms = self.timed_generate(1, bench_tokens)
            tps = bench_tokens / (ms / 1e3)
            nbytes = sum(self.shape.token_bytes(pos + i) for i in range(bench_tokens))
            gbps = nbytes / (ms / 1e3) / 1e9
            results.append({"position": pos, "tok_per_sec": tps, "latency_us": ms * 1e3 / bench_tokens,
                            "bw_gbps": gbps, "bw_util": gbps / HBM_PEAK_GBPS})
        return results

    # --------------------------------------------------------- extensions
    def timed_generate(self, first_token: int, n: int) -> float:
        """Decode n tokens in one launch; returns the kernel's device time (ms)."""
        self.decode_many(first_token, n)
        return float(self.lib.megakernel_last_kernel_ms(self._handle))

    def fill_kv_synthetic(self, length: int, seed: int, std: float = 1.0):
        _lib.check(self.lib, self.lib.megakernel_fill_kv_synthetic(self._handle, length, seed, std),
                   "fill_kv_synthetic")

    def set_kv(self, kv_bits: np.ndarray):
        """kv_bits: uint16 [L][2][NKV][len][D] (bf16 bits)."""
        kv_bits = np.ascontiguousarray(kv_bits, dtype=np.uint16)
        _lib.check(self.lib, self.lib.megakernel_set_kv(
            self._handle, kv_bits.ctypes.data_as(ctypes.c_void_p), kv_bits.shape[3]), "set_kv")

    def get_kv(self, length: int) -> np.ndarray:
        s = self.shape
        out = np.empty((s.n_layers, 2, s.n_kv_heads, length, s.head_dim), dtype=np.uint16)
        _lib.check(self.lib, self.lib.megakernel_get_kv(
            self._handle, out.ctypes.data_as(ctypes.c_void_p), length), "get_kv")
        return out

    def set_pos(self, pos: int):
        _lib.check(self.lib, self.lib.megakernel_set_pos(self._handle, pos), "set_pos")

    def debug_forward(self, token: int):
        """One step returning (next_token, layers[(L+1), H], logits[V])."""
        s = self.shape
        layers = np.empty((s.n_layers + 1, s.hidden), dtype=np.float32)
        logits = np.empty(s.vocab, dtype=np.float32)
        nxt = self.lib.megakernel_debug_forward(
            self._handle, int(token), layers.ctypes.data_as(_lib.P_float),
            logits.ctypes.data_as(_lib.P_float))
        _lib.check(self.lib, nxt, "debug_forward")
        return nxt, layers, logits

    def set_attention_chunk(self, chunk_min: int):
        _lib.check(self.lib, self.lib.megakernel_set_attention_chunk(self._handle, chunk_min),
                   "set_attention_chunk")

    def set_attention_merge(self, merge_min: int):
        """Above merge_min splits per kv head the first split's workgroup merges them (default 20)."""
        _lib.check(self.lib, self.lib.megakernel_set_attention_merge(self._handle, merge_min),
                   "set_attention_merge")

    def set_decode_kernel(self, variant: int):
        """_lib.KERNEL_AUTO (class-specialised kernel where it applies) or
        _lib.KERNEL_SPREAD (always the spread kernel)."""
        _lib.check(self.lib, self.lib.megakernel_set_decode_kernel(self._handle, int(variant)), "set_decode_kernel")

    def decode_kernel_for(self, n_tokens: int) -> int:
        """The kernel (_lib.KERNEL_CLASS or _lib.KERNEL_SPREAD) a launch of
        n_tokens from the current position uses."""
        return _lib.check(self.lib, self.lib.megakernel_decode_kernel_for(self._handle, int(n_tokens)),
                          "decode_kernel_for")

    def set_lmhead_fp8(self, enable=True):
        """LM head mode: False / _lib.LMHEAD_BF16, True / _lib.LMHEAD_FP8 (stream
        the FP8 copy: OCP e4m3, power-of-two row scales), or
        _lib.LMHEAD_SCREENED (the FP8 copy screens the rows, the possible
        argmax rows are scored again in bf16: the bf16 head's tokens)."""
        mode = int(enable) if not isinstance(enable, bool) else (_lib.LMHEAD_FP8 if enable else _lib.LMHEAD_BF16)
        _lib.check(self.lib, self.lib.megakernel_set_lmhead_fp8(self._handle, mode), "set_lmhead_fp8")

    def set_kv_fp8(self, enable: bool = True):
        """Switch the KV cache to FP8 (OCP e4m3, power-of-two scale per row of
        K and V); the cache is emptied and the position reset."""
        _lib.check(self.lib, self.lib.megakernel_set_kv_fp8(self._handle, int(bool(enable))), "set_kv_fp8")

    def lmhead_fp8(self):
        """(codes uint8 [V, H], scales float32 [V]) of the FP8 LM head."""
        s = self.shape
        codes = np.empty((s.vocab, s.hidden), dtype=np.uint8)
        scales = np.empty(s.vocab, dtype=np.float32)
        _lib.check(self.lib, self.lib.megakernel_get_lmhead_fp8(
            self._handle, codes.ctypes.data_as(ctypes.c_void_p),
            scales.ctypes.data_as(ctypes.POINTER(ctypes.c_float))), "get_lmhead_fp8")
        return codes, scales

    def set_layer_fp8(self, enable: bool = True):
        """Stream FP8 (OCP e4m3, power-of-two row scales) copies of the layer
        matrices (class-specialised kernel only)."""
        _lib.check(self.lib, self.lib.megakernel_set_layer_fp8(self._handle, int(bool(enable))), "set_layer_fp8")

    LAYER_MATRICES = ("qkv", "o", "gate", "up", "down")

    def layer_fp8(self, layer: int, which: str):
        """(codes uint8 [R, K], scales float32 [R]) of FP8 layer matrix `which`
        (one of LAYER_MATRICES; "qkv" is the fused q | k | v rows)."""
        s = self.shape
        q, kv = s.n_q_heads * s.head_dim, s.n_kv_heads * s.head_dim
        rk = {"qkv": (q + 2 * kv, s.hidden), "o": (s.hidden, q), "gate": (s.ffn, s.hidden),
              "up": (s.ffn, s.hidden), "down": (s.hidden, s.ffn)}[which]
        codes = np.empty(rk, dtype=np.uint8)
        scales = np.empty(rk[0], dtype=np.float32)
        _lib.check(self.lib, self.lib.megakernel_get_layer_fp8(
            self._handle, int(layer), self.LAYER_MATRICES.index(which), codes.ctypes.data_as(ctypes.c_void_p),
            scales.ctypes.data_as(ctypes.POINTER(ctypes.c_float))), "get_layer_fp8")
        return codes, scales

    @property
    def grid_size(self) -> int:
        return self.lib.megakernel_grid_size(self._handle)

    def close(self):
        """Free GPU resources."""
        if getattr(self, "_handle", None):
            self.lib.megakernel_free(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
