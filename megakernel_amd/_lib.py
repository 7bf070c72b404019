"""ctypes binding of megakernel.so (declarations mirror include/megakernel.h).

The six reference entry points are declared exactly as the reference bridge
declares them (/root/reference/host/bridge.py:39-67); the rest are the
additive extensions.  Loading fails loudly if the library is missing: there is
no fallback path.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT_LIB = os.path.join(_HERE, "megakernel.so")

c_void_p, c_int, c_float = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
c_ll, c_ull, c_char_p = ctypes.c_longlong, ctypes.c_ulonglong, ctypes.c_char_p
P_ll = ctypes.POINTER(ctypes.c_longlong)
P_int = ctypes.POINTER(ctypes.c_int)
P_float = ctypes.POINTER(ctypes.c_float)

# name -> (restype, argtypes)
SIGNATURES = {
    # reference entry points (src/megakernel.cu:544-622)
    "megakernel_init": (c_void_p, [c_void_p, P_ll, c_int]),
    "megakernel_decode": (c_int, [c_void_p, c_int]),
    "megakernel_reset": (None, [c_void_p]),
    "megakernel_get_pos": (c_int, [c_void_p]),
    "megakernel_free": (None, [c_void_p]),
    "megakernel_sync": (None, []),
    # extensions
    "megakernel_last_error": (c_char_p, []),
    "megakernel_init_ex": (c_void_p, [c_void_p, P_ll, c_int, c_int, c_int, c_int]),
    "megakernel_init_from_host": (c_void_p, [c_void_p, c_ull, P_ll, c_int, c_int, c_int, c_int]),
    "megakernel_generate": (c_int, [c_void_p, c_int, c_int, P_int]),
    "megakernel_debug_forward": (c_int, [c_void_p, c_int, P_float, P_float]),
    "megakernel_set_pos": (c_int, [c_void_p, c_int]),
    "megakernel_set_kv": (c_int, [c_void_p, c_void_p, c_int]),
    "megakernel_get_kv": (c_int, [c_void_p, c_void_p, c_int]),
    "megakernel_fill_kv_synthetic": (c_int, [c_void_p, c_int, c_ull, c_float]),
    "megakernel_trace_generate": (c_int, [c_void_p, c_int, c_int, c_int, ctypes.POINTER(ctypes.c_ulonglong)]),
    "megakernel_last_kernel_ms": (c_float, [c_void_p]),
    "megakernel_grid_size": (c_int, [c_void_p]),
    "megakernel_set_attention_chunk": (c_int, [c_void_p, c_int]),
    "megakernel_set_attention_merge": (c_int, [c_void_p, c_int]),
    "megakernel_set_decode_kernel": (c_int, [c_void_p, c_int]),
    "megakernel_decode_kernel_for": (c_int, [c_void_p, c_int]),
    "megakernel_set_lmhead_fp8": (c_int, [c_void_p, c_int]),
    "megakernel_set_kv_fp8": (c_int, [c_void_p, c_int]),
    "megakernel_get_lmhead_fp8": (c_int, [c_void_p, c_void_p, P_float]),
    "megakernel_set_layer_fp8": (c_int, [c_void_p, c_int]),
    "megakernel_get_layer_fp8": (c_int, [c_void_p, c_int, c_int, c_void_p, P_float]),
    "megakernel_prefill_attach": (c_int, [c_void_p, c_void_p, P_ll, c_int]),
    "megakernel_prefill": (c_int, [c_void_p, P_int, c_int, P_int]),
    "megakernel_synth_fill": (c_int, [c_void_p, c_ull, c_ull, c_float, c_int]),
    "megakernel_synth_key": (c_ull, [c_ull, c_ull]),
    "megakernel_rope_inv_freq": (c_int, [c_int, P_float, c_int]),
    "megakernel_device_alloc": (c_void_p, [c_ull]),
    "megakernel_device_free": (None, [c_void_p]),
    "megakernel_memcpy": (c_int, [c_void_p, c_void_p, c_ull, c_int]),
    "megakernel_device_info": (c_int, [P_int, P_int, c_char_p, c_int]),
    # batched decode
    "megakernel_batch_init": (c_void_p, [c_void_p, P_ll, c_int, c_int, c_int, c_int, c_int]),
    "megakernel_batch_free": (None, [c_void_p]),
    "megakernel_batch_set_pos": (c_int, [c_void_p, c_int, c_int]),
    "megakernel_batch_get_pos": (c_int, [c_void_p, P_int]),
    "megakernel_batch_fill_kv_synthetic": (c_int, [c_void_p, c_int, c_int, c_ull, c_float]),
    "megakernel_batch_set_kv": (c_int, [c_void_p, c_int, c_void_p, c_int]),
    "megakernel_batch_get_kv": (c_int, [c_void_p, c_int, c_void_p, c_int]),
    "megakernel_decode_batch": (c_int, [c_void_p, P_int, P_int]),
    "megakernel_generate_batch": (c_int, [c_void_p, P_int, c_int, P_int]),
    "megakernel_batch_debug_logits": (c_int, [c_void_p, P_int, P_int, P_float]),
    "megakernel_batch_prefill": (c_int, [c_void_p, c_int, P_int, c_int, P_int, P_float]),
    "megakernel_batch_set_kv_fp8": (c_int, [c_void_p, c_int]),
    "megakernel_batch_set_lmhead_fp8": (c_int, [c_void_p, c_int]),
    "megakernel_batch_set_step_kernel": (c_int, [c_void_p, c_int]),
    "megakernel_batch_trace_step": (c_int, [c_void_p, P_int, ctypes.POINTER(ctypes.c_ulonglong), ctypes.c_longlong]),
    "megakernel_batch_last_ms": (c_float, [c_void_p]),
    # operator microbench
    "megakernel_op_packed_bytes": (c_ll, [c_int, c_int]),
    "megakernel_op_pack": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p]),
    "megakernel_op_rmsnorm": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_float]),
    "megakernel_op_gemv": (c_int, [c_void_p, c_ll, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_int,
                                   c_void_p, c_int, c_int]),
    "megakernel_op_rope": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_float]),
    "megakernel_op_lmhead_argmax": (c_int, [c_void_p, c_ll, c_int, c_int, c_int, c_void_p, c_int, c_void_p,
                                            c_void_p, c_void_p, c_int, c_int]),
    "megakernel_op_lmhead_argmax_noalloc": (c_int, [c_void_p, c_ll, c_int, c_int, c_int, c_void_p, c_int,
                                                    c_void_p, c_void_p, c_int, c_int]),
    "megakernel_op_last_ms": (c_float, []),
    # self-test
    "megakernel_selftest_dataflow": (c_int, [c_int, P_int, P_float]),
}

PRESET_BASELINE, PRESET_QWEN3_06B, PRESET_TINY = 0, 1, 2
KERNEL_AUTO, KERNEL_SPREAD, KERNEL_CLASS = 0, 1, 2  # megakernel_set_decode_kernel / _decode_kernel_for
BATCH_STEP_PERSISTENT, BATCH_STEP_PER_PHASE = 0, 1  # megakernel_batch_set_step_kernel
LMHEAD_BF16, LMHEAD_FP8, LMHEAD_SCREENED = 0, 1, 2  # megakernel_set_lmhead_fp8
H2D, D2H, D2D = 0, 1, 2

_cache: dict[str, ctypes.CDLL] = {}


class MegakernelError(RuntimeError):
    pass


def load(path: str | None = None) -> ctypes.CDLL:
    path = os.path.abspath(path or os.environ.get("MEGAKERNEL_LIB", DEFAULT_LIB))
    if path in _cache:
        return _cache[path]
    if not os.path.exists(path):
        raise MegakernelError(
            f"{path} not found: build it first (`make lib` or __graft_entry__.build()); "
            "there is no CPU fallback")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _cache[path] = lib
    return lib


def last_error(lib: ctypes.CDLL) -> str:
    msg = lib.megakernel_last_error()
    return msg.decode() if msg else ""


def check(lib: ctypes.CDLL, rc: int, what: str) -> int:
    if rc is None or rc < 0:
        raise MegakernelError(f"{what} failed: {last_error(lib)}")
    return rc
