"""Operator microbench over the library's
``megakernel_op_*`` entry points.

Each op of one decode step runs as a standalone launch that repeats the op
``reps`` times in-kernel; instance ``r`` reads weight copy ``r % n_copies``,
input ``r % n_in`` and writes output slot ``r % n_out``.  The reference has
these ops only as device functions of its kernel:

=================  ==========================================================
rmsnorm            /root/reference/src/rmsnorm.cuh:87-108
gemv (QKV, O)      /root/reference/src/gemv.cuh:118-199, :36-104
gemv + residual    /root/reference/src/gemv.cuh:36-104, src/megakernel.cu:288-290
gate/up + SiLU     /root/reference/src/gemv.cuh:212-279
rope               /root/reference/src/attention.cuh:22-44
lm head + argmax   /root/reference/src/sampling.cuh:32-117
=================  ==========================================================

Buffers are device memory passed as anything with ``data_ptr()`` (a torch
tensor) or as an integer address; the caller owns them.  Every function
returns the device time of the call in milliseconds.
"""
from __future__ import annotations

from . import _lib

LAYOUT_TILE, LAYOUT_GATE_UP = 1, 2
GEMV_PLAIN, GEMV_RESIDUAL, GEMV_GATE_UP = 0, 1, 2


def _p(t) -> int | None:
    if t is None:
        return None
    return t.data_ptr() if hasattr(t, "data_ptr") else int(t)


def _lib_():
    return _lib.load()


def packed_bytes(rows: int, k: int) -> int:
    lib = _lib_()
    return _lib.check(lib, lib.megakernel_op_packed_bytes(rows, k), "op_packed_bytes")


def pack(src, rows: int, k: int, layout: int, dst) -> float:
    """Row-major bf16 [rows][k] -> packed layout (LAYOUT_GATE_UP: rows = 2F, gate then up)."""
    lib = _lib_()
    _lib.check(lib, lib.megakernel_op_pack(_p(src), rows, k, layout, _p(dst)), "op_pack")
    return float(lib.megakernel_op_last_ms())


def rmsnorm(x, gain, y, n: int, n_in: int, n_out: int, reps: int, eps: float = 1e-6) -> float:
    lib = _lib_()
    _lib.check(lib, lib.megakernel_op_rmsnorm(_p(x), _p(gain), _p(y), n, n_in, n_out, reps, eps), "op_rmsnorm")
    return float(lib.megakernel_op_last_ms())


def gemv(w, copy_bytes: int, n_copies: int, rows: int, k: int, kind: int, x, res, n_in: int, y, n_out: int,
         reps: int) -> float:
    lib = _lib_()
    _lib.check(lib, lib.megakernel_op_gemv(_p(w), copy_bytes, n_copies, rows, k, kind, _p(x), _p(res), n_in,
                                           _p(y), n_out, reps), "op_gemv")
    return float(lib.megakernel_op_last_ms())


def rope(x, pos, y, n_heads: int, head_dim: int, n_in: int, n_out: int, reps: int, theta: float = 1e6) -> float:
    lib = _lib_()
    _lib.check(lib, lib.megakernel_op_rope(_p(x), _p(pos), _p(y), n_heads, head_dim, n_in, n_out, reps, theta),
               "op_rope")
    return float(lib.megakernel_op_last_ms())


def lmhead_argmax(w, copy_bytes: int, n_copies: int, vocab: int, k: int, h, n_in: int, logits, keys, tokens,
                  n_out: int, reps: int) -> float:
    lib = _lib_()
    _lib.check(lib, lib.megakernel_op_lmhead_argmax(_p(w), copy_bytes, n_copies, vocab, k, _p(h), n_in,
                                                    _p(logits), _p(keys), _p(tokens), n_out, reps),
               "op_lmhead_argmax")
    return float(lib.megakernel_op_last_ms())
