"""The C-ABI library on the CPU: it loads, exports every function that
include/megakernel.h declares (and the ctypes table matches the header), and
its host-only entry points and argument checks behave.  No GPU work is
launched here."""
import ctypes
import os
import re

import numpy as np
import pytest

from megakernel_amd import _lib
from oracle import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "megakernel.h")


def header_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"\b(megakernel_[a-z_0-9]+)\s*\(", text)


@pytest.fixture(scope="module")
def clib():
    if not os.path.exists(_lib.DEFAULT_LIB):
        from megakernel_amd import launcher
        launcher.compile_shared_library()
    return _lib.load()


def test_header_declares_the_reference_entry_points():
    fns = header_functions()
    for name in ("megakernel_init", "megakernel_decode", "megakernel_reset", "megakernel_get_pos",
                 "megakernel_free", "megakernel_sync"):
        assert name in fns
    assert len(fns) == len(set(fns))


def test_library_exports_every_declared_symbol(clib):
    raw = ctypes.CDLL(_lib.DEFAULT_LIB)
    for name in header_functions():
        assert hasattr(raw, name), name
    assert set(header_functions()) == set(_lib.SIGNATURES)


def test_reference_signatures_unchanged():
    # host/bridge.py:41-67 of the reference declares exactly these
    S = _lib.SIGNATURES
    assert S["megakernel_init"] == (ctypes.c_void_p, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_longlong),
                                                      ctypes.c_int])
    assert S["megakernel_decode"] == (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int])
    assert S["megakernel_reset"] == (None, [ctypes.c_void_p])
    assert S["megakernel_get_pos"] == (ctypes.c_int, [ctypes.c_void_p])
    assert S["megakernel_free"] == (None, [ctypes.c_void_p])
    assert S["megakernel_sync"] == (None, [])


def test_synth_key_matches_oracle(clib):
    for seed, tid in [(0, 0), (2024, 7), (123, 0x40000003), (2**63 + 5, 0x7F000000)]:
        assert clib.megakernel_synth_key(seed, tid) == synth.stream_key(seed, tid)


@pytest.mark.parametrize("preset,d", [(_lib.PRESET_BASELINE, 64), (_lib.PRESET_QWEN3_06B, 128),
                                      (_lib.PRESET_TINY, 64)])
def test_rope_inv_freq_table(clib, preset, d):
    out = (ctypes.c_float * d)()
    n = clib.megakernel_rope_inv_freq(preset, out, d)
    assert n == d // 2
    got = np.frombuffer(out, dtype=np.float32)[:n].astype(np.float64)
    ref = 1.0 / (1e6 ** (np.arange(0, d, 2) / d))
    np.testing.assert_allclose(got, ref, rtol=3e-7)
    assert clib.megakernel_rope_inv_freq(preset, out, 1) == -1  # buffer too small


def test_null_handle_errors_are_reported(clib):
    assert clib.megakernel_decode(None, 1) == -1
    assert "handle" in _lib.last_error(clib)
    assert clib.megakernel_get_pos(None) == -1
    assert clib.megakernel_set_pos(None, 0) == -1
    assert clib.megakernel_generate(None, 1, 1, None) == -1
    assert clib.megakernel_set_attention_chunk(None, 64) == -1
    assert clib.megakernel_set_attention_merge(None, 8) == -1
    assert clib.megakernel_grid_size(None) == -1
    assert clib.megakernel_set_lmhead_fp8(None, 1) == -1
    assert "handle" in _lib.last_error(clib)
    assert clib.megakernel_get_lmhead_fp8(None, None, None) == -1
    assert "FP8 LM head" in _lib.last_error(clib)
    assert clib.megakernel_set_kv_fp8(None, 1) == -1
    assert "handle" in _lib.last_error(clib)
    assert clib.megakernel_batch_set_kv_fp8(None, 1) == -1
    assert "handle" in _lib.last_error(clib)
    clib.megakernel_reset(None)  # no-ops, as in the reference
    clib.megakernel_free(None)


def test_op_argument_checks(clib):
    """The operator-microbench entry points reject bad arguments before any
    GPU work (the pointers below are never dereferenced)."""
    fake = 0x10000
    assert clib.megakernel_op_packed_bytes(16, 1024) == 16 * 1024 * 2
    assert clib.megakernel_op_packed_bytes(15, 1024) == -1
    assert clib.megakernel_op_pack(None, 16, 256, 1, fake) == -1
    assert "null" in _lib.last_error(clib)
    assert clib.megakernel_op_pack(fake, 16, 100, 1, fake) == -1  # tiles need k % 32
    assert clib.megakernel_op_pack(fake, 16, 256, 0, fake) == -1  # no row-pair layout any more
    assert clib.megakernel_op_pack(fake, 16, 256, 7, fake) == -1
    assert "layout" in _lib.last_error(clib)
    assert clib.megakernel_op_pack(fake, 48, 256, 2, fake) == -1  # gate/up needs rows % 32
    assert clib.megakernel_op_rmsnorm(fake, fake, fake, 1000, 1, 1, 1, 1e-6) == -1
    assert clib.megakernel_op_rmsnorm(fake, fake, fake, 1024, 0, 1, 1, 1e-6) == -1
    assert "n_in" in _lib.last_error(clib)
    assert clib.megakernel_op_gemv(fake, 0, 1, 2048, 1000, 0, fake, None, 1, fake, 1, 1) == -1
    assert clib.megakernel_op_gemv(fake, 0, 1, 1024, 2816, 1, fake, None, 1, fake, 1, 1) == -1
    assert "res" in _lib.last_error(clib)
    assert clib.megakernel_op_gemv(fake, 1024, 2, 2048, 1024, 0, fake, None, 1, fake, 1, 1) == -1
    assert "copy_bytes" in _lib.last_error(clib)
    assert clib.megakernel_op_gemv(fake, 0, 1, 2048, 1024, 5, fake, None, 1, fake, 1, 1) == -1
    assert clib.megakernel_op_rope(fake, fake, fake, 24, 32, 1, 1, 1, 1e6) == -1
    assert clib.megakernel_op_lmhead_argmax(fake, 0, 1, 151936, 2048, fake, 1, None, fake, fake, 1, 1) == -1
    assert clib.megakernel_op_lmhead_argmax(fake, 0, 1, 100, 1024, fake, 1, None, fake, fake, 1, 1) == -1
    assert clib.megakernel_op_lmhead_argmax(fake, 0, 1, 4096, 1024, fake, 1, None, None, fake, 1, 1) == -1
    assert clib.megakernel_selftest_dataflow(0, ctypes.byref(ctypes.c_int()), None) == -1
    assert "rounds" in _lib.last_error(clib)


def _offsets(shape) -> list[int]:
    from megakernel_amd.weights import flat_layout
    return flat_layout(shape).ordered_offsets()


def test_init_infers_or_rejects_the_shape_before_gpu_work(clib):
    """megakernel_init takes no shape (reference src/megakernel.cu:544): the
    library infers it from the offsets of the contiguous weights.bin, and
    rejects offsets that match no compiled preset or contradict an explicit
    one -- before any GPU call (the weight pointer is never dereferenced)."""
    from megakernel_amd.config import BASELINE, QWEN3_06B
    fake = ctypes.c_void_p(0x10000)
    bad = [0, 1, 2] + list(range(100, 100 + 307))  # 310 offsets, no shape's layout
    arr = (ctypes.c_longlong * len(bad))(*bad)
    assert clib.megakernel_init(fake, arr, len(bad)) is None
    assert "contiguous weights.bin" in _lib.last_error(clib)
    q = _offsets(QWEN3_06B)
    qa = (ctypes.c_longlong * len(q))(*q)
    # a QWEN3_06B-shaped file (head_dim 128, ffn 3072) is not read as BASELINE
    assert clib.megakernel_init_ex(fake, qa, len(q), _lib.PRESET_BASELINE, 151936, 64) is None
    assert "QWEN3_06B" in _lib.last_error(clib)
    b = _offsets(BASELINE.with_(vocab=4096))
    ba = (ctypes.c_longlong * len(b))(*b)
    assert clib.megakernel_init_ex(fake, ba, len(b), _lib.PRESET_BASELINE, 151936, 64) is None
    assert "vocab 4096" in _lib.last_error(clib)
    # a non-contiguous layout whose tensors overlap at the requested preset's sizes
    over = list(b)
    over[4] = over[3] + 16  # w_k starts inside w_q
    oa = (ctypes.c_longlong * len(over))(*over)
    assert clib.megakernel_init_ex(fake, oa, len(over), _lib.PRESET_BASELINE, 4096, 64) is None
    assert "overlap" in _lib.last_error(clib)
    assert clib.megakernel_init(fake, ba, 14) is None  # count is not 2 + 11 * layers
    assert "num_offsets" in _lib.last_error(clib)


def test_engine_infers_shape_from_offsets_file(tmp_path):
    """MegakernelEngine(weights_path, offsets_path), as the reference bridge
    is constructed, infers the preset, layer count and vocabulary."""
    import json

    from megakernel_amd.config import BASELINE, QWEN3_06B, TINY
    from megakernel_amd.weights import flat_layout, infer_shape
    for s in (BASELINE, QWEN3_06B, TINY.with_(n_layers=3, vocab=2048)):
        p = tmp_path / "offs.json"
        p.write_text(json.dumps(flat_layout(s).offsets))
        from megakernel_amd.weights import load_offsets
        assert infer_shape(load_offsets(str(p))) == s
    offs = dict(flat_layout(BASELINE).offsets)
    offs["layer.3.w_up"] += 2
    with pytest.raises(ValueError, match="contiguous"):
        infer_shape(offs)
