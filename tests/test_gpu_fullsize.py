"""GPU parity of exactly the workloads that are timed, at their real sizes,
and of the reference's own drop-in path.

* configs[0] through the reference's six entry points, bound the way the
  reference bridge binds them (/root/reference/host/bridge.py:41-67): the full
  28-layer model is uploaded to a device buffer, megakernel_init infers its
  shape from the 310 offsets, a 16-token prompt is fed with megakernel_decode
  and 64 greedy tokens follow (the reference's validate.py greedy-match rule,
  /root/reference/host/validate.py:95-118: identical wherever the oracle's
  top-1/top-2 margin exceeds 2e-2), then reset / get_pos / free / sync.
* the plain (benchmarked) kernel instantiation on the full model
  with 1,024 prefilled positions, 64 tokens in one resident launch, teacher-
  forced against the oracle, plus the per-layer and logit bars at two steps.
* the full model at 8,192 and 32,768 prefilled positions.

The oracle's prefilled cache is the device's own synthetic prefill read back
with megakernel_get_kv (bit-exactness of that prefill against the CPU
generator is tested in test_gpu_parity.py); everything after it is computed
independently by both sides.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from megakernel_amd import _lib
from megakernel_amd.config import BASELINE, QWEN3_06B, TINY
from megakernel_amd.weights import DeviceWeights, flat_layout
from oracle import qwen3_ref, synth

from ._helpers import LOGIT_ABS, MARGIN, check_step, check_tokens_teacher_forced, make_pair, oracle_shape

pytestmark = pytest.mark.gpu


def _print(*a):
    print(*a, flush=True)


def _reference_binding():
    """megakernel.so with exactly the reference bridge's declarations."""
    lib = ctypes.CDLL(_lib.DEFAULT_LIB)
    lib.megakernel_init.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_longlong), ctypes.c_int]
    lib.megakernel_init.restype = ctypes.c_void_p
    lib.megakernel_decode.argtypes = [ctypes.c_void_p, ctypes.c_int]
    lib.megakernel_decode.restype = ctypes.c_int
    lib.megakernel_reset.argtypes = [ctypes.c_void_p]
    lib.megakernel_reset.restype = None
    lib.megakernel_get_pos.argtypes = [ctypes.c_void_p]
    lib.megakernel_get_pos.restype = ctypes.c_int
    lib.megakernel_free.argtypes = [ctypes.c_void_p]
    lib.megakernel_free.restype = None
    lib.megakernel_sync.argtypes = []
    lib.megakernel_sync.restype = None
    return lib


def _upload_like_reference(host: np.ndarray) -> torch.Tensor:
    """The reference uploads weights.bin into a torch cuda uint8 tensor
    (bridge.py:77-84); its data_ptr() is what megakernel_init receives."""
    t = torch.empty(host.nbytes, dtype=torch.uint8, device="cuda")
    t.copy_(torch.from_numpy(host))
    torch.cuda.synchronize()
    return t


def _oracle_for(shape, host, max_seq):
    osh = oracle_shape(shape)
    bits = qwen3_ref.unpack_flat(osh, host, flat_layout(shape).offsets)
    return qwen3_ref.Qwen3Oracle(osh, bits, max_seq)


def test_reference_binding_configs0_full_model():
    """configs[0] (16-token prompt, 64 greedy tokens, full BASELINE model)
    through megakernel_init / decode / reset / get_pos / free / sync."""
    shape = BASELINE
    dw = DeviceWeights(shape, 2024, std=0.02, gain_std=0.0)
    host = dw.to_host()
    dw.free()
    buf = _upload_like_reference(host)
    orc = _oracle_for(shape, host, 128)
    lib = _reference_binding()
    offs = flat_layout(shape).ordered_offsets()
    assert len(offs) == 310
    arr = (ctypes.c_longlong * len(offs))(*offs)
    h = lib.megakernel_init(ctypes.c_void_p(buf.data_ptr()), arr, len(offs))
    assert h, _lib.last_error(_lib.load())
    try:
        prompt = synth.prompt_tokens(2024, 16, shape.vocab)
        _print(f"configs[0] via the reference ABI: prompt {prompt}")
        outs = [lib.megakernel_decode(h, t) for t in prompt]
        assert min(outs) >= 0
        assert lib.megakernel_get_pos(h) == 16
        gen = [outs[-1]]
        for _ in range(63):
            gen.append(lib.megakernel_decode(h, gen[-1]))
        assert min(gen) >= 0 and lib.megakernel_get_pos(h) == 16 + 63
        for t in prompt[:-1]:
            orc.step(t)
        same, low = check_tokens_teacher_forced([prompt[-1]] + gen[:-1], gen, orc)
        _print(f"  64 greedy tokens: {same} identical to the oracle, {low} low-margin differences")
        # reset: the cache and position start over, the first step repeats
        lib.megakernel_reset(h)
        assert lib.megakernel_get_pos(h) == 0
        assert lib.megakernel_decode(h, prompt[0]) == outs[0]
        assert lib.megakernel_get_pos(h) == 1
    finally:
        lib.megakernel_free(h)
        lib.megakernel_sync()
        del buf


def test_reference_binding_infers_qwen3_shape():
    """megakernel_init on a QWEN3_06B-shaped weights.bin (head_dim 128, ffn
    3072: the reference's config.cuh shapes) picks that preset from the
    offsets and decodes it correctly."""
    shape = QWEN3_06B.with_(n_layers=2, vocab=4096)
    dw = DeviceWeights(shape, 77, std=0.02, gain_std=0.1)
    host = dw.to_host()
    dw.free()
    buf = _upload_like_reference(host)
    orc = _oracle_for(shape, host, 64)
    lib = _reference_binding()
    offs = flat_layout(shape).ordered_offsets()
    arr = (ctypes.c_longlong * len(offs))(*offs)
    h = lib.megakernel_init(ctypes.c_void_p(buf.data_ptr()), arr, len(offs))
    assert h, _lib.last_error(_lib.load())
    try:
        toks = [5, 900, 4095, 17]
        outs = []
        for t in toks:
            outs.append(lib.megakernel_decode(h, t))
        gen = [outs[-1]]
        for _ in range(8):
            gen.append(lib.megakernel_decode(h, gen[-1]))
        kin, kout = toks + gen[:-1], outs + gen[1:]
        same, low = check_tokens_teacher_forced(kin, kout, orc)
        _print(f"QWEN3_06B shape via megakernel_init: {same} identical, {low} low-margin")
    finally:
        lib.megakernel_free(h)
        lib.megakernel_sync()
        del buf


def test_init_from_host_failure_after_upload():
    """A failure after the library has uploaded the weights (here: a vocab
    that is not a multiple of 16 on a padded, non-contiguous layout) returns
    NULL with a message and frees the upload exactly once; the next init
    works."""
    lib = _lib.load()
    shape = TINY.with_(n_layers=1, vocab=1000)
    lay = flat_layout(shape)
    offs = lay.ordered_offsets()
    padded = [offs[0]] + [o + 16 * (i + 1) for i, o in enumerate(offs[1:])]
    host = np.zeros(lay.total_bytes + 16 * len(offs), dtype=np.uint8)
    arr = (ctypes.c_longlong * len(padded))(*padded)
    h = lib.megakernel_init_from_host(host.ctypes.data_as(ctypes.c_void_p), host.nbytes, arr, len(padded),
                                      _lib.PRESET_TINY, shape.vocab, 64)
    assert not h
    assert "vocab" in _lib.last_error(lib)
    eng, orc, dw = make_pair(TINY, 3, 32)
    try:
        nxt = eng.decode_token(7)
        r = orc.step(7, capture=True)
        assert nxt == r["token"] or qwen3_ref.top2_margin(r["logits"]) <= 2e-2
    finally:
        eng.close()
        dw.free()


def _prefilled_pair(ctx: int, seed: int, extra: int):
    eng, orc, dw = make_pair(BASELINE, seed, ctx + extra, gain_std=0.0, bits_from_device=True)
    eng.fill_kv_synthetic(ctx, seed)
    kv = eng.get_kv(ctx)  # [L][2][NKV][ctx][D]
    orc.set_kv(kv[:, 0], kv[:, 1])
    del kv
    return eng, orc, dw


def test_prefill_full_model_1024_tokens():
    """The prefill bench's workload: the full model consumes a 1,024-token
    prompt (one pass of 64 column groups) from an empty cache through the
    batch-1 handle's prefill context; the token after it against the oracle
    stepped through the same prompt (logits within the bar through the batch
    handle's own prefill, same weights), then 16 decoded tokens
    teacher-forced."""
    from megakernel_amd.batch import BatchEngine
    n = 1024
    eng, orc, dw = make_pair(BASELINE, 1025, n + 64, gain_std=0.0, bits_from_device=True)
    try:
        rng = np.random.default_rng(1025)
        prompt = [int(t) for t in rng.integers(0, BASELINE.vocab, size=n)]
        ref = None
        for i, t in enumerate(prompt):
            ref = orc.step(t, capture=i == n - 1)
            if i % 256 == 255:
                _print(f"  oracle: {i + 1} prompt tokens")
        be = BatchEngine(dw, 1, n + 16, BASELINE)
        try:
            nxt_b, logits = be.prefill(0, prompt, with_logits=True)
        finally:
            be.close()
        err = float(np.abs(logits - ref["logits"].numpy()).max())
        _print(f"prefill {n}: next token {nxt_b} (oracle {ref['token']}), logits max abs err {err:.2e}")
        assert err <= LOGIT_ABS
        if nxt_b != ref["token"]:
            assert qwen3_ref.top2_margin(ref["logits"]) <= MARGIN
        eng.attach_prefill(dw)
        nxt = eng.prefill(prompt)
        assert nxt == nxt_b and eng.pos == n
        gen = eng.decode_many(ref["token"], 16)
        same, low = check_tokens_teacher_forced([ref["token"]] + gen[:-1], gen, orc)
        _print(f"  16 decoded tokens after the prefill: {same} identical, {low} low-margin")
    finally:
        eng.close()
        dw.free()


def test_configs2_full_model_ctx1024_plain_launch():
    """The benchmarked workload's own instantiation: full model, 1,024
    prefilled positions, two debug steps at the per-layer / logit bars, then
    64 tokens in one resident launch of the plain kernel, teacher-forced."""
    eng, orc, dw = _prefilled_pair(1024, 2024, 80)
    try:
        tok = 11
        for i in range(2):
            nxt, layers, logits = eng.debug_forward(tok)
            ref = orc.step(tok, capture=True)
            l2, la = check_step(layers, logits, ref, f"ctx 1024 step {i}")
            _print(f"configs[2] debug step {i}: layer relL2 {l2:.2e} logits abs {la:.2e}")
            tok = ref["token"]
        gen = eng.decode_many(tok, 64)
        assert eng.pos == 1024 + 2 + 64
        same, low = check_tokens_teacher_forced([tok] + gen[:-1], gen, orc)
        _print(f"configs[2] plain launch, 64 tokens: {same} identical, {low} low-margin")
    finally:
        eng.close()
        dw.free()


@pytest.mark.parametrize("ctx", [8192, 32768])
def test_configs3_full_model_long_context(ctx):
    """the full model at 8,192 / 32,768 prefilled positions (16 and
    32 attention splits per kv head; the long-context merge above 20), two
    debug steps at the bars, then 8 tokens in one resident launch."""
    eng, orc, dw = _prefilled_pair(ctx, 31 + ctx, 16)
    try:
        tok = 3
        for i in range(2):
            _print(f"configs[3] ctx {ctx} step {i}")
            nxt, layers, logits = eng.debug_forward(tok)
            ref = orc.step(tok, capture=True)
            l2, la = check_step(layers, logits, ref, f"ctx {ctx} step {i}")
            _print(f"  layer relL2 {l2:.2e} logits abs {la:.2e}")
            tok = ref["token"]
        gen = eng.decode_many(tok, 8)
        same, low = check_tokens_teacher_forced([tok] + gen[:-1], gen, orc)
        _print(f"  8-token launch: {same} identical, {low} low-margin")
    finally:
        eng.close()
        dw.free()


@pytest.mark.parametrize("ctx", [0, 100, 600, 1024, 1500, 3000, 4000])
def test_class_kernel_equals_spread_kernel(ctx):
    """The class-specialised kernel (MK_KERNEL_AUTO at up to 8 splits per kv
    head) and the spread kernel run the same arithmetic: per-layer residuals,
    logits and tokens of the same steps are bitwise identical; and the class
    kernel is the one AUTO picks for these launches."""
    shape = BASELINE.with_(n_layers=3, vocab=8192)
    eng, orc, dw = make_pair(shape, 71, ctx + 40)
    try:
        if ctx:
            eng.fill_kv_synthetic(ctx, 9)
        assert eng.decode_kernel_for(20) == _lib.KERNEL_CLASS
        runs = []
        for variant in (_lib.KERNEL_AUTO, _lib.KERNEL_SPREAD):
            eng.set_decode_kernel(variant)
            eng.set_pos(ctx)
            _, layers, logits = eng.debug_forward(5)
            gen = eng.decode_many(7, 20)
            runs.append((layers, logits, gen))
        assert np.array_equal(runs[0][0], runs[1][0]), "per-layer residuals differ"
        assert np.array_equal(runs[0][1], runs[1][1]), "logits differ"
        assert runs[0][2] == runs[1][2], "tokens differ"
        _print(f"ctx {ctx}: class == spread, tokens {runs[0][2][:6]}")
    finally:
        eng.close()
        dw.free()
