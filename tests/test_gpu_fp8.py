"""GPU parity of the FP8 LM head (megakernel_set_lmhead_fp8) through the C ABI.

The library quantises the tied table to OCP e4m3 with power-of-two row scales
on the device; the codes and scales must equal the oracle's (oracle/fp8.py,
pinned against torch's float8_e4m3fn) bit for bit.  Decoding then streams the
FP8 copy: hidden states are unchanged (the embedding gather keeps the bf16
table) and the logits must match the oracle run with the same dequantised
table, at the north_star bars (layer rel-L2 1e-2, logits 2e-2 abs, greedy
tokens identical where the oracle's top-1/top-2 margin exceeds 2e-2).
"""
from __future__ import annotations

import numpy as np
import pytest

from megakernel_amd.config import BASELINE, QWEN3_06B, TINY
from oracle import qwen3_ref, synth

from ._helpers import check_step, check_tokens_teacher_forced, make_pair

pytestmark = pytest.mark.gpu

BASELINE_2L = BASELINE.with_(n_layers=2, vocab=4096)


def _print(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("name,shape", [("tiny", TINY), ("baseline_2l", BASELINE_2L),
                                        ("qwen3_2l", QWEN3_06B.with_(n_layers=2, vocab=4096)),
                                        ("baseline_full_vocab", BASELINE.with_(n_layers=1))])
def test_fp8_lmhead_codes_bit_exact(name, shape):
    eng, orc, dw = make_pair(shape, 13, 32)
    try:
        _print(f"fp8 codes {name} vocab {shape.vocab}")
        eng.set_lmhead_fp8(True)
        codes, scales = eng.lmhead_fp8()
        want_codes, want_scales = orc.use_fp8_lm_head()
        assert np.array_equal(scales, want_scales), "row scales differ"
        diff = codes != want_codes
        assert not diff.any(), f"{int(diff.sum())} FP8 codes differ (first at {np.argwhere(diff)[0]})"
    finally:
        eng.close()
        dw.free()


def test_fp8_lmhead_decode_parity():
    eng, orc, dw = make_pair(BASELINE_2L, 17, 128)
    try:
        eng.set_lmhead_fp8(True)
        orc.use_fp8_lm_head()
        prompt = synth.prompt_tokens(17, 6, BASELINE_2L.vocab)
        tok = prompt[0]
        for i in range(12):
            tin = prompt[i] if i < len(prompt) else tok
            _print(f"fp8 step {i} token {tin}")
            nxt, layers, logits = eng.debug_forward(tin)
            ref = orc.step(tin, capture=True)
            check_step(layers, logits, ref, f"fp8 step {i}")
            if nxt != ref["token"]:
                assert qwen3_ref.top2_margin(ref["logits"]) <= 2e-2
            tok = nxt
    finally:
        eng.close()
        dw.free()


def test_fp8_lmhead_long_context():
    """Long-context instantiation (32 splits per kv head, first-split merge)
    with the FP8 LM head."""
    shape = BASELINE.with_(n_layers=2, vocab=2048)
    ctx = 2000
    eng, orc, dw = make_pair(shape, 23, ctx + 16)
    try:
        eng.set_attention_chunk(64)
        eng.set_lmhead_fp8(True)
        orc.use_fp8_lm_head()
        eng.fill_kv_synthetic(ctx, 9)
        ks = np.stack([synth.kv_prefill_bits(9, l, 0, ctx, shape.n_kv_heads, shape.head_dim)
                       for l in range(shape.n_layers)])
        vs = np.stack([synth.kv_prefill_bits(9, l, 1, ctx, shape.n_kv_heads, shape.head_dim)
                       for l in range(shape.n_layers)])
        orc.set_kv(ks, vs)
        tok = 4
        for i in range(3):
            _print(f"fp8 ctx {ctx} step {i}")
            _, layers, logits = eng.debug_forward(tok)
            ref = orc.step(tok, capture=True)
            check_step(layers, logits, ref, f"fp8 ctx {ctx} step {i}")
            tok = ref["token"]
    finally:
        eng.close()
        dw.free()


def test_fp8_lmhead_generate_toggle_and_oracle():
    """One resident launch == per-token decoding with the FP8 head; greedy
    tokens agree with the FP8 oracle (teacher-forced); switching back to bf16
    reproduces the bf16 logits bit for bit."""
    eng, orc, dw = make_pair(BASELINE_2L, 19, 256)
    try:
        _, _, bf16_logits = eng.debug_forward(7)
        eng.set_lmhead_fp8(True)
        eng.set_pos(0)
        _, _, f8_logits = eng.debug_forward(7)
        assert not np.array_equal(f8_logits, bf16_logits)
        dq = float(np.abs(f8_logits - bf16_logits).max())
        _print(f"fp8 vs bf16 LM head: max |logit difference| {dq:.3e}")
        eng.set_pos(0)
        a0 = eng.decode_token(7)
        gen = eng.decode_many(a0, 40)
        eng.set_pos(0)
        b = [eng.decode_token(7)]
        for _ in range(40):
            b.append(eng.decode_token(b[-1]))
        assert [a0] + gen == b, "generate() and per-token decode disagree with the FP8 head"
        orc.use_fp8_lm_head()
        same, low = check_tokens_teacher_forced([7, a0] + gen[:-1], [a0] + gen, orc)
        _print(f"fp8 teacher-forced: {same} identical, {low} low-margin differences")
        eng.set_lmhead_fp8(False)
        eng.set_pos(0)
        _, _, back = eng.debug_forward(7)
        assert np.array_equal(back, bf16_logits), "bf16 logits changed after the FP8 head was switched off"
    finally:
        eng.close()
        dw.free()
