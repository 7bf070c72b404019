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


# ---------------------------------------------------------------- FP8 KV cache
def _synthetic_kv(shape, seed, ctx):
    ks = np.stack([synth.kv_prefill_bits(seed, l, 0, ctx, shape.n_kv_heads, shape.head_dim)
                   for l in range(shape.n_layers)])
    vs = np.stack([synth.kv_prefill_bits(seed, l, 1, ctx, shape.n_kv_heads, shape.head_dim)
                   for l in range(shape.n_layers)])
    return ks, vs


def _bf16_bits(t) -> np.ndarray:
    import torch
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("name,shape", [("tiny", TINY), ("baseline_2l", BASELINE_2L),
                                        ("qwen3_2l", QWEN3_06B.with_(n_layers=2, vocab=4096))])
def test_fp8_kv_fill_and_set_exact(name, shape):
    """fill_kv_synthetic and set_kv quantise each K / V row as the oracle does;
    get_kv returns bf16 of code x scale, which is exact: bit-equal to the
    oracle's dequantised rows."""
    ctx = 300
    eng, orc, dw = make_pair(shape, 29, ctx + 8, kv_fp8=True)
    try:
        _print(f"fp8 kv fill {name}")
        ks, vs = _synthetic_kv(shape, 41, ctx)
        orc.set_kv(ks, vs)
        eng.fill_kv_synthetic(ctx, 41)
        got = eng.get_kv(ctx)
        assert np.array_equal(got[:, 0], _bf16_bits(orc.k_cache[:, :, :ctx])), "K codes / scales differ"
        assert np.array_equal(got[:, 1], _bf16_bits(orc.v_cache[:, :, :ctx])), "V codes / scales differ"
        # set_kv of other bf16 rows (a wide dynamic range across rows)
        rng = np.random.default_rng(3)
        vals = (rng.standard_normal((shape.n_layers, 2, shape.n_kv_heads, 40, shape.head_dim)) *
                np.exp(rng.uniform(-6, 6, size=(shape.n_layers, 2, shape.n_kv_heads, 40, 1)))).astype(np.float32)
        import torch
        bits = _bf16_bits(torch.from_numpy(vals))
        eng.set_kv(bits)
        orc.set_kv(bits[:, 0], bits[:, 1])
        got = eng.get_kv(40)
        assert np.array_equal(got[:, 0], _bf16_bits(orc.k_cache[:, :, :40]))
        assert np.array_equal(got[:, 1], _bf16_bits(orc.v_cache[:, :, :40]))
    finally:
        eng.close()
        dw.free()


@pytest.mark.parametrize("ctx,chunk", [(100, 512), (1500, 64), (2000, 64)])
def test_fp8_kv_decode_parity(ctx, chunk):
    """Decoding over an FP8 cache (split attention; ctx 2000 at chunk 64 runs
    the long-context merge) against the oracle on the same dequantised cache;
    the appended rows are the oracle's quantised k / v (the kernel's fp32 k
    differs in summation order, so a code may sit one step away)."""
    shape = BASELINE.with_(n_layers=2, vocab=2048)
    eng, orc, dw = make_pair(shape, 37, ctx + 16, kv_fp8=True)
    try:
        eng.set_attention_chunk(chunk)
        eng.fill_kv_synthetic(ctx, 43)
        orc.set_kv(*_synthetic_kv(shape, 43, ctx))
        tok = 5
        for i in range(4):
            _print(f"fp8 kv ctx {ctx} chunk {chunk} step {i}")
            _, layers, logits = eng.debug_forward(tok)
            ref = orc.step(tok, capture=True)
            check_step(layers, logits, ref, f"fp8 kv ctx {ctx} step {i}")
            tok = ref["token"]
        got = eng.get_kv(ctx + 4)[:, :, :, ctx:].astype(np.uint32)
        from oracle import synth as osynth
        gk = osynth.bf16_bits_to_f32(got[:, 0].astype(np.uint16))
        gv = osynth.bf16_bits_to_f32(got[:, 1].astype(np.uint16))
        wk = orc.k_cache[:, :, ctx:ctx + 4].numpy()
        wv = orc.v_cache[:, :, ctx:ctx + 4].numpy()
        for g_, w_, nm in ((gk, wk, "K"), (gv, wv, "V")):
            rel = np.linalg.norm(g_ - w_, axis=-1) / np.maximum(np.linalg.norm(w_, axis=-1), 1e-30)
            assert rel.max() <= 2.0 ** -4, f"appended {nm} rows off by rel-L2 {rel.max():.3e}"
            assert (g_ != w_).mean() < 0.02, f"{(g_ != w_).mean():.3%} of appended {nm} entries differ"
    finally:
        eng.close()
        dw.free()


def test_fp8_kv_generate_and_fp8_head_together():
    """FP8 cache and FP8 LM head together: one resident launch == per-token
    decoding; greedy tokens agree with the oracle (teacher-forced)."""
    eng, orc, dw = make_pair(BASELINE_2L, 47, 256, kv_fp8=True)
    try:
        eng.set_lmhead_fp8(True)
        orc.use_fp8_lm_head()
        prompt = synth.prompt_tokens(47, 6, BASELINE_2L.vocab)
        for t in prompt[:-1]:
            eng.decode_token(t)
        a0 = eng.decode_token(prompt[-1])
        gen = eng.decode_many(a0, 40)
        eng.set_pos(len(prompt) - 1)
        b = [eng.decode_token(prompt[-1])]
        for _ in range(40):
            b.append(eng.decode_token(b[-1]))
        assert [a0] + gen == b, "generate() and per-token decode disagree on the FP8 cache"
        for t in prompt[:-1]:
            orc.step(t)
        same, low = check_tokens_teacher_forced([prompt[-1], a0] + gen[:-1], [a0] + gen, orc)
        _print(f"fp8 kv + fp8 head teacher-forced: {same} identical, {low} low-margin differences")
    finally:
        eng.close()
        dw.free()


@pytest.mark.parametrize("which,prefix,prompt_len", [("tiny", 20, 37), ("baseline_2l", 300, 70)])
def test_fp8_kv_batch1_prefill_then_decode(which, prefix, prompt_len):
    """megakernel_prefill into an FP8 cache (the prefill context appends FP8
    rows with the handle's scales), then decode, against the oracle on the
    same dequantised cache."""
    shape = TINY if which == "tiny" else BASELINE.with_(n_layers=2, vocab=2048)
    eng, orc, dw = make_pair(shape, 53, prefix + prompt_len + 16, kv_fp8=True)
    try:
        eng.attach_prefill(dw)
        if prefix:
            eng.fill_kv_synthetic(prefix, 11)
            orc.set_kv(*_synthetic_kv(shape, 11, prefix))
        prompt = [int(t) for t in np.random.default_rng(prompt_len).integers(0, shape.vocab, size=prompt_len)]
        _print(f"fp8 kv batch-1 prefill {which} prefix {prefix} prompt {prompt_len}")
        nxt = eng.prefill(prompt)
        assert eng.pos == prefix + prompt_len
        ref = None
        for t in prompt:
            ref = orc.step(t, capture=True)
        if nxt != ref["token"]:
            assert qwen3_ref.top2_margin(ref["logits"]) <= 2e-2, f"prefill token {nxt} != oracle {ref['token']}"
        tok = ref["token"]
        for i in range(3):
            _, layers, logits = eng.debug_forward(tok)
            r = orc.step(tok, capture=True)
            check_step(layers, logits, r, f"fp8 kv decode {i} after prefill")
            tok = r["token"]
    finally:
        eng.close()
        dw.free()


# ------------------------------------------------------------ FP8 layer weights
@pytest.mark.parametrize("name,shape", [("tiny", TINY), ("baseline_2l", BASELINE_2L)])
def test_fp8_layer_codes_bit_exact(name, shape):
    """Every layer matrix (fused QKV, O, gate, up, down) quantised on the
    device equals the oracle's e4m3 codes and power-of-two row scales bit for
    bit, read back through megakernel_get_layer_fp8."""
    eng, orc, dw = make_pair(shape, 47, 32)
    try:
        _print(f"fp8 layer codes {name}")
        eng.set_layer_fp8(True)
        want = orc.use_fp8_layers()
        for li in range(shape.n_layers):
            for m in eng.LAYER_MATRICES:
                codes, scales = eng.layer_fp8(li, m)
                wc, ws = want[li][m]
                assert codes.shape == wc.shape, (li, m)
                assert np.array_equal(scales, ws), f"layer {li} {m}: row scales differ"
                diff = codes != wc
                assert not diff.any(), f"layer {li} {m}: {int(diff.sum())} codes differ (first {np.argwhere(diff)[0]})"
    finally:
        eng.close()
        dw.free()


def test_fp8_layer_decode_parity():
    """Decoding with FP8 layer weights against the oracle run on the same
    dequantised matrices (exact: code x 2^e is a bf16 value), per layer and
    per logit, at the bf16 path's bars."""
    eng, orc, dw = make_pair(BASELINE_2L, 53, 128)
    try:
        eng.set_layer_fp8(True)
        orc.use_fp8_layers()
        prompt = synth.prompt_tokens(53, 6, BASELINE_2L.vocab)
        tok = prompt[0]
        for i in range(12):
            tin = prompt[i] if i < len(prompt) else tok
            _print(f"fp8 layers step {i} token {tin}")
            nxt, layers, logits = eng.debug_forward(tin)
            ref = orc.step(tin, capture=True)
            check_step(layers, logits, ref, f"fp8 layers step {i}")
            if nxt != ref["token"]:
                assert qwen3_ref.top2_margin(ref["logits"]) <= 2e-2
            tok = nxt
    finally:
        eng.close()
        dw.free()


def test_fp8_layers_lmhead_and_kv_together():
    """All three FP8 formats at once (layers, LM head, KV cache) over a split
    context, against the oracle with all three; then a resident launch equals
    per-token decoding and switching the layers back to bf16 reproduces the
    bf16 logits bit for bit."""
    shape = BASELINE_2L
    ctx = 700
    eng, orc, dw = make_pair(shape, 59, ctx + 64, kv_fp8=True)
    try:
        eng.set_attention_chunk(256)
        eng.fill_kv_synthetic(ctx, 61)
        orc.set_kv(*_synthetic_kv(shape, 61, ctx))
        _, _, bf16_logits = eng.debug_forward(9)
        eng.set_pos(ctx)
        eng.set_layer_fp8(True)
        eng.set_lmhead_fp8(True)
        orc.use_fp8_layers()
        orc.use_fp8_lm_head()
        tok = 9
        for i in range(4):
            _print(f"fp8 layers+head+kv ctx {ctx} step {i}")
            _, layers, logits = eng.debug_forward(tok)
            ref = orc.step(tok, capture=True)
            check_step(layers, logits, ref, f"fp8 all step {i}")
            tok = ref["token"]
        eng.set_pos(ctx)
        a0 = eng.decode_token(9)
        gen = eng.decode_many(a0, 20)
        eng.set_pos(ctx)
        b = [eng.decode_token(9)]
        for _ in range(20):
            b.append(eng.decode_token(b[-1]))
        assert [a0] + gen == b, "generate() and per-token decode disagree with FP8 layers"
        eng.set_layer_fp8(False)
        eng.set_lmhead_fp8(False)
        eng.set_pos(ctx)
        _, _, back = eng.debug_forward(9)
        assert np.array_equal(back, bf16_logits), "bf16 logits changed after FP8 layers were switched off"
    finally:
        eng.close()
        dw.free()


def test_fp8_layers_need_class_kernel():
    """FP8 layer weights are served by the class-specialised kernel only: the
    spread kernel variant refuses the launch with a message, the QWEN3 preset
    (no class kernel) refuses the switch, and the handle keeps working."""
    from megakernel_amd import _lib
    eng, orc, dw = make_pair(BASELINE_2L, 67, 64)
    try:
        eng.set_layer_fp8(True)
        eng.set_decode_kernel(_lib.KERNEL_SPREAD)
        with pytest.raises(RuntimeError, match="class kernel"):
            eng.decode_token(3)
        eng.set_decode_kernel(_lib.KERNEL_AUTO)
        eng.set_pos(0)
        eng.decode_token(3)
        assert eng.pos == 1
    finally:
        eng.close()
        dw.free()
    shape = QWEN3_06B.with_(n_layers=1, vocab=1024)
    eng, orc, dw = make_pair(shape, 67, 16)
    try:
        with pytest.raises(RuntimeError, match="class kernel"):
            eng.set_layer_fp8(True)
        eng.decode_token(3)
    finally:
        eng.close()
        dw.free()


def test_fp8_layers_full_model_ctx1024():
    """The FP8 bench line's workload: full BASELINE model, 1,024 prefilled
    positions, FP8 layers and LM head; every matrix's codes of the first and
    last layer bit-exact, two debug steps at the bars, then 64 tokens in one
    resident launch teacher-forced against the FP8 oracle."""
    ctx = 1024
    eng, orc, dw = make_pair(BASELINE, 2024, ctx + 80, gain_std=0.0, bits_from_device=True)
    try:
        eng.fill_kv_synthetic(ctx, 2024)
        kv = eng.get_kv(ctx)
        orc.set_kv(kv[:, 0], kv[:, 1])
        del kv
        eng.set_layer_fp8(True)
        eng.set_lmhead_fp8(True)
        want = orc.use_fp8_layers()
        orc.use_fp8_lm_head()
        for li in (0, BASELINE.n_layers - 1):
            for m in eng.LAYER_MATRICES:
                codes, scales = eng.layer_fp8(li, m)
                assert np.array_equal(scales, want[li][m][1]) and np.array_equal(codes, want[li][m][0]), (li, m)
        del want
        tok = 11
        for i in range(2):
            _, layers, logits = eng.debug_forward(tok)
            ref = orc.step(tok, capture=True)
            l2, la = check_step(layers, logits, ref, f"fp8 full ctx 1024 step {i}")
            _print(f"fp8 full model step {i}: layer relL2 {l2:.2e} logits abs {la:.2e}")
            tok = ref["token"]
        gen = eng.decode_many(tok, 64)
        same, low = check_tokens_teacher_forced([tok] + gen[:-1], gen, orc)
        _print(f"fp8 full model, 64 tokens: {same} identical, {low} low-margin")
    finally:
        eng.close()
        dw.free()


# -------------------------------------------------------- screened LM head
@pytest.mark.parametrize("name,ctx", [("baseline_2l", 300), ("baseline_full", 1024)])
def test_screened_lmhead_tokens_equal_bf16_head(name, ctx):
    """MK_LMHEAD_SCREENED: the FP8 copy screens the rows, the rows whose bound
    reaches the threshold are scored again from the bf16 tiles; the argmax is
    then the bf16 head's, so a resident launch of 64 tokens (and the per-token
    path) produces exactly the bf16 head's tokens.  The full model also checks
    them teacher-forced against the oracle."""
    from megakernel_amd import _lib
    shape = BASELINE_2L if name == "baseline_2l" else BASELINE
    eng, orc, dw = make_pair(shape, 71, ctx + 80, gain_std=0.0, bits_from_device=name == "baseline_full")
    try:
        eng.fill_kv_synthetic(ctx, 71)
        ref = eng.decode_many(5, 64)
        eng.set_lmhead_fp8(_lib.LMHEAD_SCREENED)
        eng.set_pos(ctx)
        got = eng.decode_many(5, 64)
        _print(f"screened {name}: first tokens {got[:6]} / bf16 {ref[:6]}")
        assert got == ref, f"screened tokens differ from the bf16 head's (first at {next(i for i, (a, b) in enumerate(zip(got, ref)) if a != b)})"
        eng.set_pos(ctx)
        per = [eng.decode_token(5)]
        for _ in range(15):
            per.append(eng.decode_token(per[-1]))
        assert per == ref[:16], "per-token screened decoding differs"
        if name == "baseline_full":
            kv = eng.get_kv(ctx)
            orc.set_kv(kv[:, 0], kv[:, 1])
            del kv
            same, low = check_tokens_teacher_forced([5] + ref[:-1], ref, orc)
            _print(f"screened full model, 64 tokens: {same} identical, {low} low-margin")
        eng.set_lmhead_fp8(_lib.LMHEAD_BF16)
        eng.set_pos(ctx)
        assert eng.decode_many(5, 64) == ref
    finally:
        eng.close()
        dw.free()


def test_screened_threshold_words_never_alias():
    """The screened LM head's threshold words (second half of the argmax
    slots) are written only by screened launches; launches with the bf16 head
    in between advance the phase tags.  Here the gap is chosen so that a
    14-bit tag would repeat: a screened launch of 8 tokens (TINY: 11 phases
    per token; its last writes per slot parity are tokens 6 and 7), 8 + 16,373
    tokens with the bf16 head, then a screened launch whose first two tokens
    sit 11 * 16,383 phases after those writes.  The words carry the full
    32-bit tag, so the screened launch waits for its own thresholds and its
    tokens equal the bf16 head's."""
    from megakernel_amd import _lib
    eng, orc, dw = make_pair(TINY, 29, 4200, gain_std=0.0)
    try:
        eng.set_lmhead_fp8(_lib.LMHEAD_SCREENED)
        eng.set_pos(0)
        first = eng.decode_many(5, 8)  # writes the threshold words
        eng.set_lmhead_fp8(_lib.LMHEAD_BF16)
        eng.set_pos(0)
        ref = eng.decode_many(3, 8)
        left = 16373
        while left:
            n = min(left, 4000)
            eng.set_pos(0)
            eng.decode_many(7, n)
            left -= n
        eng.set_lmhead_fp8(_lib.LMHEAD_SCREENED)
        eng.set_pos(0)
        got = eng.decode_many(3, 8)
        _print(f"screened after 16,381 bf16-head tokens: {got} / bf16 {ref} (first launch {first[:4]})")
        assert got == ref
    finally:
        eng.close()
        dw.free()
