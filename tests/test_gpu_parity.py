"""GPU parity of the megakernel (through the C ABI) against the CPU oracle.

Bars: residual stream after every layer within
rel-L2 1e-2, fp32 logits within 2e-2 abs, greedy tokens identical wherever the
oracle's top-1/top-2 margin exceeds 2e-2.  Bit-exact: synthetic generator,
KV-cache bytes (bf16 of the oracle's post-norm, post-RoPE K and V), argmax
tie-break.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from megakernel_amd import _lib
from megakernel_amd.config import BASELINE, QWEN3_06B, TINY
from oracle import qwen3_ref, synth

from ._helpers import check_kv_bf16, check_step, check_tokens_teacher_forced, make_pair, rel_l2

pytestmark = pytest.mark.gpu

BASELINE_2L = BASELINE.with_(n_layers=2, vocab=4096)


def _print(*a):
    print(*a, flush=True)


def test_synth_fill_bit_exact(lib):
    """Device generator == numpy restatement (incl. indices past 2^32)."""
    n = 1 << 20
    for std, add_one in [(0.02, 0), (1.0, 0), (0.1, 1)]:
        key = synth.stream_key(123, 7)
        c = float(synth.scale_const(std))
        d = lib.megakernel_device_alloc(2 * n)
        assert d
        _lib.check(lib, lib.megakernel_synth_fill(ctypes.c_void_p(d), n, key, c, add_one), "fill")
        got = np.empty(n, dtype=np.uint16)
        _lib.check(lib, lib.megakernel_memcpy(got.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(d),
                                              2 * n, _lib.D2H), "d2h")
        lib.megakernel_device_free(ctypes.c_void_p(d))
        ref = synth.normal_bf16_bits(key, n, std, add_one=bool(add_one))
        assert np.array_equal(got, ref), f"std={std} add_one={add_one}"


def test_tiny_matches_hf_golden_and_oracle():
    """TINY preset against the committed HF fixture (inputs and outputs)."""
    z = np.load("tests/golden/hf_qwen3_tiny.npz")
    eng, orc, dw = make_pair(TINY, int(z["seed"]), 64, gain_std=float(z["gain_std"]))
    try:
        worst_l = worst_g = 0.0
        for i, tok in enumerate(z["tokens_fed"]):
            _print(f"tiny step {i} token {tok}")
            nxt, layers, logits = eng.debug_forward(int(tok))
            ref = orc.step(int(tok), capture=True)
            l2, la = check_step(layers, logits, ref, f"tiny step {i}")
            worst_l, worst_g = max(worst_l, l2), max(worst_g, la)
            # HF fixture (fp32 KV) is within the same bars
            assert rel_l2(layers, z["layers"][i]).max() <= 1e-2
            assert np.abs(logits - z["logits"][i]).max() <= 2e-2
            if nxt != ref["token"]:
                assert qwen3_ref.top2_margin(ref["logits"]) <= 2e-2
        _print(f"tiny worst layer relL2 {worst_l:.2e} logits abs {worst_g:.2e}")
    finally:
        eng.close()
        dw.free()


def test_baseline_2l_matches_hf_golden():
    z = np.load("tests/golden/hf_qwen3_baseline_2l.npz")
    eng, orc, dw = make_pair(BASELINE_2L, int(z["seed"]), 64, gain_std=float(z["gain_std"]))
    try:
        for i, tok in enumerate(z["tokens_fed"]):
            _print(f"baseline_2l step {i} token {tok}")
            nxt, layers, logits = eng.debug_forward(int(tok))
            ref = orc.step(int(tok), capture=True)
            l2, la = check_step(layers, logits, ref, f"step {i}")
            _print(f"  relL2 {l2:.2e} logits {la:.2e}")
            assert rel_l2(layers, z["layers"][i]).max() <= 1e-2
            assert np.abs(logits - z["logits"][i]).max() <= 2e-2
    finally:
        eng.close()
        dw.free()


def test_generate_equals_decode_and_oracle():
    """One resident launch of n tokens == n single-token launches == oracle."""
    eng, orc, dw = make_pair(BASELINE_2L, 5, 256)
    try:
        prompt = synth.prompt_tokens(5, 8, BASELINE_2L.vocab)
        for t in prompt[:-1]:
            eng.decode_token(t)
        a0 = eng.decode_token(prompt[-1])
        gen = eng.decode_many(a0, 40)
        eng.reset()
        for t in prompt[:-1]:
            eng.decode_token(t)
        b = [eng.decode_token(prompt[-1])]
        for _ in range(40):
            b.append(eng.decode_token(b[-1]))
        assert [a0] + gen == b, "generate() and per-token decode disagree"
        assert eng.pos == len(prompt) + 40
        for t in prompt[:-1]:
            orc.step(t)
        same, low = check_tokens_teacher_forced([prompt[-1], a0] + gen[:-1], [a0] + gen, orc)
        _print(f"teacher-forced: {same} identical, {low} low-margin differences")
    finally:
        eng.close()
        dw.free()


def test_kv_cache_bytes_exact():
    """Cache bytes appended by the kernel == bf16 of the oracle's K/V."""
    eng, orc, dw = make_pair(TINY, 3, 64)
    try:
        toks = [5, 77, 901, 13]
        for t in toks:
            eng.decode_token(t)
            orc.step(t)
        kv = eng.get_kv(len(toks))  # [L][2][NKV][len][D]
        ref_k = orc.k_cache[:, :, :len(toks)].contiguous().view(torch.int16).numpy().view(np.uint16)
        ref_v = orc.v_cache[:, :, :len(toks)].contiguous().view(torch.int16).numpy().view(np.uint16)
        # fp32 accumulation order differs, so a value can land on the other
        # side of a bf16 rounding boundary: allow 1 ulp, require >= 99% exact.
        for got, ref, name in [(kv[:, 0], ref_k, "K"), (kv[:, 1], ref_v, "V")]:
            diff = np.abs(got.astype(np.int32) - ref.astype(np.int32))
            assert diff.max() <= 1, f"{name} cache differs by {diff.max()} bf16 ulps"
            assert (diff == 0).mean() >= 0.99, f"{name} exact fraction {(diff == 0).mean()}"
    finally:
        eng.close()
        dw.free()


def test_set_get_kv_roundtrip_and_synthetic_prefill():
    eng, orc, dw = make_pair(TINY, 9, 300)
    try:
        s = TINY
        n = 200
        eng.fill_kv_synthetic(n, 42)
        got = eng.get_kv(n)
        for layer in range(s.n_layers):
            for kv in range(2):
                ref = synth.kv_prefill_bits(42, layer, kv, n, s.n_kv_heads, s.head_dim)
                assert np.array_equal(got[layer, kv], ref), (layer, kv)
        rng = np.random.default_rng(0)
        host = rng.integers(0, 1 << 15, size=got.shape, dtype=np.uint16)
        eng.set_kv(host)
        assert eng.pos == n
        assert np.array_equal(eng.get_kv(n), host)
    finally:
        eng.close()
        dw.free()


@pytest.mark.parametrize("ctx,chunk,merge", [(200, 256, None), (1500, 64, None), (1500, 64, 64), (5000, 256, 4),
                                             (8192, 256, None), (8192, 256, 8), (32768, 256, None)])
def test_long_context_split_attention(ctx, chunk, merge):
    """Prefilled cache + multi-split attention vs the oracle (BASELINE configs[3]
    positions 8192 and 32768 included: 32 splits of up to 32 blocks).  Beyond
    `merge` splits per kv head (default 20) the first split's workgroup merges
    them and the O phase reads one merged partial; at or below it every O
    workgroup merges the splits."""
    shape = BASELINE.with_(n_layers=2, vocab=2048)
    eng, orc, dw = make_pair(shape, 21, ctx + 8)
    try:
        eng.set_attention_chunk(chunk)
        if merge is not None:
            eng.set_attention_merge(merge)
        eng.fill_kv_synthetic(ctx, 77)
        ks = np.stack([synth.kv_prefill_bits(77, l, 0, ctx, shape.n_kv_heads, shape.head_dim)
                       for l in range(shape.n_layers)])
        vs = np.stack([synth.kv_prefill_bits(77, l, 1, ctx, shape.n_kv_heads, shape.head_dim)
                       for l in range(shape.n_layers)])
        orc.set_kv(ks, vs)
        tok = 3
        for i in range(3):
            _print(f"ctx {ctx} chunk {chunk} step {i}")
            nxt, layers, logits = eng.debug_forward(tok)
            ref = orc.step(tok, capture=True)
            check_step(layers, logits, ref, f"ctx {ctx} step {i}")
            tok = ref["token"]
    finally:
        eng.close()
        dw.free()


def test_long_context_class_kernel_chunk():
    """Past eight 512-position splits per kv head the launch widens its
    attention chunk (at most 640 positions) so that eight splits hold the
    context and the class kernel runs: ctx 4,200 takes chunks of 544, then
    launches ending past 4,352 positions take 576 (a new split layout, the
    packed-pair words cleared between them).  Debug steps at the bars, then
    three 60-token launches teacher-forced against the oracle."""
    shape = BASELINE.with_(n_layers=2, vocab=2048)
    ctx = 4200
    eng, orc, dw = make_pair(shape, 23, ctx + 256)
    try:
        eng.fill_kv_synthetic(ctx, 78)
        ks = np.stack([synth.kv_prefill_bits(78, l, 0, ctx, shape.n_kv_heads, shape.head_dim)
                       for l in range(shape.n_layers)])
        vs = np.stack([synth.kv_prefill_bits(78, l, 1, ctx, shape.n_kv_heads, shape.head_dim)
                       for l in range(shape.n_layers)])
        orc.set_kv(ks, vs)
        assert eng.decode_kernel_for(1) == _lib.KERNEL_CLASS
        tok = 3
        for i in range(2):
            _print(f"ctx {ctx} step {i}")
            nxt, layers, logits = eng.debug_forward(tok)
            ref = orc.step(tok, capture=True)
            check_step(layers, logits, ref, f"ctx {ctx} step {i}")
            tok = ref["token"]
        for j in range(3):
            assert eng.decode_kernel_for(60) == _lib.KERNEL_CLASS
            gen = eng.decode_many(tok, 60)
            same, low = check_tokens_teacher_forced([tok] + gen[:-1], gen, orc)
            _print(f"  launch {j} at {eng.pos - 60}: {same} identical, {low} low-margin")
            tok = gen[-1]
    finally:
        eng.close()
        dw.free()


def test_reconfigure_and_rewind_between_launches():
    """The packed-pair hand-off words are not cleared before each launch, only
    when the position moves back or the split / merge configuration changes.
    Toggling the merge off for five tokens (the merged row's 4-bit tag then
    repeats: 5 x 141 phases is a multiple of 15) and back on, then rewinding,
    must still match the oracle and reproduce earlier steps bit for bit; a
    rewound resident launch must equal per-token decoding from the same point."""
    shape = BASELINE.with_(n_layers=2, vocab=2048)
    ctx = 2000
    eng, orc, dw = make_pair(shape, 31, ctx + 64)
    try:
        eng.set_attention_chunk(64)  # 32 splits per kv head at ctx 2000: above merge_min 20
        eng.fill_kv_synthetic(ctx, 5)
        ks = np.stack([synth.kv_prefill_bits(5, l, 0, ctx, shape.n_kv_heads, shape.head_dim)
                       for l in range(shape.n_layers)])
        vs = np.stack([synth.kv_prefill_bits(5, l, 1, ctx, shape.n_kv_heads, shape.head_dim)
                       for l in range(shape.n_layers)])
        orc.set_kv(ks, vs)
        tok, first = 9, []
        for i, merge in enumerate([20, 20, 20, 64, 64, 64, 64, 64, 20, 20]):
            eng.set_attention_merge(merge)
            _print(f"step {i} pos {eng.pos} merge_min {merge}")
            nxt, layers, logits = eng.debug_forward(tok)
            ref = orc.step(tok, capture=True)
            check_step(layers, logits, ref, f"step {i} merge_min {merge}")
            first.append((tok, logits))
            tok = ref["token"]
        # rewind to step 1 (same merge_min as then): bitwise the same step
        eng.set_attention_merge(20)
        eng.set_pos(ctx + 1)
        _, _, again = eng.debug_forward(first[1][0])
        assert np.array_equal(again, first[1][1]), "rewound step differs from the first pass"
        eng.set_pos(ctx)
        gen = eng.decode_many(first[0][0], 8)
        eng.set_pos(ctx)
        b = [eng.decode_token(first[0][0])]
        for _ in range(7):
            b.append(eng.decode_token(b[-1]))
        assert gen == b, "rewound resident launch and per-token decode disagree"
    finally:
        eng.close()
        dw.free()


def test_full_baseline_model_parity():
    """The BASELINE model at full size (28 layers, vocab 151936)."""
    eng, orc, dw = make_pair(BASELINE, 2024, 64, gain_std=0.0, bits_from_device=True)
    try:
        prompt = synth.prompt_tokens(2024, 4, BASELINE.vocab)
        tok = prompt[0]
        for i in range(6):
            tin = prompt[i] if i < len(prompt) else tok
            _print(f"full model step {i} token {tin}")
            nxt, layers, logits = eng.debug_forward(tin)
            ref = orc.step(tin, capture=True)
            l2, la = check_step(layers, logits, ref, f"full step {i}")
            _print(f"  relL2 {l2:.2e} logits abs {la:.2e} margin {qwen3_ref.top2_margin(ref['logits']):.3f}")
            if nxt != ref["token"]:
                assert qwen3_ref.top2_margin(ref["logits"]) <= 2e-2
            tok = nxt
    finally:
        eng.close()
        dw.free()


def test_determinism_bitwise():
    """Two identical runs produce bitwise-identical logits and tokens."""
    eng, _, dw = make_pair(BASELINE_2L, 8, 128)
    try:
        outs = []
        for _ in range(2):
            eng.reset()
            eng.fill_kv_synthetic(60, 1)
            _, layers, logits = eng.debug_forward(17)
            toks = eng.decode_many(5, 20)
            outs.append((layers, logits, toks))
        assert np.array_equal(outs[0][0], outs[1][0])
        assert np.array_equal(outs[0][1], outs[1][1])
        assert outs[0][2] == outs[1][2]
    finally:
        eng.close()
        dw.free()


def test_error_paths():
    """Bad inputs are rejected on the host with an error, not run."""
    eng, _, dw = make_pair(TINY, 1, 16)
    lib = eng.lib
    try:
        assert lib.megakernel_decode(eng._handle, TINY.vocab) == -1
        assert "token id" in _lib.last_error(lib)
        eng.set_pos(16)
        assert lib.megakernel_decode(eng._handle, 1) == -1
        assert "exceeds KV capacity" in _lib.last_error(lib)
        eng.reset()
        assert eng.pos == 0
        assert eng.decode_token(1) >= 0
    finally:
        eng.close()
        dw.free()


@pytest.mark.parametrize("chunk,merge", [(64, None), (32, 4)])
def test_qwen3_preset_head_dim_128(chunk, merge):
    """The reference's own config.cuh shapes (head_dim 128, ffn 3072); chunk 32
    gives 10 splits, merged by the first split's workgroup (merge threshold 4)."""
    shape = QWEN3_06B.with_(n_layers=2, vocab=2048)
    eng, orc, dw = make_pair(shape, 31, 400)
    try:
        eng.set_attention_chunk(chunk)
        if merge is not None:
            eng.set_attention_merge(merge)
        eng.fill_kv_synthetic(300, 5)
        ks = np.stack([synth.kv_prefill_bits(5, l, 0, 300, shape.n_kv_heads, shape.head_dim) for l in range(2)])
        vs = np.stack([synth.kv_prefill_bits(5, l, 1, 300, shape.n_kv_heads, shape.head_dim) for l in range(2)])
        orc.set_kv(ks, vs)
        tok = 11
        for i in range(3):
            nxt, layers, logits = eng.debug_forward(tok)
            ref = orc.step(tok, capture=True)
            check_step(layers, logits, ref, f"qwen3 step {i}")
            tok = ref["token"]
    finally:
        eng.close()
        dw.free()


@pytest.mark.parametrize("which,prefix,prompt_len", [("tiny", 20, 37), ("baseline_2l", 300, 70), ("tiny", 0, 1)])
def test_batch1_prefill_then_decode(which, prefix, prompt_len):
    """megakernel_prefill on a batch-1 handle (up to 1,024 prompt tokens per weight
    pass, the batched kernels on this handle's own cache), then decode: the
    token after the prompt and the following steps against the oracle stepped
    through the same prompt; the prompt's layer-0 K / V (which depend on each
    token alone) equal bf16 of the oracle's (check_kv_bf16)."""
    shape = TINY if which == "tiny" else BASELINE.with_(n_layers=2, vocab=2048)
    eng, orc, dw = make_pair(shape, 51, prefix + prompt_len + 16)
    try:
        eng.attach_prefill(dw)
        if prefix:
            eng.fill_kv_synthetic(prefix, 9)
            ks = np.stack([synth.kv_prefill_bits(9, l, 0, prefix, shape.n_kv_heads, shape.head_dim)
                           for l in range(shape.n_layers)])
            vs = np.stack([synth.kv_prefill_bits(9, l, 1, prefix, shape.n_kv_heads, shape.head_dim)
                           for l in range(shape.n_layers)])
            orc.set_kv(ks, vs)
        rng = np.random.default_rng(prompt_len)
        prompt = [int(t) for t in rng.integers(0, shape.vocab, size=prompt_len)]
        print(f"batch-1 prefill {which} prefix {prefix} prompt {prompt_len}", flush=True)
        nxt = eng.prefill(prompt)
        assert eng.pos == prefix + prompt_len
        ref = None
        for t in prompt:
            ref = orc.step(t, capture=True)
        if nxt != ref["token"]:
            assert qwen3_ref.top2_margin(ref["logits"]) <= 2e-2, f"prefill token {nxt} != oracle {ref['token']}"
        got = eng.get_kv(prefix + prompt_len)[0, :, :, prefix:, :]  # layer 0: [2][NKV][len][D]
        want = np.stack([orc.k_cache[0, :, prefix:prefix + prompt_len].contiguous().view(torch.int16).numpy(),
                         orc.v_cache[0, :, prefix:prefix + prompt_len].contiguous().view(torch.int16).numpy()]
                        ).view(np.uint16)
        check_kv_bf16(got, want, "layer-0 prompt KV")
        tok = ref["token"]
        for i in range(3):
            _, layers, logits = eng.debug_forward(tok)
            r = orc.step(tok, capture=True)
            check_step(layers, logits, r, f"decode {i} after prefill")
            tok = r["token"]
    finally:
        eng.close()
        dw.free()


def test_batch1_generate_with_prefill_matches_oracle():
    """generate_ids with the prefill context: the prompt in one call, then the
    greedy continuation in one resident launch, against the oracle."""
    shape = TINY
    eng, orc, dw = make_pair(shape, 52, 128, gain_std=0.0)
    try:
        eng.attach_prefill(dw)
        prompt = synth.prompt_tokens(52, 21, shape.vocab)
        gen, _ = eng.generate_ids(prompt, max_tokens=12)
        ref = None
        for t in prompt:
            ref = orc.step(t, capture=True)
        toks = [ref["token"]]
        margins = [qwen3_ref.top2_margin(ref["logits"])]
        for _ in range(11):
            r = orc.step(toks[-1], capture=True)
            toks.append(r["token"])
            margins.append(qwen3_ref.top2_margin(r["logits"]))
        for i, (a, b) in enumerate(zip(gen, toks)):
            if a != b:  # a near-tie may flip; everything after it is a different continuation
                assert margins[i] <= 2e-2, f"token {i}: {a} != oracle {b} (margin {margins[i]:.4f})"
                break
    finally:
        eng.close()
        dw.free()


def test_batch1_prefill_errors():
    shape = TINY
    eng, _, dw = make_pair(shape, 53, 32)
    try:
        with pytest.raises(_lib.MegakernelError, match="attach"):
            eng.prefill([1, 2])
        eng.attach_prefill(dw)
        with pytest.raises(_lib.MegakernelError, match="capacity"):
            eng.prefill([1] * 33)
        with pytest.raises(_lib.MegakernelError, match="token"):
            eng.prefill([shape.vocab])
        assert eng.pos == 0
        eng.prefill([3] * 32)
        assert eng.pos == 32
    finally:
        eng.close()
        dw.free()
    q = QWEN3_06B.with_(n_layers=1, vocab=256)
    eng, _, dw = make_pair(q, 54, 16)
    try:
        with pytest.raises(_lib.MegakernelError, match="BASELINE and TINY"):
            eng.attach_prefill(dw)
    finally:
        eng.close()
        dw.free()


@pytest.mark.parametrize("use_prefill", [False, True])
def test_generate_text_stops_at_eos(use_prefill, capsys):
    """MegakernelEngine.generate (reference host/bridge.py:118-192) with a
    byte tokenizer.  The engine's greedy ids, fed back to the oracle after the
    same prompt, equal the oracle's argmax wherever its top-1/top-2 margin
    exceeds 2e-2.  With EOS set to the engine's k-th token (its first
    occurrence; k >= 2 when the continuation has a new token there) generation
    stops right after it (EOS included), print_stream prints each token as it
    comes, and the returned text is the decoded prompt + generation with
    special tokens skipped."""
    from megakernel_amd.tokenizer import ByteTokenizer
    shape = TINY
    eng, orc, dw = make_pair(shape, 61, 128)
    try:
        if use_prefill:
            eng.attach_prefill(dw)
        prompt = "greedy decode on gfx950"
        ids = ByteTokenizer(shape.vocab).encode(prompt)
        free, _ = eng.generate_ids(ids, max_tokens=12)  # no EOS: 12 tokens
        for t in ids[:-1]:
            orc.step(t)
        check_tokens_teacher_forced([ids[-1]] + free[:-1], free, orc)
        firsts = [i for i in range(len(free)) if free[i] not in free[:i]]
        k = next((i for i in firsts if i >= 2), firsts[-1])
        tok = ByteTokenizer(shape.vocab, eos_token_id=free[k])
        eng.tokenizer = tok
        gen, _ = eng.generate_ids(ids, max_tokens=12, eos_id=tok.eos_token_id)
        assert gen == free[:k + 1], f"with EOS {free[k]}: {gen}, expected {free[:k + 1]}"
        capsys.readouterr()
        text, tps = eng.generate(prompt, max_tokens=12, print_stream=True)
        printed = capsys.readouterr().out
        assert text == tok.decode(ids + free[:k + 1], skip_special_tokens=True)
        assert printed == "".join(tok.decode([t]) for t in free[:k + 1]) + "\n"
        assert k == 0 or tps > 0
    finally:
        eng.close()
        dw.free()


def test_dataflow_handoff_selftest():
    """The hand-off primitive on its own, across every CU and XCD: 20,000
    all-gather rounds of tagged words (full tags and 4-bit packed pairs) with
    the decode kernel's write-through stores and agent-scope polling loads;
    no word may be accepted with the right tag and a wrong value."""
    lib = _lib.load()
    bad, us = ctypes.c_int(-1), ctypes.c_float(0.0)
    rc = lib.megakernel_selftest_dataflow(20000, ctypes.byref(bad), ctypes.byref(us))
    print(f"selftest: mismatches {bad.value}, {us.value:.2f} us per all-gather round", flush=True)
    assert rc == 0, _lib.last_error(lib)
    assert bad.value == 0
    assert 0.0 < us.value < 100.0


def test_bridge_benchmark_and_sweep():
    """MegakernelEngine.benchmark (the reference bridge's per-call loop: five
    warm-up tokens, reset, num_tokens timed calls) and benchmark_sweep (KV
    prefilled to each position, one timed resident launch): positive finite
    rates, the position they leave behind, and bandwidth figures under the
    HBM peak; the per-call loop's tokens are those of one resident launch."""
    eng, orc, dw = make_pair(BASELINE_2L, 83, 640)
    try:
        tps = eng.benchmark(num_tokens=20, prompt_token=3)
        _print(f"benchmark: {tps:.1f} tok/s")
        assert np.isfinite(tps) and tps > 0 and eng.pos == 20
        eng.reset()
        per_call = [eng.decode_token(3)]
        for _ in range(19):
            per_call.append(eng.decode_token(per_call[-1]))
        eng.reset()
        assert eng.decode_many(3, 20) == per_call
        res = eng.benchmark_sweep(positions=[1, 100, 500], bench_tokens=8)
        _print("sweep: " + ", ".join(f"{r['position']}: {r['tok_per_sec']:.0f} tok/s" for r in res))
        assert [r["position"] for r in res] == [1, 100, 500]
        for r in res:
            assert r["tok_per_sec"] > 0 and r["latency_us"] > 0 and 0 < r["bw_util"] < 1.0
        assert eng.pos == 500 + 8
    finally:
        eng.close()
        dw.free()
