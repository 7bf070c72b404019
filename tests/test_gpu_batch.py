"""GPU parity of the batched decode (megakernel_decode_batch and friends,
BASELINE configs[4]) against the CPU oracle, one oracle state per sequence.

Bars: fp32 logits within 2e-2 abs, greedy tokens
identical wherever the oracle's top-1/top-2 margin exceeds 2e-2; KV bytes
appended by a step equal the oracle's bf16 K / V (at most 1 ulp on < 1 % of
entries, fp32 summation order).  Sequences have different cache lengths,
including an empty cache and lengths that straddle the 128-position
attention splits.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from megakernel_amd import _lib
from megakernel_amd.batch import PREFILL_PASS_TOKENS, BatchEngine
from megakernel_amd.config import BASELINE, TINY
from megakernel_amd.weights import DeviceWeights
from oracle import qwen3_ref, synth

from ._helpers import LOGIT_ABS, MARGIN, check_kv_bf16, oracle_shape

pytestmark = pytest.mark.gpu


def _print(*a):
    print(*a, flush=True)


class MultiOracle:
    """One Qwen3Oracle (one copy of the weights) serving several sequences:
    each sequence has its own KV cache tensors and position."""

    def __init__(self, shape, dw, n_seq: int, max_seq: int, kv_fp8: bool = False):
        osh = oracle_shape(shape)
        bits = qwen3_ref.unpack_flat(osh, dw.to_host(), dw.layout.offsets)
        self.orc = qwen3_ref.Qwen3Oracle(osh, bits, max_seq, kv_fp8=kv_fp8)
        self.caches = [(self.orc.k_cache.clone(), self.orc.v_cache.clone()) for _ in range(n_seq)]
        self.pos = [0] * n_seq
        self.shape = shape

    def prefill(self, seq: int, length: int, seed: int):
        s = self.shape
        ks = np.stack([synth.kv_prefill_bits(seed, l, 0, length, s.n_kv_heads, s.head_dim)
                       for l in range(s.n_layers)])
        vs = np.stack([synth.kv_prefill_bits(seed, l, 1, length, s.n_kv_heads, s.head_dim)
                       for l in range(s.n_layers)])
        k, v = self.caches[seq]
        k.zero_()
        v.zero_()
        k[:, :, :length] = self.orc._kv_rows(qwen3_ref.bits_to_torch(ks).float())
        v[:, :, :length] = self.orc._kv_rows(qwen3_ref.bits_to_torch(vs).float())
        self.pos[seq] = length

    def step(self, seq: int, token: int) -> dict:
        self.orc.k_cache, self.orc.v_cache = self.caches[seq]
        self.orc.pos = self.pos[seq]
        r = self.orc.step(int(token), capture=True)
        self.pos[seq] = self.orc.pos
        return r


def _setup(shape, seed, lengths, max_seq, kv_fp8: bool = False):
    dw = DeviceWeights(shape, seed, std=0.02, gain_std=0.1)
    eng = BatchEngine(dw, len(lengths), max_seq, shape)
    if kv_fp8:
        eng.set_kv_fp8(True)
    mo = MultiOracle(shape, dw, len(lengths), max_seq, kv_fp8=kv_fp8)
    for b, n in enumerate(lengths):
        eng.fill_kv_synthetic(b, n, 500 + b)
        mo.prefill(b, n, 500 + b)
    assert eng.positions() == list(lengths)
    return dw, eng, mo


def _check_step(logits, toks, refs, label):
    worst = 0.0
    for b, r in enumerate(refs):
        err = float(np.abs(logits[b] - r["logits"].numpy()).max())
        worst = max(worst, err)
        assert err <= LOGIT_ABS, f"{label} seq {b}: logits max abs err {err:.3e}"
        if toks[b] != r["token"]:
            m = qwen3_ref.top2_margin(r["logits"])
            assert m <= MARGIN, f"{label} seq {b}: token {toks[b]} != oracle {r['token']} (margin {m:.4f})"
    return worst


def test_batch_tiny_parity():
    """4 sequences (empty cache, 5, 127 and 200 cached positions), 4 steps."""
    lengths = [0, 5, 127, 200]
    dw, eng, mo = _setup(TINY, 31, lengths, 256)
    try:
        toks = [7, 100, 3, 999]
        for i in range(4):
            _print(f"batch tiny step {i} tokens {toks}")
            out, logits = eng.debug_logits(toks)
            refs = [mo.step(b, toks[b]) for b in range(len(lengths))]
            worst = _check_step(logits, out, refs, f"step {i}")
            _print(f"  worst logits abs err {worst:.2e}")
            toks = out
        assert eng.positions() == [n + 4 for n in lengths]
    finally:
        eng.close()
        dw.free()


def test_batch_generate_equals_decode_and_oracle():
    """generate (graph replays) == repeated decode == oracle, teacher-forced."""
    lengths = [3, 130, 64, 1]
    dw, eng, mo = _setup(TINY, 32, lengths, 256)
    eng2 = BatchEngine(dw, len(lengths), 256, TINY)
    try:
        for b, n in enumerate(lengths):
            eng2.fill_kv_synthetic(b, n, 500 + b)
        first = [11, 22, 33, 44]
        n_steps = 6
        gen = eng.generate(first, n_steps)
        _print(f"batch generate {gen.tolist()}")
        toks = first
        for i in range(n_steps):
            out = eng2.decode(toks)
            assert out == gen[i].tolist(), f"step {i}: decode {out} != generate {gen[i].tolist()}"
            refs = [mo.step(b, toks[b]) for b in range(len(lengths))]
            for b, r in enumerate(refs):
                if out[b] != r["token"]:
                    assert qwen3_ref.top2_margin(r["logits"]) <= MARGIN
            toks = out
    finally:
        eng.close()
        eng2.close()
        dw.free()


def test_batch_kv_append_bytes():
    """The K / V a step appends equal bf16 of the oracle's post-norm, post-RoPE k and v."""
    lengths = [0, 40, 129]
    dw, eng, mo = _setup(TINY, 33, lengths, 256)
    try:
        toks = [5, 6, 7]
        eng.decode(toks)
        for b, n in enumerate(lengths):
            mo.step(b, toks[b])
            got = eng.get_kv(b, n + 1)[:, :, :, n, :]  # [L][2][NKV][D]
            k, v = mo.caches[b]
            want = np.stack([k[:, :, n].contiguous().view(torch.int16).numpy(),
                             v[:, :, n].contiguous().view(torch.int16).numpy()], axis=1).view(np.uint16)
            diff = np.abs(got.astype(np.int32) - want.astype(np.int32))
            assert diff.max() <= 1, f"seq {b}: KV bytes differ by up to {diff.max()} ulp"
            assert (diff > 0).mean() < 0.01, f"seq {b}: {(diff > 0).mean():.3%} of KV entries off by 1 ulp"
            # the prefix is untouched
            pre = eng.get_kv(b, n)
            ks = np.stack([synth.kv_prefill_bits(500 + b, l, 0, n, TINY.n_kv_heads, TINY.head_dim)
                           for l in range(TINY.n_layers)])
            assert np.array_equal(pre[:, 0], ks)
    finally:
        eng.close()
        dw.free()


def test_batch_baseline_2l_16_sequences():
    """BASELINE shapes, 2 layers, 16 sequences with lengths drawn from a seed."""
    shape = BASELINE.with_(n_layers=2, vocab=4096)
    rng = np.random.default_rng(7)
    lengths = [int(x) for x in rng.integers(0, 700, size=16)]
    dw, eng, mo = _setup(shape, 34, lengths, 720)
    try:
        toks = [int(t) for t in rng.integers(0, shape.vocab, size=16)]
        for i in range(3):
            _print(f"batch baseline-2l step {i} lengths {eng.positions()}")
            out, logits = eng.debug_logits(toks)
            refs = [mo.step(b, toks[b]) for b in range(16)]
            worst = _check_step(logits, out, refs, f"step {i}")
            _print(f"  worst logits abs err {worst:.2e}")
            toks = out
    finally:
        eng.close()
        dw.free()


def test_batch_full_model_16_sequences():
    """The full 28-layer BASELINE model (vocab 151936), 16 sequences, 2 steps."""
    rng = np.random.default_rng(8)
    lengths = [int(x) for x in rng.integers(1, 300, size=16)]
    dw, eng, mo = _setup(BASELINE, 35, lengths, 320)
    try:
        toks = [int(t) for t in rng.integers(0, BASELINE.vocab, size=16)]
        for i in range(2):
            _print(f"batch full model step {i}")
            out, logits = eng.debug_logits(toks)
            refs = [mo.step(b, toks[b]) for b in range(16)]
            worst = _check_step(logits, out, refs, f"step {i}")
            _print(f"  worst logits abs err {worst:.2e}")
            toks = out
    finally:
        eng.close()
        dw.free()


def test_batch_error_paths():
    dw = DeviceWeights(TINY, 36)
    try:
        with pytest.raises(_lib.MegakernelError, match="n_seq"):
            BatchEngine(dw, 17, 64, TINY)
        eng = BatchEngine(dw, 2, 16, TINY)
        try:
            with pytest.raises(_lib.MegakernelError, match="token id"):
                eng.decode([0, TINY.vocab])
            eng.fill_kv_synthetic(1, 16, 1)
            with pytest.raises(_lib.MegakernelError, match="exceeds KV capacity"):
                eng.decode([1, 2])
            with pytest.raises(_lib.MegakernelError):
                eng.fill_kv_synthetic(2, 1, 1)
        finally:
            eng.close()
    finally:
        dw.free()


# ------------------------------------------------------------------ prefill
def _prefill_case(shape, seed, prefix, prompt_len, other_len, max_seq):
    """Sequence 1 gets a synthetic prefix of `prefix` positions and then a
    prompt of prompt_len tokens through megakernel_batch_prefill; sequence 0
    (other_len cached positions) must be left untouched."""
    lengths = [other_len, prefix]
    dw, eng, mo = _setup(shape, seed, lengths, max_seq)
    rng = np.random.default_rng(seed)
    prompt = [int(t) for t in rng.integers(0, shape.vocab, size=prompt_len)]
    before0 = eng.get_kv(0, other_len)
    _print(f"prefill prefix={prefix} prompt={prompt_len} ({(prompt_len + 15) // 16} column groups)")
    nxt, logits = eng.prefill(1, prompt, with_logits=True)
    ref = None
    for t in prompt:
        ref = mo.step(1, t)
    err = float(np.abs(logits - ref["logits"].numpy()).max())
    _print(f"  next token {nxt} (oracle {ref['token']}), logits max abs err {err:.2e}")
    assert err <= LOGIT_ABS
    if nxt != ref["token"]:
        assert qwen3_ref.top2_margin(ref["logits"]) <= MARGIN
    assert eng.positions() == [other_len, prefix + prompt_len]
    # the prompt's K / V against the oracle's: layer 0 depends on each token
    # alone (bf16 of the same fp32 values, check_kv_bf16);
    # deeper layers carry the earlier tokens' attention, so they are held to
    # the per-layer bar (relative L2 <= 1e-2)
    got = eng.get_kv(1, prefix + prompt_len)[:, :, :, prefix:, :]
    k, v = mo.caches[1]
    want = np.stack([k[:, :, prefix:prefix + prompt_len].contiguous().view(torch.int16).numpy(),
                     v[:, :, prefix:prefix + prompt_len].contiguous().view(torch.int16).numpy()],
                    axis=1).view(np.uint16)
    check_kv_bf16(got[0], want[0], "layer-0 prompt KV")
    gf, wf = synth.bf16_bits_to_f32(got), synth.bf16_bits_to_f32(want)
    for layer in range(1, shape.n_layers):
        rel = float(np.linalg.norm(gf[layer] - wf[layer]) / np.linalg.norm(wf[layer]))
        _print(f"  layer {layer} prompt KV rel-L2 {rel:.2e}")
        assert rel <= 1e-2, f"layer {layer} prompt KV rel-L2 {rel:.3e}"
    assert np.array_equal(eng.get_kv(0, other_len), before0)
    return dw, eng, mo, nxt


def test_batch_prefill_tiny_multi_chunk():
    """37 prompt tokens (one pass, column groups of 16, 16, 5) after a 40-position prefix,
    then 3 decode steps of both sequences against the oracle."""
    dw, eng, mo, nxt = _prefill_case(TINY, 41, prefix=40, prompt_len=37, other_len=9, max_seq=128)
    try:
        toks = [3, nxt]
        for i in range(3):
            out, logits = eng.debug_logits(toks)
            refs = [mo.step(b, toks[b]) for b in range(2)]
            worst = _check_step(logits, out, refs, f"after prefill, step {i}")
            _print(f"  decode step {i}: worst logits abs err {worst:.2e}")
            toks = out
    finally:
        eng.close()
        dw.free()


@pytest.mark.parametrize("prompt_len", [1, 16])
def test_batch_prefill_tiny_edges(prompt_len):
    """One token, and exactly one full chunk, from an empty cache."""
    dw, eng, _, _ = _prefill_case(TINY, 42 + prompt_len, prefix=0, prompt_len=prompt_len, other_len=0,
                                  max_seq=64)
    eng.close()
    dw.free()


def test_batch_prefill_baseline_2l():
    """BASELINE shapes (2 layers): 70 prompt tokens after a 300-position prefix
    (five column groups of one pass straddle the 256-position attention
    splits)."""
    shape = BASELINE.with_(n_layers=2, vocab=4096)
    dw, eng, _, _ = _prefill_case(shape, 43, prefix=300, prompt_len=70, other_len=17, max_seq=400)
    eng.close()
    dw.free()


def test_batch_prefill_baseline_2l_two_passes():
    """A prompt longer than one pass (PREFILL_PASS_TOKENS): 1,030 tokens after
    a 100-position prefix are a full pass of 64 column groups and a second
    pass of one partial group, whose attention reads the first pass's K / V."""
    assert PREFILL_PASS_TOKENS == 1024
    shape = BASELINE.with_(n_layers=2, vocab=4096)
    dw, eng, _, _ = _prefill_case(shape, 45, prefix=100, prompt_len=1030, other_len=5, max_seq=1200)
    eng.close()
    dw.free()


def test_batch_prefill_baseline_2l_odd_large_pass():
    """A pass of 33 column groups (520 tokens after a 37-position prefix): the
    large-pass GEMM tiles (more than 32 groups) with column tiles that are
    only partly filled (2-group tiles of QKV / O / down and 8-group tiles of
    gate / up each end on one group, the last group half full), so the
    direct-to-LDS K loops load a stand-in group for the missing ones."""
    shape = BASELINE.with_(n_layers=2, vocab=4096)
    dw, eng, _, _ = _prefill_case(shape, 46, prefix=37, prompt_len=520, other_len=3, max_seq=600)
    eng.close()
    dw.free()


def test_batch_prefill_errors():
    dw = DeviceWeights(TINY, 44)
    eng = BatchEngine(dw, 2, 32, TINY)
    try:
        with pytest.raises(_lib.MegakernelError, match="exceeds KV capacity"):
            eng.prefill(0, [1] * 33)
        with pytest.raises(_lib.MegakernelError, match="token"):
            eng.prefill(0, [1, TINY.vocab])
        with pytest.raises(_lib.MegakernelError, match="sequence"):
            eng.prefill(2, [1])
        with pytest.raises(_lib.MegakernelError):
            eng.prefill(0, [])
        assert eng.positions() == [0, 0]
        eng.prefill(0, [5] * 32)  # fills the capacity exactly
        assert eng.positions() == [32, 0]
    finally:
        eng.close()
        dw.free()


# ------------------------------------------------------- FP8 KV caches (batch)
def test_batch_fp8_kv_16_sequences():
    """FP8 caches (e4m3, power-of-two row scales) for 16 BASELINE-shaped
    sequences against per-sequence oracles on the same dequantised caches:
    eager steps (logits), then graph steps (tokens)."""
    shape = BASELINE.with_(n_layers=2, vocab=4096)
    rng = np.random.default_rng(9)
    lengths = [int(x) for x in rng.integers(0, 700, size=16)]
    dw, eng, mo = _setup(shape, 35, lengths, 720, kv_fp8=True)
    try:
        toks = [int(t) for t in rng.integers(0, shape.vocab, size=16)]
        for i in range(3):
            _print(f"batch fp8 kv step {i} lengths {eng.positions()}")
            out, logits = eng.debug_logits(toks)
            refs = [mo.step(b, toks[b]) for b in range(16)]
            worst = _check_step(logits, out, refs, f"fp8 step {i}")
            _print(f"  worst logits abs err {worst:.2e}")
            toks = out
        out = eng.decode(toks)  # the captured step graph
        refs = [mo.step(b, toks[b]) for b in range(16)]
        for b, r in enumerate(refs):
            if out[b] != r["token"]:
                assert qwen3_ref.top2_margin(r["logits"]) <= MARGIN, f"graph step seq {b}"
    finally:
        eng.close()
        dw.free()


def test_batch_fp8_kv_fill_exact_and_prefill():
    """FP8 fills bit-exact against the oracle; a prompt prefilled into an FP8
    cache (bk_append quantising each row) gives the oracle's next token and
    logits on the same dequantised cache, and leaves the other sequences'
    caches untouched."""
    lengths = [0, 40, 129]
    dw, eng, mo = _setup(TINY, 36, lengths, 256, kv_fp8=True)
    try:
        for b, n in enumerate(lengths):
            if n == 0:
                continue
            got = eng.get_kv(b, n)
            k, v = mo.caches[b]
            for plane, want in ((0, k), (1, v)):
                wb = want[:, :, :n].to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)
                assert np.array_equal(got[:, plane], wb), f"seq {b} plane {plane}: FP8 rows differ"
        before2 = eng.get_kv(2, 129)
        prompt = [int(t) for t in np.random.default_rng(36).integers(0, TINY.vocab, size=37)]
        nxt, logits = eng.prefill(1, prompt, with_logits=True)
        ref = None
        for t in prompt:
            ref = mo.step(1, t)
        err = float(np.abs(logits - ref["logits"].numpy()).max())
        _print(f"fp8 prefill: next token {nxt} (oracle {ref['token']}), logits max abs err {err:.2e}")
        assert err <= LOGIT_ABS
        if nxt != ref["token"]:
            assert qwen3_ref.top2_margin(ref["logits"]) <= MARGIN
        assert eng.positions() == [0, 40 + 37, 129]
        assert np.array_equal(eng.get_kv(2, 129), before2)
        # decode continues on the FP8 caches after the prefill
        toks = [3, nxt, 5]
        out, logits = eng.debug_logits(toks)
        refs = [mo.step(b, toks[b]) for b in range(3)]
        _check_step(logits, out, refs, "decode after fp8 prefill")
    finally:
        eng.close()
        dw.free()


@pytest.mark.parametrize("which", ["tiny", "baseline_2l"])
def test_batch_fp8_lmhead(which):
    """The batched LM head on the FP8 copy (two MFMA k-steps per lane load, the
    row scale in the conversion) against per-sequence oracles using the same
    dequantised table; eager steps, then a graph step."""
    shape = TINY if which == "tiny" else BASELINE.with_(n_layers=2, vocab=4096)
    rng = np.random.default_rng(12)
    lengths = [int(x) for x in rng.integers(0, 200, size=16 if which != "tiny" else 4)]
    dw, eng, mo = _setup(shape, 37, lengths, 256)
    try:
        eng.set_lmhead_fp8(True)
        mo.orc.use_fp8_lm_head()
        toks = [int(t) for t in rng.integers(0, shape.vocab, size=len(lengths))]
        for i in range(2):
            _print(f"batch fp8 head {which} step {i}")
            out, logits = eng.debug_logits(toks)
            refs = [mo.step(b, toks[b]) for b in range(len(lengths))]
            worst = _check_step(logits, out, refs, f"fp8 head step {i}")
            _print(f"  worst logits abs err {worst:.2e}")
            toks = out
        out = eng.decode(toks)
        refs = [mo.step(b, toks[b]) for b in range(len(lengths))]
        for b, r in enumerate(refs):
            if out[b] != r["token"]:
                assert qwen3_ref.top2_margin(r["logits"]) <= MARGIN, f"graph step seq {b}"
    finally:
        eng.close()
        dw.free()



def _bench_lengths(seed: int = 2024, kv_min: int = 512, kv_max: int = 4096, n: int = 16):
    """The lengths bench.py --batch draws (same generator, same order)."""
    rng = np.random.default_rng(seed)
    return [int(x) for x in rng.integers(kv_min, kv_max + 1, size=n)], rng


@pytest.mark.parametrize("kv_fp8", [False, True])
def test_batch_bench_lengths_cross_17_splits(kv_fp8):
    """configs[4] at its real lengths: the 16 cache lengths bench.py draws
    (seed 2024, uniform in [512, 4096]); the longest sequence is moved to
    4,090 positions so that the steps carry it past 4,096 positions, i.e. 17
    attention splits of 256 and a second round of the last split's merge
    (16 splits per round).  BASELINE shapes, 2 layers, bf16 and FP8 caches."""
    shape = BASELINE.with_(n_layers=2, vocab=4096)
    lengths, rng = _bench_lengths()
    lengths[int(np.argmax(lengths))] = 4090
    dw, eng, mo = _setup(shape, 36, lengths, 4200, kv_fp8=kv_fp8)
    try:
        toks = [int(t) for t in rng.integers(0, shape.vocab, size=16)]
        for i in range(9):
            _print(f"batch bench lengths step {i} (fp8 {kv_fp8}): max position {max(eng.positions())}")
            out, logits = eng.debug_logits(toks)
            refs = [mo.step(b, toks[b]) for b in range(16)]
            worst = _check_step(logits, out, refs, f"step {i}")
            _print(f"  worst logits abs err {worst:.2e}")
            toks = out
        assert max(eng.positions()) == 4099
    finally:
        eng.close()
        dw.free()


def test_batch_full_model_long_sequences():
    """The full 28-layer model with 6 sequences, 4 of them above 3,000 cached
    positions (13-16 splits), 2 steps; the oracles' prefixes are the device's
    own synthetic prefill read back (the prefill itself is bit-exact against
    the CPU generator, test_batch_kv_append_bytes)."""
    lengths = [3100, 4001, 3555, 4090, 700, 1]
    dw = DeviceWeights(BASELINE, 37, std=0.02, gain_std=0.1)
    eng = BatchEngine(dw, len(lengths), 4100, BASELINE)
    mo = MultiOracle(BASELINE, dw, len(lengths), 4100)
    try:
        for b, n in enumerate(lengths):
            eng.fill_kv_synthetic(b, n, 600 + b)
            kv = eng.get_kv(b, n)  # [L][2][NKV][n][D]
            k, v = mo.caches[b]
            k[:, :, :n] = qwen3_ref.bits_to_torch(kv[:, 0]).to(k.dtype)
            v[:, :, :n] = qwen3_ref.bits_to_torch(kv[:, 1]).to(v.dtype)
            mo.pos[b] = n
        toks = [1, 2000, 151935, 77, 4096, 65000]
        for i in range(2):
            _print(f"batch full model long step {i} positions {eng.positions()}")
            out, logits = eng.debug_logits(toks)
            refs = [mo.step(b, toks[b]) for b in range(len(lengths))]
            worst = _check_step(logits, out, refs, f"step {i}")
            _print(f"  worst logits abs err {worst:.2e}")
            toks = out
    finally:
        eng.close()
        dw.free()


@pytest.mark.parametrize("name,kv_fp8,n_seq", [("tiny", False, 16), ("baseline_2l", False, 16),
                                               ("baseline_2l", True, 16), ("baseline_full", False, 16),
                                               ("tiny", False, 1), ("tiny", False, 5), ("tiny", False, 15),
                                               ("baseline_2l", False, 1), ("baseline_2l", False, 5),
                                               ("baseline_2l", False, 15)])
def test_batch_persistent_step_equals_per_phase_kernels(name, kv_fp8, n_seq):
    """The one-kernel step (bk_step: every layer in one persistent kernel,
    hand-offs through agent-scope counters) and the per-phase kernels compute
    the same sums in the same order: logits and tokens of 3 debug steps and a
    6-step graph generate are bit-identical, at the bench's cache lengths
    (seed 2024, 512-4096 positions: up to 16 attention splits per sequence),
    for 16 sequences and for 1, 5 and 15 (the first n_seq of the lengths:
    partial sequence tiles of the step's work split)."""
    shape = {"tiny": TINY, "baseline_2l": BASELINE.with_(n_layers=2, vocab=4096),
             "baseline_full": BASELINE}[name]
    lengths, rng = _bench_lengths()
    if name == "tiny":
        lengths = [0, 5, 127, 200, 31, 32, 33, 255, 256, 257, 400, 511, 1, 90, 300, 64]
    first = [int(t) for t in rng.integers(0, shape.vocab, size=16)][:n_seq]
    lengths = lengths[:n_seq]
    dw = DeviceWeights(shape, 41, std=0.02, gain_std=0.1)
    eng = BatchEngine(dw, n_seq, max(lengths) + 16, shape)
    try:
        if kv_fp8:
            eng.set_kv_fp8(True)
        runs = {}
        for variant in (_lib.BATCH_STEP_PER_PHASE, _lib.BATCH_STEP_PERSISTENT):
            eng.set_step_kernel(variant)
            for b, n in enumerate(lengths):
                eng.fill_kv_synthetic(b, n, 700 + b)
            toks, steps = list(first), []
            for i in range(3):
                _print(f"batch step variant {variant} {name} fp8 {kv_fp8} n_seq {n_seq} debug step {i}")
                out, logits = eng.debug_logits(toks)
                steps.append((list(out), logits.copy()))
                toks = out
            gen = eng.generate(toks, 6)
            runs[variant] = (steps, np.asarray(gen).copy(), eng.positions())
        (sa, ga, pa), (sb, gb, pb) = runs[_lib.BATCH_STEP_PER_PHASE], runs[_lib.BATCH_STEP_PERSISTENT]
        for i, ((ta, la), (tb, lb)) in enumerate(zip(sa, sb)):
            assert ta == tb, f"step {i}: tokens differ"
            assert np.array_equal(la, lb), f"step {i}: logits differ (max {np.abs(la - lb).max():.3e})"
        assert np.array_equal(ga, gb), "generated tokens differ"
        assert pa == pb == [n + 9 for n in lengths]
    finally:
        eng.close()
        dw.free()


@pytest.mark.parametrize("step", ["per-phase", "persistent"])
def test_batch_full_model_bench_workload_graph(step):
    """configs[4] as bench.py --batch 16 runs it: the full 28-layer model
    (vocab 151936, bench weights: seed 2024, gains 1), 16 sequences at the
    bench's cache lengths (seed 2024, uniform in [512, 4096]) and synthetic
    prefixes, the bench's first tokens, stepped through the captured step
    graph (decode: one replay; generate: chained replays).  Per-sequence
    oracles hold the device's own prefixes read back (layer 0 of each prefix
    is checked against the CPU generator first).  Two teacher-forced replays
    (both sides consume the oracle's tokens), then a two-step generate (the
    oracles consume the device's tokens); every device token must equal the
    oracle's argmax unless the oracle's top-1/top-2 margin is within 2e-2, and
    the K / V rows the four graph steps appended are held to the layer bar
    (relative L2 <= 1e-2 per layer, bf16 of the same fp32 values in layer 0)."""
    seed = 2024
    lengths, rng = _bench_lengths(seed)
    first = [int(t) for t in rng.integers(0, BASELINE.vocab, size=16)]
    dw = DeviceWeights(BASELINE, seed, std=0.02, gain_std=0.0)
    eng = BatchEngine(dw, 16, max(lengths) + 16, BASELINE)
    mo = MultiOracle(BASELINE, dw, 16, max(lengths) + 16)
    s = BASELINE
    try:
        eng.set_step_kernel(_lib.BATCH_STEP_PER_PHASE if step == "per-phase" else _lib.BATCH_STEP_PERSISTENT)
        for b, n in enumerate(lengths):
            eng.fill_kv_synthetic(b, n, seed + 1000 + b)
            kv = eng.get_kv(b, n)  # [L][2][NKV][n][D]
            if b in (0, 15):
                assert np.array_equal(kv[0, 0], synth.kv_prefill_bits(seed + 1000 + b, 0, 0, n, s.n_kv_heads,
                                                                      s.head_dim)), f"seq {b}: prefix K"
            k, v = mo.caches[b]
            k[:, :, :n] = qwen3_ref.bits_to_torch(kv[:, 0]).to(k.dtype)
            v[:, :, :n] = qwen3_ref.bits_to_torch(kv[:, 1]).to(v.dtype)
            mo.pos[b] = n
            del kv
        _print(f"batch bench workload ({step}): lengths {lengths}")
        mismatches = 0

        def check(out, refs, label):
            nonlocal mismatches
            for b, r in enumerate(refs):
                if out[b] != r["token"]:
                    m = qwen3_ref.top2_margin(r["logits"])
                    gap = float(r["logits"][r["token"]] - r["logits"][out[b]])
                    assert m <= MARGIN and gap <= MARGIN, (
                        f"{label} seq {b}: token {out[b]} != oracle {r['token']} (margin {m:.4f})")
                    mismatches += 1

        toks = list(first)
        for i in range(2):  # teacher-forced graph replays
            out = eng.decode(toks)
            refs = [mo.step(b, toks[b]) for b in range(16)]
            check(out, refs, f"decode replay {i}")
            _print(f"  replay {i}: tokens {out[:4]}... oracle {[r['token'] for r in refs[:4]]}...")
            toks = [r["token"] for r in refs]
        gen = eng.generate(toks, 2)  # chained replays
        for i in range(2):
            refs = [mo.step(b, toks[b]) for b in range(16)]
            check(gen[i].tolist(), refs, f"generate step {i}")
            toks = gen[i].tolist()
        _print(f"  generate: {gen[:, :4].tolist()}; low-margin mismatches {mismatches} of 64")
        assert eng.positions() == [n + 4 for n in lengths] == mo.pos
        for b in (0, 5, 10, 15):  # the rows the graph steps appended
            n = lengths[b]
            got = eng.get_kv(b, n + 4)[:, :, :, n:, :]
            k, v = mo.caches[b]
            want = np.stack([k[:, :, n:n + 4].contiguous().view(torch.int16).numpy(),
                             v[:, :, n:n + 4].contiguous().view(torch.int16).numpy()], axis=1).view(np.uint16)
            check_kv_bf16(got[0], want[0], f"seq {b} layer-0 KV of the graph steps")
            gf, wf = synth.bf16_bits_to_f32(got), synth.bf16_bits_to_f32(want)
            rel = [float(np.linalg.norm(gf[l] - wf[l]) / np.linalg.norm(wf[l])) for l in range(s.n_layers)]
            _print(f"  seq {b}: appended KV worst layer rel-L2 {max(rel):.2e}")
            assert max(rel) <= 1e-2, f"seq {b}: appended KV rel-L2 {max(rel):.3e}"
    finally:
        eng.close()
        dw.free()
