"""The oracle against the committed HF transformers Qwen3 fixtures.

Fixtures (tests/golden/make_golden.py) were produced by HF's own
Qwen3ForCausalLM (fp32, eager attention, fp32 KV cache) on the repo's
synthetic weights.  In fp32-KV mode the oracle must reproduce them to fp32
round-off; in its default bf16-KV mode (the reference's cache policy) it must
stay within the north_star bars.
"""
import numpy as np
import pytest
import torch

from oracle import layout, qwen3_ref, synth

FIXTURES = ["tiny", "baseline_2l"]


def _load(name):
    z = np.load(f"tests/golden/hf_qwen3_{name}.npz")
    sh = layout.Shape(*[int(v) for v in z["shape"]])
    bits = qwen3_ref.synthetic_bits(sh, int(z["seed"]), std=float(z["std"]), gain_std=float(z["gain_std"]))
    return z, sh, bits


@pytest.mark.parametrize("name", FIXTURES)
def test_fixture_inputs_are_the_synthetic_prompt(name):
    z, sh, _ = _load(name)
    n_prompt = {"tiny": 5, "baseline_2l": 4}[name]
    assert z["tokens_fed"][:n_prompt].tolist() == synth.prompt_tokens(int(z["seed"]), n_prompt, sh.vocab)


@pytest.mark.parametrize("name", FIXTURES)
def test_oracle_fp32_kv_reproduces_hf(name):
    z, sh, bits = _load(name)
    o = qwen3_ref.Qwen3Oracle(sh, bits, 64, kv_dtype=torch.float32)
    for i, t in enumerate(z["tokens_fed"]):
        r = o.step(int(t), capture=True)
        np.testing.assert_allclose(r["layers"].numpy(), z["layers"][i], rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(r["logits"].numpy(), z["logits"][i], rtol=1e-5, atol=1e-5)
        assert r["token"] == int(z["next_tokens"][i])


@pytest.mark.parametrize("name", FIXTURES)
def test_oracle_bf16_kv_within_bars(name):
    z, sh, bits = _load(name)
    o = qwen3_ref.Qwen3Oracle(sh, bits, 64)
    for i, t in enumerate(z["tokens_fed"]):
        r = o.step(int(t), capture=True)
        ref = z["layers"][i]
        rel = np.linalg.norm(r["layers"].numpy() - ref, axis=1) / np.linalg.norm(ref, axis=1)
        assert rel.max() <= 1e-2
        assert np.abs(r["logits"].numpy() - z["logits"][i]).max() <= 2e-2
        if r["token"] != int(z["next_tokens"][i]):
            lg = torch.from_numpy(z["logits"][i])
            assert qwen3_ref.top2_margin(lg) <= 2e-2


def test_planted_mistake_is_caught():
    """A plausible oracle bug (RoPE pairs rotated the wrong way) must fail the
    HF comparison, i.e. the fixture actually pins the rotation direction."""
    z, sh, bits = _load("tiny")
    orig = qwen3_ref.rope
    try:
        qwen3_ref.rope = lambda x, pos, theta: orig(x, -pos, theta)
        o = qwen3_ref.Qwen3Oracle(sh, bits, 64, kv_dtype=torch.float32)
        errs = []
        for i, t in enumerate(z["tokens_fed"]):
            r = o.step(int(t), capture=True)
            errs.append(np.abs(r["logits"].numpy() - z["logits"][i]).max())
        assert max(errs) > 1e-3
    finally:
        qwen3_ref.rope = orig
