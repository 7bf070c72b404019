"""Closed-form and invariant checks of every op of the oracle
(oracle/qwen3_ref.py), each chosen so that a plausible slip fails it: sum for
mean in RMSNorm, a flipped or mis-paired RoPE rotation, a wrong GQA head
mapping, a missing 1/sqrt(D), a wrong SiLU, the last instead of the first
index on argmax ties."""
import numpy as np
import pytest
import torch

from oracle import qwen3_ref as q

RNG = np.random.default_rng(5)


def test_rmsnorm_brute_force_scale_invariance_unit_rms():
    x = torch.from_numpy(RNG.standard_normal(1024).astype(np.float32))
    w = torch.from_numpy((1 + 0.1 * RNG.standard_normal(1024)).astype(np.float32))
    y = q.rmsnorm(x, w, 1e-6)
    xd = x.double().numpy()
    ref = xd / np.sqrt(np.mean(xd * xd) + 1e-6) * w.double().numpy()
    np.testing.assert_allclose(y.numpy(), ref, rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(q.rmsnorm(7.25 * x, w, 1e-6).numpy(), y.numpy(), rtol=1e-5, atol=1e-6)
    u = q.rmsnorm(x, torch.ones(1024), 1e-6)
    assert abs(float(u.pow(2).mean().sqrt()) - 1.0) < 1e-5


def test_inv_freq_closed_form():
    for d in (64, 128):
        got = q.inv_freq(d, 1e6).double().numpy()
        ref = 1.0 / (1e6 ** (np.arange(0, d, 2) / d))
        np.testing.assert_allclose(got, ref, rtol=2e-6)


@pytest.mark.parametrize("d", [64, 128])
def test_rope_rotate_half_pairs_and_direction(d):
    """out_i = x_i cos - x_{i+h} sin, out_{i+h} = x_{i+h} cos + x_i sin with
    angle pos * theta^(-2i/D) (reference src/attention.cuh:22-44)."""
    h = d // 2
    x = torch.from_numpy(RNG.standard_normal((3, d)).astype(np.float32))
    pos = 37
    y = q.rope(x, pos, 1e6).double().numpy()
    ang = pos * (1.0 / (1e6 ** (np.arange(h) * 2 / d)))
    xd = x.double().numpy()
    ref = np.concatenate([xd[:, :h] * np.cos(ang) - xd[:, h:] * np.sin(ang),
                          xd[:, h:] * np.cos(ang) + xd[:, :h] * np.sin(ang)], axis=1)
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5)


def test_rope_identity_norm_and_composition():
    x = torch.from_numpy(RNG.standard_normal((4, 64)).astype(np.float32))
    assert torch.equal(q.rope(x, 0, 1e6), x)
    y = q.rope(x, 1234, 1e6)
    pair = lambda t: (t[:, :32] ** 2 + t[:, 32:] ** 2).sqrt()
    np.testing.assert_allclose(pair(y).numpy(), pair(x).numpy(), rtol=1e-5)
    np.testing.assert_allclose(q.rope(q.rope(x, 3, 1e6), 5, 1e6).numpy(), q.rope(x, 8, 1e6).numpy(),
                               rtol=1e-5, atol=1e-5)


def _attn_fp64(qh, k, v):
    nq, d = qh.shape
    rep = nq // k.shape[0]
    out = np.zeros((nq, d))
    for h in range(nq):
        kh, vh = k[h // rep], v[h // rep]
        s = kh @ qh[h] / np.sqrt(d)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ vh
    return out


def test_attention_brute_force_and_gqa_mapping():
    nq, nkv, s, d = 16, 8, 37, 64
    qh = RNG.standard_normal((nq, d)).astype(np.float32)
    k = RNG.standard_normal((nkv, s, d)).astype(np.float32)
    v = RNG.standard_normal((nkv, s, d)).astype(np.float32)
    got = q.attention(torch.from_numpy(qh), torch.from_numpy(k), torch.from_numpy(v)).double().numpy()
    np.testing.assert_allclose(got, _attn_fp64(qh.astype(np.float64), k.astype(np.float64),
                                                v.astype(np.float64)), rtol=1e-5, atol=1e-5)


def test_attention_special_cases():
    nq, nkv, d = 4, 2, 64
    qh = torch.from_numpy(RNG.standard_normal((nq, d)).astype(np.float32))
    v = torch.from_numpy(RNG.standard_normal((nkv, 5, d)).astype(np.float32))
    # one position: the output is that position's V (of the head's kv group)
    k1 = torch.from_numpy(RNG.standard_normal((nkv, 1, d)).astype(np.float32))
    out = q.attention(qh, k1, v[:, :1])
    for h in range(nq):
        np.testing.assert_allclose(out[h].numpy(), v[h // 2, 0].numpy(), rtol=1e-6)
    # identical keys: uniform weights, the output is the mean of V
    kk = torch.from_numpy(np.repeat(RNG.standard_normal((nkv, 1, d)), 5, axis=1).astype(np.float32))
    out = q.attention(qh, kk, v)
    for h in range(nq):
        np.testing.assert_allclose(out[h].numpy(), v[h // 2].mean(0).numpy(), rtol=1e-5, atol=1e-6)


def test_silu_mul_closed_form():
    g = torch.linspace(-20, 20, 401)
    u = torch.linspace(3, -1, 401)
    ref = g.double() / (1 + torch.exp(-g.double())) * u.double()
    np.testing.assert_allclose(q.silu_mul(g, u).double().numpy(), ref.numpy(), rtol=1e-6, atol=1e-6)


def test_argmax_first_index_on_ties():
    assert q.argmax_first(torch.tensor([1.0, 3.0, 3.0, 2.0])) == 1
    assert q.argmax_first(torch.tensor([-1.0, -1.0])) == 0


def test_bf16_round_is_rne():
    x = torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 3 * 2 ** -9])
    assert q.bf16_round(x).tolist() == [1.0, 1.0 + 2 ** -6, 1.0 + 2 ** -7]
