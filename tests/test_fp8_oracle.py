"""The FP8 (OCP e4m3) restatement used by the FP8 LM head, pinned on the CPU:
against torch's own float8_e4m3fn conversion (an independent implementation),
closed-form code values, brute-force nearest / ties-to-even, and the
minimality of the power-of-two row scales."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8


def _torch_codes(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_decode_table_closed_form_and_torch():
    t = fp8.e4m3_decode_table()
    assert t[0x00] == 0.0 and np.signbit(t[0x80])
    assert t[0x01] == 2.0 ** -9 and t[0x07] == 7 * 2.0 ** -9
    assert t[0x08] == 2.0 ** -6
    assert t[0x38] == 1.0 and t[0x39] == 1.125 and t[0x40] == 2.0
    assert t[0x7E] == 448.0 and t[0xFE] == -448.0
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    ok = ~np.isnan(t)
    assert np.array_equal(np.isnan(t), np.isnan(ref))
    assert np.array_equal(t[ok], ref[ok])
    # the finite positive codes are strictly increasing
    pos = t[:0x7F]
    assert np.all(np.diff(pos) > 0)


@pytest.mark.parametrize("scale", [1e-4, 1e-2, 1.0, 60.0])
def test_encode_matches_torch(scale):
    rng = np.random.default_rng(7)
    x = np.clip(rng.standard_normal(200_000) * scale, -448, 448).astype(np.float32)
    assert np.array_equal(fp8.e4m3_encode(x), _torch_codes(x))


def test_encode_nearest_and_ties_to_even_brute_force():
    t = fp8.e4m3_decode_table()
    pos = t[:0x7F].astype(np.float64)  # codes 0..126, increasing
    # exact midpoints between neighbours: ties go to the even code
    mid = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)
    assert np.all(mid.astype(np.float64) == (pos[:-1] + pos[1:]) / 2)  # representable in fp32
    c = fp8.e4m3_encode(mid).astype(np.int64)
    lo = np.arange(126)
    assert np.all(c == np.where(lo % 2 == 0, lo, lo + 1))
    assert np.array_equal(fp8.e4m3_encode(-mid), (c | 0x80).astype(np.uint8))
    # random values: the chosen code is a nearest one
    rng = np.random.default_rng(3)
    x = (rng.random(20_000) * 448).astype(np.float32)
    x[:2000] *= 2.0 ** -8  # subnormal range too
    c = fp8.e4m3_encode(x)
    err = np.abs(t[c].astype(np.float64) - x)
    best = np.abs(pos[None, :] - x[:, None].astype(np.float64)).min(axis=1)
    assert np.all(err == best)


def test_row_exponents_are_minimal_powers_of_two():
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((64, 96)) * np.exp(rng.uniform(-12, 8, size=(64, 1)))).astype(np.float32)
    w[5] = 0.0
    w[6, 3] = 448.0  # exactly at the limit with e = 0
    w[6, 4:] = 0.0
    w[6, :3] = 1.0
    e = fp8.row_exponents(w)
    amax = np.abs(w).max(axis=1).astype(np.float64)
    nz = amax > 0
    assert np.all(amax[nz] <= 448.0 * 2.0 ** e[nz])
    assert np.all(amax[nz] > 448.0 * 2.0 ** (e[nz] - 1))
    assert e[5] == 0 and e[6] == 0
    codes, scales = fp8.quantize_rows(w)
    assert np.all(scales == np.ldexp(1.0, e))
    deq = fp8.dequantize_rows(codes, scales)
    # relative error of normal-range values <= 2^-4 (half an ulp of a 3-bit mantissa)
    big = np.abs(w) >= 2.0 ** -6 * scales[:, None]
    rel = np.abs(deq - w)[big] / np.abs(w)[big]
    assert rel.max() <= 2.0 ** -4
    # row maxima never saturate past 448 * scale and map to codes <= 0x7e
    assert np.all((codes & 0x7F) <= 0x7E)
    assert np.all(np.abs(deq).max(axis=1) <= 448.0 * scales)


def test_quantize_rows_equals_torch_on_scaled_rows():
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((32, 256)) * 0.02).astype(np.float32)
    codes, scales = fp8.quantize_rows(w)
    assert np.array_equal(codes, _torch_codes(w / scales[:, None]))


def test_oracle_fp8_layers_row_wise_and_exact_dequantisation():
    """Qwen3Oracle.use_fp8_layers: the fused "qkv" codes are those of the
    stacked q | k | v matrix (row-wise quantisation does not mix rows), every
    dequantised weight is within half an e4m3 step of the bf16 weight (relative
    2^-4 of its binade, or 2^-10 of the row scale below the normal range), and
    the matrices the oracle then multiplies by are exactly code x scale."""
    from oracle import qwen3_ref
    from oracle.layout import Shape
    sh = Shape(hidden=256, n_q_heads=4, n_kv_heads=2, head_dim=64, ffn=512, n_layers=2, vocab=512)
    bits = qwen3_ref.synthetic_bits(sh, 5, std=0.02, gain_std=0.1)
    orc = qwen3_ref.Qwen3Oracle(sh, bits, 8)
    orig = [{n: w[n].clone() for n in ("w_q", "w_k", "w_v", "w_o", "w_gate", "w_up", "w_down")} for w in orc.layers]
    q = orc.use_fp8_layers()
    table = fp8.e4m3_decode_table()
    for li, w in enumerate(orc.layers):
        stacked = torch.cat([orig[li]["w_q"], orig[li]["w_k"], orig[li]["w_v"]]).numpy()
        c, s = fp8.quantize_rows(stacked)
        assert np.array_equal(q[li]["qkv"][0], c) and np.array_equal(q[li]["qkv"][1], s)
        for n in ("q", "k", "v", "o", "gate", "up", "down"):
            codes, scales = q[li][n]
            a = orig[li]["w_" + n].numpy()
            b = w["w_" + n].numpy()
            assert np.array_equal(b, table[codes] * scales[:, None])
            _, ex = np.frexp(np.where(a != 0, a, 1.0))
            step = np.maximum(np.ldexp(1.0, ex - 4), scales[:, None] * 2.0 ** -9)
            assert (np.abs(b - a) <= 0.5 * step).all(), n
