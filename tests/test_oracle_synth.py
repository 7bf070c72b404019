"""Pins of the synthetic generator (oracle/synth.py)."""
import numpy as np

from oracle import synth


def test_splitmix64_published_vectors():
    # Vigna's splitmix64 seeded with 0: first outputs (reference implementation).
    assert [synth.h_int(0, i) for i in range(4)] == [
        0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    # ... and seeded with 1234567 (the test vectors of java.util.SplittableRandom's mixer).
    assert [synth.h_int(1234567, i) for i in range(3)] == [
        6457827717110365317, 3203168211198807973, 9817491932198370423]


def test_vectorised_matches_scalar():
    key = synth.stream_key(99, 12345)
    v = synth.h_vec(key, 1000, 64)
    assert [int(x) for x in v] == [synth.h_int(key, 1000 + i) for i in range(64)]
    # indices past 2^32 wrap the 64-bit counter the same way
    v = synth.h_vec(key, (1 << 33) - 3, 6)
    assert [int(x) for x in v] == [synth.h_int(key, (1 << 33) - 3 + i) for i in range(6)]


def test_bf16_rne():
    f = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 2 ** -9, 1.0 + 3 * 2 ** -9, 1.0 + 3 * 2 ** -8,
                  -2.5, 0.0, 65504.0], np.float32)
    # exact; tie -> even (down); below half; above half; tie -> even (up);
    # exact negative; zero; rounds up into the next binade
    ref = [0x3F80, 0x3F80, 0x3F80, 0x3F81, 0x3F82, 0xC020, 0x0000, 0x4780]
    got = synth.f32_to_bf16_bits(f)
    assert got.tolist() == ref
    assert synth.bf16_bits_to_f32(got)[[0, 5, 6]].tolist() == [1.0, -2.5, 0.0]


def test_irwin_hall_moments_and_bounds():
    key = synth.stream_key(7, 3)
    x = synth.normal_f32(key, 0, 1 << 20, 1.0)
    assert abs(float(x.mean())) < 5e-3
    assert abs(float(x.std()) - 1.0) < 5e-3
    assert float(np.abs(x).max()) <= 2 * np.sqrt(3.0) + 1e-6  # bounded support of IH(4)
    g = synth.normal_f32(key, 0, 1 << 16, 0.1, add_one=True)
    assert abs(float(g.mean()) - 1.0) < 5e-3


def test_prompt_tokens_in_range_and_deterministic():
    t = synth.prompt_tokens(2024, 16, 151936)
    assert t == synth.prompt_tokens(2024, 16, 151936)
    assert all(0 <= x < 151936 for x in t) and len(set(t)) == 16


def test_kv_prefill_layout_independent_of_length():
    a = synth.kv_prefill_bits(5, 1, 0, 10, 8, 64)
    b = synth.kv_prefill_bits(5, 1, 0, 30, 8, 64)
    assert a.shape == (8, 10, 64) and np.array_equal(a, b[:, :10])
    assert not np.array_equal(a, synth.kv_prefill_bits(5, 1, 1, 10, 8, 64))
