"""Shared helpers of the test-suite: build an engine and an oracle on the same
synthetic weights, and the tolerance checks north_star states."""
from __future__ import annotations

import numpy as np

from megakernel_amd.config import ModelShape
from oracle import layout as olayout
from oracle import qwen3_ref

# north_star tolerances
LAYER_REL_L2 = 1e-2
LOGIT_ABS = 2e-2
MARGIN = 2e-2


def oracle_shape(s: ModelShape) -> olayout.Shape:
    return olayout.Shape(s.hidden, s.n_q_heads, s.n_kv_heads, s.head_dim, s.ffn, s.n_layers, s.vocab)


def make_pair(shape: ModelShape, seed: int, max_seq: int, gain_std: float = 0.1,
              bits_from_device: bool = False, kv_fp8: bool = False):
    """(engine, oracle, device_weights) on identical synthetic weights."""
    from megakernel_amd.bridge import MegakernelEngine
    from megakernel_amd.weights import DeviceWeights
    dw = DeviceWeights(shape, seed, std=0.02, gain_std=gain_std)
    eng = MegakernelEngine(shape=shape, max_seq=max_seq, device_weights=dw)
    osh = oracle_shape(shape)
    if bits_from_device:
        bits = qwen3_ref.unpack_flat(osh, dw.to_host(), dw.layout.offsets)
    else:
        bits = qwen3_ref.synthetic_bits(osh, seed, std=0.02, gain_std=gain_std)
    orc = qwen3_ref.Qwen3Oracle(osh, bits, max_seq, kv_fp8=kv_fp8)
    if kv_fp8:
        eng.set_kv_fp8(True)
    return eng, orc, dw


def rel_l2(a: np.ndarray, b: np.ndarray, axis=-1) -> np.ndarray:
    return np.linalg.norm(a - b, axis=axis) / np.maximum(np.linalg.norm(b, axis=axis), 1e-30)


def check_step(kernel_layers, kernel_logits, ref: dict, label: str = ""):
    """Per-layer rel-L2 and logit abs error of one step against the oracle."""
    rl = rel_l2(kernel_layers, ref["layers"].numpy())
    la = float(np.abs(kernel_logits - ref["logits"].numpy()).max())
    assert rl.max() <= LAYER_REL_L2, f"{label} layer rel-L2 {rl.max():.3e} (per layer {rl})"
    assert la <= LOGIT_ABS, f"{label} logits max abs err {la:.3e}"
    return float(rl.max()), la


def check_tokens_teacher_forced(kernel_in: list[int], kernel_out: list[int], orc) -> tuple[int, int]:
    """Feed the kernel's own input tokens to the oracle; every kernel output must
    equal the oracle argmax unless the oracle's top1-top2 margin <= MARGIN.
    Returns (#identical, #low-margin mismatches)."""
    same = low = 0
    for i, (tin, tout) in enumerate(zip(kernel_in, kernel_out)):
        r = orc.step(int(tin), capture=True)
        if r["token"] == tout:
            same += 1
            continue
        m = qwen3_ref.top2_margin(r["logits"])
        gap = float(r["logits"][r["token"]] - r["logits"][tout])
        assert m <= MARGIN and gap <= MARGIN, (
            f"step {i}: kernel token {tout} != oracle {r['token']} with margin {m:.4f}")
        low += 1
    return same, low


def check_kv_bf16(got_bits: np.ndarray, want_bits: np.ndarray, label: str = "") -> None:
    """K / V bytes against bf16 of the oracle's fp32 k / v (same inputs, fp32
    summation order differs): at most 1 ulp wherever |want| >= 1e-3 x RMS of
    the plane; entries below that come from near-cancelling sums, where the
    order decides the low bits, and are held to 1e-3 x RMS absolute; fewer
    than 1 % of entries may differ at all."""
    from oracle import synth
    d = np.abs(got_bits.astype(np.int32) - want_bits.astype(np.int32))
    gf, wf = synth.bf16_bits_to_f32(got_bits), synth.bf16_bits_to_f32(want_bits)
    rms = float(np.sqrt(np.mean(wf.astype(np.float64) ** 2)))
    big = np.abs(wf) >= 1e-3 * rms
    assert d[big].max(initial=0) <= 1, f"{label}: K/V bytes differ by up to {d[big].max()} ulp"
    small_err = float(np.abs(gf - wf)[~big].max(initial=0.0))
    assert small_err <= 1e-3 * rms, f"{label}: near-zero K/V entries off by {small_err:.3e} (rms {rms:.3e})"
    assert (d > 0).mean() < 0.01, f"{label}: {(d > 0).mean():.3%} of K/V entries differ"
