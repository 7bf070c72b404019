"""FP8 (OCP e4m3) restatement for the FP8 LM head.  TEST INFRASTRUCTURE.

The reference has no FP8 implementation; it plans FP8 weights
(/root/reference/RESEARCH.md:434-436,463).  The format is the OCP 8-bit
floating point e4m3 ("e4m3fn"): sign, 4 exponent bits with bias 7, 3 mantissa
bits, no infinities, largest finite 448, subnormals m * 2^-9, NaN only at
0x7f / 0xff.

Quantisation of a weight matrix W[R][C] (the library's lmhead_fp8_kernel):
  * per row r the power-of-two scale 2^e_r, e_r the smallest integer with
    max|W[r]| <= 448 * 2^e_r (e_r = 0 for an all-zero row);
  * code = e4m3(W[r][c] * 2^-e_r), rounded to nearest, ties to even (the
    scaling is exact, so this is the only rounding);
  * dequantised weight = decode(code) * 2^e_r.
"""
from __future__ import annotations

import numpy as np

MAX_E4M3 = 448.0


def e4m3_decode_table() -> np.ndarray:
    """float32 value of each of the 256 codes (NaN at 0x7f, 0xff)."""
    c = np.arange(256)
    mag = c & 0x7F
    e, m = mag >> 3, mag & 7
    v = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * 2.0 ** (e - 7.0))
    v = np.where(c & 0x80, -v, v)
    v[mag == 0x7F] = np.nan
    return v.astype(np.float32)


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """Codes of float32 values with |x| <= 448: nearest, ties to even."""
    x = np.asarray(x, dtype=np.float32)
    sign = np.where(np.signbit(x), 0x80, 0).astype(np.int64)
    a = np.abs(x)
    sub = a < np.float32(2.0 ** -6)
    # subnormal range: m = rint(a * 2^9) in 0..8 (8 is the smallest normal code)
    c_sub = np.rint(a * np.float32(512.0)).astype(np.int64)
    # normal range: a = 2^E * f, f in [1, 2); code = ((E + 7) << 3) + rint(8 f) - 8
    _, ex = np.frexp(np.where(sub, np.float32(1.0), a))
    E = ex.astype(np.int64) - 1
    r = np.rint(np.ldexp(a, (3 - E).astype(np.int32)).astype(np.float32)).astype(np.int64)
    c_norm = ((E + 7) << 3) + r - 8
    c = np.where(sub, c_sub, c_norm)
    return (sign | np.minimum(c, 0x7E)).astype(np.uint8)


def row_exponents(w: np.ndarray) -> np.ndarray:
    """e_r: smallest integer with max|W[r]| <= 448 * 2^e_r (0 for zero rows)."""
    amax = np.abs(np.asarray(w, dtype=np.float32)).max(axis=1)
    _, ex = np.frexp(np.where(amax > 0, amax, np.float32(1.0)))
    e = ex.astype(np.int64) - 1 - 8  # ilogb(amax) - 8, as 448 = 1.75 * 2^8
    e = e + (amax > np.ldexp(np.float32(MAX_E4M3), e.astype(np.int32)).astype(np.float32))
    return np.where(amax > 0, e, 0).astype(np.int64)


def quantize_rows(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(codes uint8 [R][C], scales float32 [R] = 2^e_r) of a float32 matrix."""
    w = np.asarray(w, dtype=np.float32)
    e = row_exponents(w)
    scaled = np.ldexp(w, (-e)[:, None].astype(np.int32)).astype(np.float32)
    return e4m3_encode(scaled), np.ldexp(np.float32(1.0), e.astype(np.int32)).astype(np.float32)


def dequantize_rows(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """float32 [R][C] = decode(codes) * scale_r (exact: the scales are powers of two)."""
    return e4m3_decode_table()[codes] * np.asarray(scales, dtype=np.float32)[:, None]
