"""The fp8 (OCP e4m3) pool format, restated in numpy. TEST INFRASTRUCTURE ONLY.

The reference plans a quantised KV cache (liteinfer docs/roadmap.md, section
2.5: "storage-level quant of K and V; dequant on read") and has no code for
it; this is the format the build's fp8 pool stores, written from the format's
definition:

* e4m3 ("e4m3fn" in torch): 1 sign bit, 4 exponent bits with bias 7, 3
  mantissa bits; exponent field 0 holds subnormals m/8 * 2^-6; no infinity;
  0x7f and 0xff are NaN, so the largest finite magnitude is
  1.75 * 2^8 = 448.
* Quantising x with a scale: q = e4m3(clamp(float32(x) * float32(1 / scale),
  -448, 448)), the reciprocal and the product rounded to float32, the
  conversion rounding to nearest, ties to even.
* Reading: x' = decode(q) * scale.

Pinned in tests/test_fp8_oracle.py against torch's float8_e4m3fn
conversion, the closed form of all 256 codes, and round-trip properties.
"""

from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0
_MIN_NORMAL = 2.0 ** -6
_SUBNORMAL_STEP = 2.0 ** -9


def decode_table() -> np.ndarray:
    """float64 value of each of the 256 codes (NaN for 0x7f and 0xff)."""
    out = np.empty(256, dtype=np.float64)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exp = (code >> 3) & 0xF
        man = code & 0x7
        if exp == 0xF and man == 0x7:
            out[code] = np.nan
        elif exp == 0:
            out[code] = sign * man * _SUBNORMAL_STEP
        else:
            out[code] = sign * (1.0 + man / 8.0) * 2.0 ** (exp - 7)
    return out


_TABLE = decode_table()


def decode(codes: np.ndarray) -> np.ndarray:
    """Codes (uint8) to float64 values."""
    return _TABLE[np.asarray(codes, dtype=np.uint8)]


def encode(x: np.ndarray) -> np.ndarray:
    """float32 values, already within [-448, 448], to codes: nearest e4m3, ties to even."""
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    if np.any(np.abs(x) > E4M3_MAX) or np.any(np.isnan(x)):
        raise ValueError("encode takes finite values within [-448, 448]; clamp first")
    sign = np.signbit(x)
    a = np.abs(x)
    # The grid step at a: 2^(e - 3) in the binade [2^e, 2^(e+1)), 2^-9 below
    # the smallest normal. a / step is exact (a power-of-two division), so
    # np.round (half to even) rounds exactly as the format does.
    _, e2 = np.frexp(np.where(a > 0, a, 1.0))  # a = f * 2^e2, f in [0.5, 1)
    e = e2 - 1
    step = np.where(a >= _MIN_NORMAL, np.ldexp(1.0, e - 3), _SUBNORMAL_STEP)
    q = np.round(a / step) * step  # may round up into the next binade
    # Bits of q.
    codes = np.zeros(x.shape, dtype=np.uint8)
    sub = q < _MIN_NORMAL
    codes[sub] = np.round(q[sub] / _SUBNORMAL_STEP).astype(np.uint8)
    norm = ~sub
    if np.any(norm):
        _, qe2 = np.frexp(q[norm])
        qe = qe2 - 1
        man = np.round(q[norm] / np.ldexp(1.0, qe - 3)).astype(np.int64) - 8
        codes[norm] = (((qe + 7) << 3) | man).astype(np.uint8)
    codes[sign & (q > 0)] |= 0x80
    codes[sign & (q == 0)] |= 0x80  # -0 keeps its sign
    return codes


def quantize(x: np.ndarray, scale: float) -> np.ndarray:
    """Pool codes of x (any float array) for a positive scale, as the slot-write stores them.

    A NaN stays a NaN (0x7f, or 0xff with its sign bit set), as torch's
    float8_e4m3fn cast keeps it; everything else is clamped to +-448 first.
    """
    x = np.asarray(x, dtype=np.float32)
    inv = np.float32(1.0) / np.float32(scale)
    y = x * inv
    nan = np.isnan(y)
    codes = encode(np.clip(np.where(nan, 0.0, y), -E4M3_MAX, E4M3_MAX).astype(np.float32))
    # The sign a NaN keeps is the input's (a product's NaN sign is not fixed
    # by IEEE 754, so it is taken before the scaling).
    codes[nan] = np.where(np.signbit(x[nan]), 0xFF, 0x7F).astype(np.uint8)
    return codes


def dequantize(codes: np.ndarray, scale: float) -> np.ndarray:
    """float64 values the readers see: decode(codes) * scale."""
    return decode(codes) * float(np.float32(scale))
