"""The fp8 (e4m3) pool format of the oracle, pinned.

Against torch's float8_e4m3fn conversion (an independent implementation of
the same OCP format), against the format's closed form, and by brute force:
every quantised value is the nearest finite e4m3 value, ties to the even
mantissa.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import fp8


def _finite_values() -> np.ndarray:
    t = fp8.decode_table()
    return np.unique(t[np.isfinite(t)])


def test_decode_table_is_torchs_e4m3fn():
    codes = torch.arange(256, dtype=torch.uint8)
    want = codes.view(torch.float8_e4m3fn).to(torch.float64).numpy()
    got = fp8.decode_table()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[~np.isnan(got)], want[~np.isnan(want)])
    assert np.isnan(got[[0x7F, 0xFF]]).all() and np.nanmax(got) == 448.0 and np.nanmin(got) == -448.0


def test_closed_form_corners():
    t = fp8.decode_table()
    assert t[0x00] == 0.0 and t[0x80] == 0.0 and np.signbit(t[0x80])
    assert t[0x01] == 2.0 ** -9          # smallest subnormal
    assert t[0x07] == 7 * 2.0 ** -9      # largest subnormal
    assert t[0x08] == 2.0 ** -6          # smallest normal
    assert t[0x38] == 1.0                # exponent field 7 = bias
    assert t[0x7E] == 448.0


def test_encode_matches_torch_on_random_ties_and_boundaries():
    g = torch.Generator().manual_seed(0)
    x = torch.cat([torch.randn(1 << 16, generator=g) * s for s in (1e-3, 0.05, 1.0, 20.0, 300.0)])
    vals = torch.tensor(_finite_values(), dtype=torch.float32)
    mids = (vals[1:] + vals[:-1]) / 2  # exact ties
    x = torch.cat([x, vals, mids, torch.tensor([448.0, -448.0, 0.0, -0.0, 2.0 ** -10, -(2.0 ** -10), 1e-30])])
    x = x.clamp(-448, 448)
    want = x.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = fp8.encode(x.numpy())
    assert np.array_equal(got, want)


def test_quantize_with_a_scale_is_torch_on_the_scaled_clamped_values():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1 << 15, generator=g, dtype=torch.float32).to(torch.bfloat16).to(torch.float32) * 40
    for scale in (1.0, 0.25, 3.0, 0.1):
        inv = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(scale, dtype=torch.float32)
        want = (x * inv).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        assert np.array_equal(fp8.quantize(x.numpy(), scale), want)


def test_every_value_is_its_own_code_and_the_nearest_value_wins():
    vals = _finite_values()
    assert np.array_equal(fp8.decode(fp8.encode(vals.astype(np.float32))), vals)
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.uniform(-448, 448, 4000), rng.uniform(-0.05, 0.05, 4000)]).astype(np.float32)
    q = fp8.decode(fp8.encode(x))
    xd = x.astype(np.float64)
    dist = np.abs(vals[None, :] - xd[:, None])
    best = dist.min(axis=1)
    assert np.allclose(np.abs(q - xd), best, rtol=0, atol=0)


def test_dequantize_applies_the_scale():
    codes = np.arange(256, dtype=np.uint8)
    t = fp8.decode_table()
    ok = np.isfinite(t)
    assert np.array_equal(fp8.dequantize(codes, 0.5)[ok], t[ok] * 0.5)


def test_quantize_keeps_a_nan_as_torchs_cast_does():
    """NaN (either sign) becomes the e4m3 NaN code torch's float8_e4m3fn cast
    gives it; the clamp applies to numbers only (+-inf saturate to +-448,
    where torch's unsaturated cast would give NaN)."""
    x = np.array([np.nan, -np.nan, 3.0, -2.5], dtype=np.float32)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(fp8.quantize(x, 1.0), want)
    assert np.array_equal(fp8.quantize(np.array([np.inf, -np.inf], dtype=np.float32), 1.0), [0x7E, 0xFE])
