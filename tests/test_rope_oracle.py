"""The RoPE oracle against torch's own ops and the geometry of a rotation."""

import numpy as np
import pytest
import torch

from oracle import rope as R

DTYPES = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _angles(tokens, dim, rng):
    half = dim // 2
    theta = rng.uniform(-np.pi, np.pi, size=(tokens, half))
    return np.concatenate((theta, theta), axis=-1)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_round_to_matches_torch_conversion(dtype):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10,
        # ties and carries: the low 16 (bf16) bits exactly 0x8000 / 0x7fff / 0xffff
        (rng.integers(0, 2**15, 3000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
        (rng.integers(0, 2**15, 3000, dtype=np.uint32) << 16 | 0xFFFF).view(np.float32),
        np.array([0.0, -0.0, 1.0, 65504.0, 1e-8, -3.0e38], dtype=np.float32),
    ])
    x = x[np.isfinite(x)]
    want = torch.from_numpy(x).to(DTYPES[dtype]).float().numpy()
    np.testing.assert_array_equal(R.round_to(x, dtype).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("dim", [64, 128])
def test_rope_is_torch_ops_bit_for_bit(dtype, dim):
    rng = np.random.default_rng(1)
    td = DTYPES[dtype]
    x = torch.from_numpy(rng.standard_normal((2, 4, 7, dim)).astype(np.float32)).to(td)
    ang = torch.from_numpy(_angles(7, dim, rng))
    cos = ang.cos()[None].to(td)
    sin = ang.sin()[None].to(td)
    half = dim // 2
    c, s = cos.unsqueeze(1), sin.unsqueeze(1)
    # torch's ops, one rounding each, as the reference's model evaluates them
    want = (x * c) + (torch.cat((-x[..., half:], x[..., :half]), dim=-1) * s)
    got = R.rope(x.float().numpy(), c.float().numpy(), s.float().numpy(), dtype)
    np.testing.assert_array_equal(got, want.float().numpy())


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_zero_angle_is_identity_and_quarter_turn_is_rotate_half(dtype):
    rng = np.random.default_rng(2)
    x = R.round_to(rng.standard_normal((3, 5, 64)).astype(np.float32), dtype)
    one, zero = np.ones((5, 64), np.float32), np.zeros((5, 64), np.float32)
    np.testing.assert_array_equal(R.rope(x, one, zero, dtype), x)
    np.testing.assert_array_equal(R.rope(x, zero, one, dtype), R.rotate_half(x))


def test_exact_rotation_keeps_pair_lengths_and_composes():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 9, 128))
    a, b = _angles(9, 128, rng), _angles(9, 128, rng)
    y = R.rope(x, np.cos(a), np.sin(a), "f64")
    norm = lambda t: np.hypot(t[..., :64], t[..., 64:])
    np.testing.assert_allclose(norm(y), norm(x), rtol=1e-12)
    z = R.rope(y, np.cos(b), np.sin(b), "f64")
    np.testing.assert_allclose(z, R.rope(x, np.cos(a + b), np.sin(a + b), "f64"), rtol=1e-10, atol=1e-12)


def test_rope_kv_write_stores_rotated_k_and_plain_v():
    rng = np.random.default_rng(4)
    q = rng.standard_normal((2, 4, 3, 8)).astype(np.float32)
    k = rng.standard_normal((2, 2, 3, 8)).astype(np.float32)
    v = rng.standard_normal((2, 2, 3, 8)).astype(np.float32)
    ang = _angles(3, 8, rng)[None].repeat(2, 0)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    slots = np.array([5, 0, 9, 2, 7, 11])
    kp0 = np.full((12, 2, 8), 7.0, np.float32)
    vp0 = np.full((12, 2, 8), -7.0, np.float32)
    q_out, kp, vp = R.rope_kv_write(q, k, v, cos, sin, slots, kp0, vp0, "f32")
    np.testing.assert_array_equal(q_out, R.rope(q, cos[:, None], sin[:, None], "f32"))
    k_rot = R.rope(k, cos[:, None], sin[:, None], "f32")
    for i, s in enumerate(slots):
        b, t = divmod(i, 3)
        np.testing.assert_array_equal(kp[s], k_rot[b, :, t])
        np.testing.assert_array_equal(vp[s], v[b, :, t])
    untouched = sorted(set(range(12)) - set(slots.tolist()))
    assert (kp[untouched] == 7.0).all() and (vp[untouched] == -7.0).all()
