"""The engine's fused elementwise kernels against the torch ops they replace.

`add_rms_norm` is the residual add and RMSNorm of liteinfer/models/llama.py:
34-48 (fp32 statistics, the normalised row rounded to the model dtype before
the weight); `silu_mul` the SiLU gate of llama.py:101-116. The residual add is
bit-exact (one rounding of an fp32 sum). The normalised row is rounded to
the dtype before the weight multiplies it, so where the fp32 sum of squares
(summed in another order) moves that first rounding by one unit in the last
place, the weight can carry the product to two; the same holds for the
gate, whose exponential can move the rounded silu by one before `up`
multiplies it. Almost every element agrees exactly.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from liteinfer_amd.engine.ops import add_rms_norm, silu_mul

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _ref_norm(h, w, eps):
    xf = h.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return w * xf.to(h.dtype)


def _ulps_apart(a, b, dtype):
    """Largest distance in units in the last place between two 16-bit tensors of one sign pattern."""
    ia, ib = a.view(torch.int16).int(), b.view(torch.int16).int()
    same_sign = (ia < 0) == (ib < 0)
    return int(((ia - ib).abs() * same_sign + (~same_sign) * 1000).max())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("rows", "hidden"), [(1, 4096), (7, 4096), (300, 4096), (5, 8), (3, 8192), (64, 1000 * 8)])
def test_add_rms_norm_matches_the_torch_ops(dtype, rows, hidden):
    g = torch.Generator(device=DEV).manual_seed(rows + hidden)
    h = torch.randn(rows, hidden, generator=g, device=DEV).to(dtype)
    delta = torch.randn(rows, hidden, generator=g, device=DEV).to(dtype)
    w = (1 + 0.1 * torch.randn(hidden, generator=g, device=DEV)).to(dtype)
    want_h = h + delta
    want = _ref_norm(want_h, w, 1e-5)
    got_h = h.clone()
    got = add_rms_norm(got_h, w, 1e-5, delta)
    torch.cuda.synchronize()
    assert torch.equal(got_h.view(torch.int16), want_h.view(torch.int16)), "the residual add is one rounding"
    assert _ulps_apart(got, want, dtype) <= 2
    # without a delta: the norm alone, h untouched
    h2 = h.clone()
    got2 = add_rms_norm(h2, w, 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(h2, h)
    assert _ulps_apart(got2, _ref_norm(h, w, 1e-5), dtype) <= 2
    # most elements agree exactly
    assert (got2 == _ref_norm(h, w, 1e-5)).float().mean() > 0.99


def test_add_rms_norm_on_a_batch_view_of_three_dims():
    h = torch.randn(4, 5, 512, device=DEV).to(torch.bfloat16)
    w = torch.ones(512, device=DEV, dtype=torch.bfloat16)
    got = add_rms_norm(h.clone(), w, 1e-6)
    assert _ulps_apart(got, _ref_norm(h, w, 1e-6), torch.bfloat16) <= 2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("rows", "ffn"), [(1, 14336), (33, 14336), (2, 8)])
def test_silu_mul_matches_the_torch_ops(dtype, rows, ffn):
    g = torch.Generator(device=DEV).manual_seed(rows * 7 + ffn)
    gu = (3 * torch.randn(rows, 2 * ffn, generator=g, device=DEV)).to(dtype)
    gate, up = gu.chunk(2, dim=-1)
    want = F.silu(gate) * up
    got = silu_mul(gu)
    torch.cuda.synchronize()
    assert got.shape == want.shape
    # a one-unit move of the rounded silu can become two in the product
    assert _ulps_apart(got, want, dtype) <= 2
    assert (got == want).float().mean() > 0.99


def test_bad_shapes_are_refused():
    with pytest.raises(ValueError):
        add_rms_norm(torch.zeros(2, 12, device=DEV, dtype=torch.bfloat16), torch.ones(12, device=DEV,
                                                                                       dtype=torch.bfloat16), 1e-5)
    with pytest.raises(ValueError):
        add_rms_norm(torch.zeros(2, 16, device=DEV), torch.ones(16, device=DEV), 1e-5)
    with pytest.raises(ValueError):
        silu_mul(torch.zeros(2, 12, device=DEV, dtype=torch.bfloat16))
