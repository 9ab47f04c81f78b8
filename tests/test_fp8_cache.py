"""The fp8 cache on the CPU path: the store quantises as the oracle does, and the
dense kernels read the dequantised rows."""

from __future__ import annotations

import numpy as np
import torch

from liteinfer_amd.attention import PagedKV, eager_attention, sdpa_attention
from liteinfer_amd.cache.block_pool import BlockPool
from liteinfer_amd.cache.kv_cache import quantize_fp8, scatter_into
from oracle import fp8
from oracle.attention import attend


def test_quantize_fp8_is_the_oracles_quantiser():
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(4096, generator=g) * 50).to(torch.bfloat16)
    for scale in (1.0, 0.3, 7.0):
        got = quantize_fp8(x, scale).view(torch.uint8).numpy()
        assert np.array_equal(got, fp8.quantize(x.float().numpy(), scale))


def test_block_pool_fp8_storage_and_validation():
    pool = BlockPool(4, 16, 2, 2, 8, torch.bfloat16, torch.device("cpu"), cache_quant="fp8", k_scale=2.0)
    k, v = pool.slots(0)
    assert k.dtype == torch.float8_e4m3fn and v.dtype == torch.float8_e4m3fn and pool.dtype == torch.bfloat16
    assert pool.nbytes == 2 * 2 * 64 * 2 * 8
    for bad in ({"cache_quant": "int4"}, {"cache_quant": "fp8", "k_scale": 0.0}):
        try:
            BlockPool(4, 16, 2, 2, 8, torch.bfloat16, torch.device("cpu"), **bad)
        except ValueError:
            continue
        raise AssertionError(f"{bad} accepted")


def test_dense_kernels_over_an_fp8_pool_read_the_dequantised_rows():
    g = torch.Generator().manual_seed(1)
    slots_n, heads, kvh, d = 64, 4, 2, 16
    kp = torch.zeros(slots_n, kvh, d, dtype=torch.float8_e4m3fn)
    vp = torch.zeros_like(kp)
    k = torch.randn(1, kvh, 40, d, generator=g)
    v = torch.randn(1, kvh, 40, d, generator=g)
    slots = torch.randperm(slots_n, generator=g)[:40].view(1, -1)
    scatter_into(kp, vp, slots, k, v, k_scale=0.5, v_scale=3.0)
    table = torch.cat([slots.view(1, -1), torch.zeros(1, 0, dtype=torch.int64)], dim=1).repeat(2, 1)
    ctx = torch.tensor([40, 17], dtype=torch.int32)
    q = torch.randn(2, heads, 1, d, generator=g)
    kv = PagedKV(kp, vp, table, ctx, k_scale=0.5, v_scale=3.0)
    kd = fp8.dequantize(kp.view(torch.uint8).numpy(), 0.5)
    vd = fp8.dequantize(vp.view(torch.uint8).numpy(), 3.0)
    want = attend(q.squeeze(2).numpy(), kd, vd, table.numpy(), ctx.numpy(), d ** -0.5, heads // kvh, dtype=np.float64)
    for kernel in (eager_attention, sdpa_attention):
        out = kernel(q, kv, d ** -0.5, heads // kvh).squeeze(2).numpy()
        np.testing.assert_allclose(out, want, rtol=1e-5, atol=1e-5)
