"""The library shares torch's HIP runtime, so torch streams are valid handles for it."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_one_hip_runtime_is_mapped_after_a_launch():
    from liteinfer_amd.paged_kernels import kv_scatter

    pool = torch.zeros(16, 1, 8, device="cuda")
    k = torch.ones(1, 1, 2, 8, device="cuda")
    kv_scatter(pool, pool.clone(), torch.tensor([[3, 5]], device="cuda"), k, k)
    torch.cuda.synchronize()
    maps = open("/proc/self/maps").read().splitlines()
    paths = {line.split()[-1] for line in maps if "libamdhip64" in line}
    assert len(paths) == 1, paths
    assert pool[3].sum().item() == 8.0 and pool[5].sum().item() == 8.0


def test_a_launch_on_a_side_stream_lands_on_that_stream():
    from liteinfer_amd.paged_kernels import kv_scatter

    side = torch.cuda.Stream()
    pool = torch.zeros(1024, 8, 128, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(64, 8, 1, 128, device="cuda").to(torch.bfloat16)
    slots = torch.arange(64, device="cuda").view(1, 64) * 3
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        kv_scatter(pool, pool.clone(), slots, k, k)
    side.synchronize()
    assert torch.equal(pool[slots.view(-1)], k.squeeze(2))
