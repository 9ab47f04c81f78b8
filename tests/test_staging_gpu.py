"""Host-to-device staging on a copy stream (`block_pool.to_device`): what the engine's
loop uses to stage a step while the step before it runs."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from liteinfer_amd.cache.block_pool import to_device

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def test_staged_values_arrive_while_the_stream_is_busy():
    """Values staged while the current stream still runs earlier work are there for the work
    queued after them, over many sizes (the staging buffers and device blocks are reused)."""
    rng = np.random.default_rng(3)
    a = torch.randn(2048, 2048, device=DEV)
    for i in range(40):
        for _ in range(3):
            a = a @ a / 2048.0  # keep the stream busy
        n = int(rng.integers(1, 5000))
        host = rng.integers(-2 ** 40, 2 ** 40, size=(n % 7 + 1, n)).astype(np.int64)
        got = to_device(host, torch.int64, DEV)
        # work on the current stream that reads the staged values
        doubled = got * 2
        assert np.array_equal(doubled.cpu().numpy(), host * 2), i
        lists = host[0].tolist()
        got_l = to_device([lists], torch.long, DEV)
        assert torch.equal(got_l.cpu(), torch.tensor([lists])), i


def test_staging_is_refused_inside_a_capture():
    """A captured copy would read its pinned staging buffer again on every replay: refused."""
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        graph.capture_begin()
        try:
            with pytest.raises(RuntimeError, match="graph capture"):
                to_device([[1, 2, 3]], torch.long, DEV)
        finally:
            graph.capture_end()
    torch.cuda.current_stream().wait_stream(side)
