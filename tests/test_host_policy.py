"""Host-side scheduling choices of the paged path (no GPU needed)."""

from __future__ import annotations

import numpy as np

from liteinfer_amd.attention import _one_query_rows_to_decode_kernel as to_decode_kernel
from liteinfer_amd.workloads import c3_shapes

GEOMETRY = dict(num_heads=32, num_kv_heads=8, head_dim=128)


def _lens(chunks, rows):
    return [q for q, _ in chunks] + [1] * len(rows), [q + p for q, p in chunks] + list(rows)


def test_no_one_query_rows_means_no_decode_launch():
    q, c = _lens([(100, 20), (64, 0)], [])
    assert to_decode_kernel(q, c, pool_element_size=2, **GEOMETRY) is False


def test_config_3_folds_its_rows_beside_the_chunks():
    chunks, rows = c3_shapes(0)
    q, c = _lens(chunks, rows)
    assert to_decode_kernel(q, c, pool_element_size=2, **GEOMETRY) is False


def test_a_decode_heavy_pass_sends_its_rows_to_the_decode_kernel():
    rows = np.random.default_rng(3).integers(1000, 8000, size=200).tolist()
    q, c = _lens([(256, 1000)] * 4, rows)
    assert to_decode_kernel(q, c, pool_element_size=2, **GEOMETRY) is True


def test_fp8_pools_and_long_rows_always_use_the_decode_kernel():
    chunks, rows = c3_shapes(0)
    q, c = _lens(chunks, rows)
    assert to_decode_kernel(q, c, pool_element_size=1, **GEOMETRY) is True
    q, c = _lens([(2048, 4000)] * 8, [9000])
    assert to_decode_kernel(q, c, pool_element_size=2, **GEOMETRY) is True


def _roofline_ratio(q, c):
    rows = sum(cc for qq, cc in zip(q, c) if qq == 1) * 8 * 128 * 2 * 2 / 8.0e12
    flops = sum(4 * 32 * 128 * (qq * (cc - qq) + qq * (qq + 1) / 2) for qq, cc in zip(q, c) if qq > 1) / 2.5e15
    return rows / flops


def test_the_split_is_where_the_rows_roofline_time_passes_the_chunks():
    """Rows fold while their HBM roofline time is at most the chunks' MFMA roofline time."""
    chunks = [(512, 1024)] * 4
    rng = np.random.default_rng(5)
    for n in range(1, 400, 7):
        rows = rng.integers(256, 4096, size=n).tolist()
        q, c = _lens(chunks, rows)
        want = _roofline_ratio(q, c) > 1.0
        assert to_decode_kernel(q, c, pool_element_size=2, **GEOMETRY) is want
    # config 3 sits well inside the fold region
    q, c = _lens(*c3_shapes(0))
    assert 0.3 < _roofline_ratio(q, c) < 0.8
