"""Host-side scheduling choices of the paged path (no GPU needed)."""

from __future__ import annotations

import numpy as np

from liteinfer_amd.attention import _one_query_rows_to_decode_kernel as to_decode_kernel
from liteinfer_amd.workloads import c3_shapes

def _lens(chunks, rows):
    return [q for q, _ in chunks] + [1] * len(rows), [q + p for q, p in chunks] + list(rows)


def test_no_one_query_rows_means_no_decode_split():
    q, _ = _lens([(100, 20), (64, 0)], [])
    assert to_decode_kernel(q) is False


def test_any_one_query_row_goes_to_the_decode_split():
    """Config 3, a decode-heavy pass, a single short row: all take the split."""
    chunks, rows = c3_shapes(0)
    assert to_decode_kernel(_lens(chunks, rows)[0]) is True
    rows = np.random.default_rng(3).integers(1000, 8000, size=200).tolist()
    assert to_decode_kernel(_lens([(256, 1000)] * 4, rows)[0]) is True
    assert to_decode_kernel(_lens([(2048, 4000)] * 8, [9])[0]) is True
    assert to_decode_kernel([1]) is True
