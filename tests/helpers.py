"""Builders of seeded paged-attention inputs shared by the tests."""

from __future__ import annotations

import numpy as np
import torch


def to_numpy(t: torch.Tensor) -> np.ndarray:
    """fp32 numpy copy (bf16/fp16 widen exactly)."""
    return t.detach().float().cpu().numpy()


class PagedBatch:
    """One decode step (query_lens None) or packed pass over a seeded random pool.

    Each sequence's first context_len table columns are random slots in
    [1, num_slots); the columns after them hold other random slots, which no
    kernel may read. The table is `width` columns wide when that is more
    than the longest context (the width is what a decode call's kernel
    choice sees: a wide table takes a short batch to the balanced split).
    """

    def __init__(self, context_lens, query_lens=None, dtype=torch.float32, num_heads=8, num_kv_heads=2,
                 head_dim=16, num_slots=512, seed=0, device="cuda", shuffled_blocks=None, width=None):
        g = torch.Generator().manual_seed(seed)
        self.device = torch.device(device)
        self.dtype = dtype
        self.context_lens = list(context_lens)
        self.query_lens = None if query_lens is None else list(query_lens)
        self.groups = num_heads // num_kv_heads
        self.num_heads, self.num_kv_heads, self.head_dim = num_heads, num_kv_heads, head_dim
        self.scaling = head_dim ** -0.5

        def randn(*shape):
            return torch.randn(*shape, generator=g, dtype=torch.float32).to(dtype).to(self.device)

        self.key_pool = randn(num_slots, num_kv_heads, head_dim)
        self.value_pool = randn(num_slots, num_kv_heads, head_dim)
        rows = len(self.context_lens) if self.query_lens is None else sum(self.query_lens)
        self.query = randn(rows, num_heads, head_dim)
        width = max(max(self.context_lens), width or 0)
        table = torch.randint(1, num_slots, (len(self.context_lens), width), generator=g, dtype=torch.int64)
        self.slot_table = table.to(self.device)

    @property
    def context_lens_t(self) -> torch.Tensor:
        return torch.tensor(self.context_lens, dtype=torch.int32, device=self.device)

    @property
    def query_start_loc(self) -> torch.Tensor | None:
        if self.query_lens is None:
            return None
        return torch.tensor([0, *self.query_lens], device=self.device).cumsum(0).to(torch.int32)

    def oracle(self, dtype=np.float64) -> np.ndarray:
        from oracle.attention import attend

        qsl = None if self.query_lens is None else to_numpy(self.query_start_loc).astype(np.int32)
        return attend(to_numpy(self.query), to_numpy(self.key_pool), to_numpy(self.value_pool),
                      self.slot_table.cpu().numpy(), np.asarray(self.context_lens), self.scaling, self.groups,
                      query_start_loc=qsl, dtype=dtype)


def assert_within(actual: torch.Tensor, expected: np.ndarray, max_abs: float, mean_abs: float | None = None):
    """max |actual - expected| <= max_abs (and mean <= mean_abs when given), no NaN."""
    a = to_numpy(actual).astype(np.float64)
    assert a.shape == expected.shape, (a.shape, expected.shape)
    assert np.isfinite(a).all(), "non-finite output"
    err = np.abs(a - expected)
    assert err.max() <= max_abs, f"max abs error {err.max():.3e} > {max_abs:.3e}"
    if mean_abs is not None:
        assert err.mean() <= mean_abs, f"mean abs error {err.mean():.3e} > {mean_abs:.3e}"
