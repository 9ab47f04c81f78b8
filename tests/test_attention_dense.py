"""The boundary's dense kernels and selection policy (CPU)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from liteinfer_amd.attention import (
    IMPLEMENTATIONS,
    PagedKV,
    eager_attention,
    paged_attention,
    reads_pool_in_place,
    resolve,
    sdpa_attention,
    select_implementation,
    unsupported_reason,
)
from tests.helpers import PagedBatch, to_numpy


def _kv(b: PagedBatch) -> PagedKV:
    return PagedKV(b.key_pool, b.value_pool, b.slot_table, b.context_lens_t, query_start_loc=b.query_start_loc,
                   max_query_len=max(b.query_lens or [1]), host_context_lens=tuple(b.context_lens),
                   host_query_lens=tuple(b.query_lens or ()))


def _run(kernel, b: PagedBatch) -> torch.Tensor:
    if b.query_lens is None:
        return kernel(b.query.unsqueeze(2), _kv(b), b.scaling, b.groups).squeeze(2)
    return kernel(b.query.transpose(0, 1).unsqueeze(0), _kv(b), b.scaling, b.groups).squeeze(0).transpose(0, 1)


CASES = [
    ([6, 4, 1], None),
    ([23], [5]),
    ([37], [37]),
    ([90, 60, 3, 7], [1, 40, 1, 7]),
]


@pytest.mark.parametrize("kernel", [eager_attention, sdpa_attention], ids=["eager", "sdpa"])
@pytest.mark.parametrize(("ctxs", "qlens"), CASES)
def test_dense_kernels_match_the_oracle(kernel, ctxs, qlens):
    b = PagedBatch(ctxs, qlens, device="cpu", seed=5)
    np.testing.assert_allclose(to_numpy(_run(kernel, b)), b.oracle(), rtol=1e-5, atol=1e-5)


def test_packed_dense_kernel_without_host_lengths_is_refused():
    b = PagedBatch([6, 4], [2, 4], device="cpu")
    with pytest.raises(ValueError, match="host_context_lens"):
        eager_attention(b.query.transpose(0, 1).unsqueeze(0), _kv(b)._replace(host_context_lens=()), b.scaling, b.groups)


def test_paged_decode_rejects_more_than_one_query_per_sequence():
    b = PagedBatch([6, 4], device="cpu")
    q = b.query.unsqueeze(2)
    with pytest.raises(ValueError, match="one query per sequence"):
        paged_attention(torch.cat([q, q], dim=2), _kv(b), b.scaling, b.groups)


def test_registry_names_and_lookup():
    assert sorted(IMPLEMENTATIONS) == ["eager", "paged", "sdpa"]
    assert resolve("paged") is paged_attention
    with pytest.raises(ValueError, match="unknown attn_implementation"):
        resolve("flash")


def test_the_choice_falls_back_off_rocm():
    assert select_implementation(None, torch.device("cpu")) == "sdpa"


def test_a_named_kernel_that_cannot_run_is_refused_rather_than_downgraded():
    with pytest.raises(ValueError, match="cannot run here"):
        select_implementation("paged", torch.device("cpu"))


def test_the_reason_names_the_precondition():
    reason = unsupported_reason("paged", torch.device("cpu"))
    assert reason is not None and "ROCm" in reason
    assert unsupported_reason("sdpa", torch.device("cpu")) is None


def test_only_paged_reads_the_pool_in_place():
    assert reads_pool_in_place("paged") and not reads_pool_in_place("eager") and not reads_pool_in_place("sdpa")


def test_paged_kernels_refuse_a_cpu_device():
    from liteinfer_amd.paged_kernels import paged_decode

    b = PagedBatch([4], device="cpu")
    with pytest.raises(RuntimeError, match="ROCm device"):
        paged_decode(b.query, b.key_pool, b.value_pool, b.slot_table, b.context_lens_t, b.scaling, b.groups)
