"""Parity at the benchmark configurations, full size, through the layer's own call sequence.

Each step writes its new K/V with the slot-write kernel, then attends through
the `paged` boundary, and is compared with the fp64 oracle on the same
(bf16-valued) inputs: max-abs <= 2e-2 and mean-abs <= 2e-3. The oracle's
pools are host copies taken before the HIP write, with the new rows stored by
the oracle's own scatter, so the write is checked as part of the step.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from liteinfer_amd.attention import PagedKV, paged_attention
from liteinfer_amd.cache.kv_cache import scatter_into
from liteinfer_amd.workloads import decode_step, packed_step
from oracle.addressing import tokens_first
from oracle.attention import attend
from tests.helpers import assert_within, to_numpy

pytestmark = pytest.mark.gpu


def _host_pools_after_write(step):
    """fp32 host copies of the pools with the step's new rows stored by numpy (before any HIP write)."""
    kp, vp = to_numpy(step.key_pool), to_numpy(step.value_pool)
    flat = step.write_slots.reshape(-1).cpu().numpy()
    kp[flat] = tokens_first(to_numpy(step.new_k))
    vp[flat] = tokens_first(to_numpy(step.new_v))
    return kp, vp


def _decode_oracle(step, pools, dtype=np.float64):
    return attend(to_numpy(step.query), pools[0], pools[1],
                  step.slot_table.cpu().numpy(), np.asarray(step.host_context_lens),
                  step.geometry.scaling, step.geometry.groups, dtype=dtype)


def _decode(step):
    scatter_into(step.key_pool, step.value_pool, step.write_slots, step.new_k, step.new_v)
    kv = PagedKV(step.key_pool, step.value_pool, step.slot_table, step.context_lens)
    return paged_attention(step.query.unsqueeze(2), kv, step.geometry.scaling, step.geometry.groups).squeeze(2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_c1_llama_1b_geometry(dtype):
    step = decode_step("c1", dtype=dtype, seed=0)
    pools = _host_pools_after_write(step)
    out = _decode(step)
    want = _decode_oracle(step, pools)
    if dtype == torch.float32:
        np.testing.assert_allclose(to_numpy(out), want, rtol=1e-5, atol=1e-5)
    else:
        assert_within(out, want, 2e-2, 2e-3)


def test_c2_llama_8b_batch_64():
    step = decode_step("c2", seed=0)
    pools = _host_pools_after_write(step)
    out = _decode(step)
    assert_within(out, _decode_oracle(step, pools), 2e-2, 2e-3)


def test_c4_long_context_partitions():
    step = decode_step("c4", seed=0)
    pools = _host_pools_after_write(step)
    out = _decode(step)
    assert_within(out, _decode_oracle(step, pools, dtype=np.float32), 2e-2, 2e-3)


def test_c3_mixed_chunks_and_decode_rows():
    step = packed_step("c3", seed=0)
    pools = _host_pools_after_write(step)
    scatter_into(step.key_pool, step.value_pool, step.write_slots, step.new_k, step.new_v)
    kv = PagedKV(step.key_pool, step.value_pool, step.slot_table, step.context_lens,
                 query_start_loc=step.query_start_loc, max_query_len=step.max_query_len,
                 host_context_lens=tuple(step.host_context_lens), host_query_lens=tuple(step.host_query_lens))
    q = step.query.transpose(0, 1).unsqueeze(0)
    out = paged_attention(q, kv, step.geometry.scaling, step.geometry.groups).squeeze(0).transpose(0, 1)
    want = attend(to_numpy(step.query), pools[0], pools[1],
                  step.slot_table.cpu().numpy(), np.asarray(step.host_context_lens), step.geometry.scaling,
                  step.geometry.groups, query_start_loc=step.query_start_loc.cpu().numpy())
    assert_within(out, want, 2e-2, 2e-3)
