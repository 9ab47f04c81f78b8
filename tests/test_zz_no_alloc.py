"""The allocation-free decode entry point answers what li_paged_decode answers.

``li_paged_decode_noalloc`` runs li_paged_decode's kernels with the
partials in a device array the library holds. Two calls in a row (the second
smaller, so it reads what the first left behind in the shared scratch) must
each equal li_paged_decode on the same inputs bit for bit, and meet the fp64
oracle's bar; a call needing more scratch than the library holds is refused
before anything runs.
"""

from __future__ import annotations

import pytest
import torch

from liteinfer_amd.paged_kernels import paged_decode, paged_decode_noalloc
from liteinfer_amd.workloads import decode_step
from tests.helpers import PagedBatch, assert_within

pytestmark = pytest.mark.gpu


def _both(step_query, key_pool, value_pool, slot_table, context_lens, scaling, groups, **kw):
    want = paged_decode(step_query, key_pool, value_pool, slot_table, context_lens, scaling, groups, **kw)
    out = torch.full_like(step_query, float("nan"))
    got = paged_decode_noalloc(step_query, key_pool, value_pool, slot_table, context_lens, scaling, groups, out=out,
                               **kw)
    torch.cuda.synchronize()
    assert got.data_ptr() == out.data_ptr()
    return want, got


def test_two_calls_in_a_row_equal_the_workspace_entry_point():
    print("no-alloc decode: Llama-3-8B geometry, 48 sequences then 5", flush=True)
    big = decode_step("custom", context_lens=[int(c) for c in torch.randint(1, 6000, (48,),
                      generator=torch.Generator().manual_seed(3))], seed=3)
    geo = big.geometry
    want, got = _both(big.query, big.key_pool, big.value_pool, big.slot_table, big.context_lens, geo.scaling,
                      geo.groups)
    assert torch.equal(got, want)

    small = decode_step("custom", context_lens=[700, 1, 65, 4096, 33], seed=4)
    want, got = _both(small.query, small.key_pool, small.value_pool, small.slot_table, small.context_lens,
                      geo.scaling, geo.groups)
    assert torch.equal(got, want)


def test_a_narrow_table_takes_the_short_kernel_through_either_entry_point():
    print("no-alloc decode: a narrow table (the one-launch short kernel), then a wide one", flush=True)
    for width in (None, 4096):
        b = PagedBatch([37, 128, 500, 1000], dtype=torch.bfloat16, num_heads=32, num_kv_heads=8, head_dim=128,
                       num_slots=8192, seed=9, width=width)
        want, got = _both(b.query, b.key_pool, b.value_pool, b.slot_table, b.context_lens_t, b.scaling, b.groups)
        assert torch.equal(got, want)
        assert_within(got, b.oracle(), 2e-2, 2e-3)


@pytest.mark.parametrize("kernel", ["auto", "equal_splits", "generic"])
def test_every_schedule_meets_the_oracle(kernel):
    print(f"no-alloc decode: kernel={kernel}", flush=True)
    b = PagedBatch([37, 128, 500, 1023, 3000], dtype=torch.bfloat16, num_heads=32, num_kv_heads=8, head_dim=128,
                   num_slots=8192, seed=7)
    splits = 4 if kernel == "equal_splits" else None
    want, got = _both(b.query, b.key_pool, b.value_pool, b.slot_table, b.context_lens_t, b.scaling, b.groups,
                      num_splits=splits, kernel=kernel)
    assert torch.equal(got, want)
    assert_within(got, b.oracle(), 2e-2, 2e-3)


def test_a_call_needing_more_scratch_is_refused_before_it_runs():
    # 16 query heads per KV head at head_dim 128: the balanced split's partials
    # (4 waves per CU, two partial slots of two KV heads each) outgrow 32 MiB.
    b = PagedBatch([100], dtype=torch.bfloat16, num_heads=32, num_kv_heads=2, head_dim=128, num_slots=256, seed=1)
    out = torch.zeros_like(b.query)
    with pytest.raises(ValueError, match="scratch"):
        paged_decode_noalloc(b.query, b.key_pool, b.value_pool, b.slot_table, b.context_lens_t, b.scaling, b.groups,
                             out=out)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0
