"""The HIP paged decode answers what the oracle answers.

Restates the reference's decode tests (tests/unit/test_paged_decode.py) with
the fp64 oracle as the answer: fp32 within rtol = atol = 1e-5, bf16 within
atol 2^-6, and BASELINE's bar for bf16 (max-abs 2e-2, mean-abs 2e-3). Both
kernels are checked: the MFMA kernel (bf16/fp16, head_dim 64/128, groups up to
16) and the general-shape kernel (everything, fp32 above all).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from liteinfer_amd.paged_kernels import paged_decode
from tests.helpers import PagedBatch, assert_within, to_numpy

pytestmark = pytest.mark.gpu

# A slot table this wide takes any batch to the balanced split (the short
# kernel serves tables up to 2,048 columns).
WIDE = 4096


def _run(b: PagedBatch, **kw) -> torch.Tensor:
    return paged_decode(b.query, b.key_pool, b.value_pool, b.slot_table, b.context_lens_t, b.scaling, b.groups, **kw)


def _fp32_close(actual, expected):
    np.testing.assert_allclose(to_numpy(actual), expected, rtol=1e-5, atol=1e-5)


# --- the reference's cases, fp32 through the general-shape kernel ----------------------


def test_float32_matches_the_oracle():
    b = PagedBatch([6, 4, 1])
    _fp32_close(_run(b), b.oracle())


@pytest.mark.parametrize("block_kv", [16, 32, 64, 128])
def test_the_answer_does_not_depend_on_the_key_tile(block_kv):
    b = PagedBatch([200, 65, 64, 63, 17, 1])
    _fp32_close(_run(b, block_kv=block_kv), b.oracle())


def test_a_group_that_is_not_a_power_of_two():
    b = PagedBatch([70, 5], num_heads=10, num_kv_heads=2)
    _fp32_close(_run(b), b.oracle())


def test_no_grouped_query_heads():
    b = PagedBatch([9, 3], num_kv_heads=8)
    _fp32_close(_run(b), b.oracle())


@pytest.mark.parametrize("head_dim", [96, 80, 48, 24])
def test_head_dims_off_the_fast_path(head_dim):
    b = PagedBatch([70, 5], head_dim=head_dim)
    _fp32_close(_run(b), b.oracle())


@pytest.mark.parametrize("num_splits", [1, 2, 3, 5, 8, 32])
def test_the_answer_does_not_depend_on_the_split_count(num_splits):
    b = PagedBatch([200, 65, 64, 63, 17, 1])
    _fp32_close(_run(b, num_splits=num_splits), b.oracle())


def test_split_and_unsplit_agree():
    b = PagedBatch([300, 129, 7])
    torch.testing.assert_close(_run(b, num_splits=11), _run(b, num_splits=1), rtol=1e-5, atol=1e-5)


def test_splits_past_a_short_context_contribute_nothing():
    b = PagedBatch([200, 3])
    _fp32_close(_run(b, num_splits=8), b.oracle())


def test_padding_columns_are_never_read():
    b = PagedBatch([200, 65, 3], dtype=torch.bfloat16)
    for kernel in ("auto", "equal_splits", "generic"):
        first = _run(b, kernel=kernel, num_splits=3 if kernel == "equal_splits" else None)
        table = b.slot_table.clone()
        cols = torch.arange(table.shape[1], device=table.device)
        pad = cols[None, :] >= b.context_lens_t[:, None]
        table[pad] = torch.randint(1, 512, (int(pad.sum()),), device=table.device)
        b2 = b
        b2.slot_table = table
        assert torch.equal(_run(b2, kernel=kernel, num_splits=3 if kernel == "equal_splits" else None), first)


def test_pools_laid_out_differently_are_refused():
    b = PagedBatch([4])
    with pytest.raises(ValueError, match="laid out identically"):
        paged_decode(b.query, b.key_pool, b.value_pool.transpose(1, 2), b.slot_table, b.context_lens_t, b.scaling,
                     b.groups)


def test_pools_of_2_pow_31_slots_are_refused():
    """The attention kernels hold slot indices in 32 bits; a bigger pool is refused, not wrapped."""
    from liteinfer_amd.paged_kernels import paged_prefill

    b = PagedBatch([4])
    huge_k = b.key_pool[:1].expand(1 << 31, *b.key_pool.shape[1:])
    huge_v = b.value_pool[:1].expand(1 << 31, *b.value_pool.shape[1:])
    with pytest.raises(ValueError, match="fewer than 2\\*\\*31 slots"):
        paged_decode(b.query, huge_k, huge_v, b.slot_table, b.context_lens_t, b.scaling, b.groups)
    qsl = torch.tensor([0, 1], dtype=torch.int32, device=b.query.device)
    with pytest.raises(ValueError, match="fewer than 2\\*\\*31 slots"):
        paged_prefill(b.query, huge_k, huge_v, b.slot_table, b.context_lens_t, qsl, 1, b.scaling, b.groups)


def test_fewer_than_one_split_is_refused():
    b = PagedBatch([4])
    with pytest.raises(ValueError, match="num_splits must be >= 1"):
        _run(b, num_splits=0)


# --- bf16 / fp16 through both kernels --------------------------------------------------


@pytest.mark.parametrize("kernel", ["auto", "equal_splits", "generic"])
@pytest.mark.parametrize("num_splits", [None, 1, 11])
def test_bfloat16_within_rounding(kernel, num_splits):
    b = PagedBatch([300, 129, 7], dtype=torch.bfloat16)
    assert_within(_run(b, kernel=kernel, num_splits=num_splits), b.oracle(), 2 ** -6)


@pytest.mark.parametrize("width", [None, WIDE])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize(("num_heads", "num_kv_heads"), [(32, 8), (8, 8), (10, 2), (32, 4), (16, 1)])
def test_mfma_kernel_shapes(dtype, head_dim, num_heads, num_kv_heads, width):
    """Every group the MFMA kernel takes (1, 4, 5, 8, 16), contexts straddling 32-key tiles;
    a table as wide as the longest context (the short kernel) and a wide one (the balanced split)."""
    b = PagedBatch([1, 31, 32, 33, 100, 257, 1000], dtype=dtype, num_heads=num_heads, num_kv_heads=num_kv_heads,
                   head_dim=head_dim, num_slots=4096, seed=2, width=width)
    want = b.oracle()
    for kernel in ("auto", "equal_splits"):
        for splits in (None, 1, 3):
            assert_within(_run(b, kernel=kernel, num_splits=splits), want, 2 ** -6, 2e-3)


@pytest.mark.parametrize(("num_heads", "num_kv_heads"), [(64, 16), (24, 12), (12, 6), (16, 4)])
def test_head_groups_sharing_work_groups(num_heads, num_kv_heads):
    """KV head counts whose pairs the head-grouped decode runs four (16),
    two (12, 4) or one (6) to a work-group, with more than one set of
    work-group groups where the pair count exceeds four (16, 12): long and
    short contexts, so that work-groups cross both sequence and head-group
    boundaries."""
    b = PagedBatch([5000, 1, 77, 2100, 32, 9000, 640], dtype=torch.bfloat16, num_heads=num_heads,
                   num_kv_heads=num_kv_heads, head_dim=128, num_slots=1 << 15, seed=4)
    assert_within(_run(b), b.oracle(), 2 ** -6, 2e-3)


@pytest.mark.parametrize("width", [None, WIDE])
@pytest.mark.parametrize("num_kv_heads", [8, 2])
def test_thousands_of_short_contexts(num_kv_heads, width):
    """2,500 sequences of 1-80 keys: every work-group of the balanced grid
    walks about ten segments, and its starting sequence is found past the
    first 64 of the batch's key counts."""
    rng = np.random.default_rng(11)
    ctx = rng.integers(1, 81, size=2500).tolist()
    b = PagedBatch(ctx, dtype=torch.bfloat16, num_heads=4 * num_kv_heads, num_kv_heads=num_kv_heads,
                   head_dim=128, num_slots=1 << 17, seed=11, width=width)
    assert_within(_run(b), b.oracle(), 2 ** -6, 2e-3)


def test_mfma_and_general_kernels_agree():
    b = PagedBatch([513, 64, 2000, 1], dtype=torch.bfloat16, num_heads=32, num_kv_heads=8, head_dim=128,
                   num_slots=8192, seed=4)
    fast = _run(b)
    slow = _run(b, kernel="generic")
    assert_within(fast, to_numpy(slow).astype(np.float64), 2 ** -7)


def test_strided_query_is_served():
    b = PagedBatch([77, 5], dtype=torch.bfloat16, num_heads=32, num_kv_heads=8, head_dim=128, num_slots=1024)
    wide = torch.zeros(b.query.shape[0], b.query.shape[1], 256, dtype=b.query.dtype, device=b.query.device)
    wide[..., :128] = b.query
    b.query = wide[..., :128]
    assert_within(_run(b), b.oracle(), 2 ** -6)


def test_long_context_is_partitioned_and_combined():
    b = PagedBatch([20000, 3000], dtype=torch.bfloat16, num_heads=32, num_kv_heads=8, head_dim=128,
                   num_slots=32768, seed=9)
    assert_within(_run(b), b.oracle(), 2e-2, 2e-3)


@pytest.mark.parametrize(("context_lens", "num_kv_heads"), [([60000], 1), ([40000, 9], 2), ([120000], 2)])
def test_a_context_cut_into_hundreds_of_pieces(context_lens, num_kv_heads):
    """One long sequence over one or two KV heads: the balanced grid cuts each
    (sequence, KV head) into hundreds of pieces, which the combine folds in
    rounds of 32 with a running maximum (dozens of rounds here); a 9-key
    sequence beside it stays whole in one wave."""
    b = PagedBatch(context_lens, dtype=torch.bfloat16, num_heads=4 * num_kv_heads, num_kv_heads=num_kv_heads,
                   head_dim=128, num_slots=131072, seed=23)
    assert_within(_run(b), b.oracle(), 2e-2, 2e-3)


@pytest.mark.parametrize(("num_heads", "num_kv_heads", "head_dim"), [(32, 8, 128), (16, 1, 64), (12, 6, 128)])
def test_more_sequences_than_a_wave_has_lanes(num_heads, num_kv_heads, head_dim):
    """150 sequences: the balanced kernels find a wave's first sequence and
    count keys 64 sequences at a time, so this takes three passes; some
    contexts are shorter than a share, some span several waves. KV heads in
    pairs (8, 6) run the head-grouped kernel, a single KV head the per-head one."""
    rng = np.random.default_rng(31)
    ctx = rng.integers(1, 600, size=150).tolist()
    b = PagedBatch(ctx, dtype=torch.bfloat16, num_heads=num_heads, num_kv_heads=num_kv_heads, head_dim=head_dim,
                   num_slots=8192, seed=31, width=WIDE)
    assert_within(_run(b), b.oracle(), 2 ** -6, 2e-3)


@pytest.mark.parametrize("width", [None, WIDE])
@pytest.mark.parametrize("kernel", ["auto", "equal_splits", "generic"])
def test_a_row_with_no_keys_is_nan_like_the_reference(kernel, width):
    """A context of 0 keys: the reference's softmax over nothing gives 0 / 0
    (NaN) for that row; the other rows are unaffected."""
    b = PagedBatch([300, 0, 45], dtype=torch.bfloat16, num_heads=32, num_kv_heads=8, head_dim=128, num_slots=2048,
                   seed=9, width=width)
    out = paged_decode(b.query, b.key_pool, b.value_pool, b.slot_table, b.context_lens_t, b.scaling, b.groups,
                       num_splits=2 if kernel == "equal_splits" else None, kernel=kernel)
    assert torch.isnan(out[1].float()).all()
    want = b.oracle()
    assert_within(out[[0, 2]], want[[0, 2]], 2e-2, 2e-3)


# --- the short kernel: one work-group per (sequence, KV head) ---------------------------


@pytest.mark.parametrize(("context_lens", "num_heads", "num_kv_heads", "head_dim", "width"), [
    ([1], 32, 8, 64, None),                  # one key: seven of eight waves fold nothing
    ([128], 32, 8, 64, None),                # the reference's batch-1 shape
    ([190] * 32, 32, 8, 64, None),
    ([1024], 32, 8, 128, None),              # the widest table at any segment count
    ([31, 32, 33, 255, 256, 257, 1000], 16, 1, 64, None),  # runs that end inside a tile
    ([2048] * 16, 32, 8, 64, None),          # 128 segments: a 2,048-wide table still short
    ([700, 5, 2048] + [64] * 29, 32, 4, 128, 2048),
    ([1024] * 64, 32, 8, 64, None),          # segments x width at the rule's limit
    ([33, 600, 1], 64, 4, 128, None),        # 16 heads per KV head
    ([100, 513], 10, 2, 128, None),          # a group of 5
])
def test_short_contexts_in_one_launch(context_lens, num_heads, num_kv_heads, head_dim, width):
    """Batches whose table is at most 1,024 (or, over 128 segments, 2,048) columns wide run the short
    kernel: its waves split each context into equal runs of whole tiles and merge their softmax
    states in LDS. Runs ending inside a tile, waves with no keys, groups of 1-16, both head_dims."""
    b = PagedBatch(context_lens, dtype=torch.bfloat16, num_heads=num_heads, num_kv_heads=num_kv_heads,
                   head_dim=head_dim, num_slots=1 << 16, seed=41, width=width)
    assert_within(_run(b), b.oracle(), 2 ** -6, 2e-3)


@pytest.mark.parametrize("head_dim", [64, 128])
def test_short_and_balanced_kernels_in_half_precision(head_dim):
    """fp16 through both kernels (a tight table and a wide one), each within the bar of the oracle."""
    b = PagedBatch([3, 77, 640, 1024], dtype=torch.float16, num_heads=32, num_kv_heads=8, head_dim=head_dim,
                   num_slots=8192, seed=43)
    short = _run(b)
    wide = PagedBatch([3, 77, 640, 1024], dtype=torch.float16, num_heads=32, num_kv_heads=8, head_dim=head_dim,
                      num_slots=8192, seed=43, width=WIDE)
    balanced = _run(wide)
    assert_within(short, b.oracle(), 2 ** -6, 2e-3)
    assert_within(balanced, wide.oracle(), 2 ** -6, 2e-3)


@pytest.mark.parametrize("head_dim", [64, 128])
def test_contexts_past_a_narrowed_tables_width_are_still_folded(head_dim):
    """A table passed as a narrower view of a wider one (its rows keep the wider pitch), with
    contexts past the view's width: every kernel reads slot_table[i, :ctx] through the row pitch,
    as the reference's pointer arithmetic does, so the answer is the wide table's."""
    b = PagedBatch([1000, 300, 700], dtype=torch.bfloat16, num_heads=32, num_kv_heads=8, head_dim=head_dim,
                   num_slots=8192, seed=47)
    want = b.oracle()
    narrow = b.slot_table[:, :512]
    assert narrow.stride(0) == b.slot_table.shape[1]
    out = paged_decode(b.query, b.key_pool, b.value_pool, narrow, b.context_lens_t, b.scaling, b.groups)
    assert_within(out, want, 2 ** -6, 2e-3)
