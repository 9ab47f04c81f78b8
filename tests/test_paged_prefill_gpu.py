"""The HIP packed/chunked prefill answers what the oracle answers.

Restates the reference's prefill tests (tests/unit/test_paged_prefill.py)
with the fp64 oracle as the answer, for both the general-shape kernel and the
MFMA kernel.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from liteinfer_amd.paged_kernels import paged_decode, paged_prefill
from tests.helpers import PagedBatch, assert_within, to_numpy

pytestmark = pytest.mark.gpu


def _run(b: PagedBatch, **kw) -> torch.Tensor:
    return paged_prefill(b.query, b.key_pool, b.value_pool, b.slot_table, b.context_lens_t, b.query_start_loc,
                         max(b.query_lens), b.scaling, b.groups, **kw)


def _fp32_close(actual, expected):
    np.testing.assert_allclose(to_numpy(actual), expected, rtol=1e-5, atol=1e-5)


def test_a_chunk_reads_its_prefix_and_its_own_past():
    b = PagedBatch([23], [5], num_slots=2048)
    _fp32_close(_run(b), b.oracle())


def test_a_whole_prompt_is_the_chunk_whose_context_is_itself():
    b = PagedBatch([37], [37], num_slots=2048)
    _fp32_close(_run(b), b.oracle())


def test_decode_rows_beside_chunks_in_one_launch():
    b = PagedBatch([90, 60, 3, 7], [1, 40, 1, 7], num_slots=2048)
    _fp32_close(_run(b), b.oracle())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_long_rows_beside_a_chunk_cut_into_many_pieces(dtype):
    """Two one-query rows over 20,000 and 9,000 keys beside a 64-query chunk:
    the rows' split cuts each (row, KV head) into many pieces, which the
    many-piece combine (several waves per head) folds."""
    b = PagedBatch([20000, 300, 9000], [1, 64, 1], dtype=dtype, num_heads=32, num_kv_heads=8, head_dim=128,
                   num_slots=1 << 15, seed=21)
    assert_within(_run(b), b.oracle(), 2 ** -6, 2e-3)


@pytest.mark.parametrize(
    ("contexts", "query_lens", "dtype", "head_dim", "num_heads", "num_kv_heads"),
    [
        ([4160], [64], torch.bfloat16, 128, 32, 8),  # one block over a long prefix: cut into pieces
        ([15512], [512], torch.bfloat16, 64, 32, 8),  # eight blocks, each cut
        ([2100, 9000], [100, 37], torch.float16, 128, 32, 8),  # two sequences, partial blocks
        ([6000], [300], torch.bfloat16, 128, 16, 2),  # two KV heads: one queue, eight groups
        ([700, 5000, 90], [700, 64, 1], torch.bfloat16, 128, 32, 8),  # a one-query row keeps the pass whole
        ([200], [150], torch.bfloat16, 128, 32, 8),  # too short to cut
        ([5032], [32], torch.bfloat16, 128, 64, 4),  # 16 heads per KV head: 16-query blocks
        ([3300, 2100], [300, 5], torch.bfloat16, 128, 8, 8),  # one head per KV head: 256-query blocks
        ([1100 + 37 * i for i in range(16)], [20 + i for i in range(16)], torch.float16, 64, 32, 8),  # 16 sequences
    ],
    ids=["64-over-4096", "512-over-15000", "two-f16", "two-kv-heads", "with-a-row", "short", "g16", "g1",
         "sixteen"],
)
def test_a_small_pass_cut_into_pieces(contexts, query_lens, dtype, head_dim, num_heads, num_kv_heads):
    """A pass whose blocks would leave most of the grid idle has each
    block's fully visible key stages cut into pieces folded by different
    work-groups and merged after the launch: same answer as the oracle."""
    b = PagedBatch(contexts, query_lens, dtype=dtype, num_heads=num_heads, num_kv_heads=num_kv_heads,
                   head_dim=head_dim, num_slots=1 << 15, seed=len(contexts) + head_dim)
    assert_within(_run(b), b.oracle(), 2 ** -6, 2e-3)


@pytest.mark.parametrize("block_q", [1, 4, 16, 32])
def test_the_answer_does_not_depend_on_the_query_block(block_q):
    b = PagedBatch([100, 16, 47, 9], [33, 16, 15, 1], num_slots=2048)
    _fp32_close(_run(b, block_q=block_q), b.oracle())


@pytest.mark.parametrize("block_kv", [16, 64, 128])
def test_the_answer_does_not_depend_on_the_key_tile(block_kv):
    b = PagedBatch([200, 65], [70, 3], num_slots=2048)
    _fp32_close(_run(b, block_kv=block_kv), b.oracle())


@pytest.mark.parametrize(
    ("num_heads", "num_kv_heads", "head_dim"),
    [(8, 8, 16), (8, 1, 16), (10, 2, 16), (8, 2, 80)],
    ids=["no-grouping", "one-kv-head", "group-not-a-power-of-two", "head-dim-not-a-power-of-two"],
)
def test_groupings_and_head_dims(num_heads, num_kv_heads, head_dim):
    b = PagedBatch([50, 30], [19, 1], num_heads=num_heads, num_kv_heads=num_kv_heads, head_dim=head_dim,
                   num_slots=2048)
    _fp32_close(_run(b), b.oracle())


def test_one_query_per_sequence_equals_decode():
    b = PagedBatch([90, 17, 1], [1, 1, 1], num_slots=2048)
    decode = paged_decode(b.query, b.key_pool, b.value_pool, b.slot_table, b.context_lens_t, b.scaling, b.groups,
                          num_splits=1)
    _fp32_close(_run(b), to_numpy(decode).astype(np.float64))


def test_strided_query_and_output_layout_are_kept():
    """The boundary hands over `query.squeeze(0).transpose(0, 1)`, a strided view."""
    b = PagedBatch([130, 64, 12], [33, 1, 12], dtype=torch.bfloat16, num_slots=2048)
    heads_first = b.query.transpose(0, 1).contiguous()  # [H, T, D]
    b.query = heads_first.transpose(0, 1)               # [T, H, D] view, token stride D
    out = _run(b)
    assert out.stride() == b.query.stride()
    assert_within(out, b.oracle(), 2 ** -6)


@pytest.mark.parametrize("kernel", ["auto", "generic"])
def test_bfloat16_within_rounding(kernel):
    b = PagedBatch([130, 64, 12], [33, 1, 12], dtype=torch.bfloat16, num_slots=2048)
    assert_within(_run(b, kernel=kernel), b.oracle(), 2 ** -6)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize(("num_heads", "num_kv_heads"), [(32, 8), (8, 8), (10, 2), (16, 1), (32, 16)])
@pytest.mark.parametrize("one_query_rows", [None, False])
def test_mfma_kernel_shapes(dtype, head_dim, num_heads, num_kv_heads, one_query_rows):
    """Chunks straddling every tile boundary, over prefixes and alone, beside decode rows.

    ``one_query_rows=False`` has the prefill kernel serve the one-query
    sequences too (the decode kernel is not launched): same answer.
    """
    b = PagedBatch([1, 40, 300, 129, 64, 700], [1, 33, 200, 1, 64, 31], dtype=dtype, num_heads=num_heads,
                   num_kv_heads=num_kv_heads, head_dim=head_dim, num_slots=4096, seed=6)
    assert_within(_run(b, one_query_rows=one_query_rows), b.oracle(), 2 ** -6, 2e-3)


@pytest.mark.parametrize(("num_heads", "num_kv_heads"), [(32, 8), (32, 16), (8, 2)])
def test_persistent_grid_takes_every_unit_on_every_call(num_heads, num_kv_heads):
    """More (query block, KV head) units than work-groups, in per-XCD queues or one
    queue; the queues restart empty on every launch, so repeated calls agree bit for bit."""
    rng = np.random.default_rng(11)
    q = rng.integers(1, 200, size=24).tolist()
    p = rng.integers(0, 300, size=24).tolist()
    b = PagedBatch([qq + pp for qq, pp in zip(q, p)], q, dtype=torch.bfloat16, num_heads=num_heads,
                   num_kv_heads=num_kv_heads, head_dim=128, num_slots=32768, seed=12)
    first = _run(b)
    assert_within(first, b.oracle(), 2 ** -6, 2e-3)
    for _ in range(3):
        again = _run(b)
        assert torch.equal(again, first)


@pytest.mark.parametrize(("num_heads", "num_kv_heads"), [(32, 8), (16, 4)])
def test_more_sequences_than_the_work_list_kernel_has_threads(num_heads, num_kv_heads):
    """1,100 sequences (one to three queries each over short prefixes): the
    work-list kernel walks them in strides of its 1,024 threads, keeps each
    sequence's blocks together, and the one-query ones go to the decode
    kernel; Hkv 4 runs the single-queue grid."""
    rng = np.random.default_rng(21)
    n = 1100
    q = rng.integers(1, 4, size=n).tolist()
    p = rng.integers(0, 40, size=n).tolist()
    b = PagedBatch([qq + pp for qq, pp in zip(q, p)], q, dtype=torch.bfloat16, num_heads=num_heads,
                   num_kv_heads=num_kv_heads, head_dim=128, num_slots=65536, seed=21)
    assert_within(_run(b), b.oracle(), 2 ** -6, 2e-3)
    assert_within(_run(b, one_query_rows=False), b.oracle(), 2 ** -6, 2e-3)


@pytest.mark.parametrize("one_query_rows", [None, False])
@pytest.mark.parametrize("pool", ["bf16", "fp8"])
def test_a_packed_pass_writes_its_rows_and_nothing_around_them(one_query_rows, pool):
    """Chunks beside one-query rows (one of them with a context of one key),
    into an output that is a window of a larger buffer: every row outside the
    window keeps its sentinel, bit for bit (no kernel of the pass may store
    outside the rows it owns)."""
    from oracle import fp8

    b = PagedBatch([1, 40, 300, 129, 64, 700], [1, 33, 200, 1, 64, 31], dtype=torch.bfloat16, num_heads=32,
                   num_kv_heads=8, head_dim=128, num_slots=4096, seed=13)
    from oracle.attention import attend

    kp, vp, k_scale, v_scale = b.key_pool, b.value_pool, 1.0, 1.0
    if pool == "fp8":
        k_scale, v_scale = 0.5, 0.25
        kc, vc = fp8.quantize(to_numpy(b.key_pool), k_scale), fp8.quantize(to_numpy(b.value_pool), v_scale)
        kp = torch.from_numpy(kc).cuda().view(torch.float8_e4m3fn)
        vp = torch.from_numpy(vc).cuda().view(torch.float8_e4m3fn)
        # the attention of the rows the fp8 pool holds, dequantised
        want = attend(to_numpy(b.query), fp8.dequantize(kc, k_scale), fp8.dequantize(vc, v_scale),
                      b.slot_table.cpu().numpy(), np.asarray(b.context_lens), b.scaling, b.groups,
                      query_start_loc=to_numpy(b.query_start_loc).astype(np.int32), dtype=np.float64)
    else:
        want = b.oracle()
    t = b.query.shape[0]
    big = torch.full((t + 8, 32, 128), 7.0, dtype=torch.bfloat16, device="cuda")
    out = big[4:4 + t]
    got = paged_prefill(b.query, kp, vp, b.slot_table, b.context_lens_t, b.query_start_loc, max(b.query_lens),
                        b.scaling, b.groups, one_query_rows=one_query_rows, k_scale=k_scale, v_scale=v_scale,
                        out=out)
    torch.cuda.synchronize()
    assert got.data_ptr() == out.data_ptr()
    assert torch.equal(big[:4], torch.full_like(big[:4], 7.0))
    assert torch.equal(big[4 + t:], torch.full_like(big[4 + t:], 7.0))
    # the bf16 pool to the bf16 bar; the fp8 pool to the bar its own tests use
    assert_within(got, want, 2 ** -6 if pool == "bf16" else 2e-2, 2e-3)


_RNG = np.random.default_rng(11)
_MANY_ROWS = _RNG.integers(200, 3000, size=160).tolist()


@pytest.mark.parametrize(
    ("contexts", "query_lens"),
    [
        ([700] + _MANY_ROWS, [300] + [1] * len(_MANY_ROWS)),
        ([2100, 1500, 1800, 999], [2000, 1500, 700, 1]),
        ([30000, 45000, 600, 2600], [1, 1, 512, 1]),
        ([5000, 77, 1], [1, 77, 1]),
    ],
    ids=["rows-outweigh-one-chunk", "one-row-beside-chunks", "long-rows-in-pieces", "a-one-key-row"],
)
@pytest.mark.parametrize(
    ("dtype", "head_dim", "num_heads", "num_kv_heads"),
    [(torch.bfloat16, 128, 32, 8), (torch.float16, 64, 16, 8), (torch.bfloat16, 128, 12, 3)],
    ids=["bf16-d128", "f16-d64", "three-kv-heads"],
)
def test_rows_and_chunks_share_the_prefill_launch(contexts, query_lens, dtype, head_dim, num_heads, num_kv_heads):
    """16-bit pools: the one-query rows are folded by the prefill launch's first
    work-groups (the decode split, as many work-groups as the rows' bytes
    against the chunks' flops ask for), which then join the chunks' queues."""
    b = PagedBatch(contexts, query_lens, dtype=dtype, num_heads=num_heads, num_kv_heads=num_kv_heads,
                   head_dim=head_dim, num_slots=65536)
    expected = b.oracle()
    assert_within(_run(b), expected, 2 ** -6, 2e-3)
    # Folding the rows as query blocks of the prefill instead gives the same attention.
    assert_within(_run(b, one_query_rows=False), expected, 2 ** -6, 2e-3)


@pytest.mark.parametrize(("num_seqs", "num_heads", "num_kv_heads", "head_dim", "dtype", "max_q", "max_prefix"), [
    (64, 8, 2, 128, torch.bfloat16, 60, 300),     # the most sequences the direct schedule scans
    (32, 32, 8, 128, torch.bfloat16, 64, 3000),   # 256 units: every CU one, prefixes past 1,024 keys
    (5, 32, 8, 64, torch.float16, 150, 90),       # several blocks a sequence, the first partial
    (65, 8, 1, 128, torch.bfloat16, 40, 200),     # one sequence too many: the work list again
    (3, 16, 1, 128, torch.bfloat16, 16, 0),       # 16 heads per KV head, no prefix
])
def test_a_small_pass_runs_one_work_group_per_unit(num_seqs, num_heads, num_kv_heads, head_dim, dtype, max_q,
                                                   max_prefix):
    """A pass whose (query block, KV head) units all fit the grid at once, with no one-query rows
    in the launch, skips the work-list kernel: work-group i scans the query counts for its own
    unit. One-query sequences are folded by the prefill kernel here (``one_query_rows=False``);
    repeated calls agree bit for bit."""
    rng = np.random.default_rng(num_seqs + head_dim)
    q = rng.integers(1, max_q + 1, size=num_seqs).tolist()
    p = rng.integers(0, max_prefix + 1, size=num_seqs).tolist()
    b = PagedBatch([qq + pp for qq, pp in zip(q, p)], q, dtype=dtype, num_heads=num_heads,
                   num_kv_heads=num_kv_heads, head_dim=head_dim, num_slots=1 << 17, seed=num_seqs)
    first = _run(b, one_query_rows=False)
    assert_within(first, b.oracle(), 2 ** -6, 2e-3)
    assert torch.equal(_run(b, one_query_rows=False), first)


@pytest.mark.parametrize("width", [None, 4096])
def test_a_pass_of_only_one_query_rows_runs_as_a_decode_step(width):
    """paged_attention over a packed payload whose host query lengths are all 1: the pass is a
    decode step and runs as one (the same attention as the packed kernels give it)."""
    from liteinfer_amd.attention import PagedKV, paged_attention

    ctx = [5, 300, 1, 2000, 77]
    b = PagedBatch(ctx, [1] * len(ctx), dtype=torch.bfloat16, num_heads=32, num_kv_heads=8, head_dim=128,
                   num_slots=8192, seed=51, width=width)
    q = b.query.transpose(0, 1).unsqueeze(0)  # [1, heads, tokens, dim], as the model's packed pass holds it
    kv = PagedKV(b.key_pool, b.value_pool, b.slot_table, b.context_lens_t, query_start_loc=b.query_start_loc,
                 max_query_len=1, host_context_lens=tuple(ctx), host_query_lens=tuple([1] * len(ctx)))
    out = paged_attention(q, kv, b.scaling, b.groups)
    assert out.shape == q.shape
    want = b.oracle()
    assert_within(out.squeeze(0).transpose(0, 1), want, 2 ** -6, 2e-3)
    # without the host lengths the packed kernels serve it: the same attention
    kv_dev = PagedKV(b.key_pool, b.value_pool, b.slot_table, b.context_lens_t, query_start_loc=b.query_start_loc,
                     max_query_len=1)
    assert_within(paged_attention(q, kv_dev, b.scaling, b.groups).squeeze(0).transpose(0, 1), want, 2 ** -6, 2e-3)
