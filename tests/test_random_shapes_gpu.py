"""Seeded random shapes for the HIP decode and packed prefill, against the fp64 oracle.

The hand-picked cases in the other files pin the rules one at a time; these
draw the shape itself (batch, contexts, query lengths, KV heads, group size,
head_dim, query dtype, fp8 pools) from a fixed seed per case, so the
kernels' scheduling (balanced shares, head-grouped segments, persistent
prefill queues, one-query rows beside chunks) meets combinations no listed
case names. Every case is at the bf16 bar: max-abs 2^-6 and mean-abs 2e-3
against the fp64 oracle (fp8 pools: the oracle over the dequantised rows,
max-abs 2e-2).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from liteinfer_amd.paged_kernels import paged_decode, paged_prefill
from oracle import fp8
from oracle.attention import attend
from tests.helpers import PagedBatch, assert_within, to_numpy

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn


def _heads(rng):
    num_kv_heads = int(rng.choice([1, 2, 3, 4, 8]))
    groups = int(rng.choice([1, 2, 4, 5, 8, 16]))
    return num_kv_heads * groups, num_kv_heads


def _contexts(rng, batch, longest):
    """Mostly short contexts, some long, a few at 1 and at tile edges."""
    ctx = rng.integers(1, longest // 4 + 2, size=batch)
    long_ones = rng.random(batch) < 0.2
    ctx[long_ones] = rng.integers(longest // 2, longest + 1, size=int(long_ones.sum()))
    edges = rng.random(batch) < 0.1
    ctx[edges] = rng.choice([1, 31, 32, 33, 63, 64, 65], size=int(edges.sum()))
    return [int(c) for c in ctx]


@pytest.mark.parametrize("case", range(16))
def test_decode_random_shapes(case):
    rng = np.random.default_rng(7000 + case)
    num_heads, num_kv_heads = _heads(rng)
    head_dim = int(rng.choice([64, 128]))
    dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float16
    batch = int(rng.integers(1, 200))
    ctx = _contexts(rng, batch, int(rng.choice([600, 3000])))
    b = PagedBatch(ctx, dtype=dtype, num_heads=num_heads, num_kv_heads=num_kv_heads, head_dim=head_dim,
                   num_slots=16384, seed=7000 + case)
    splits = None if rng.random() < 0.7 else int(rng.integers(1, 9))
    out = paged_decode(b.query, b.key_pool, b.value_pool, b.slot_table, b.context_lens_t, b.scaling, b.groups,
                       num_splits=splits)
    assert_within(out, b.oracle(), 2 ** -6, 2e-3)


@pytest.mark.parametrize("case", range(12))
def test_prefill_random_shapes(case):
    rng = np.random.default_rng(8000 + case)
    num_heads, num_kv_heads = _heads(rng)
    head_dim = int(rng.choice([64, 128]))
    dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float16
    batch = int(rng.integers(1, 12))
    ctx = _contexts(rng, batch, int(rng.choice([400, 1500])))
    # Each sequence's queries are the last of its context: one (a decode row)
    # for about a third, up to the whole context for the rest.
    q = [1 if rng.random() < 0.35 else int(rng.integers(1, min(c, 300) + 1)) for c in ctx]
    b = PagedBatch(ctx, q, dtype=dtype, num_heads=num_heads, num_kv_heads=num_kv_heads, head_dim=head_dim,
                   num_slots=16384, seed=8000 + case)
    out = paged_prefill(b.query, b.key_pool, b.value_pool, b.slot_table, b.context_lens_t, b.query_start_loc,
                        max(q), b.scaling, b.groups, one_query_rows=(1 in q))
    assert_within(out, b.oracle(), 2 ** -6, 2e-3)


@pytest.mark.parametrize("case", range(8))
def test_fp8_decode_random_shapes(case):
    rng = np.random.default_rng(9000 + case)
    num_heads, num_kv_heads = _heads(rng)
    k_scale, v_scale = float(rng.choice([0.25, 1.0])), float(rng.choice([0.5, 1.0]))
    batch = int(rng.integers(1, 150))
    ctx = _contexts(rng, batch, 2000)
    b = PagedBatch(ctx, dtype=torch.bfloat16, num_heads=num_heads, num_kv_heads=num_kv_heads, head_dim=128,
                   num_slots=16384, seed=9000 + case)
    kc = fp8.quantize(to_numpy(b.key_pool), k_scale)
    vc = fp8.quantize(to_numpy(b.value_pool), v_scale)
    want = attend(to_numpy(b.query), fp8.dequantize(kc, k_scale), fp8.dequantize(vc, v_scale),
                  b.slot_table.cpu().numpy(), np.asarray(ctx), b.scaling, b.groups, dtype=np.float64)
    kp = torch.from_numpy(kc).to(b.device).view(FP8)
    vp = torch.from_numpy(vc).to(b.device).view(FP8)
    out = paged_decode(b.query, kp, vp, b.slot_table, b.context_lens_t, b.scaling, b.groups, k_scale=k_scale,
                       v_scale=v_scale)
    assert_within(out, want, 2e-2, 2e-3)


@pytest.mark.parametrize("case", range(4))
def test_decode_random_long_contexts(case):
    """Fewer sequences, contexts up to 20,000 keys: many slot chunks per
    segment, pieces spread over many waves."""
    rng = np.random.default_rng(7500 + case)
    num_heads, num_kv_heads = _heads(rng)
    head_dim = int(rng.choice([64, 128]))
    batch = int(rng.integers(1, 17))
    ctx = _contexts(rng, batch, 20000)
    b = PagedBatch(ctx, dtype=torch.bfloat16, num_heads=num_heads, num_kv_heads=num_kv_heads, head_dim=head_dim,
                   num_slots=65536, seed=7500 + case)
    out = paged_decode(b.query, b.key_pool, b.value_pool, b.slot_table, b.context_lens_t, b.scaling, b.groups)
    assert_within(out, b.oracle(), 2 ** -6, 2e-3)


@pytest.mark.parametrize("case", range(3))
def test_prefill_random_long_chunks(case):
    """Chunks of up to 600 queries over prefixes of up to 4,000 keys, beside one-query rows."""
    rng = np.random.default_rng(8500 + case)
    num_heads, num_kv_heads = _heads(rng)
    batch = int(rng.integers(2, 5))
    ctx = _contexts(rng, batch, 4600)
    q = [1 if i % 2 else int(rng.integers(1, min(c, 600) + 1)) for i, c in enumerate(ctx)]
    b = PagedBatch(ctx, q, dtype=torch.bfloat16, num_heads=num_heads, num_kv_heads=num_kv_heads, head_dim=128,
                   num_slots=65536, seed=8500 + case)
    for one_query_rows in (True, False):
        out = paged_prefill(b.query, b.key_pool, b.value_pool, b.slot_table, b.context_lens_t, b.query_start_loc,
                            max(q), b.scaling, b.groups, one_query_rows=one_query_rows)
        assert_within(out, b.oracle(), 2 ** -6, 2e-3)


@pytest.mark.parametrize("case", range(12))
def test_decode_step_with_newest_rows_random_shapes(case):
    """paged_decode(new_key=, new_value=) against the scatter-then-decode pair on the same pools: the
    pools and the attention bit for bit, whatever the shape (each sequence's slots its own, as a cache
    hands them out)."""
    from liteinfer_amd.cache.kv_cache import scatter_into

    rng = np.random.default_rng(7500 + case)
    num_heads, num_kv_heads = _heads(rng)
    head_dim = int(rng.choice([64, 128]))
    dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float16
    batch = int(rng.integers(1, 120))
    ctx = _contexts(rng, batch, int(rng.choice([600, 3000])))
    num_slots = sum(ctx) + max(ctx) + 64
    g = torch.Generator().manual_seed(7500 + case)
    kp = torch.randn(num_slots, num_kv_heads, head_dim, generator=g).to(dtype).cuda()
    vp = torch.randn(num_slots, num_kv_heads, head_dim, generator=g).to(dtype).cuda()
    q = torch.randn(batch, num_heads, head_dim, generator=g).to(dtype).cuda()
    nk = torch.randn(batch, num_kv_heads, head_dim, generator=g).to(dtype).cuda()
    nv = torch.randn(batch, num_kv_heads, head_dim, generator=g).to(dtype).cuda()
    perm = torch.randperm(num_slots, generator=g)
    width = max(ctx)
    table = torch.empty(batch, width, dtype=torch.int64)
    at = 0
    for i, c in enumerate(ctx):
        table[i, :c] = perm[at:at + c]
        table[i, c:] = perm[-(width - c):] if width > c else table[i, c:]
        at += c
    table = table.cuda()
    lens = torch.tensor(ctx, dtype=torch.int32, device="cuda")
    groups, scale = num_heads // num_kv_heads, head_dim ** -0.5
    kp1, vp1 = kp.clone(), vp.clone()
    fused = paged_decode(q, kp1, vp1, table, lens, scale, groups, new_key=nk, new_value=nv)
    newest = table.gather(1, (lens.long() - 1)[:, None]).view(1, -1)
    scatter_into(kp, vp, newest, nk.unsqueeze(2), nv.unsqueeze(2))
    paired = paged_decode(q, kp, vp, table, lens, scale, groups)
    torch.cuda.synchronize()
    assert torch.equal(kp1.view(torch.int16), kp.view(torch.int16))
    assert torch.equal(vp1.view(torch.int16), vp.view(torch.int16))
    assert torch.equal(fused.view(torch.int16), paired.view(torch.int16))


@pytest.mark.parametrize("case", range(10))
def test_small_prefill_passes_without_a_work_list_random_shapes(case):
    """Passes of at most 64 sequences, the caller saying no row is served elsewhere, sized so that
    their (query block, KV head) units fit the grid where batch x KV heads allows (one launch,
    each work-group finding its unit from the query counts; otherwise the listed schedule).
    One-query sequences are folded as blocks too."""
    rng = np.random.default_rng(9500 + case)
    num_kv_heads = int(rng.choice([1, 2, 4, 8]))
    groups = int(rng.choice([1, 2, 4, 8, 16]))
    head_dim = int(rng.choice([64, 128]))
    dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float16
    block_q = 256 // groups
    batch = int(rng.integers(1, 65))
    # keep batch x KV heads x blocks of the longest query run within the grid's 256 work-groups
    max_blocks = max(1, 256 // (batch * num_kv_heads))
    q = [int(rng.integers(1, block_q * max_blocks + 1)) for _ in range(batch)]
    ctx = [qq + int(rng.integers(0, 900)) for qq in q]
    b = PagedBatch(ctx, q, dtype=dtype, num_heads=num_kv_heads * groups, num_kv_heads=num_kv_heads,
                   head_dim=head_dim, num_slots=1 << 16, seed=9500 + case)
    out = paged_prefill(b.query, b.key_pool, b.value_pool, b.slot_table, b.context_lens_t, b.query_start_loc,
                        max(q), b.scaling, b.groups, one_query_rows=False)
    assert_within(out, b.oracle(), 2 ** -6, 2e-3)
