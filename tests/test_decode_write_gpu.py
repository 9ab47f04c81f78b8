"""A decode step that writes each sequence's newest K / V rows and attends in one call.

`paged_decode(..., new_key=, new_value=)` is the decode pair of the
reference's layer step: ``KVCache.scatter`` at the slots ``newest_slots``
gives for position ``context_len - 1`` (liteinfer/cache/kv_cache.py:236-253,
liteinfer/cache/block_pool.py:151-170), then ``paged_decode``
(liteinfer/models/paged_kernels.py:696-818). On the head-grouped kernel over a
16-bit pool both happen in the decode launch; elsewhere a write launch runs
first. Either way the pool must end bit-identical to the scatter's, and the
attention bit-identical to the same decode run after the scatter (the fused
kernel folds the new rows from registers, which hold the same bits the pool
then holds). Tables hand each sequence slots of its own, as a cache does.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from liteinfer_amd import paged_kernels
from liteinfer_amd.cache.kv_cache import scatter_into
from liteinfer_amd.paged_kernels import paged_decode
from tests.helpers import assert_within, to_numpy

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


class _Step:
    def __init__(self, contexts, num_heads=32, num_kv_heads=8, head_dim=128, dtype=torch.bfloat16,
                 num_slots=1 << 15, seed=0, fill=None, width=None):
        g = torch.Generator().manual_seed(seed)
        self.contexts = list(contexts)
        batch = len(self.contexts)
        self.groups = num_heads // num_kv_heads
        self.scaling = head_dim ** -0.5
        self.dtype = dtype

        def randn(*shape):
            return torch.randn(*shape, generator=g).to(dtype).to(DEV)

        self.key_pool = randn(num_slots, num_kv_heads, head_dim)
        self.value_pool = randn(num_slots, num_kv_heads, head_dim)
        if fill is not None:
            self.key_pool.fill_(fill)
            self.value_pool.fill_(fill)
        self.query = randn(batch, num_heads, head_dim)
        self.new_k = randn(batch, num_kv_heads, head_dim)
        self.new_v = randn(batch, num_kv_heads, head_dim)
        width = max(max(self.contexts), 1, width or 0)
        assert sum(self.contexts) + width <= num_slots
        perm = torch.randperm(num_slots, generator=g)
        table = torch.empty(batch, width, dtype=torch.int64)
        at = 0
        for i, c in enumerate(self.contexts):
            # each sequence's context slots are its own; columns past the
            # context repeat other slots (stale entries, never read)
            table[i, :c] = perm[at:at + c]
            table[i, c:] = perm[(at + torch.arange(width - c)) % num_slots]
            at += c
        self.slot_table = table.to(DEV)
        self.context_lens = torch.tensor(self.contexts, dtype=torch.int32, device=DEV)

    def write_slots(self):
        idx = (self.context_lens.long() - 1).clamp(min=0)[:, None]
        return self.slot_table.gather(1, idx).view(1, -1)

    def pools(self):
        return self.key_pool.clone(), self.value_pool.clone()


def _two_ways(step: _Step, **kw):
    """The fused call and the scatter-then-decode pair, on copies of the same pools."""
    kp1, vp1 = step.pools()
    fused = paged_decode(step.query, kp1, vp1, step.slot_table, step.context_lens, step.scaling, step.groups,
                         new_key=step.new_k, new_value=step.new_v, **kw)
    kp2, vp2 = step.pools()
    live = [i for i, c in enumerate(step.contexts) if c > 0]
    rows = torch.tensor(live, device=DEV)
    scatter_into(kp2, vp2, step.write_slots()[:, rows], step.new_k[rows].unsqueeze(2),
                 step.new_v[rows].unsqueeze(2))
    paired = paged_decode(step.query, kp2, vp2, step.slot_table, step.context_lens, step.scaling, step.groups, **kw)
    torch.cuda.synchronize()
    return (fused, kp1, vp1), (paired, kp2, vp2)


def _bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


@pytest.mark.parametrize(
    ("contexts", "heads", "kv_heads", "dim", "dtype"),
    [
        ([1, 31, 32, 33, 64, 500, 4097, 8191], 32, 8, 128, torch.bfloat16),  # head-grouped, fused
        ([2000, 1, 77, 6000], 16, 8, 64, torch.float16),  # head-grouped at head_dim 64
        ([700, 33, 1, 5000], 12, 3, 128, torch.bfloat16),  # an odd KV head count: per-head kernel, write first
        ([300, 5000, 12], 64, 4, 128, torch.bfloat16),  # 16 heads per KV head
        ([4000, 2, 900, 33], 32, 16, 128, torch.bfloat16),  # eight head pairs: two sets of four per work-group
        ([1, 31, 32, 33, 64, 500], 32, 8, 128, torch.bfloat16),  # a short table: the short kernel writes them
        ([1000, 1, 77], 16, 8, 64, torch.float16),  # short, head_dim 64
        ([700, 33, 1], 12, 3, 128, torch.bfloat16),  # short, odd KV head count
        ([2048] * 15 + [1], 64, 8, 128, torch.bfloat16),  # 128 segments of a 2,048-wide table: short
    ],
    ids=["bf16-8kv", "f16-d64", "three-kv-heads", "g16", "16kv", "short", "short-d64", "short-3kv", "short-wide"],
)
def test_fused_write_equals_scatter_then_decode(contexts, heads, kv_heads, dim, dtype):
    step = _Step(contexts, heads, kv_heads, dim, dtype, seed=len(contexts), num_slots=1 << 16)
    (fused, kp1, vp1), (paired, kp2, vp2) = _two_ways(step)
    assert torch.equal(_bits(kp1), _bits(kp2)) and torch.equal(_bits(vp1), _bits(vp2))
    assert torch.equal(_bits(fused), _bits(paired))


def test_fused_write_over_thousands_of_sequences():
    """2,000 sequences of 1-70 keys (about ten segments per work-group):
    every newest row lands in its slot and the attention matches the
    scatter-then-decode pair bit for bit."""
    rng = np.random.default_rng(13)
    step = _Step(rng.integers(1, 71, size=2000).tolist(), seed=13, num_slots=1 << 17)
    (fused, kp1, vp1), (paired, kp2, vp2) = _two_ways(step)
    assert torch.equal(_bits(kp1), _bits(kp2)) and torch.equal(_bits(vp1), _bits(vp2))
    assert torch.equal(_bits(fused), _bits(paired))


@pytest.mark.parametrize("kernel", ["equal_splits", "generic"])
def test_other_kernels_write_first(kernel):
    step = _Step([100, 1, 4000], seed=3)
    kw = {"kernel": kernel, "num_splits": 4 if kernel == "equal_splits" else None}
    (fused, kp1, vp1), (paired, kp2, vp2) = _two_ways(step, **kw)
    assert torch.equal(_bits(kp1), _bits(kp2)) and torch.equal(_bits(vp1), _bits(vp2))
    assert torch.equal(_bits(fused), _bits(paired))


def test_fused_write_matches_the_oracle():
    from oracle.attention import attend

    step = _Step([1, 17, 900, 4096, 2500, 64], seed=5)
    kp, vp = step.pools()
    out = paged_decode(step.query, kp, vp, step.slot_table, step.context_lens, step.scaling, step.groups,
                       new_key=step.new_k, new_value=step.new_v)
    # the oracle over the pools as the scatter leaves them
    kref, vref = step.pools()
    scatter_into(kref, vref, step.write_slots(), step.new_k.unsqueeze(2), step.new_v.unsqueeze(2))
    want = attend(to_numpy(step.query), to_numpy(kref), to_numpy(vref), step.slot_table.cpu().numpy(),
                  np.asarray(step.contexts), step.scaling, step.groups)
    assert_within(out, want, 2e-2, 2e-3)


@pytest.mark.parametrize("width", [None, 4096])
def test_rows_past_the_newest_key_never_carry_what_the_pool_held(width):
    """A pool full of NaN: the newest key's tile also stages its slot for the
    masked keys past it, which must fold the new (finite) rows too (a short
    table: the short kernel; a wide one: the head-grouped kernel)."""
    step = _Step([1, 5, 32, 40, 1000], seed=7, fill=float("nan"), width=width)
    kp, vp = step.pools()
    # give every context slot but the newest finite rows
    for i, c in enumerate(step.contexts):
        slots = step.slot_table[i, :c - 1]
        kp[slots] = step.query[i, :step.new_k.shape[1]].unsqueeze(0)
        vp[slots] = step.query[i, :step.new_k.shape[1]].unsqueeze(0)
    out = paged_decode(step.query, kp, vp, step.slot_table, step.context_lens, step.scaling, step.groups,
                       new_key=step.new_k, new_value=step.new_v)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()


def test_empty_contexts_write_nothing_and_read_nan():
    step = _Step([0, 50, 0, 3000], seed=9)
    (fused, kp1, vp1), (paired, kp2, vp2) = _two_ways(step)
    assert torch.equal(_bits(kp1), _bits(kp2)) and torch.equal(_bits(vp1), _bits(vp2))
    assert torch.isnan(fused[0].float()).all() and torch.isnan(fused[2].float()).all()
    assert torch.equal(_bits(fused[[1, 3]]), _bits(paired[[1, 3]]))


@pytest.mark.parametrize("contexts", [[300, 1, 2049], [300, 1, 900]], ids=["balanced", "short"])
def test_fp8_pool_writes_quantised_rows_first(contexts):
    from liteinfer_amd.cache.kv_cache import quantize_fp8

    step = _Step(contexts, seed=11)
    ks, vs = 0.5, 0.25
    kp1 = quantize_fp8(step.key_pool, ks)
    vp1 = quantize_fp8(step.value_pool, vs)
    kp2, vp2 = kp1.clone(), vp1.clone()
    fused = paged_decode(step.query, kp1, vp1, step.slot_table, step.context_lens, step.scaling, step.groups,
                         k_scale=ks, v_scale=vs, new_key=step.new_k, new_value=step.new_v)
    paged_kernels.kv_scatter(kp2, vp2, step.write_slots(), step.new_k.unsqueeze(2), step.new_v.unsqueeze(2),
                             k_scale=ks, v_scale=vs)
    paired = paged_decode(step.query, kp2, vp2, step.slot_table, step.context_lens, step.scaling, step.groups,
                          k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    assert torch.equal(kp1.view(torch.uint8), kp2.view(torch.uint8))
    assert torch.equal(vp1.view(torch.uint8), vp2.view(torch.uint8))
    assert torch.equal(_bits(fused), _bits(paired))


def test_the_noalloc_entry_point_agrees_with_the_write_entry_point():
    """paged_decode (li_paged_decode_write, no rows to write) and the
    no-allocation entry point run the same kernels and the same combine: the
    bits agree on a batch with many split contexts."""
    from liteinfer_amd import _native

    step = _Step([8191, 5000, 64, 7000, 1, 2900, 33, 4000] * 4, seed=15, num_slots=1 << 18)
    got = paged_decode(step.query, step.key_pool, step.value_pool, step.slot_table, step.context_lens,
                                 step.scaling, step.groups)
    out = torch.empty_like(step.query)
    paged_kernels.paged_decode_noalloc(step.query, step.key_pool, step.value_pool, step.slot_table,
                                       step.context_lens, step.scaling, step.groups, out=out)
    torch.cuda.synchronize()
    assert _native.is_built()
    assert torch.equal(_bits(got), _bits(out))
