"""A decode step (and a packed pass) captured into a HIP graph replays correctly for changing contexts.

The reference captures its decode steps (liteinfer/engine/cuda_graphs.py:
105-260): the slot table and context lengths are static buffers rewritten
before each replay, columns past a row's context hold stale slots, and the
kernels' grids may depend on host integers only. This captures the fused RoPE
+ slot-write and the paged decode of one layer, then replays it with new
contexts, queries and slot tables, checking every replay against the same
calls run eagerly, with eager work and synchronisations between replays.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from liteinfer_amd.paged_kernels import paged_decode
from liteinfer_amd.rope import rope_kv_write

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


class _Step:
    def __init__(self, batch=16, width=2048, heads=32, kv_heads=8, dim=128, num_slots=1 << 16, seed=0):
        self.g = torch.Generator(device=DEV).manual_seed(seed)
        self.batch, self.width, self.heads, self.kv_heads, self.dim = batch, width, heads, kv_heads, dim
        self.num_slots = num_slots
        bf = torch.bfloat16
        self.key_pool = torch.randn(num_slots, kv_heads, dim, generator=self.g, device=DEV).to(bf)
        self.value_pool = torch.randn(num_slots, kv_heads, dim, generator=self.g, device=DEV).to(bf)
        # static inputs of the captured step
        self.q = torch.empty(batch, 1, heads, dim, dtype=bf, device=DEV)
        self.k = torch.empty(batch, 1, kv_heads, dim, dtype=bf, device=DEV)
        self.v = torch.empty_like(self.k)
        self.cos = torch.empty(batch, 1, dim, dtype=bf, device=DEV)
        self.sin = torch.empty_like(self.cos)
        self.slot_table = torch.empty(batch, width, dtype=torch.int64, device=DEV)
        self.context_lens = torch.empty(batch, dtype=torch.int32, device=DEV)
        self.write_slots = torch.empty(1, batch, dtype=torch.int64, device=DEV)

    def refill(self, seed):
        """New contexts, tables (stale columns past each context), projections and angles."""
        g = torch.Generator(device=DEV).manual_seed(1000 + seed)
        ctx = torch.randint(1, self.width + 1, (self.batch,), generator=g, device=DEV, dtype=torch.int32)
        table = torch.randint(0, self.num_slots, (self.batch, self.width), generator=g, device=DEV)
        self.context_lens.copy_(ctx)
        self.slot_table.copy_(table)
        self.write_slots.copy_(table.gather(1, (ctx.long() - 1)[:, None]).view(1, -1))
        for t in (self.q, self.k, self.v):
            t.copy_(torch.randn(t.shape, generator=g, device=DEV).to(t.dtype))
        ang = torch.rand(self.batch, 1, self.dim // 2, generator=g, device=DEV) * 6.28
        emb = torch.cat((ang, ang), dim=-1)
        self.cos.copy_(emb.cos().to(self.cos.dtype))
        self.sin.copy_(emb.sin().to(self.sin.dtype))

    def run(self):
        q = rope_kv_write(self.q.transpose(1, 2), self.k.transpose(1, 2), self.v.transpose(1, 2), self.cos, self.sin,
                          self.write_slots, self.key_pool, self.value_pool)
        return paged_decode(q.squeeze(2), self.key_pool, self.value_pool, self.slot_table, self.context_lens,
                            self.dim ** -0.5, self.heads // self.kv_heads)


@pytest.mark.parametrize("width", [2048, 4096])
def test_captured_decode_step_matches_eager_on_every_replay(width):
    """16 sequences over a 2,048-wide table run the one-launch short kernel; over a 4,096-wide
    one, the balanced split and its combine."""
    step = _Step(width=width)
    step.refill(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step.run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step.run()
    for r in range(1, 6):
        step.refill(r)
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = step.run()  # the same inputs: the slot-write rewrites identical rows
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), f"replay {r} differs from the eager step"
        # unrelated eager work between replays
        torch.randn(1024, 1024, device=DEV).sum().item()


def test_captured_grid_does_not_depend_on_contexts():
    """Replays cover contexts from 1 key to the full table width with one capture."""
    step = _Step(batch=8, width=4096, seed=1)
    step.refill(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step.run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step.run()
    for lens in ([1] * 8, [4096] * 8, [1, 4096, 33, 2048, 7, 100, 4095, 64]):
        step.refill(len(lens) + sum(lens))
        step.context_lens.copy_(torch.tensor(lens, dtype=torch.int32))
        step.write_slots.copy_(step.slot_table.gather(1, (step.context_lens.long() - 1)[:, None]).view(1, -1))
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = step.run()
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager)
        assert np.isfinite(replayed.float().cpu().numpy()).all()


def test_captured_packed_pass_with_rows_matches_eager_on_every_replay():
    """A packed pass (chunks and one-query rows in one prefill launch) captured
    once: the rows' work-group count and the work list are computed on the
    device on every replay, so new lengths need no new capture."""
    from liteinfer_amd.paged_kernels import paged_prefill

    g = torch.Generator(device=DEV).manual_seed(7)
    batch, tokens, width, heads, kv_heads, dim, num_slots = 6, 600, 4096, 32, 8, 128, 1 << 16
    bf = torch.bfloat16
    key_pool = torch.randn(num_slots, kv_heads, dim, generator=g, device=DEV).to(bf)
    value_pool = torch.randn(num_slots, kv_heads, dim, generator=g, device=DEV).to(bf)
    query = torch.empty(tokens, heads, dim, dtype=bf, device=DEV)
    slot_table = torch.empty(batch, width, dtype=torch.int64, device=DEV)
    context_lens = torch.empty(batch, dtype=torch.int32, device=DEV)
    qsl = torch.empty(batch + 1, dtype=torch.int32, device=DEV)
    max_query_len = 400

    def refill(qlens, seed):
        gg = torch.Generator(device=DEV).manual_seed(seed)
        assert sum(qlens) == tokens and max(qlens) <= max_query_len
        ctx = [q + int(torch.randint(0, width - q + 1, (1,), generator=gg, device=DEV)) for q in qlens]
        context_lens.copy_(torch.tensor(ctx, dtype=torch.int32))
        qsl.copy_(torch.tensor([0, *np.cumsum(qlens).tolist()], dtype=torch.int32))
        slot_table.copy_(torch.randint(0, num_slots, (batch, width), generator=gg, device=DEV))
        query.copy_(torch.randn(query.shape, generator=gg, device=DEV).to(bf))

    def run():
        return paged_prefill(query, key_pool, value_pool, slot_table, context_lens, qsl, max_query_len,
                             dim ** -0.5, heads // kv_heads)

    refill([400, 100, 97, 1, 1, 1], 0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run()
    for i, qlens in enumerate(([400, 100, 97, 1, 1, 1], [300, 296, 1, 1, 1, 1], [1, 1, 1, 1, 196, 400],
                               [200, 200, 197, 1, 1, 1], [100, 100, 100, 100, 100, 100])):
        refill(qlens, 10 + i)
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = run()
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), qlens
        assert np.isfinite(replayed.float().cpu().numpy()).all()


def test_captured_small_pass_cut_into_pieces_matches_eager_on_every_replay():
    """A pass small enough to be cut into pieces (two sequences of at most
    64 queries over up to 8,192 keys), captured once: the pieces are chosen
    on the device on every replay from the lengths it finds, and the merge
    after the launch folds however many there are (none when a one-query
    row keeps the pass whole)."""
    from liteinfer_amd.paged_kernels import paged_prefill

    g = torch.Generator(device=DEV).manual_seed(9)
    batch, width, heads, kv_heads, dim, num_slots = 2, 8192, 32, 8, 128, 1 << 15
    bf = torch.bfloat16
    key_pool = torch.randn(num_slots, kv_heads, dim, generator=g, device=DEV).to(bf)
    value_pool = torch.randn(num_slots, kv_heads, dim, generator=g, device=DEV).to(bf)
    query = torch.empty(128, heads, dim, dtype=bf, device=DEV)
    slot_table = torch.empty(batch, width, dtype=torch.int64, device=DEV)
    context_lens = torch.empty(batch, dtype=torch.int32, device=DEV)
    qsl = torch.empty(batch + 1, dtype=torch.int32, device=DEV)
    max_query_len = 64

    def refill(qlens, ctx, seed):
        gg = torch.Generator(device=DEV).manual_seed(seed)
        context_lens.copy_(torch.tensor(ctx, dtype=torch.int32))
        qsl.copy_(torch.tensor([0, *np.cumsum(qlens).tolist()], dtype=torch.int32))
        slot_table.copy_(torch.randint(0, num_slots, (batch, width), generator=gg, device=DEV))
        query.copy_(torch.randn(query.shape, generator=gg, device=DEV).to(bf))

    def run():
        return paged_prefill(query, key_pool, value_pool, slot_table, context_lens, qsl, max_query_len,
                             dim ** -0.5, heads // kv_heads)

    refill([64, 64], [8192, 3000], 0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run()
    cases = (([64, 64], [8192, 3000]), ([10, 50], [600, 7000]), ([64, 1], [5000, 4000]),
             ([33, 64], [64, 8192]), ([64, 64], [2048, 2048]))
    for i, (qlens, ctx) in enumerate(cases):
        refill(qlens, ctx, 20 + i)
        graph.replay()
        torch.cuda.synchronize()
        replayed = out[:sum(qlens)].clone()
        eager = run()[:sum(qlens)]
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), (qlens, ctx)
        assert np.isfinite(replayed.float().cpu().numpy()).all()


def test_plain_capture_after_an_engine_capture():
    """An engine that captured its decode graphs leaves no state that breaks a later capture.

    The reference captures outside any inference-mode context
    (liteinfer/engine/cuda_graphs.py:232-260). A capture made under
    ``torch.inference_mode`` registers the default generator's graph state as
    inference tensors, and every later capture outside that mode then fails in
    ``capture_begin``; this runs both in one process, in that order.
    """
    from liteinfer_amd.engine.llm import LLM, EngineConfig
    from liteinfer_amd.engine.model import LlamaShape, RandomLlama

    shape = LlamaShape(hidden_size=256, num_layers=1, num_heads=4, num_kv_heads=2, head_dim=64,
                       intermediate_size=512, vocab_size=500)
    model = RandomLlama(shape, dtype=torch.bfloat16, seed=3, std=0.05)
    config = EngineConfig(max_num_seqs=4, max_model_len=128, max_num_batched_tokens=64, num_gpu_blocks=64,
                          use_graphs=True)
    llm = LLM(model, config)
    outputs, stats = llm.generate_ids([[1, 2, 3, 4], [5, 6, 7]], max_tokens=4)
    assert [len(o) for o in outputs] == [4, 4] and stats.decode_steps > 0
    assert llm.runner.graphs.captured_widths, "the engine captured no decode graph"

    step = _Step(batch=4, width=256, seed=5)
    step.refill(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step.run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step.run()
    step.refill(1)
    graph.replay()
    torch.cuda.synchronize()
    replayed = out.clone()
    assert torch.equal(replayed, step.run())


def test_captured_small_pass_without_a_work_list_matches_eager_on_every_replay():
    """A pass whose units all fit the grid at once, the caller saying it holds no one-query rows:
    one launch, each work-group finding its unit from the query counts it reads on the device,
    so one capture replays for any lengths within the shapes it was captured at."""
    from liteinfer_amd.paged_kernels import paged_prefill

    g = torch.Generator(device=DEV).manual_seed(10)
    batch, width, heads, kv_heads, dim, num_slots = 6, 700, 32, 8, 128, 1 << 14
    bf = torch.bfloat16
    key_pool = torch.randn(num_slots, kv_heads, dim, generator=g, device=DEV).to(bf)
    value_pool = torch.randn(num_slots, kv_heads, dim, generator=g, device=DEV).to(bf)
    query = torch.empty(6 * 128, heads, dim, dtype=bf, device=DEV)
    slot_table = torch.empty(batch, width, dtype=torch.int64, device=DEV)
    context_lens = torch.empty(batch, dtype=torch.int32, device=DEV)
    qsl = torch.empty(batch + 1, dtype=torch.int32, device=DEV)
    max_query_len = 128

    def refill(qlens, ctx, seed):
        gg = torch.Generator(device=DEV).manual_seed(seed)
        context_lens.copy_(torch.tensor(ctx, dtype=torch.int32))
        qsl.copy_(torch.tensor([0, *np.cumsum(qlens).tolist()], dtype=torch.int32))
        slot_table.copy_(torch.randint(0, num_slots, (batch, width), generator=gg, device=DEV))
        query.copy_(torch.randn(query.shape, generator=gg, device=DEV).to(bf))

    def run():
        return paged_prefill(query, key_pool, value_pool, slot_table, context_lens, qsl, max_query_len,
                             dim ** -0.5, heads // kv_heads, one_query_rows=False)

    refill([128] * 6, [700] * 6, 0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run()
    cases = (([128] * 6, [700] * 6), ([1, 64, 65, 2, 128, 30], [1, 600, 65, 2, 700, 31]),
             ([0, 5, 0, 128, 0, 1], [0, 5, 0, 300, 0, 9]))
    for i, (qlens, ctx) in enumerate(cases):
        refill(qlens, ctx, 30 + i)
        graph.replay()
        torch.cuda.synchronize()
        replayed = out[:sum(qlens)].clone()
        eager = run()[:sum(qlens)]
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), (qlens, ctx)
        assert np.isfinite(replayed.float().cpu().numpy()).all()
