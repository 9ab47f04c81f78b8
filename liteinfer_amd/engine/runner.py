"""Model runner and captured decode graphs (liteinfer/engine/model_runner.py,
liteinfer/engine/cuda_graphs.py), over this build's paged path.

`execute` runs one scheduled step. A step where every sequence computes one
token is a decode batch, one sequence per row; it replays a graph captured for
the smallest width that holds it (powers of two up to ``max_num_seqs``),
padding the extra rows with a one-token context in a reserved slot. Anything
else is one packed pass: prompts, chunks and sampled tokens side by side.
Every address is built before the forward, so the forward holds no host work.
"""

from __future__ import annotations

import contextlib
import gc
from dataclasses import dataclass

import torch

from liteinfer_amd.cache.block_pool import to_device
from liteinfer_amd.cache.kv_cache import KVCache
from liteinfer_amd.engine.model import RandomLlama
from liteinfer_amd.engine.scheduler import PENDING_TOKEN, Sequence

_PAD = "__pad__"


@dataclass
class PendingTokens:
    """Token ids a step sampled, still on the device: `tokens[index[request_id]]` is that sequence's."""

    tokens: torch.Tensor
    index: dict[str, int]


@dataclass
class _Chunk:
    token_ids: list[int]
    start: int

    @property
    def end(self) -> int:
        return self.start + len(self.token_ids)


@contextlib.contextmanager
def graph_capture(graph: torch.cuda.CUDAGraph, pool=None):
    """`torch.cuda.graph(graph, pool)` with Python's cyclic garbage collector off
    for the capture: a collection inside it would run the destructors of
    whatever unreachable cycles hold (device tensors, graphs) while the stream
    captures, and such a collection inside a captured decode forward has
    aborted the process. (torch collects once just before the capture
    begins; the collector is on again after it.)"""
    was_enabled = gc.isenabled()
    gc.disable()
    try:
        with torch.cuda.graph(graph, pool=pool):
            yield
    finally:
        if was_enabled:
            gc.enable()


class DecodeGraphs:
    """Decode forwards captured per batch width; static inputs rewritten before each replay."""

    def __init__(self, model: RandomLlama, cache: KVCache, max_num_seqs: int, max_model_len: int,
                 pad_slot: int) -> None:
        self.model = model
        self.cache = cache
        self.pad_slot = pad_slot
        widths, w = [], 1
        while w < max_num_seqs:
            widths.append(w)
            w *= 2
        widths.append(max_num_seqs)
        self.widths = widths
        dev = model.device
        n = max_num_seqs
        self.input_ids = torch.zeros(n, 1, dtype=torch.long, device=dev)
        self.positions = torch.zeros(n, 1, dtype=torch.long, device=dev)
        self.write_slots = torch.full((1, n), pad_slot, dtype=torch.long, device=dev)
        self.slot_table = torch.full((n, max_model_len), pad_slot, dtype=torch.long, device=dev)
        self.context_lens = torch.ones(n, dtype=torch.int32, device=dev)
        self._graphs: dict[int, tuple[torch.cuda.CUDAGraph, torch.Tensor]] = {}
        self._pool = None
        self.captured_widths: list[int] = []

    @torch.no_grad()
    def capture_all(self) -> None:
        """Capture every width now (so no capture lands inside a timed run)."""
        for w in self.widths:
            if w not in self._graphs:
                self._capture(w)

    def has_capacity_for(self, n: int) -> bool:
        return n <= self.widths[-1]

    def _width_for(self, n: int) -> int:
        return next(w for w in self.widths if w >= n)

    def _forward(self, width: int) -> torch.Tensor:
        payload = self.cache.make_decode_payload(self.write_slots[:, :width], self.slot_table[:width],
                                                 self.context_lens[:width], None)
        return self.model.forward(self.input_ids[:width], self.positions[:width], payload)

    def _capture(self, width: int) -> None:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self._forward(width)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        if self._pool is None:
            self._pool = torch.cuda.graph_pool_handle()
        with graph_capture(graph, pool=self._pool):
            out = self._forward(width)
        self._graphs[width] = (graph, out)
        self.captured_widths.append(width)

    def run(self, input_ids, positions, write_slots, slots, context_lens) -> torch.Tensor:
        n, cols = slots.shape
        width = self._width_for(n)
        self.input_ids[:n].copy_(input_ids)
        self.positions[:n].copy_(positions)
        self.write_slots[:, :n].copy_(write_slots)
        self.slot_table[:n, :cols].copy_(slots)
        self.context_lens[:n].copy_(context_lens)
        if n < width:  # padding rows: one key in the reserved slot
            self.input_ids[n:width].zero_()
            self.positions[n:width].zero_()
            self.write_slots[:, n:width].fill_(self.pad_slot)
            self.slot_table[n:width, 0].fill_(self.pad_slot)
            self.context_lens[n:width].fill_(1)
        if width not in self._graphs:
            self._capture(width)
        graph, out = self._graphs[width]
        graph.replay()
        return out[:n]


class ModelRunner:
    def __init__(self, model: RandomLlama, cache: KVCache, max_num_seqs: int, max_model_len: int,
                 use_graphs: bool = True) -> None:
        self.model = model
        self.cache = cache
        self.device = model.device
        cache.reserve([_PAD], [1])
        pad_slot = cache.block_table(_PAD)[0] * cache.pool.block_size
        self.graphs = DecodeGraphs(model, cache, max_num_seqs, max_model_len, pad_slot) if use_graphs else None

    def release(self, seq: Sequence) -> None:
        self.cache.release(seq.request_id)

    @torch.no_grad()
    def execute(self, seqs: list[Sequence], num_tokens: list[int], pending: PendingTokens | None = None
                ) -> torch.Tensor:
        """One step over the next `num_tokens` of each sequence; logits at each one's last token.

        A token id still on the device (`PENDING_TOKEN` in the sequence,
        sampled by the step before and not read back yet) is taken from
        `pending` on the device, so the step is staged and launched without
        waiting for the one before it.
        """
        ids = [s.request_id for s in seqs]
        chunks = []
        for seq, count in zip(seqs, num_tokens, strict=True):
            start = seq.num_computed_tokens
            if count < 1 or start + count > len(seq):
                raise ValueError(f"{seq.request_id}: cannot compute {count} tokens from position {start}")
            chunks.append(_Chunk([seq.token_at(p) for p in range(start, start + count)], start))
        self.cache.reserve(ids, [c.end for c in chunks])
        # Where a token is pending: its index in pending.tokens (-1: the id is on the host).
        sources = [[pending.index[i] if t == PENDING_TOKEN else -1 for t in c.token_ids]
                   for i, c in zip(ids, chunks)] if pending is not None else None
        if all(len(c.token_ids) == 1 for c in chunks):
            logits = self._decode(ids, chunks, sources, pending)
        else:
            logits = self._packed(ids, chunks, sources, pending)
        for seq, c in zip(seqs, chunks):
            seq.num_computed_tokens = c.end
        return logits

    def _token_ids(self, host_ids: torch.Tensor, sources: torch.Tensor | None,
                   pending: PendingTokens | None) -> torch.Tensor:
        """The step's token ids on the device, the pending ones gathered from `pending.tokens`."""
        if sources is None:
            return host_ids
        return torch.where(sources >= 0, pending.tokens[sources.clamp(min=0)], host_ids)

    def _packed(self, ids: list[str], chunks: list[_Chunk], sources, pending) -> torch.Tensor:
        counts = [len(c.token_ids) for c in chunks]
        payload = self.cache.make_packed_payload(ids, [c.start for c in chunks], counts)
        rows = [[t for c in chunks for t in c.token_ids]]
        if sources is not None:
            rows.append([k for per in sources for k in per])
        staged = to_device(rows, torch.long, self.device)
        tokens = self._token_ids(staged[0:1], staged[1:2] if sources is not None else None, pending)
        qsl = payload.addresses.query_start_loc
        return self.model.forward(tokens, payload.addresses.positions, payload, logits_positions=qsl[1:].long() - 1)

    def _decode(self, ids: list[str], chunks: list[_Chunk], sources, pending) -> torch.Tensor:
        totals = [c.end for c in chunks]
        rows = [[c.token_ids[0] for c in chunks], [c.start for c in chunks], totals]
        if sources is not None:
            rows.append([per[0] for per in sources])
        staged = to_device(rows, torch.long, self.device)
        input_ids = self._token_ids(staged[0], staged[3] if sources is not None else None, pending).unsqueeze(1)
        positions = staged[1].unsqueeze(1)
        write_slots = self.cache.newest_slots_for(ids, [c.start for c in chunks])
        slots = self.cache.slot_table_for(ids, totals)
        context_lens = staged[2].to(torch.int32)
        if self.graphs is not None and self.graphs.has_capacity_for(len(ids)):
            return self.graphs.run(input_ids, positions, write_slots, slots, context_lens)
        payload = self.cache.make_decode_payload(write_slots, slots, context_lens, None)
        return self.model.forward(input_ids, positions, payload)
