"""Per-sequence paged KV cache and the payloads a forward pass is handed.

The protocol is liteinfer's (liteinfer/cache/kv_cache.py): a pass first
`reserve`s room for what each sequence will hold, then gets a payload whose
``update(k, v, layer_idx)`` stores this pass's K/V and returns a `PagedKV` —
the layer's pool plus every address attention needs. Every address is built
when the payload is made, so the forward holds no host work and a decode
step can be captured.

On a ROCm device the store is the HIP slot-write kernel (`kv_scatter`); the
CPU path is torch's indexed assignment, which is what the HIP kernel is
checked against bit for bit.
"""

from __future__ import annotations

from typing import Protocol

import torch

from liteinfer_amd.attention import PagedKV
from liteinfer_amd.cache.block_pool import (
    BlockPool,
    BlockPoolExhaustedError,
    PackedAddresses,
    newest_slots,
    packed_addresses,
    slot_table,
)


class KVPayload(Protocol):
    """What one forward pass is handed in place of a KV cache (kv_cache.py:50-59)."""

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int) -> PagedKV: ...


def tokens_first(states: torch.Tensor) -> torch.Tensor:
    """``[B, H, T, D]`` -> ``[B * T, H, D]`` batch-major, the order slots are in (kv_cache.py:250-253)."""
    batch, heads, tokens, dim = states.shape
    return states.transpose(1, 2).reshape(batch * tokens, heads, dim)


def quantize_fp8(x: torch.Tensor, scale: float) -> torch.Tensor:
    """Rows as an fp8 pool stores them: ``e4m3(clamp(float32(x) * float32(1 / scale), +-448))``."""
    inv = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(scale, dtype=torch.float32)
    return (x.to(torch.float32) * inv.to(x.device)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)


def scatter_into(key_pool: torch.Tensor, value_pool: torch.Tensor, slots: torch.Tensor,
                 k: torch.Tensor, v: torch.Tensor, k_scale: float = 1.0, v_scale: float = 1.0,
                 bad_slots: torch.Tensor | None = None) -> None:
    """Store ``[B, H, T, D]`` K/V rows at `slots` (B*T entries, batch-major) of one layer's pools.

    An fp8 pool stores each row quantised with its scale (`quantize_fp8`).
    On the device a slot outside the pool is skipped and counted into
    `bad_slots`; torch's indexed assignment raises for it on the CPU.
    """
    if key_pool.device.type == "cuda":
        from liteinfer_amd.paged_kernels import kv_scatter

        kv_scatter(key_pool, value_pool, slots, k, v, k_scale=k_scale, v_scale=v_scale, bad_slots=bad_slots)
        return
    flat = slots.reshape(-1)
    if key_pool.dtype == torch.float8_e4m3fn:
        key_pool[flat] = quantize_fp8(tokens_first(k), k_scale)
        value_pool[flat] = quantize_fp8(tokens_first(v), v_scale)
        return
    key_pool[flat] = tokens_first(k)
    value_pool[flat] = tokens_first(v)


class KVCache:
    """Block tables per request over one `BlockPool` (kv_cache.py:129-247)."""

    def __init__(self, pool: BlockPool) -> None:
        self._pool = pool
        self._block_tables: dict[str, list[int]] = {}

    @property
    def pool(self) -> BlockPool:
        return self._pool

    def release(self, request_id: str) -> None:
        """Return every block of a finished sequence to the pool."""
        for block in self._block_tables.pop(request_id, []):
            self._pool.free(block)

    def reserve(self, request_ids: list[str], totals: list[int]) -> None:
        """Grow each sequence's block table to cover `totals[i]` tokens, all or nothing.

        The shortfall of every entry is added up first and checked against the
        pool's free blocks, so a step that cannot be served takes no block
        (the reference's contract, kv_cache.py:145-169, with its message).
        """
        entries = list(zip(request_ids, totals, strict=True))
        missing = sum(self._missing_blocks(rid, total) for rid, total in entries)
        free = self._pool.num_free_blocks
        if missing > free:
            raise BlockPoolExhaustedError(
                f"KV block pool exhausted: this step needs {missing} more blocks and "
                f"{free} of {self._pool.num_blocks} are free. "
                "Increase num_gpu_blocks or reduce max_num_seqs / max_model_len."
            )
        for rid, total in entries:
            grow = self._missing_blocks(rid, total)
            if grow:
                self._block_tables.setdefault(rid, []).extend(self._pool.allocate() for _ in range(grow))
            else:
                self._block_tables.setdefault(rid, [])

    def _missing_blocks(self, request_id: str, total: int) -> int:
        """Blocks `request_id` lacks to hold `total` tokens (0 if it has enough)."""
        needed = (total + self._pool.block_size - 1) // self._pool.block_size
        return max(0, needed - len(self._block_tables.get(request_id, ())))

    def block_table(self, request_id: str) -> list[int]:
        return self._block_tables[request_id]

    def make_packed_payload(self, request_ids: list[str], starts: list[int], counts: list[int]) -> _PackedPayload:
        """Payload for each sequence's `counts[i]` tokens from `starts[i]`, laid end to end."""
        addresses = packed_addresses(self._tables(request_ids), starts, counts, self._pool.block_size, self._pool.device)
        totals = tuple(s + c for s, c in zip(starts, counts, strict=True))
        return _PackedPayload(self, addresses, totals, tuple(counts))

    def make_decode_payload(
        self,
        write_slots: torch.Tensor,
        slots: torch.Tensor,
        context_lens: torch.Tensor,
        num_splits: int | None = None,
    ) -> _DecodePayload:
        """Payload for one decode pass writing `write_slots` and reading `slots`."""
        return _DecodePayload(self, write_slots, slots, context_lens, num_splits)

    def newest_slots_for(self, request_ids: list[str], positions: list[int]) -> torch.Tensor:
        """``[1, B]`` slot of each sequence's token at `positions[i]` — where a decode step writes."""
        return newest_slots(self._tables(request_ids), positions, self._pool.block_size, self._pool.device)

    def slot_table_for(self, request_ids: list[str], totals: list[int]) -> torch.Tensor:
        """Each sequence's first `totals[i]` positions as slots, left-aligned."""
        return slot_table(self._tables(request_ids), totals, self._pool.block_size, self._pool.device)

    def _tables(self, request_ids: list[str]) -> list[list[int]]:
        return [self._block_tables[rid] for rid in request_ids]

    def layer_storage(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        return self._pool.slots(layer_idx)

    def scatter(self, layer_idx: int, slots: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
        """Store one K/V column per slot, in the order the pass holds its tokens (kv_cache.py:236-247)."""
        keys, values = self._pool.slots(layer_idx)
        scatter_into(keys, values, slots, k, v, self._pool.k_scale, self._pool.v_scale, self._pool.bad_slots)

    def rotate_and_scatter(self, layer_idx: int, slots: torch.Tensor, q: torch.Tensor, k: torch.Tensor,
                           v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        """RoPE on q and k, then `scatter` of k and v; returns the rotated q.

        One HIP launch on a ROCm device (`rope.rope_kv_write`); the torch ops
        of llama.py:85-98 and `scatter` on the CPU.
        """
        keys, values = self._pool.slots(layer_idx)
        if keys.device.type == "cuda":
            from liteinfer_amd.rope import rope_kv_write

            return rope_kv_write(q, k, v, cos, sin, slots, keys, values,
                                 k_scale=self._pool.k_scale, v_scale=self._pool.v_scale,
                                 bad_slots=self._pool.bad_slots)
        from liteinfer_amd.rope import apply_rotary_pos_emb

        q_embed, k_embed = apply_rotary_pos_emb(q, k, cos, sin)
        scatter_into(keys, values, slots, k_embed, v, self._pool.k_scale, self._pool.v_scale)
        return q_embed


class _PackedPayload:
    """A pass packed end to end: whole prompts, chunks and sampled tokens (kv_cache.py:256-293)."""

    def __init__(self, cache: KVCache, addresses: PackedAddresses,
                 host_context_lens: tuple[int, ...], host_query_lens: tuple[int, ...]) -> None:
        self._cache = cache
        self.addresses = addresses
        self._host_context_lens = host_context_lens
        self._host_query_lens = host_query_lens
        self._max_query_len = max(host_query_lens)

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int) -> PagedKV:
        self._cache.scatter(layer_idx, self.addresses.slots, key_states, value_states)
        return self._paged_kv(layer_idx)

    def update_rotated(self, query_states: torch.Tensor, key_states: torch.Tensor, value_states: torch.Tensor,
                       cos: torch.Tensor, sin: torch.Tensor, layer_idx: int) -> tuple[torch.Tensor, PagedKV]:
        """`update` with the layer's RoPE fused in: returns (rotated q, PagedKV)."""
        q = self._cache.rotate_and_scatter(layer_idx, self.addresses.slots, query_states, key_states, value_states,
                                           cos, sin)
        return q, self._paged_kv(layer_idx)

    def _paged_kv(self, layer_idx: int) -> PagedKV:
        key_pool, value_pool = self._cache.layer_storage(layer_idx)
        return PagedKV(
            key_pool,
            value_pool,
            self.addresses.slot_table,
            self.addresses.context_lens,
            query_start_loc=self.addresses.query_start_loc,
            max_query_len=self._max_query_len,
            host_context_lens=self._host_context_lens,
            host_query_lens=self._host_query_lens,
            k_scale=self._cache.pool.k_scale,
            v_scale=self._cache.pool.v_scale,
        )


class _DecodePayload:
    """A decode pass: store each sequence's new token, then point at the pool (kv_cache.py:296-321)."""

    def __init__(self, cache: KVCache, write_slots: torch.Tensor, slots: torch.Tensor,
                 context_lens: torch.Tensor, num_splits: int | None) -> None:
        self._cache = cache
        self._write_slots = write_slots
        self._slots = slots
        self._context_lens = context_lens
        self._num_splits = num_splits

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int) -> PagedKV:
        self._cache.scatter(layer_idx, self._write_slots, key_states, value_states)
        return self._paged_kv(layer_idx)

    def update_rotated(self, query_states: torch.Tensor, key_states: torch.Tensor, value_states: torch.Tensor,
                       cos: torch.Tensor, sin: torch.Tensor, layer_idx: int) -> tuple[torch.Tensor, PagedKV]:
        """`update` with the layer's RoPE fused in: returns (rotated q, PagedKV)."""
        q = self._cache.rotate_and_scatter(layer_idx, self._write_slots, query_states, key_states, value_states,
                                           cos, sin)
        return q, self._paged_kv(layer_idx)

    def _paged_kv(self, layer_idx: int) -> PagedKV:
        key_pool, value_pool = self._cache.layer_storage(layer_idx)
        pool = self._cache.pool
        return PagedKV(key_pool, value_pool, self._slots, self._context_lens, self._num_splits,
                       k_scale=pool.k_scale, v_scale=pool.v_scale)
