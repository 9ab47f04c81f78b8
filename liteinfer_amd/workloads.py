"""Seeded synthetic inputs for the paged path at the benchmark geometries.

Each builder returns the pool, addresses and new K/V rows a layer of
liteinfer holds at that step, built through this package's own addressing
(`cache.block_pool`) exactly as the engine builds them: every sequence owns
blocks taken from a seeded permutation of the pool, its slot table is
`slot_table(...)`, and a decode step's new token is written at
`newest_slots(...)`. Values are N(0, 1).

Geometries:
  c1  Llama-3.2-1B attention: 32/8 heads, head_dim 64, block 16, batch 4,
      contexts {37, 128, 500, 1023}, pool 512 blocks.
  c2  Llama-3-8B: 32/8 heads, head_dim 128, block 16, batch 64, contexts
      uniform in [512, 8192], pool 65,536 blocks.
  c3  Llama-3-8B mixed packed step: 8 prompt chunks of U[64, 2048] queries
      over U[0, 4096] cached keys, plus 56 decode rows over U[256, 4096].
  c4  Llama-3-8B long context: batch 8, contexts U[32768, 131072], pool
      65,536 blocks.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from liteinfer_amd.cache.block_pool import newest_slots, packed_addresses, slot_table

BLOCK_SIZE = 16


@dataclass
class Geometry:
    num_heads: int
    num_kv_heads: int
    head_dim: int

    @property
    def groups(self) -> int:
        return self.num_heads // self.num_kv_heads

    @property
    def scaling(self) -> float:
        return self.head_dim ** -0.5


LLAMA_3_2_1B = Geometry(32, 8, 64)
LLAMA_3_8B = Geometry(32, 8, 128)


@dataclass
class DecodeStep:
    """A decode step: write one new K/V per sequence, then attend one query per sequence."""

    name: str
    geometry: Geometry
    query: torch.Tensor          # [B, Hq, D]
    key_pool: torch.Tensor       # [S, Hkv, D]
    value_pool: torch.Tensor
    slot_table: torch.Tensor     # [B, max ctx] int64
    context_lens: torch.Tensor   # [B] int32, the new token included
    new_k: torch.Tensor          # [B, Hkv, 1, D]
    new_v: torch.Tensor
    write_slots: torch.Tensor    # [1, B] int64
    host_context_lens: list[int]

    @property
    def batch(self) -> int:
        return len(self.host_context_lens)


@dataclass
class PackedStep:
    """A packed pass: write every new token's K/V, then attend all queries causally."""

    name: str
    geometry: Geometry
    query: torch.Tensor          # [T, Hq, D]
    key_pool: torch.Tensor
    value_pool: torch.Tensor
    slot_table: torch.Tensor
    context_lens: torch.Tensor
    query_start_loc: torch.Tensor
    new_k: torch.Tensor          # [1, Hkv, T, D]
    new_v: torch.Tensor
    write_slots: torch.Tensor    # [1, T]
    host_context_lens: list[int]
    host_query_lens: list[int]

    @property
    def max_query_len(self) -> int:
        return max(self.host_query_lens)


def _randn(shape, dtype, device, generator) -> torch.Tensor:
    return torch.randn(shape, generator=generator, dtype=torch.float32, device=device).to(dtype)


def _assign_blocks(totals: list[int], num_blocks: int, rng: np.random.Generator) -> list[list[int]]:
    order = rng.permutation(num_blocks)
    tables, at = [], 0
    for total in totals:
        n = -(-total // BLOCK_SIZE)
        if at + n > num_blocks:
            raise ValueError(f"pool of {num_blocks} blocks cannot hold contexts of {sum(totals)} tokens")
        tables.append(order[at:at + n].tolist())
        at += n
    return tables


def _pool(geo: Geometry, num_blocks: int, dtype, device, gen):
    shape = (num_blocks * BLOCK_SIZE, geo.num_kv_heads, geo.head_dim)
    return _randn(shape, dtype, device, gen), _randn(shape, dtype, device, gen)


def decode_step(config: str, dtype=torch.bfloat16, device="cuda", seed: int = 0,
                context_lens: list[int] | None = None, num_blocks: int | None = None,
                geometry: Geometry = LLAMA_3_8B) -> DecodeStep:
    """Inputs of the c1, c2 or c4 decode step (or custom contexts, at `geometry`)."""
    rng = np.random.default_rng(seed)
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(seed)
    if config == "c1":
        geo, ctxs, blocks = LLAMA_3_2_1B, [37, 128, 500, 1023], 512
    elif config == "c2":
        geo, ctxs, blocks = LLAMA_3_8B, rng.integers(512, 8192 + 1, size=64).tolist(), 65536
    elif config == "c4":
        geo, ctxs, blocks = LLAMA_3_8B, rng.integers(32768, 131072 + 1, size=8).tolist(), 65536
    elif config == "custom":
        geo, ctxs = geometry, list(context_lens or [])
        blocks = num_blocks or -(-sum(ctxs) // BLOCK_SIZE) + len(ctxs)
    else:
        raise ValueError(f"unknown decode config {config!r}")
    ctxs = [int(c) for c in ctxs]
    tables = _assign_blocks(ctxs, blocks, rng)
    key_pool, value_pool = _pool(geo, blocks, dtype, device, gen)
    b = len(ctxs)
    return DecodeStep(
        name=config,
        geometry=geo,
        query=_randn((b, geo.num_heads, geo.head_dim), dtype, device, gen),
        key_pool=key_pool,
        value_pool=value_pool,
        slot_table=slot_table(tables, ctxs, BLOCK_SIZE, device),
        context_lens=torch.tensor(ctxs, dtype=torch.int32, device=device),
        new_k=_randn((b, geo.num_kv_heads, 1, geo.head_dim), dtype, device, gen),
        new_v=_randn((b, geo.num_kv_heads, 1, geo.head_dim), dtype, device, gen),
        write_slots=newest_slots(tables, [c - 1 for c in ctxs], BLOCK_SIZE, device),
        host_context_lens=ctxs,
    )


def c3_shapes(seed: int = 0) -> tuple[list[tuple[int, int]], list[int]]:
    """Config 3's (queries, cached prefix) chunks and its decode-row contexts, as packed_step draws them."""
    return _c3_shapes(np.random.default_rng(seed))


def _c3_shapes(rng: np.random.Generator) -> tuple[list[tuple[int, int]], list[int]]:
    chunks = list(zip(rng.integers(64, 2048 + 1, size=8).tolist(), rng.integers(0, 4096 + 1, size=8).tolist()))
    decode_contexts = rng.integers(256, 4096 + 1, size=56).tolist()
    return [(int(q), int(p)) for q, p in chunks], [int(c) for c in decode_contexts]


def packed_step(config: str = "c3", dtype=torch.bfloat16, device="cuda", seed: int = 0,
                chunks: list[tuple[int, int]] | None = None, decode_contexts: list[int] | None = None,
                geometry: Geometry = LLAMA_3_8B, num_blocks: int = 65536) -> PackedStep:
    """Inputs of the c3 mixed step: chunk (queries, prefix) pairs first, then one-query decode rows."""
    rng = np.random.default_rng(seed)
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(seed)
    geo = geometry
    if config == "c3":
        chunks, decode_contexts = _c3_shapes(rng)
    elif config != "custom":
        raise ValueError(f"unknown packed config {config!r}")
    chunks = [(int(q), int(p)) for q, p in (chunks or [])]
    decode_contexts = [int(c) for c in (decode_contexts or [])]
    starts = [p for _, p in chunks] + [c - 1 for c in decode_contexts]
    counts = [q for q, _ in chunks] + [1] * len(decode_contexts)
    totals = [s + c for s, c in zip(starts, counts)]
    tables = _assign_blocks(totals, num_blocks, rng)
    key_pool, value_pool = _pool(geo, num_blocks, dtype, device, gen)
    addr = packed_addresses(tables, starts, counts, BLOCK_SIZE, device)
    t = sum(counts)
    return PackedStep(
        name=config,
        geometry=geo,
        query=_randn((t, geo.num_heads, geo.head_dim), dtype, device, gen),
        key_pool=key_pool,
        value_pool=value_pool,
        slot_table=addr.slot_table,
        context_lens=addr.context_lens,
        query_start_loc=addr.query_start_loc,
        new_k=_randn((1, geo.num_kv_heads, t, geo.head_dim), dtype, device, gen),
        new_v=_randn((1, geo.num_kv_heads, t, geo.head_dim), dtype, device, gen),
        write_slots=addr.slots,
        host_context_lens=totals,
        host_query_lens=counts,
    )
