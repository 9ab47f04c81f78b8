"""The package's pool addressing and payloads agree with the oracle and the reference's known answers (CPU)."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from liteinfer_amd.cache.block_pool import BlockPool, BlockPoolExhaustedError, newest_slots, packed_addresses, slot_table
from liteinfer_amd.cache.kv_cache import KVCache
from oracle import addressing

CPU = torch.device("cpu")
KATS = json.loads((Path(__file__).resolve().parent / "golden" / "addressing_kats.json").read_text())


@pytest.mark.parametrize("case", KATS["slot_table"], ids=lambda c: str(c["block_tables"]))
def test_slot_table_known_answers(case):
    table = slot_table(case["block_tables"], case["totals"], case["block_size"], CPU)
    np.testing.assert_array_equal(table.numpy(), addressing.slot_table(case["block_tables"], case["totals"], case["block_size"]))
    if "expected" in case:
        assert table.tolist() == case["expected"]


@pytest.mark.parametrize("case", KATS["packed"])
def test_packed_addresses_known_answers(case):
    got = packed_addresses(case["block_tables"], case["starts"], case["counts"], case["block_size"], CPU)
    assert got.positions.tolist() == case["positions"]
    assert got.slots.tolist() == case["slots"]
    assert got.query_start_loc.tolist() == case["query_start_loc"]
    assert got.query_start_loc.dtype == torch.int32
    assert got.context_lens.tolist() == case["context_lens"]
    assert got.context_lens.dtype == torch.int32


def test_random_addresses_match_the_oracle():
    rng = np.random.default_rng(7)
    bs = 16
    for _ in range(20):
        n = int(rng.integers(1, 9))
        tables = [rng.permutation(500)[: rng.integers(1, 12)].tolist() for _ in range(n)]
        counts = [int(rng.integers(1, len(t) * bs + 1)) for t in tables]
        starts = [int(rng.integers(0, len(t) * bs - c + 1)) for t, c in zip(tables, counts)]
        got = packed_addresses(tables, starts, counts, bs, CPU)
        want = addressing.packed_addresses(tables, starts, counts, bs)
        for key in ("slots", "positions", "query_start_loc", "slot_table", "context_lens"):
            np.testing.assert_array_equal(getattr(got, key).numpy(), want[key], err_msg=key)
        positions = [s + c - 1 for s, c in zip(starts, counts)]
        np.testing.assert_array_equal(newest_slots(tables, positions, bs, CPU).numpy(),
                                      addressing.newest_slots(tables, positions, bs))


def _cache(num_blocks=16, bs=4, layers=2, heads=2, dim=8):
    return KVCache(BlockPool(num_blocks, bs, layers, heads, dim, torch.float32, CPU))


def test_reserve_is_all_or_nothing():
    cache = _cache(num_blocks=3)
    cache.reserve(["a"], [8])
    with pytest.raises(BlockPoolExhaustedError):
        cache.reserve(["a", "b"], [9, 4])  # needs 1 + 1 blocks, 1 free
    assert cache.pool.num_free_blocks == 1
    assert len(cache.block_table("a")) == 2


def test_reserve_allocates_only_when_the_last_block_fills():
    cache = _cache()
    cache.reserve(["r"], [4])
    assert len(cache.block_table("r")) == 1
    cache.reserve(["r"], [5])
    assert len(cache.block_table("r")) == 2
    cache.release("r")
    assert cache.pool.num_free_blocks == 16


def test_packed_then_decode_payload_reads_back_what_was_written():
    """A prompt chunked over two passes plus a decode token all land where the read table says."""
    cache = _cache()
    g = torch.Generator().manual_seed(0)
    prompt = torch.randn(1, 2, 7, 8, generator=g)
    cache.reserve(["s"], [4])
    cache.make_packed_payload(["s"], [0], [4]).update(prompt[:, :, :4], prompt[:, :, :4] + 1, 0)
    cache.reserve(["s"], [7])
    kv = cache.make_packed_payload(["s"], [4], [3]).update(prompt[:, :, 4:], prompt[:, :, 4:] + 1, 0)
    assert kv.key_pool.data_ptr() == cache.layer_storage(0)[0].data_ptr()
    read = kv.key_pool[kv.slot_table[0, :7]].permute(1, 0, 2).unsqueeze(0)
    torch.testing.assert_close(read, prompt, rtol=0, atol=0)
    cache.reserve(["s"], [8])
    token = torch.randn(1, 2, 1, 8, generator=g)
    payload = cache.make_decode_payload(cache.newest_slots_for(["s"], [7]), cache.slot_table_for(["s"], [8]),
                                        torch.tensor([8], dtype=torch.int32), num_splits=3)
    kv = payload.update(token, token, 1)
    assert kv.num_splits == 3
    torch.testing.assert_close(kv.key_pool[kv.slot_table[0, 7]], token[0, :, 0], rtol=0, atol=0)
