"""Paged-pool addressing and the KV slot-write, restated in numpy. TEST INFRASTRUCTURE ONLY.

Follows liteinfer/cache/block_pool.py:103-223 and liteinfer/cache/kv_cache.py:
236-253. Integer arithmetic only; results are exact.
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np


def position_slot(table: Sequence[int], position: int, block_size: int) -> int:
    """Slot of a logical position: block table entry times block size plus offset (block_pool.py:36-38)."""
    return int(table[position // block_size]) * block_size + position % block_size


def slot_table(block_tables: Sequence[Sequence[int]], totals: Sequence[int], block_size: int) -> np.ndarray:
    """``[B, max(totals)]`` int64, left-aligned; padding past a table's end reads block 0
    (block_pool.py:103-148)."""
    width = max(totals)
    out = np.zeros((len(block_tables), width), dtype=np.int64)
    for i, table in enumerate(block_tables):
        for p in range(width):
            block = p // block_size
            b = int(table[block]) if block < len(table) else 0
            out[i, p] = b * block_size + p % block_size
    return out


def newest_slots(block_tables: Sequence[Sequence[int]], positions: Sequence[int], block_size: int) -> np.ndarray:
    """``[1, B]`` int64 slot of one position per sequence (block_pool.py:151-170)."""
    return np.array([[position_slot(t, p, block_size) for t, p in zip(block_tables, positions, strict=True)]],
                    dtype=np.int64)


def packed_addresses(block_tables, starts, counts, block_size) -> dict[str, np.ndarray]:
    """Write slots, positions, query_start_loc, read table and context lengths of a packed
    pass (block_pool.py:191-223)."""
    totals = [s + c for s, c in zip(starts, counts, strict=True)]
    positions = [s + j for s, c in zip(starts, counts, strict=True) for j in range(c)]
    owners = [i for i, c in enumerate(counts) for _ in range(c)]
    table = slot_table(block_tables, totals, block_size)
    return {
        "slots": np.array([[table[o, p] for o, p in zip(owners, positions, strict=True)]], dtype=np.int64),
        "positions": np.array([positions], dtype=np.int64),
        "query_start_loc": np.concatenate([[0], np.cumsum(counts)]).astype(np.int32),
        "slot_table": table,
        "context_lens": np.array(totals, dtype=np.int32),
    }


def tokens_first(states: np.ndarray) -> np.ndarray:
    """``[B, H, T, D]`` -> ``[B * T, H, D]`` batch-major (kv_cache.py:250-253)."""
    b, h, t, d = states.shape
    return np.ascontiguousarray(states.transpose(0, 2, 1, 3)).reshape(b * t, h, d)


def scatter(key_pool: np.ndarray, value_pool: np.ndarray, slots: np.ndarray, k: np.ndarray, v: np.ndarray):
    """Return copies of the pools with token i's rows stored at slots[i] (kv_cache.py:236-247).

    Works on any dtype, bf16 included when passed as a uint16 view: bytes move,
    nothing is converted. Later tokens win when slots repeat.
    """
    kp, vp = key_pool.copy(), value_pool.copy()
    flat = np.asarray(slots).reshape(-1)
    rows_k, rows_v = tokens_first(k), tokens_first(v)
    for i, s in enumerate(flat):
        kp[s] = rows_k[i]
        vp[s] = rows_v[i]
    return kp, vp
