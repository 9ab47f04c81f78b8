"""Attention over a paged KV pool, restated in numpy. TEST INFRASTRUCTURE ONLY.

The answer liteinfer's `eager` kernel computes (liteinfer/models/attention.py:
97-164), evaluated in a chosen float dtype (float64 for the reference answer):

* query head h reads KV head h // groups (_repeat_kv, attention.py:69-78);
* sequence i attends to the pool rows at slot_table[i, :context_lens[i]]
  (_gathered / _decode_batch, attention.py:86-112);
* its nq queries are the last positions of its context, so query j sees keys
  0 .. ctx - nq + j (_future_keys, attention.py:81-84); a decode query (nq = 1)
  sees the whole context;
* out = softmax(q k^T * scale over the visible keys) v.

Inputs are numpy arrays; bf16 tensors are passed already widened to float32
(bf16 -> float32 is exact).
"""

from __future__ import annotations

import numpy as np


def attend(
    query: np.ndarray,
    key_pool: np.ndarray,
    value_pool: np.ndarray,
    slot_table: np.ndarray,
    context_lens: np.ndarray,
    scale: float,
    groups: int,
    query_start_loc: np.ndarray | None = None,
    dtype=np.float64,
    query_block: int = 256,
) -> np.ndarray:
    """Attention output, ``[rows, num_heads, head_dim]`` in `dtype`.

    `query` is ``[rows, num_heads, head_dim]``: one row per sequence for a
    decode step (`query_start_loc` None), or the packed rows of every
    sequence, sequence i owning ``[query_start_loc[i], query_start_loc[i+1])``.
    Queries are processed `query_block` at a time to bound memory.
    """
    rows, num_heads, head_dim = query.shape
    num_kv_heads = key_pool.shape[1]
    if num_heads != num_kv_heads * groups:
        raise ValueError(f"{num_heads} heads != {num_kv_heads} KV heads x {groups}")
    batch = len(context_lens)
    out = np.zeros((rows, num_heads, head_dim), dtype=dtype)
    for i in range(batch):
        if query_start_loc is None:
            first, nq = i, 1
        else:
            first, nq = int(query_start_loc[i]), int(query_start_loc[i + 1] - query_start_loc[i])
        if nq == 0:
            continue
        ctx = int(context_lens[i])
        if ctx <= 0:
            # Nothing to attend to: the reference's softmax over all-masked
            # scores is 0 / 0 (liteinfer/models/attention.py:158-164).
            out[first:first + nq] = np.nan
            continue
        slots = np.asarray(slot_table[i, :ctx], dtype=np.int64)
        keys = key_pool[slots].astype(dtype)      # [ctx, Hkv, D]
        values = value_pool[slots].astype(dtype)
        k_h = keys.transpose(1, 2, 0)             # [Hkv, D, ctx]
        v_h = values.transpose(1, 0, 2)           # [Hkv, ctx, D]
        for b0 in range(0, nq, query_block):
            b1 = min(b0 + query_block, nq)
            q = query[first + b0:first + b1].astype(dtype)            # [n, Hq, D]
            n = b1 - b0
            # [Hkv, G * n, D]: rows of one KV head's query heads, head-major.
            qg = q.reshape(n, num_kv_heads, groups, head_dim).transpose(1, 2, 0, 3).reshape(
                num_kv_heads, groups * n, head_dim)
            scores = np.matmul(qg, k_h) * dtype(scale)                # [Hkv, G*n, ctx]
            positions = ctx - nq + np.arange(b0, b1)                  # [n]
            visible = np.arange(ctx)[None, :] <= positions[:, None]   # [n, ctx]
            visible = np.tile(visible, (groups, 1))                   # [G*n, ctx]
            scores = np.where(visible[None], scores, -np.inf)
            top = scores.max(axis=-1, keepdims=True)
            weights = np.exp(scores - top)
            weights /= weights.sum(axis=-1, keepdims=True)
            o = np.matmul(weights, v_h)                               # [Hkv, G*n, D]
            o = o.reshape(num_kv_heads, groups, n, head_dim).transpose(2, 0, 1, 3).reshape(n, num_heads, head_dim)
            out[first + b0:first + b1] = o
    return out


def attention_bytes(context_lens, num_kv_heads: int, head_dim: int, elem_size: int,
                    num_heads: int, query_rows: int) -> int:
    """Algorithmic HBM bytes of one decode-style pass: every context token's K and V row
    for every KV head, its int64 slot, and each query row read once and written once."""
    tokens = int(np.sum(np.asarray(context_lens, dtype=np.int64)))
    return tokens * (2 * num_kv_heads * head_dim * elem_size + 8) + 2 * query_rows * num_heads * head_dim * elem_size


def causal_pairs(query_lens, context_lens) -> int:
    """Visible (query, key) pairs of a packed pass: query j of nq over ctx keys sees ctx - nq + j + 1."""
    total = 0
    for nq, ctx in zip(query_lens, context_lens, strict=True):
        nq, ctx = int(nq), int(ctx)
        prefix = ctx - nq
        total += nq * prefix + nq * (nq + 1) // 2
    return total
