"""Writes the golden fixtures under tests/golden/. Re-run to regenerate them.

addressing_kats.json
    The known-answer vectors liteinfer's own tests hold for the pool
    addressing (tests/unit/test_slot_table.py in the reference): inputs and
    expected outputs, as data.

attention_bruteforce.npz
    Small paged-attention cases (decode, chunk over a prefix, whole prompt,
    mixed rows, GQA groups of 1/4/5) with outputs computed by a pure-Python
    scalar brute force in float64 — explicit loops, math.exp, no numpy
    matmul — so they pin the numpy oracle through an independent code path.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent

# Reference: tests/unit/test_slot_table.py. BLOCK_SIZE = 4 there (:11) unless
# a case says otherwise.
ADDRESSING_KATS = {
    "slot_table": [
        # (:30-32) block 2, three tokens -> 8, 9, 10
        {"block_tables": [[2]], "totals": [3], "block_size": 4, "expected": [[8, 9, 10]]},
        # (:35-37) blocks 0 then 3, five tokens -> 0..3 then 12
        {"block_tables": [[0, 3]], "totals": [5], "block_size": 4, "expected": [[0, 1, 2, 3, 12]]},
        # (:40-43) left-aligned: row 1 of [[0],[1]] totals [1,3] is [4,5,6]
        {"block_tables": [[0], [1]], "totals": [1, 3], "block_size": 4, "expected_row": [1, [4, 5, 6]],
         "expected_shape": [2, 3]},
        # (:50-53) unequal tables: row 1 of [[0,1],[2]] totals [5,2] starts [8,9]
        {"block_tables": [[0, 1], [2]], "totals": [5, 2], "block_size": 4, "expected_row_prefix": [1, [8, 9]]},
        # (:56-60) width from the counts: block size 16, totals [3,9] -> 9 columns
        {"block_tables": [[1], [1]], "totals": [3, 9], "block_size": 16, "expected_shape": [2, 9]},
    ],
    "packed": [
        # (:108-146) three sequences, two blocks each, block size 4
        {
            "block_tables": [[2, 5], [1, 7], [3, 6]],
            "starts": [5, 0, 3],
            "counts": [3, 2, 1],
            "block_size": 4,
            "positions": [[5, 6, 7, 0, 1, 3]],
            "slots": [[21, 22, 23, 4, 5, 15]],
            "query_start_loc": [0, 3, 5, 6],
            "context_lens": [8, 2, 4],
        },
    ],
    "newest": [
        # (:88-95) the decode write slot is the read table's last column
        {"block_tables": [[2, 7], [5, 1, 3]], "totals": [6, 9], "block_size": 4},
    ],
}


def brute_force(query, key_pool, value_pool, slot_table, context_lens, scale, groups, query_start_loc):
    """Scalar float64 attention, one (query, head) at a time."""
    rows, heads, dim = query.shape
    out = np.zeros((rows, heads, dim), dtype=np.float64)
    for i, ctx in enumerate(context_lens):
        first, last = (i, i + 1) if query_start_loc is None else (int(query_start_loc[i]), int(query_start_loc[i + 1]))
        nq = last - first
        for j in range(nq):
            pos = int(ctx) - nq + j
            for h in range(heads):
                kvh = h // groups
                scores = []
                for key in range(pos + 1):
                    slot = int(slot_table[i, key])
                    dot = 0.0
                    for d in range(dim):
                        dot += float(query[first + j, h, d]) * float(key_pool[slot, kvh, d])
                    scores.append(dot * scale)
                top = max(scores)
                weights = [math.exp(s - top) for s in scores]
                total = sum(weights)
                for d in range(dim):
                    acc = 0.0
                    for key, w in enumerate(weights):
                        acc += w * float(value_pool[int(slot_table[i, key]), kvh, d])
                    out[first + j, h, d] = acc / total
    return out


CASES = [
    # name, query_lens (None = decode), context_lens, heads, kv_heads, head_dim
    ("decode_gqa4", None, [6, 4, 1], 8, 2, 16),
    ("decode_no_gqa", None, [9, 3], 4, 4, 8),
    ("decode_group5", None, [11, 2], 10, 2, 8),
    ("chunk_over_prefix", [5], [23], 8, 2, 16),
    ("whole_prompt", [7], [7], 4, 2, 8),
    ("mixed_rows", [1, 6, 1, 3], [12, 9, 3, 3], 8, 2, 8),
]


def attention_fixtures(seed: int = 1234) -> dict[str, np.ndarray]:
    rng = np.random.default_rng(seed)
    arrays: dict[str, np.ndarray] = {}
    num_slots = 64
    for name, qlens, ctxs, heads, kv_heads, dim in CASES:
        groups = heads // kv_heads
        rows = len(ctxs) if qlens is None else sum(qlens)
        q = rng.standard_normal((rows, heads, dim)).astype(np.float32)
        kp = rng.standard_normal((num_slots, kv_heads, dim)).astype(np.float32)
        vp = rng.standard_normal((num_slots, kv_heads, dim)).astype(np.float32)
        width = max(ctxs)
        table = np.zeros((len(ctxs), width), dtype=np.int64)
        for i, c in enumerate(ctxs):
            table[i, :c] = rng.integers(1, num_slots, size=c)
            table[i, c:] = rng.integers(1, num_slots, size=width - c)  # padding columns: never read
        qsl = None if qlens is None else np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
        scale = dim ** -0.5
        out = brute_force(q, kp, vp, table, ctxs, scale, groups, qsl)
        prefix = f"{name}__"
        arrays[prefix + "query"] = q
        arrays[prefix + "key_pool"] = kp
        arrays[prefix + "value_pool"] = vp
        arrays[prefix + "slot_table"] = table
        arrays[prefix + "context_lens"] = np.asarray(ctxs, dtype=np.int32)
        arrays[prefix + "query_start_loc"] = qsl if qsl is not None else np.zeros(0, dtype=np.int32)
        arrays[prefix + "groups"] = np.asarray(groups)
        arrays[prefix + "scale"] = np.asarray(scale)
        arrays[prefix + "expected"] = out
    return arrays


def main() -> None:
    (HERE / "addressing_kats.json").write_text(json.dumps(ADDRESSING_KATS, indent=1) + "\n")
    np.savez_compressed(HERE / "attention_bruteforce.npz", **attention_fixtures())
    print("wrote", HERE / "addressing_kats.json", HERE / "attention_bruteforce.npz")


if __name__ == "__main__":
    main()
