"""The oracle is pinned before anything is checked against it.

Each function of oracle/ is tied to something it could not have agreed with
by accident: the reference's own known-answer vectors, a scalar brute force
written separately, torch's fused attention, or a closed form that a
dropped term, a wrong sign, a transposed operand or a wrong head mapping
would break.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import addressing
from oracle.attention import attend, attention_bytes, causal_pairs

GOLDEN = Path(__file__).resolve().parent / "golden"
KATS = json.loads((GOLDEN / "addressing_kats.json").read_text())


# --- addressing: the reference's known answers ------------------------------------


@pytest.mark.parametrize("case", KATS["slot_table"], ids=lambda c: str(c["block_tables"]))
def test_oracle_slot_table_matches_the_reference_known_answers(case):
    table = addressing.slot_table(case["block_tables"], case["totals"], case["block_size"])
    if "expected" in case:
        assert table.tolist() == case["expected"]
    if "expected_shape" in case:
        assert list(table.shape) == case["expected_shape"]
    if "expected_row" in case:
        row, values = case["expected_row"]
        assert table[row].tolist() == values
    if "expected_row_prefix" in case:
        row, values = case["expected_row_prefix"]
        assert table[row, : len(values)].tolist() == values


@pytest.mark.parametrize("case", KATS["packed"])
def test_oracle_packed_addresses_match_the_reference_known_answers(case):
    got = addressing.packed_addresses(case["block_tables"], case["starts"], case["counts"], case["block_size"])
    assert got["positions"].tolist() == case["positions"]
    assert got["slots"].tolist() == case["slots"]
    assert got["query_start_loc"].tolist() == case["query_start_loc"]
    assert got["query_start_loc"].dtype == np.int32
    assert got["context_lens"].tolist() == case["context_lens"]
    totals = [s + c for s, c in zip(case["starts"], case["counts"])]
    np.testing.assert_array_equal(got["slot_table"], addressing.slot_table(case["block_tables"], totals, case["block_size"]))


@pytest.mark.parametrize("case", KATS["newest"])
def test_oracle_newest_slot_is_the_read_table_s_last_column(case):
    table = addressing.slot_table(case["block_tables"], case["totals"], case["block_size"])
    expected = [[table[i, t - 1] for i, t in enumerate(case["totals"])]]
    got = addressing.newest_slots(case["block_tables"], [t - 1 for t in case["totals"]], case["block_size"])
    assert got.tolist() == expected


def test_oracle_slot_table_is_the_closed_form_on_random_tables():
    rng = np.random.default_rng(0)
    bs = 16
    tables = [rng.permutation(100)[: rng.integers(1, 9)].tolist() for _ in range(6)]
    totals = [rng.integers(1, len(t) * bs + 1) for t in tables]
    got = addressing.slot_table(tables, totals, bs)
    for i, t in enumerate(tables):
        for p in range(totals[i]):
            assert got[i, p] == t[p // bs] * bs + p % bs


def test_oracle_scatter_is_torch_index_put_and_leaves_other_slots_alone():
    rng = np.random.default_rng(1)
    pool_k = rng.standard_normal((40, 3, 8)).astype(np.float32)
    pool_v = rng.standard_normal((40, 3, 8)).astype(np.float32)
    k = rng.standard_normal((2, 3, 5, 8)).astype(np.float32)
    v = rng.standard_normal((2, 3, 5, 8)).astype(np.float32)
    slots = rng.permutation(40)[:10].reshape(1, 10)
    got_k, got_v = addressing.scatter(pool_k, pool_v, slots, k, v)
    tk, tv = torch.from_numpy(pool_k.copy()), torch.from_numpy(pool_v.copy())
    flat = torch.from_numpy(slots.reshape(-1))
    tk[flat] = torch.from_numpy(k).permute(0, 2, 1, 3).reshape(10, 3, 8)
    tv[flat] = torch.from_numpy(v).permute(0, 2, 1, 3).reshape(10, 3, 8)
    np.testing.assert_array_equal(got_k, tk.numpy())
    np.testing.assert_array_equal(got_v, tv.numpy())
    untouched = np.setdiff1d(np.arange(40), slots)
    np.testing.assert_array_equal(got_k[untouched], pool_k[untouched])
    # batch-major: token (b=1, t=2) is entry 1 * 5 + 2
    np.testing.assert_array_equal(got_k[slots[0, 7]], k[1, :, 2, :])


# --- attention: brute force, torch, closed forms --------------------------------------

FIXTURES = np.load(GOLDEN / "attention_bruteforce.npz")
CASE_NAMES = sorted({key.split("__")[0] for key in FIXTURES.files})


@pytest.mark.parametrize("name", CASE_NAMES)
def test_oracle_matches_the_scalar_brute_force(name):
    f = {key.split("__")[1]: FIXTURES[key] for key in FIXTURES.files if key.startswith(name + "__")}
    qsl = f["query_start_loc"] if f["query_start_loc"].size else None
    got = attend(f["query"], f["key_pool"], f["value_pool"], f["slot_table"], f["context_lens"],
                 float(f["scale"]), int(f["groups"]), query_start_loc=qsl)
    np.testing.assert_allclose(got, f["expected"], rtol=1e-12, atol=1e-12)


def _random_case(ctxs, qlens, heads=8, kv_heads=2, dim=16, slots=256, seed=3):
    rng = np.random.default_rng(seed)
    rows = len(ctxs) if qlens is None else sum(qlens)
    q = rng.standard_normal((rows, heads, dim))
    kp = rng.standard_normal((slots, kv_heads, dim))
    vp = rng.standard_normal((slots, kv_heads, dim))
    table = rng.integers(0, slots, size=(len(ctxs), max(ctxs)))
    qsl = None if qlens is None else np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    return q, kp, vp, table, np.asarray(ctxs), qsl, heads // kv_heads, dim ** -0.5


def test_oracle_whole_prompt_matches_torch_causal_sdpa():
    ctx = 37
    q, kp, vp, table, ctxs, qsl, groups, scale = _random_case([ctx], [ctx])
    got = attend(q, kp, vp, table, ctxs, scale, groups, query_start_loc=qsl)
    tq = torch.from_numpy(q).permute(1, 0, 2).unsqueeze(0)
    k = torch.from_numpy(kp[table[0, :ctx]]).permute(1, 0, 2).unsqueeze(0).repeat_interleave(groups, dim=1)
    v = torch.from_numpy(vp[table[0, :ctx]]).permute(1, 0, 2).unsqueeze(0).repeat_interleave(groups, dim=1)
    want = torch.nn.functional.scaled_dot_product_attention(tq, k, v, is_causal=True, scale=scale)
    np.testing.assert_allclose(got, want.squeeze(0).permute(1, 0, 2).numpy(), rtol=1e-10, atol=1e-10)


def test_oracle_one_visible_key_returns_its_value_row():
    q, kp, vp, table, _, _, groups, scale = _random_case([1, 1], None)
    got = attend(q, kp, vp, table, np.array([1, 1]), scale, groups)
    for i in range(2):
        for h in range(q.shape[1]):
            np.testing.assert_allclose(got[i, h], vp[table[i, 0], h // groups], rtol=0, atol=1e-12)


def test_oracle_zero_scale_averages_the_visible_values():
    ctxs, qlens = [9, 5], [4, 1]
    q, kp, vp, table, ctx, qsl, groups, _ = _random_case(ctxs, qlens)
    got = attend(q, kp, vp, table, ctx, 0.0, groups, query_start_loc=qsl)
    # sequence 0: query j of 4 over 9 keys sees keys 0 .. 5 + j
    for j in range(4):
        for h in range(q.shape[1]):
            want = vp[table[0, : 6 + j], h // groups].mean(axis=0)
            np.testing.assert_allclose(got[j, h], want, rtol=0, atol=1e-12)


def test_oracle_reads_kv_head_h_over_groups():
    ctxs = [7, 3]
    q, kp, vp, table, ctx, _, groups, scale = _random_case(ctxs, None, heads=12, kv_heads=3)
    for kvh in range(3):
        vp[:, kvh, :] = float(kvh + 1)
    got = attend(q, kp, vp, table, ctx, scale, groups)
    for h in range(12):
        np.testing.assert_allclose(got[:, h, :], float(h // groups + 1), rtol=0, atol=1e-12)


def test_oracle_chunk_rows_equal_the_same_rows_of_the_whole_prompt():
    q, kp, vp, table, _, qsl_whole, groups, scale = _random_case([20], [20])
    whole = attend(q, kp, vp, table, np.array([20]), scale, groups, query_start_loc=qsl_whole)
    chunk = attend(q[-6:], kp, vp, table, np.array([20]), scale, groups, query_start_loc=np.array([0, 6], np.int32))
    np.testing.assert_allclose(chunk, whole[-6:], rtol=1e-12, atol=1e-12)


def test_oracle_ignores_slot_table_columns_past_the_context():
    q, kp, vp, table, ctx, _, groups, scale = _random_case([10, 4], None)
    before = attend(q, kp, vp, table, ctx, scale, groups)
    table[1, 4:] = (table[1, 4:] + 17) % kp.shape[0]
    after = attend(q, kp, vp, table, ctx, scale, groups)
    np.testing.assert_array_equal(before, after)


def test_oracle_query_blocking_does_not_change_the_answer():
    q, kp, vp, table, ctx, qsl, groups, scale = _random_case([50, 30], [40, 3])
    a = attend(q, kp, vp, table, ctx, scale, groups, query_start_loc=qsl, query_block=7)
    b = attend(q, kp, vp, table, ctx, scale, groups, query_start_loc=qsl, query_block=256)
    np.testing.assert_allclose(a, b, rtol=1e-13, atol=1e-13)


def test_work_counts_are_the_closed_forms():
    # 4 rows of ctx [3, 5]: 8 tokens x (2*2*4*2 + 8) + 2 * 2 rows * 4 heads * 4 * 2
    assert attention_bytes([3, 5], num_kv_heads=2, head_dim=4, elem_size=2, num_heads=4, query_rows=2) == 8 * 40 + 128
    # a whole prompt of 4 sees 1 + 2 + 3 + 4 pairs; 2 queries over 5 keys see 4 + 5
    assert causal_pairs([4, 2], [4, 5]) == 10 + 9


def test_baseline_matches_the_oracle():
    from oracle import baseline

    q, kp, vp, table, ctx, qsl, groups, scale = _random_case([12, 7], [5, 7])
    want = attend(q, kp, vp, table, ctx, scale, groups, query_start_loc=qsl)
    for kind in ("eager", "sdpa"):
        got = baseline.packed(kind, torch.from_numpy(q).float(), torch.from_numpy(kp).float(),
                              torch.from_numpy(vp).float(), torch.from_numpy(table), torch.from_numpy(ctx),
                              [5, 7], scale, groups)
        np.testing.assert_allclose(got.numpy(), want, rtol=2e-5, atol=2e-5)
    q, kp, vp, table, ctx, _, groups, scale = _random_case([12, 7], None)
    want = attend(q, kp, vp, table, ctx, scale, groups)
    for kind in ("eager", "sdpa"):
        got = baseline.decode(kind, torch.from_numpy(q).float(), torch.from_numpy(kp).float(),
                              torch.from_numpy(vp).float(), torch.from_numpy(table), torch.from_numpy(ctx),
                              scale, groups)
        np.testing.assert_allclose(got.numpy(), want, rtol=2e-5, atol=2e-5)


def test_a_row_with_no_keys_is_nan():
    """A decode row whose context is empty: the reference's eager softmax over
    nothing but -inf scores is 0 / 0, NaN (torch does the same on a fully
    masked row); the other rows are untouched by it."""
    import torch

    rng = np.random.default_rng(4)
    q = rng.standard_normal((2, 4, 8))
    kp = rng.standard_normal((16, 2, 8))
    vp = rng.standard_normal((16, 2, 8))
    table = rng.integers(0, 16, size=(2, 5))
    out = attend(q, kp, vp, table, np.array([0, 5]), 0.3, 2)
    assert np.isnan(out[0]).all() and np.isfinite(out[1]).all()
    scores = torch.full((1, 1, 1, 3), float("-inf"))
    assert torch.isnan(torch.softmax(scores, dim=-1)).all()
