"""The C-ABI library loads, exports what the header declares, and checks arguments (CPU; no kernel runs)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from liteinfer_amd import _build, _native
from liteinfer_amd.paged_kernels import _MAX_SPLITS, choose_num_splits

HEADER = Path(__file__).resolve().parent.parent / "include" / "liteinfer_amd.h"


def _declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"\b(li_[a-z0-9_]+)\s*\(", text)


def test_library_is_built_and_loads():
    assert _native.is_built(), "run `python -m liteinfer_amd._build` (or __graft_entry__.build())"
    lib = _native.load()
    assert lib.li_abi_version() == _native.ABI_VERSION


def test_library_carries_the_digest_of_its_sources():
    lib = _native.load()
    assert lib.li_build_id().decode() == _build.source_hash()


def test_a_library_built_from_other_sources_is_refused(monkeypatch):
    """A stale build (its digest differs from the sources beside it) does not load."""
    _native.load()
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setattr(_build, "source_hash", lambda: "0123456789abcdef")
    with pytest.raises(RuntimeError, match="built from other sources"):
        _native.load()
    monkeypatch.undo()
    assert _native.load().li_build_id().decode() == _build.source_hash()


def test_every_declared_symbol_is_exported_and_bound():
    declared = _declared_functions()
    assert declared, "no declarations parsed"
    assert sorted(declared) == sorted(_native.EXPORTED_SYMBOLS)
    lib = ctypes.CDLL(str(_native.library_path()))
    for name in declared:
        assert hasattr(lib, name), name


def _splits(batch, kv_heads, max_context, cus=256, block_kv=64):
    return choose_num_splits(batch, kv_heads, max_context, device_index=0, block_kv=block_kv, num_cus=cus)


# The reference's own properties of its chooser (tests/unit/test_paged_decode.py:252-281).

def test_a_batch_that_already_fills_the_device_is_not_split():
    assert _splits(batch=256, kv_heads=8, max_context=1024) == 1


def test_a_single_sequence_splits_its_key_loop():
    assert _splits(batch=1, kv_heads=1, max_context=4096) > 1


def test_the_split_count_never_exceeds_the_cap():
    assert _splits(batch=1, kv_heads=1, max_context=1 << 20) <= _MAX_SPLITS == 32


def test_a_context_with_too_little_to_cut_is_not_split():
    assert _splits(batch=1, kv_heads=1, max_context=128) == 1


def test_no_split_is_finer_than_one_key_tile():
    assert _splits(batch=1, kv_heads=1, max_context=256) == 4


def test_a_longer_context_is_cut_more_finely():
    assert _splits(batch=1, kv_heads=8, max_context=4096) > _splits(batch=1, kv_heads=8, max_context=256)


# Values the reference's chooser gives, worked by hand from paged_kernels.py:683-693
# (tiles = cdiv(W, 64); 1 under 4 tiles; else max(1, min(2 * CUs // (B * Hkv), tiles, 32))).
@pytest.mark.parametrize(
    ("batch", "kv_heads", "max_context", "cus", "want"),
    [
        (1, 8, 4096, 256, 32),     # 512 // 8 = 64, tiles 64, capped at 32
        (1, 8, 4096, 84, 21),      # an 84-SM A40: 168 // 8 = 21 (docs/benchmarks.md's 21 splits)
        (4, 8, 8192, 256, 16),     # 512 // 32
        (64, 8, 8192, 256, 1),     # 512 // 512
        (12, 8, 4096, 84, 1),      # 168 // 96: "from batch 12 up nothing is split"
        (8, 8, 256, 84, 2),        # 168 // 64 = 2, tiles 4: the batch-8, 256-token case
        (1, 1, 255, 256, 4),       # tiles = cdiv(255, 64) = 4
        (1, 1, 192, 256, 1),       # 3 tiles: under the minimum
        (3, 2, 100000, 256, 32),   # 512 // 6 = 85, capped
        (300, 8, 8192, 256, 1),    # target // programs = 0, floored at 1
    ],
)
def test_choose_num_splits_is_the_reference_rule(batch, kv_heads, max_context, cus, want):
    assert _splits(batch, kv_heads, max_context, cus=cus) == want


def test_choose_num_splits_follows_the_tile_size():
    # 4 tiles of 32 keys are worth cutting; as tiles of 64 they are 2.
    assert _splits(batch=1, kv_heads=1, max_context=128, block_kv=32) == 4
    assert _splits(batch=1, kv_heads=1, max_context=128, block_kv=64) == 1


def test_choose_num_splits_of_an_empty_batch_is_one():
    assert _splits(batch=0, kv_heads=8, max_context=4096) == 1


def _plan(**kw):
    args = dict(batch=4, num_heads=32, num_kv_heads=8, head_dim=128, max_context=4096, num_splits=0, num_cus=256,
                block_kv=64)
    args.update(kw)
    lib = _native.load()
    parts, plen, need = ctypes.c_int(), ctypes.c_int(), ctypes.c_size_t()
    status = lib.li_paged_decode_plan(*args.values(), ctypes.byref(parts), ctypes.byref(plen), ctypes.byref(need))
    return status, parts.value, plen.value, need.value


def test_plan_sizes_the_workspace_for_its_partitions():
    status, parts, plen, need = _plan()
    assert status == 0 and parts > 1 and plen % 64 == 0
    rows = 4 * 32 * parts
    assert need >= rows * 128 * 4 + rows * 4


def test_plan_pins_the_reference_split_rule_when_asked():
    status, parts, plen, _ = _plan(num_splits=5)
    assert (status, parts, plen) == (0, 5, 0)
    status, parts, _, need = _plan(num_splits=1)
    assert (status, parts) == (0, 1)
    # The MFMA kernel may still run its balanced split (a pinned count is a
    # hint there): 4 waves per CU, two fp32 partials of G = 4 heads each.
    assert need >= 256 * 4 * 2 * 4 * (128 + 1) * 4


def test_kernel_choices_map_to_flags():
    from liteinfer_amd.paged_kernels import _flags, _prefill_kernel
    assert _flags("auto") == 0
    assert _flags("generic") == _native.LI_FLAG_FORCE_GENERIC
    assert _flags("equal_splits") == _native.LI_FLAG_EQUAL_SPLITS
    with pytest.raises(ValueError):
        _flags("fast")
    with pytest.raises(ValueError):
        _prefill_kernel("equal_splits")


def test_plan_rejects_bad_arguments_with_a_message():
    status, *_ = _plan(num_heads=30)
    assert status == _native.LI_EINVAL
    assert "cannot be grouped" in _native.last_error()
    status, *_ = _plan(num_splits=-1)
    assert status == _native.LI_EINVAL
    assert "num_splits must be >= 1" in _native.last_error()


def test_check_raises_the_reported_message():
    _plan(num_heads=30)
    with pytest.raises(ValueError, match="cannot be grouped"):
        _native.check(_native.LI_EINVAL, "plan")


def test_scatter_rejects_null_pointers_before_launching():
    lib = _native.load()
    strides = _native.i64_array([0, 0, 0, 1])
    status = lib.li_kv_scatter(None, None, strides, strides, 1, 1, None, None, None, 16, 16, 8, 2, 8,
                               _native.LI_BF16, None, None)
    assert status == _native.LI_EINVAL
    assert "null pointer" in _native.last_error()


def _row_groups(row_keys, chunk_pairs, listed_blocks, grid=256, split_waves=1024, kv_heads=8, heads=32, dim=128,
                fp8=0):
    return _native.load().li_prefill_row_groups(row_keys, chunk_pairs, listed_blocks, grid, split_waves, kv_heads,
                                                heads, dim, fp8)


def test_prefill_row_groups_on_extreme_passes():
    """The count of row work-groups a packed pass's prefill launch uses (the
    rule prefill_order runs on the device), on the edges of its inputs: it
    never exceeds the grid or the workspace's partial slots (four row waves
    per work-group), whatever the passes' sizes."""
    # no rows: none
    assert _row_groups(0, 10**9, 100) == 0
    # rows only: every work-group the launch can hold
    assert _row_groups(5000, 0, 0) == 256
    assert _row_groups(5000, 0, 0, grid=256, split_waves=512) == 128
    # a workspace of exactly grid * 4 partial slots: the whole grid
    assert _row_groups(5000, 0, 0, grid=264, split_waves=264 * 4) == 264
    # a grid that is not a multiple of the four waves' slots (a CU count that
    # is not a multiple of 8: grid 264, 1040 waves): held to the slots
    assert _row_groups(5000, 0, 0, grid=264, split_waves=1040) == 260
    assert _row_groups(10**7, 1, 1, grid=264, split_waves=1040) <= 260
    # a grid smaller than the queue count: never above the grid
    for grid in range(0, 9):
        for keys, pairs, blocks in ((1, 1, 1), (10**6, 10**3, 1), (10, 10**12, 400), (10**6, 0, 0)):
            got = _row_groups(keys, pairs, blocks, grid=grid, split_waves=4 * grid)
            assert 0 <= got <= grid, (grid, keys, pairs, blocks, got)
    # one tiny chunk against huge rows: the ratio overflows no integer
    assert _row_groups(2**40, 1, 1) == 256 - 8
    # one huge chunk against one short row: the floor of one per queue
    assert _row_groups(1, 10**15, 1) == 8
    # a workspace smaller than one work-group's waves: no row work-group
    assert _row_groups(100, 100, 1, split_waves=3) == 0


def test_prefill_row_groups_properties_on_a_grid_of_passes():
    rng = __import__("random").Random(0)
    for _ in range(3000):
        grid = rng.choice([1, 7, 8, 64, 248, 256, 264, 304])
        slots = rng.choice([0, 4, 4 * grid, 4 * grid - 4, 1024, 4 * grid + 40])
        keys = rng.choice([0, 1, rng.randrange(1, 10**7), 2**50])
        pairs = rng.choice([0, 1, rng.randrange(1, 10**12), 2**62])
        blocks = rng.randrange(0, 5000)
        fp8 = rng.randrange(2)
        got = _row_groups(keys, pairs, blocks, grid=grid, split_waves=slots, fp8=fp8)
        cap = min(grid, slots // 4)
        assert 0 <= got <= cap
        if keys == 0 or cap == 0:
            assert got == 0
        elif pairs == 0:
            assert got == cap
        elif got < cap:
            assert got % 8 == 0 and got >= 8
    assert _native.load().li_prefill_row_groups(1, 1, -1, 8, 32, 8, 32, 128, 0) == _native.LI_EINVAL
