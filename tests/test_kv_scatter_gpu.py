"""The HIP slot-write is bit-exact: the pool equals torch index_put_ and the oracle's scatter."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from liteinfer_amd.cache.block_pool import BlockPool
from liteinfer_amd.cache.kv_cache import KVCache, tokens_first
from liteinfer_amd.paged_kernels import check_bad_slots, kv_scatter
from oracle import addressing

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _bits(t: torch.Tensor) -> np.ndarray:
    """Raw bit pattern as unsigned ints, so the comparison is bit-exact whatever the dtype."""
    view = {torch.float32: torch.int32, torch.float16: torch.int16, torch.bfloat16: torch.int16}[t.dtype]
    return t.detach().contiguous().view(view).cpu().numpy()


def _case(batch, heads, tokens, dim, num_slots, dtype, layout="bhtd", seed=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    kp = torch.randn(num_slots, heads, dim, generator=g, device=DEV).to(dtype)
    vp = torch.randn(num_slots, heads, dim, generator=g, device=DEV).to(dtype)
    if layout == "bthd":  # what a projection's view(B, T, H, D).transpose(1, 2) hands over
        k = torch.randn(batch, tokens, heads, dim, generator=g, device=DEV).to(dtype).transpose(1, 2)
        v = torch.randn(batch, tokens, heads, dim, generator=g, device=DEV).to(dtype).transpose(1, 2)
    else:
        k = torch.randn(batch, heads, tokens, dim, generator=g, device=DEV).to(dtype)
        v = torch.randn(batch, heads, tokens, dim, generator=g, device=DEV).to(dtype)
    perm = torch.randperm(num_slots, generator=torch.Generator().manual_seed(seed))[: batch * tokens]
    slots = perm.view(1, -1).to(DEV)
    return kp, vp, k, v, slots


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(
    ("batch", "heads", "tokens", "dim", "layout"),
    [
        (64, 8, 1, 128, "bhtd"),    # a Llama-3-8B decode step
        (1, 8, 700, 128, "bthd"),   # a packed pass, projection layout
        (4, 8, 1, 64, "bthd"),      # Llama-3.2-1B decode
        (3, 2, 5, 24, "bhtd"),      # three 16-byte units per head row in bf16
        (2, 3, 4, 6, "bthd"),       # odd everything: element path
    ],
)
def test_scatter_equals_index_put_bit_for_bit(dtype, batch, heads, tokens, dim, layout):
    kp, vp, k, v, slots = _case(batch, heads, tokens, dim, 4096, dtype, layout)
    want_k, want_v = kp.clone(), vp.clone()
    flat = slots.reshape(-1)
    want_k[flat] = tokens_first(k)
    want_v[flat] = tokens_first(v)
    kv_scatter(kp, vp, slots, k, v)
    np.testing.assert_array_equal(_bits(kp), _bits(want_k))
    np.testing.assert_array_equal(_bits(vp), _bits(want_v))


def test_scatter_equals_the_oracle_and_touches_nothing_else():
    kp, vp, k, v, slots = _case(2, 8, 9, 128, 1024, torch.bfloat16, "bthd", seed=3)
    before_k, before_v = _bits(kp), _bits(vp)
    want_k, want_v = addressing.scatter(before_k, before_v, slots.cpu().numpy(), _bits(k), _bits(v))
    kv_scatter(kp, vp, slots, k, v)
    np.testing.assert_array_equal(_bits(kp), want_k)
    np.testing.assert_array_equal(_bits(vp), want_v)


def test_scatter_into_a_layer_of_a_multi_layer_pool():
    pool = BlockPool(num_blocks=64, block_size=16, num_layers=3, num_kv_heads=8, head_dim=128,
                     dtype=torch.bfloat16, device=DEV)
    cache = KVCache(pool)
    cache.reserve(["a", "b"], [20, 7])
    payload = cache.make_packed_payload(["a", "b"], [0, 0], [20, 7])
    g = torch.Generator(device=DEV).manual_seed(1)
    k = torch.randn(1, 8, 27, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(1, 8, 27, 128, generator=g, device=DEV).to(torch.bfloat16)
    kv = payload.update(k, v, 1)
    torch.cuda.synchronize()
    read = kv.key_pool[kv.slot_table[0, :20]]
    np.testing.assert_array_equal(_bits(read), _bits(tokens_first(k)[:20]))
    untouched = pool.slots(0)[0].abs().sum().item() + pool.slots(2)[0].abs().sum().item()
    assert untouched == 0.0


def test_out_of_range_slots_are_not_written():
    kp, vp, k, v, slots = _case(1, 2, 4, 16, 64, torch.float32)
    slots = slots.clone()
    slots[0, 1] = 64
    slots[0, 2] = -1
    before = _bits(kp)
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    kv_scatter(kp, vp, slots, k, v, bad_slots=bad)
    after = _bits(kp)
    changed = np.nonzero((after != before).any(axis=(1, 2)))[0].tolist()
    assert sorted(changed) == sorted([int(slots[0, 0]), int(slots[0, 3])])
    assert int(bad.item()) == 2
    kv_scatter(kp, vp, slots, k, v)  # no counter: the same skip, nothing counted
    assert int(bad.item()) == 2
    with pytest.raises(IndexError, match="2 K/V slot writes"):
        check_bad_slots(bad)
    assert int(bad.item()) == 0
    check_bad_slots(bad)


@pytest.mark.parametrize("src", [torch.bfloat16, torch.float32])
def test_fp8_out_of_range_slots_are_counted(src):
    _, _, k, v, slots = _case(1, 2, 4, 16, 64, src)
    kp = torch.zeros(64, 2, 16, dtype=torch.float8_e4m3fn, device=DEV)
    vp = torch.zeros_like(kp)
    slots = slots.clone()
    slots[0, 0] = 1 << 40
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    kv_scatter(kp, vp, slots, k, v, k_scale=0.5, v_scale=2.0, bad_slots=bad)
    assert int(bad.item()) == 1
    written = (kp.view(torch.uint8) != 0).any(dim=(1, 2)).nonzero().reshape(-1).tolist()
    assert set(written) == set(slots[0, 1:].tolist())


def test_pool_check_slot_writes_raises_after_a_bad_decode_write():
    pool = BlockPool(num_layers=1, num_blocks=4, block_size=16, num_kv_heads=2, head_dim=64,
                     dtype=torch.bfloat16, device=DEV)
    cache = KVCache(pool)
    k = torch.randn(2, 2, 1, 64, dtype=torch.bfloat16, device=DEV)
    cache.scatter(0, torch.tensor([[5, 64]], device=DEV), k, k)
    with pytest.raises(IndexError, match="outside the pool's 64 slots"):
        pool.check_slot_writes()
    pool.check_slot_writes()


def test_c2_decode_write_is_bit_exact_at_full_pool_size():
    from liteinfer_amd.workloads import decode_step

    step = decode_step("c2", seed=11)
    kp, vp = step.key_pool.clone(), step.value_pool.clone()
    flat = step.write_slots.reshape(-1)
    kp[flat] = tokens_first(step.new_k)
    vp[flat] = tokens_first(step.new_v)
    kv_scatter(step.key_pool, step.value_pool, step.write_slots, step.new_k, step.new_v)
    assert torch.equal(step.key_pool.view(torch.int16), kp.view(torch.int16))
    assert torch.equal(step.value_pool.view(torch.int16), vp.view(torch.int16))
