"""Fused RoPE + slot-write: bit-exact against torch's separate ops and the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from liteinfer_amd.cache.block_pool import BlockPool
from liteinfer_amd.cache.kv_cache import KVCache, tokens_first
from liteinfer_amd.rope import apply_rotary_pos_emb, rope_kv_write
from oracle import rope as R

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
NAMES = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}


def _bits(t: torch.Tensor) -> np.ndarray:
    view = {torch.float32: torch.int32, torch.float16: torch.int16, torch.bfloat16: torch.int16}[t.dtype]
    return t.detach().contiguous().view(view).cpu().numpy()


def _cos_sin(batch, tokens, dim, dtype, gen, theta=500000.0):
    """What the rotary module hands over: cat(freqs, freqs) of positions times inverse frequencies."""
    inv = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float32, device=DEV) / dim))
    pos = torch.randint(0, 8192, (batch, tokens), generator=gen, device=DEV).float()
    freqs = pos[..., None] * inv
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def _case(batch, tokens, heads, kv_heads, dim, dtype, num_slots=4096, seed=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    # projections as LlamaAttention hands them over: view(B, T, H, D).transpose(1, 2)
    q = torch.randn(batch, tokens, heads, dim, generator=g, device=DEV).to(dtype).transpose(1, 2)
    k = torch.randn(batch, tokens, kv_heads, dim, generator=g, device=DEV).to(dtype).transpose(1, 2)
    v = torch.randn(batch, tokens, kv_heads, dim, generator=g, device=DEV).to(dtype).transpose(1, 2)
    cos, sin = _cos_sin(batch, tokens, dim, dtype, g)
    kp = torch.randn(num_slots, kv_heads, dim, generator=g, device=DEV).to(dtype)
    vp = torch.randn(num_slots, kv_heads, dim, generator=g, device=DEV).to(dtype)
    perm = torch.randperm(num_slots, generator=torch.Generator().manual_seed(seed))[: batch * tokens]
    return q, k, v, cos, sin, perm.view(1, -1).to(DEV), kp, vp


def _torch_reference(q, k, v, cos, sin, slots, kp, vp):
    q_embed, k_embed = apply_rotary_pos_emb(q, k, cos, sin)
    kp, vp = kp.clone(), vp.clone()
    flat = slots.reshape(-1)
    kp[flat] = tokens_first(k_embed)
    vp[flat] = tokens_first(v)
    return q_embed, kp, vp


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(("batch", "tokens", "heads", "kv_heads", "dim"), [
    (64, 1, 32, 8, 128),    # a decode step at Llama-3-8B geometry
    (1, 300, 32, 8, 128),   # a packed pass
    (3, 17, 8, 2, 64),      # small ragged shapes
    (2, 5, 10, 2, 72),      # head_dim 72: the element-wise path for 16-bit types
])
def test_bit_exact_against_torch_ops(dtype, batch, tokens, heads, kv_heads, dim):
    q, k, v, cos, sin, slots, kp, vp = _case(batch, tokens, heads, kv_heads, dim, dtype)
    want_q, want_kp, want_vp = _torch_reference(q, k, v, cos, sin, slots, kp, vp)
    got_q = rope_kv_write(q, k, v, cos, sin, slots, kp, vp)
    np.testing.assert_array_equal(_bits(got_q), _bits(want_q))
    np.testing.assert_array_equal(_bits(kp), _bits(want_kp))
    np.testing.assert_array_equal(_bits(vp), _bits(want_vp))
    # same memory order as the reference's result: token-major (strides of
    # size-1 dimensions are immaterial)
    assert [st for st, n in zip(got_q.stride(), got_q.shape) if n > 1] == \
        [st for st, n in zip(want_q.stride(), want_q.shape) if n > 1]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_bit_exact_against_the_oracle(dtype):
    q, k, v, cos, sin, slots, kp, vp = _case(2, 9, 8, 2, 64, dtype, num_slots=64, seed=3)
    name = NAMES[dtype]
    want_q, want_kp, want_vp = R.rope_kv_write(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                                               cos.float().cpu().numpy(), sin.float().cpu().numpy(),
                                               slots.cpu().numpy(), kp.float().cpu().numpy(), vp.float().cpu().numpy(),
                                               name)
    got_q = rope_kv_write(q, k, v, cos, sin, slots, kp, vp)
    np.testing.assert_array_equal(got_q.float().cpu().numpy(), want_q)
    np.testing.assert_array_equal(kp.float().cpu().numpy(), want_kp)
    np.testing.assert_array_equal(vp.float().cpu().numpy(), want_vp)


def test_broadcast_cos_and_contiguous_inputs():
    dtype = torch.bfloat16
    q, k, v, cos, sin, slots, kp, vp = _case(4, 6, 8, 2, 128, dtype, seed=5)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    cos1, sin1 = cos[:1], sin[:1]  # one table for the whole batch
    want_q, want_kp, want_vp = _torch_reference(q, k, v, cos1.expand_as(cos), sin1.expand_as(sin), slots, kp, vp)
    got_q = rope_kv_write(q, k, v, cos1, sin1, slots, kp, vp)
    np.testing.assert_array_equal(_bits(got_q), _bits(want_q))
    np.testing.assert_array_equal(_bits(kp), _bits(want_kp))
    np.testing.assert_array_equal(_bits(vp), _bits(want_vp))


def test_out_of_range_slots_are_skipped_and_others_untouched():
    dtype = torch.bfloat16
    q, k, v, cos, sin, slots, kp, vp = _case(1, 4, 8, 2, 64, dtype, num_slots=32, seed=6)
    slots = torch.tensor([[3, -1, 32, 7]], device=DEV)
    before_k, before_v = kp.clone(), vp.clone()
    q_embed, k_embed = apply_rotary_pos_emb(q, k, cos, sin)
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    got_q = rope_kv_write(q, k, v, cos, sin, slots, kp, vp, bad_slots=bad)
    assert int(bad.item()) == 2  # one count per token, not per head or element
    np.testing.assert_array_equal(_bits(got_q), _bits(q_embed))
    rows_k, rows_v = tokens_first(k_embed), tokens_first(v)
    for i, s in ((0, 3), (3, 7)):
        assert torch.equal(kp[s], rows_k[i]) and torch.equal(vp[s], rows_v[i])
    keep = [s for s in range(32) if s not in (3, 7)]
    assert torch.equal(kp[keep], before_k[keep]) and torch.equal(vp[keep], before_v[keep])


def test_payload_update_rotated_matches_rotate_then_update():
    pool = BlockPool(num_layers=2, num_blocks=64, block_size=16, num_kv_heads=8, head_dim=128,
                     dtype=torch.bfloat16, device=DEV)
    cache = KVCache(pool)
    cache.reserve(["a", "b"], [40, 3])
    payload = cache.make_packed_payload(["a", "b"], [0, 0], [40, 3])
    q, k, v, cos, sin, *_ = _case(1, 43, 32, 8, 128, torch.bfloat16, seed=7)
    q_rot, kv = payload.update_rotated(q, k, v, cos, sin, layer_idx=1)
    keys, values = pool.slots(1)
    got_k, got_v = keys.clone(), values.clone()
    keys.zero_(), values.zero_()
    q_embed, k_embed = apply_rotary_pos_emb(q, k, cos, sin)
    kv2 = payload.update(k_embed, v, layer_idx=1)
    assert torch.equal(q_rot, q_embed)
    assert torch.equal(got_k, keys) and torch.equal(got_v, values)
    assert torch.equal(kv.slot_table, kv2.slot_table) and torch.equal(kv.context_lens, kv2.context_lens)
