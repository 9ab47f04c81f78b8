"""Rotary position embedding fused with the KV slot-write.

liteinfer applies RoPE to a layer's q and k (`_apply_rotary_pos_emb`,
liteinfer/models/llama.py:79-98, called at :155-156) and then stores k and v
through the payload (`payload.update`, llama.py:160 -> `KVCache.scatter`,
liteinfer/cache/kv_cache.py:236-253). On a ROCm device `rope_kv_write` does
both in one HIP launch (`li_rope_kv_write`): it returns the rotated q and
writes the rotated k and the untouched v into their pool slots, bit for bit
what the separate torch ops produce. `apply_rotary_pos_emb` is the same
arithmetic as plain torch ops, the path for CPU tensors.
"""

from __future__ import annotations

import torch

from liteinfer_amd import _native
from liteinfer_amd.paged_kernels import _as_index, _check_pools, _require_device_tensors, bad_slots_pointer


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """``cat(-x[..., D/2:], x[..., :D/2])`` (llama.py:79-82)."""
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rotary_pos_emb(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor,
                         sin: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``x * cos + rotate_half(x) * sin`` for q and k; cos / sin broadcast over heads (llama.py:85-98)."""
    cos = cos.unsqueeze(1)
    sin = sin.unsqueeze(1)
    return (q * cos) + (rotate_half(q) * sin), (k * cos) + (rotate_half(k) * sin)


def rope_kv_write(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    slots: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    *,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    bad_slots: torch.Tensor | None = None,
) -> torch.Tensor:
    """Rotate q and k, store k and v at `slots`, return the rotated q.

    Args:
        q: ``[batch, num_heads, tokens, head_dim]`` (any strides; the
            projection's ``view(...).transpose(1, 2)`` as LlamaAttention makes it).
        k, v: ``[batch, num_kv_heads, tokens, head_dim]``.
        cos, sin: ``[batch, tokens, head_dim]`` from the rotary module (a
            batch of 1 broadcasts).
        slots: ``batch * tokens`` pool slots, batch-major (``[1, T]`` for a
            packed pass, ``[1, B]`` for a decode step).
        key_pool, value_pool: this layer's ``[num_slots, num_kv_heads,
            head_dim]`` stores, written in place. An fp8
            (``torch.float8_e4m3fn``) pool stores the rotated k (rounded to
            q's dtype, as the torch ops round it) and v quantised with
            `k_scale` / `v_scale`, exactly as `kv_scatter` would store them.
        bad_slots: optional one-element int32 counter of slots outside the
            pool (not written), as for `kv_scatter`.

    Returns:
        The rotated q, ``[batch, num_heads, tokens, head_dim]``, laid out
        token-major in memory like the reference's result (so the packed
        attention's ``squeeze(0).transpose(0, 1)`` is a free view).
    """
    device = _require_device_tensors(q, k, v, cos, sin, slots, key_pool, value_pool)
    bad_ptr = bad_slots_pointer(bad_slots, device)
    _check_pools(key_pool, value_pool)
    if q.dim() != 4 or k.dim() != 4 or k.shape != v.shape:
        raise ValueError(f"q, k, v must be [batch, heads, tokens, head_dim], got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    batch, num_heads, tokens, head_dim = q.shape
    num_kv_heads = k.shape[1]
    if k.shape[0] != batch or k.shape[2] != tokens or k.shape[3] != head_dim:
        raise ValueError(f"k {tuple(k.shape)} does not match q {tuple(q.shape)}")
    if num_kv_heads != key_pool.shape[1] or head_dim != key_pool.shape[2]:
        raise ValueError(f"k rows {num_kv_heads}x{head_dim} do not match the pool's {tuple(key_pool.shape[1:])}")
    if head_dim % 2:
        raise ValueError(f"head_dim {head_dim} must be even for rotary embedding")
    fp8 = key_pool.dtype == _native.FP8_POOL_DTYPE
    dtype = q.dtype if fp8 else key_pool.dtype
    if fp8 and dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"an fp8 pool is written from bfloat16 or float16 projections, not {dtype}")
    for name, t in (("q", q), ("k", k), ("v", v), ("cos", cos), ("sin", sin)):
        if t.dtype != dtype:
            raise ValueError(f"{name} dtype {t.dtype} does not match the pool's {dtype}")
    if cos.shape != sin.shape or cos.dim() != 3 or cos.shape[1:] != (tokens, head_dim) or cos.shape[0] not in (1, batch):
        raise ValueError(f"cos / sin must be [batch or 1, {tokens}, {head_dim}], got {tuple(cos.shape)}, {tuple(sin.shape)}")
    if cos.stride() != sin.stride():
        sin = sin.contiguous()
        cos = cos.contiguous()
    cs_strides = list(cos.stride())
    if cos.shape[0] == 1:
        cs_strides[0] = 0
    flat_slots = _as_index(slots.reshape(-1), torch.int64).contiguous()
    if flat_slots.numel() != batch * tokens:
        raise ValueError(f"{flat_slots.numel()} slots for {batch * tokens} tokens")
    out = torch.empty(batch, tokens, num_heads, head_dim, dtype=dtype, device=device).transpose(1, 2)
    lib = _native.load()
    args = (
        q.data_ptr(), _native.i64_array(q.stride()),
        k.data_ptr(), _native.i64_array(k.stride()),
        v.data_ptr(), _native.i64_array(v.stride()),
        cos.data_ptr(), sin.data_ptr(), _native.i64_array(cs_strides),
        batch, tokens, flat_slots.data_ptr(),
        out.data_ptr(), _native.i64_array(out.stride()),
        key_pool.data_ptr(), value_pool.data_ptr(),
        key_pool.shape[0], key_pool.stride(0), key_pool.stride(1),
        num_heads, num_kv_heads, head_dim, _native.dtype_code(dtype),
    )
    if fp8:
        if not (k_scale > 0 and v_scale > 0):
            raise ValueError(f"k_scale and v_scale must be > 0, got {k_scale}, {v_scale}")
        status = lib.li_rope_kv_write_fp8(*args, float(k_scale), float(v_scale), bad_ptr,
                                          _native.stream_handle(device))
    else:
        status = lib.li_rope_kv_write(*args, bad_ptr, _native.stream_handle(device))
    _native.check(status, "rope_kv_write")
    return out
