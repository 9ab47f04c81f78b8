"""The reference's dense `eager` and `sdpa` attention on CPU, fp32. TEST INFRASTRUCTURE ONLY.

Timed by bench.py beside the GPU kernels as the CPU baseline: the same
arithmetic as liteinfer/models/attention.py:97-201 (gather each context out
of the pool, expand the KV heads, attend), restated in torch and run on the
host's cores. A decode step gathers every row's context at once, bounded by
its length; a packed pass goes one sequence at a time.
"""

from __future__ import annotations

import torch
from torch.nn import functional as F


def _expand(states: torch.Tensor, groups: int) -> torch.Tensor:
    return states if groups == 1 else states.repeat_interleave(groups, dim=1)


def _visible(nq: int, ctx: int) -> torch.Tensor:
    return torch.arange(ctx)[None, :] <= (torch.arange(nq) + (ctx - nq))[:, None]


def _eager(q, k, v, mask, scale, groups):
    k, v = _expand(k, groups), _expand(v, groups)
    s = (q @ k.transpose(-2, -1)) * scale
    if mask is not None:
        s = s.masked_fill(~mask, float("-inf"))
    return torch.softmax(s, dim=-1, dtype=torch.float32).to(q.dtype) @ v


def _sdpa(q, k, v, mask, scale, groups):
    k, v = _expand(k, groups), _expand(v, groups)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=scale)


def decode(kind: str, query, key_pool, value_pool, slot_table, context_lens, scale, groups):
    """query ``[B, Hq, D]`` -> ``[B, Hq, D]``, one decode step."""
    fn = _eager if kind == "eager" else _sdpa
    width = slot_table.shape[1]
    mask = (torch.arange(width)[None, :] < context_lens[:, None])[:, None, None, :]
    k = key_pool[slot_table].transpose(1, 2)
    v = value_pool[slot_table].transpose(1, 2)
    return fn(query.unsqueeze(2), k, v, mask, scale, groups).squeeze(2)


def packed(kind: str, query, key_pool, value_pool, slot_table, context_lens, query_lens, scale, groups):
    """query ``[T, Hq, D]`` packed -> ``[T, Hq, D]``; sequences attended one at a time."""
    fn = _eager if kind == "eager" else _sdpa
    out = []
    start = 0
    for i, (nq, ctx) in enumerate(zip(query_lens, context_lens.tolist(), strict=True)):
        q = query[start:start + nq].transpose(0, 1).unsqueeze(0)
        slots = slot_table[i:i + 1, :ctx]
        k = key_pool[slots].transpose(1, 2)
        v = value_pool[slots].transpose(1, 2)
        out.append(fn(q, k, v, _visible(nq, ctx), scale, groups).squeeze(0).transpose(0, 1))
        start += nq
    return torch.cat(out, dim=0)
