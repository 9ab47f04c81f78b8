"""The attention boundary: one kernel per `attn_implementation` name.

The same operator surface as liteinfer's ``models/attention.py`` — `PagedKV`,
the registry `IMPLEMENTATIONS`, `resolve`, `unsupported_reason`,
`select_implementation`, `reads_pool_in_place` and the three kernels with the
signature ``fn(query, kv, scaling, num_kv_groups) -> Tensor`` — so a model
layer calls it exactly as it calls the reference (liteinfer/models/llama.py:161).

* ``paged`` reads the pool in place through the HIP library
  (`paged_kernels`): decode when `kv.query_start_loc` is None, otherwise a
  packed pass (attention.py:204-257 in the reference).
* ``eager`` and ``sdpa`` gather each context out of the pool and attend with
  dense torch ops. They run on any device and are the CPU path.

Causality is positional: a sequence's queries are the last positions of its
context, so query ``j`` of ``q`` sees keys ``0 .. context_len - q + j``.
"""

from __future__ import annotations

import functools
from collections.abc import Callable
from typing import NamedTuple

import torch
from torch.nn import functional as F


class PagedKV(NamedTuple):
    """A layer's KV pool plus the addresses a kernel reads it by (attention.py:41-66)."""

    key_pool: torch.Tensor
    """``[num_slots, kv_heads, head_dim]``: this layer's key store."""
    value_pool: torch.Tensor
    slot_table: torch.Tensor
    """``[batch, max_context]`` int64 slot per logical position, left-aligned;
    columns at or past a row's context length are never read."""
    context_lens: torch.Tensor
    """``[batch]`` int32 tokens each sequence holds, this pass's included."""
    num_splits: int | None = None
    """Decode partitions per sequence; None lets the kernel choose."""
    query_start_loc: torch.Tensor | None = None
    """``[batch + 1]`` int32 prefix sums of each sequence's queries in a packed
    pass; None marks a decode step (one query per batch row)."""
    max_query_len: int = 1
    """Most queries any sequence brings; sizes the prefill grid."""
    host_context_lens: tuple[int, ...] = ()
    """`context_lens` on the host, for the dense kernels' per-sequence slicing."""
    host_query_lens: tuple[int, ...] = ()
    """Each sequence's query count on the host, for the same slicing."""
    k_scale: float = 1.0
    """An fp8 (``torch.float8_e4m3fn``) pool holds K / k_scale; unused otherwise."""
    v_scale: float = 1.0
    """An fp8 pool holds V / v_scale; unused otherwise."""


# ---------------------------------------------------------------------------
# Dense kernels (gather, then attend)
# ---------------------------------------------------------------------------


def _expand_kv_heads(states: torch.Tensor, groups: int) -> torch.Tensor:
    """``[B, Hkv, S, D]`` -> ``[B, Hkv * groups, S, D]``: query head h reads KV head h // groups."""
    if groups == 1:
        return states
    return states.repeat_interleave(groups, dim=1)


def _causal_visibility(num_queries: int, num_keys: int, device: torch.device) -> torch.Tensor:
    """``[queries, keys]`` True where the key is visible: queries are the last positions."""
    key_pos = torch.arange(num_keys, device=device)
    query_pos = torch.arange(num_queries, device=device) + (num_keys - num_queries)
    return key_pos[None, :] <= query_pos[:, None]


def _gather(pool: torch.Tensor, slots: torch.Tensor, like: torch.Tensor, scale: float) -> torch.Tensor:
    """``[B, W]`` slots of a ``[S, Hkv, D]`` pool -> ``[B, Hkv, W, D]`` in `like`'s dtype.

    An fp8 pool's rows are dequantised (times `scale`) in float32, then
    rounded to the query's dtype, the values the dense arithmetic then uses.
    """
    rows = pool[slots].transpose(1, 2)
    if rows.dtype == torch.float8_e4m3fn:
        rows = (rows.to(torch.float32) * scale).to(like.dtype)
    return rows


# (query, keys, values, visible-or-None, is_causal) -> output
_Attend = Callable[[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor | None, bool], torch.Tensor]


def _eager_core(query, keys, values, visible, is_causal, *, scaling: float, num_kv_groups: int):
    """Scaled dot-product attention as explicit matmuls (attention.py:146-164).

    Scores are computed in the input dtype, softmax in fp32 and cast back to the
    input dtype before the value product — the reference's rounding sequence.
    """
    keys = _expand_kv_heads(keys, num_kv_groups)
    values = _expand_kv_heads(values, num_kv_groups)
    scores = (query @ keys.transpose(-2, -1)) * scaling
    if is_causal:
        visible = _causal_visibility(query.shape[-2], keys.shape[-2], query.device)
    if visible is not None:
        scores = scores.masked_fill(~visible, float("-inf"))
    weights = torch.softmax(scores, dim=-1, dtype=torch.float32).to(query.dtype)
    return weights @ values


def _sdpa_core(query, keys, values, visible, is_causal, *, scaling: float, num_kv_groups: int):
    """The same attention through torch's fused kernel (attention.py:167-186)."""
    keys = _expand_kv_heads(keys, num_kv_groups)
    values = _expand_kv_heads(values, num_kv_groups)
    return F.scaled_dot_product_attention(query, keys, values, attn_mask=visible, is_causal=is_causal, scale=scaling)


def _dense(query: torch.Tensor, kv: PagedKV, attend: _Attend) -> torch.Tensor:
    if kv.query_start_loc is None:
        return _dense_decode(query, kv, attend)
    return _dense_packed(query, kv, attend)


def _dense_decode(query: torch.Tensor, kv: PagedKV, attend: _Attend) -> torch.Tensor:
    """Every row's context gathered at once, each bounded by its own length."""
    width = kv.slot_table.shape[1]
    bound = torch.arange(width, device=query.device)[None, :] < kv.context_lens.to(query.device)[:, None]
    keys = _gather(kv.key_pool, kv.slot_table, query, kv.k_scale)
    values = _gather(kv.value_pool, kv.slot_table, query, kv.v_scale)
    return attend(query, keys, values, bound[:, None, None, :], False)


def _dense_packed(query: torch.Tensor, kv: PagedKV, attend: _Attend) -> torch.Tensor:
    """A packed pass sliced one sequence at a time on the host."""
    if not (kv.host_context_lens and kv.host_query_lens):
        raise ValueError(
            "a dense kernel slices each sequence of a packed pass on the host, and was "
            "handed no host_context_lens / host_query_lens"
        )
    pieces = []
    chunks = query.split(list(kv.host_query_lens), dim=2)
    for row, (chunk, ctx) in enumerate(zip(chunks, kv.host_context_lens, strict=True)):
        slots = kv.slot_table[row : row + 1, :ctx]
        nq = chunk.shape[2]
        whole_prompt = nq == ctx
        is_causal = nq > 1 and whole_prompt
        visible = _causal_visibility(nq, ctx, query.device) if (nq > 1 and not whole_prompt) else None
        keys = _gather(kv.key_pool, slots, chunk, kv.k_scale)
        values = _gather(kv.value_pool, slots, chunk, kv.v_scale)
        pieces.append(attend(chunk, keys, values, visible, is_causal))
    return torch.cat(pieces, dim=2)


def eager_attention(query: torch.Tensor, kv: PagedKV, scaling: float, num_kv_groups: int) -> torch.Tensor:
    """Attention written out in matmuls: what the arithmetic looks like."""
    return _dense(query, kv, functools.partial(_eager_core, scaling=scaling, num_kv_groups=num_kv_groups))


def sdpa_attention(query: torch.Tensor, kv: PagedKV, scaling: float, num_kv_groups: int) -> torch.Tensor:
    """The same attention through torch's fused kernel, which never holds the scores."""
    return _dense(query, kv, functools.partial(_sdpa_core, scaling=scaling, num_kv_groups=num_kv_groups))


# ---------------------------------------------------------------------------
# The paged kernel (HIP)
# ---------------------------------------------------------------------------


def paged_attention(query: torch.Tensor, kv: PagedKV, scaling: float, num_kv_groups: int) -> torch.Tensor:
    """Attend straight out of the KV pool; decode or packed is decided by `query_start_loc`."""
    if kv.query_start_loc is None:
        return _paged_decode_step(query, kv, scaling, num_kv_groups)
    return _paged_packed(query, kv, scaling, num_kv_groups)


def _paged_decode_step(query: torch.Tensor, kv: PagedKV, scaling: float, num_kv_groups: int) -> torch.Tensor:
    """``[batch, heads, 1, dim]`` in, the same out."""
    if query.shape[2] != 1:
        raise ValueError(f"paged decode takes one query per sequence, got {query.shape[2]}")
    from liteinfer_amd.paged_kernels import paged_decode

    out = paged_decode(
        query.squeeze(2), kv.key_pool, kv.value_pool, kv.slot_table, kv.context_lens,
        scaling, num_kv_groups, num_splits=kv.num_splits, k_scale=kv.k_scale, v_scale=kv.v_scale,
    )
    return out.unsqueeze(2)


def _one_query_rows_to_decode_kernel(query_lens) -> bool:
    """Whether a packed pass's one-query sequences should go to the decode split.

    True whenever there are any. Over a 16-bit pool the split runs inside the
    prefill launch: its first work-groups stream the rows' K/V while the rest
    fold the chunks on the matrix cores, then join the chunks' queues
    (``prefill_pp_rows``; config 3: 316-335 us against 341-387 us with the
    rows folded as prefill units, where each row walks its whole context
    through a 256-row work-group at matrix-core speed; no case measured
    slower; over an fp8 pool the lockstep prefill does the same: 359-365
    against 412 us, and ~382 us with the rows in a decode launch of their
    own before it).
    False (no decode launch, ``LI_FLAG_PREFILL_ONLY``) when there are none;
    a caller may still ask for the folded form with ``one_query_rows=False``.
    The answer is the same attention either way.
    """
    return any(q == 1 for q in query_lens)


def _paged_packed(query: torch.Tensor, kv: PagedKV, scaling: float, num_kv_groups: int) -> torch.Tensor:
    """``[1, heads, total_queries, dim]`` in, the same out; the kernel works token-first."""
    from liteinfer_amd.paged_kernels import paged_prefill

    # The host query lengths, when the payload carries them, say whether the
    # pass has one-query sequences (None: the kernels find out on the device).
    one_query_rows = None
    if kv.host_query_lens:
        if all(q == 1 for q in kv.host_query_lens):
            # Every sequence brings one query: the pass is a decode step (token
            # i is sequence i's query), run as one (no query offsets to read;
            # the short kernel where the table is narrow).
            out = _paged_decode_step(query.permute(2, 1, 0, 3), kv, scaling, num_kv_groups)  # [T, H, 1, D]
            return out.permute(2, 1, 0, 3)
        one_query_rows = _one_query_rows_to_decode_kernel(kv.host_query_lens)
    out = paged_prefill(
        query.squeeze(0).transpose(0, 1), kv.key_pool, kv.value_pool, kv.slot_table, kv.context_lens,
        kv.query_start_loc, kv.max_query_len, scaling, num_kv_groups, one_query_rows=one_query_rows,
        k_scale=kv.k_scale, v_scale=kv.v_scale,
    )
    return out.transpose(0, 1).unsqueeze(0)


IMPLEMENTATIONS = {
    "eager": eager_attention,
    "sdpa": sdpa_attention,
    "paged": paged_attention,
}
PAGED_IMPLEMENTATION = "paged"
"""Fastest wherever its preconditions hold."""

UNIVERSAL_IMPLEMENTATION = "sdpa"
"""Runs on any device and shape; the automatic choice's fallback."""


def resolve(name: str):
    """Look up a kernel by name."""
    if name not in IMPLEMENTATIONS:
        raise ValueError(f"unknown attn_implementation {name!r}; known: {sorted(IMPLEMENTATIONS)}")
    return IMPLEMENTATIONS[name]


def unsupported_reason(name: str, device: torch.device) -> str | None:
    """Why this kernel cannot run on `device`, or None if it can.

    Only ``paged`` has preconditions: it is a HIP kernel for ROCm devices, and
    its library must be built. Head dims up to 512 and any query-head grouping
    are served.
    """
    if name != PAGED_IMPLEMENTATION:
        return None
    device = torch.device(device)
    if device.type != "cuda" or torch.version.hip is None:
        return f"it is a HIP kernel for ROCm devices and the device is {device}"
    from liteinfer_amd import _native

    if not _native.is_built():
        return f"its HIP library is not built ({_native.library_path()} is missing)"
    return None


def select_implementation(requested: str | None, device: torch.device) -> str:
    """Resolve a kernel name; None picks `paged` where it runs, else `sdpa`.

    A named kernel that cannot run is refused rather than downgraded.
    """
    if requested is None:
        return UNIVERSAL_IMPLEMENTATION if unsupported_reason(PAGED_IMPLEMENTATION, device) else PAGED_IMPLEMENTATION
    resolve(requested)
    blocked = unsupported_reason(requested, device)
    if blocked is not None:
        raise ValueError(
            f"attn_implementation={requested!r} cannot run here: {blocked}. "
            f"Leave it unset to choose automatically, or pass {UNIVERSAL_IMPLEMENTATION!r}."
        )
    return requested


def reads_pool_in_place(name: str) -> bool:
    """Whether this kernel reads the pool where it lies (what a captured decode step needs)."""
    return name == PAGED_IMPLEMENTATION
