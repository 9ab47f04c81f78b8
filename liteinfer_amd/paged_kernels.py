"""Attention that reads the KV pool where it lies, in hand-written HIP for MI355X.

Host side of the three device kernels of liteinfer's `paged` path. The entry
points keep the reference's names, arguments, defaults and error messages
(liteinfer/models/paged_kernels.py:645-882), so the attention boundary and
its tests read the same; underneath, each call is one or two launches of the
C-ABI library in ``csrc/`` on torch's current stream:

* `kv_scatter` — the KV slot-write, a bit-exact copy of this pass's K/V rows
  into their pool slots (liteinfer/cache/kv_cache.py:236-253).
* `paged_decode` — one query per sequence. The key axis is cut into
  partitions (`choose_num_splits`); a sequence longer than one partition
  writes fp32 partials and a log-sum-exp per partition, and a second launch
  weighs them together.
* `paged_prefill` — packed queries, causal within each sequence's chunk,
  over the prefix the pool already holds. Its one-query sequences (decode
  rows beside chunks) run on the decode kernel, partitioned, in the same
  call.

bf16/fp16 pools with head_dim 64 or 128 and up to 16 query heads per KV head
run on the MFMA kernels; every other shape (fp32 above all) on a
general-shape kernel with fp32 arithmetic. Nothing here has a CPU fallback:
without the HIP library, or off a ROCm device, the calls raise.
"""

from __future__ import annotations

import functools

import torch

from liteinfer_amd import _native

# Keys per tile of the general-shape kernel, and the granularity of decode
# partitions. The MFMA kernels fold 32 keys per step whatever this is.
_BLOCK_KV = 64

# Query tokens per program of the general-shape prefill kernel, and its key
# tile (the reference's defaults, paged_kernels.py:113-114).
_PREFILL_BLOCK_Q = 16
_PREFILL_BLOCK_KV = 32

# The most programs choose_num_splits cuts one sequence's decode key loop into
# (the reference's cap, paged_kernels.py:129). The library's own schedules
# (the balanced split, and the fixed-length partitions of num_splits=None on
# the general-shape kernel) are not bound by it.
_MAX_SPLITS = 32

# Compute units assumed when no device is visible (MI355X: 8 XCDs x 32 CUs).
_MI355X_COMPUTE_UNITS = 256

_KERNELS = ("auto", "generic", "equal_splits")


def _flags(kernel: str) -> int:
    if kernel not in _KERNELS:
        raise ValueError(f"kernel must be one of {_KERNELS}, got {kernel!r}")
    return {"auto": 0, "generic": _native.LI_FLAG_FORCE_GENERIC, "equal_splits": _native.LI_FLAG_EQUAL_SPLITS}[kernel]


def _prefill_kernel(kernel: str) -> str:
    if kernel not in ("auto", "generic"):
        raise ValueError(f"kernel must be one of ('auto', 'generic'), got {kernel!r}")
    return kernel


@functools.cache
def _compute_unit_count(device_index: int) -> int:
    """Compute units of this device. Cached: the choice below is made per layer per step."""
    if torch.cuda.is_available():
        return torch.cuda.get_device_properties(device_index).multi_processor_count
    return _MI355X_COMPUTE_UNITS


def choose_num_splits(
    batch: int,
    num_kv_heads: int,
    max_context: int,
    device_index: int,
    block_kv: int = _BLOCK_KV,
    num_cus: int | None = None,
) -> int:
    """How many programs to cut each sequence's decode key loop into.

    The reference's rule (paged_kernels.py:645-693), computed by the library
    (`li_choose_num_splits`) with the device's compute units for SMs: a
    context of fewer than four `block_kv` tiles is not cut; otherwise the
    count that brings the grid of ``batch * num_kv_heads`` programs up to two
    per CU, at most one per tile and at most `_MAX_SPLITS`. The answer is a
    function of host integers only (`max_context` is the slot table's width),
    so a captured graph keeps the count it recorded. On bf16 / fp16 the
    decode kernel takes it as a scheduling hint (its balanced split runs
    whatever the count); the general-shape kernel and ``kernel="equal_splits"``
    cut each context into that many equal slices, as the reference does.
    """
    if num_cus is None:
        num_cus = _compute_unit_count(device_index)
    splits = _native.load().li_choose_num_splits(batch, num_kv_heads, max_context, num_cus, block_kv)
    if splits < 1:
        _native.check(splits, "choose_num_splits")
    return splits


def _require_device_tensors(*tensors: torch.Tensor) -> torch.device:
    device = tensors[0].device
    if device.type != "cuda" or torch.version.hip is None:
        raise RuntimeError(f"the paged kernels are HIP kernels and need a ROCm device, got {device}")
    for t in tensors:
        if t.device != device:
            raise ValueError(f"all operands must be on {device}, one is on {t.device}")
    return device


def _check_pools(key_pool: torch.Tensor, value_pool: torch.Tensor) -> None:
    if key_pool.stride() != value_pool.stride():
        raise ValueError("key and value pools must be laid out identically")
    if key_pool.dim() != 3 or key_pool.shape != value_pool.shape:
        raise ValueError(f"pools must be [num_slots, kv_heads, head_dim], got {tuple(key_pool.shape)}")
    if key_pool.stride(2) != 1:
        raise ValueError("the pools' head_dim axis must be contiguous")
    if key_pool.dtype != value_pool.dtype:
        raise ValueError("key and value pools must share a dtype")


_MAX_ATTEND_SLOTS = 1 << 31


def _check_attend_pools(key_pool: torch.Tensor, value_pool: torch.Tensor) -> None:
    """The pools' checks for an attention pass, whose kernels hold slot indices in 32 bits."""
    _check_pools(key_pool, value_pool)
    if key_pool.shape[0] >= _MAX_ATTEND_SLOTS:
        raise ValueError(f"the pools hold {key_pool.shape[0]} slots; paged attention reads pools "
                         f"of fewer than 2**31 slots")


def _kv_dtype_code(query: torch.Tensor, key_pool: torch.Tensor, k_scale: float, v_scale: float) -> int:
    """The pool's element type code: the query's, or fp8 (with checked scales)."""
    if _is_fp8(key_pool):
        if query.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError(f"an fp8 pool is read with bfloat16 or float16 queries, not {query.dtype}")
        _check_scales(k_scale, v_scale)
        return _native.LI_FP8_E4M3
    if query.dtype != key_pool.dtype:
        raise ValueError(f"query dtype {query.dtype} does not match the pool's {key_pool.dtype}")
    return _native.dtype_code(query.dtype)


def _as_index(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    return t if t.dtype == dtype else t.to(dtype)


def _last_dim_contiguous(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


def _is_fp8(pool: torch.Tensor) -> bool:
    return pool.dtype == _native.FP8_POOL_DTYPE


def _check_scales(k_scale: float, v_scale: float) -> None:
    for name, value in (("k_scale", k_scale), ("v_scale", v_scale)):
        if not (value > 0 and value != float("inf")):
            raise ValueError(f"{name} must be finite and > 0, got {value}")


def bad_slots_pointer(bad_slots: torch.Tensor | None, device: torch.device) -> int | None:
    """Device address of a slot-write miss counter (None for no counter)."""
    if bad_slots is None:
        return None
    if bad_slots.dtype != torch.int32 or bad_slots.numel() < 1 or bad_slots.device != device:
        raise ValueError(f"bad_slots must be an int32 tensor of at least one element on {device}, "
                         f"got {bad_slots.dtype} {tuple(bad_slots.shape)} on {bad_slots.device}")
    return bad_slots.data_ptr()


def check_bad_slots(bad_slots: torch.Tensor) -> None:
    """Raise IndexError if slot writes counted into `bad_slots` missed the pool; reset it.

    Reading the counter synchronises with the writes already queued, so call
    it where the caller synchronises anyway (outside captured regions).
    """
    missed = int(bad_slots.reshape(-1)[0].item())
    if missed:
        bad_slots.zero_()
        raise IndexError(f"{missed} K/V slot writes named a slot outside the pool and were not stored")


def kv_scatter(
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    slots: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    bad_slots: torch.Tensor | None = None,
) -> None:
    """Store one K/V column per slot, in the order the pass holds its tokens.

    `k` and `v` are ``[B, H, T, D]`` (any strides); `slots` holds ``B * T``
    entries taken batch-major, ``[1, T]`` for a packed pass or ``[1, B]`` for a
    decode step (kv_cache.py:236-247). The pools are this layer's
    ``[num_slots, H, D]`` stores and are written in place, bit for bit — or,
    for an fp8 (``torch.float8_e4m3fn``) pool, each element quantised as
    ``e4m3(clamp(x * (1 / scale), +-448))`` with ``k_scale`` / ``v_scale``
    (the reference's planned storage-level quantisation, roadmap section 2.5).

    A slot outside ``[0, num_slots)`` is not written. torch's ``index_put_``
    raises for it; a kernel cannot, so when `bad_slots` (a one-element int32
    tensor on the pools' device) is given, the kernel adds the number of such
    tokens to it, and the caller reads it once it synchronises
    (`check_bad_slots`).
    """
    device = _require_device_tensors(key_pool, value_pool, slots, k, v)
    bad_ptr = bad_slots_pointer(bad_slots, device)
    _check_pools(key_pool, value_pool)
    if k.dim() != 4 or k.shape != v.shape:
        raise ValueError(f"k and v must both be [batch, heads, tokens, head_dim], got {tuple(k.shape)}, {tuple(v.shape)}")
    batch, heads, tokens, head_dim = k.shape
    if heads != key_pool.shape[1] or head_dim != key_pool.shape[2]:
        raise ValueError(f"k rows {heads}x{head_dim} do not match the pool's {tuple(key_pool.shape[1:])}")
    fp8 = _is_fp8(key_pool)
    if fp8:
        if k.dtype != v.dtype or k.dtype not in _native.DTYPE_CODES:
            raise ValueError(f"an fp8 pool takes float32 / float16 / bfloat16 k and v, got {k.dtype}, {v.dtype}")
        _check_scales(k_scale, v_scale)
    elif k.dtype != key_pool.dtype or v.dtype != key_pool.dtype:
        raise ValueError(f"k/v dtype {k.dtype} does not match the pool's {key_pool.dtype}")
    flat_slots = _as_index(slots.reshape(-1), torch.int64).contiguous()
    if flat_slots.numel() != batch * tokens:
        raise ValueError(f"{flat_slots.numel()} slots for {batch * tokens} tokens")
    lib = _native.load()
    if fp8:
        status = lib.li_kv_scatter_fp8(
            k.data_ptr(), v.data_ptr(),
            _native.i64_array(k.stride()), _native.i64_array(v.stride()),
            batch, tokens, flat_slots.data_ptr(),
            key_pool.data_ptr(), value_pool.data_ptr(),
            key_pool.shape[0], key_pool.stride(0), key_pool.stride(1),
            heads, head_dim, _native.dtype_code(k.dtype), float(k_scale), float(v_scale),
            bad_ptr, _native.stream_handle(device),
        )
        _native.check(status, "kv_scatter")
        return
    status = lib.li_kv_scatter(
        k.data_ptr(), v.data_ptr(),
        _native.i64_array(k.stride()), _native.i64_array(v.stride()),
        batch, tokens, flat_slots.data_ptr(),
        key_pool.data_ptr(), value_pool.data_ptr(),
        key_pool.shape[0], key_pool.stride(0), key_pool.stride(1),
        heads, head_dim, _native.dtype_code(key_pool.dtype),
        bad_ptr, _native.stream_handle(device),
    )
    _native.check(status, "kv_scatter")


def _decode_inputs(query, key_pool, value_pool, slot_table, context_lens, num_kv_groups, num_splits,
                   k_scale, v_scale):
    """paged_decode's argument checks (the reference's messages) and the layouts its kernels take."""
    if key_pool.stride() != value_pool.stride():
        raise ValueError("key and value pools must be laid out identically")
    if num_splits is not None and num_splits < 1:
        raise ValueError(f"num_splits must be >= 1, got {num_splits}")
    device = _require_device_tensors(query, key_pool, value_pool, slot_table, context_lens)
    _check_attend_pools(key_pool, value_pool)
    _, num_heads, head_dim = query.shape
    kv_code = _kv_dtype_code(query, key_pool, k_scale, v_scale)
    if num_heads % num_kv_groups != 0 or num_heads // num_kv_groups != key_pool.shape[1]:
        raise ValueError(
            f"{num_heads} query heads in groups of {num_kv_groups} do not match {key_pool.shape[1]} KV heads"
        )
    if head_dim != key_pool.shape[2]:
        raise ValueError(f"query head_dim {head_dim} does not match the pool's {key_pool.shape[2]}")
    query = _last_dim_contiguous(query)
    slot_table = _as_index(slot_table, torch.int64)
    if slot_table.stride(-1) != 1:
        slot_table = slot_table.contiguous()
    context_lens = _as_index(context_lens, torch.int32).contiguous()
    return device, query, slot_table, context_lens, kv_code


@functools.lru_cache(maxsize=4096)
def _decode_workspace_bytes(batch: int, num_heads: int, num_kv_heads: int, head_dim: int, max_context: int,
                            num_splits: int, device_index: int, block_kv: int) -> int:
    """li_paged_decode_plan's workspace size for one shape: a function of these host integers only, so it
    is asked once per shape (a decode step calls it once per layer with the same shape)."""
    parts, plen, need = _native.ctypes.c_int(), _native.ctypes.c_int(), _native.ctypes.c_size_t()
    status = _native.load().li_paged_decode_plan(
        batch, num_heads, num_kv_heads, head_dim, max_context, num_splits, _compute_unit_count(device_index),
        block_kv, _native.ctypes.byref(parts), _native.ctypes.byref(plen), _native.ctypes.byref(need))
    _native.check(status, "paged_decode")
    return need.value


def paged_decode(
    query: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    slot_table: torch.Tensor,
    context_lens: torch.Tensor,
    scaling: float,
    num_kv_groups: int,
    block_kv: int = _BLOCK_KV,
    num_splits: int | None = None,
    *,
    kernel: str = "auto",
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    new_key: torch.Tensor | None = None,
    new_value: torch.Tensor | None = None,
) -> torch.Tensor:
    """Attend one query per sequence over the KV each sequence's slots address.

    Args:
        query: ``[batch, num_heads, head_dim]`` — the decode token's queries.
        key_pool: this layer's flat key store, ``[num_slots, num_kv_heads, head_dim]``.
        value_pool: the matching value store.
        slot_table: ``[batch, max_context]`` physical slot per logical position,
            left-aligned; columns past a row's context are never read.
        context_lens: ``[batch]`` real cached tokens per sequence.
        scaling: softmax scale, normally ``head_dim ** -0.5``.
        num_kv_groups: query heads per KV head.
        block_kv: key tile of the general-shape kernel and the granularity of
            the chosen partitions.
        num_splits: how many slices each sequence's keys are cut into. On the
            MFMA kernel (bf16 / fp16) this is a scheduling hint: it runs its
            balanced split, equal keys per wave across the whole batch, for
            any value (or, for a slot table narrow enough, one work-group per
            sequence and KV head in a single launch). On the general-shape kernel, and on the MFMA kernel
            with ``kernel="equal_splits"``, an integer is the reference's rule
            (each context cut into that many equal slices) and ``None`` picks
            fixed-length partitions. The result is the same attention either
            way, within fp32 rounding of the partial combine.
        kernel: ``"auto"`` (MFMA where it applies), ``"generic"`` (the
            general-shape kernel) or ``"equal_splits"`` (MFMA, splits pinned).
        k_scale, v_scale: the scales of an fp8 (``torch.float8_e4m3fn``) pool,
            whose rows hold K / k_scale and V / v_scale (`kv_scatter`); the
            attention is over the dequantised rows. fp8 pools run on the MFMA
            kernel (bf16 / fp16 queries, head_dim 128). Ignored otherwise.
        new_key, new_value: each sequence's newest K / V rows, ``[batch,
            num_kv_heads, head_dim]`` in the query's dtype, written into the
            pool at the slot of its last context position (the decode
            step's ``KVCache.scatter`` at ``newest_slots``, kv_cache.py:236-253)
            before the attention reads it: one launch where the head-grouped
            or the short kernel serves the shape over a 16-bit pool, a write
            launch first elsewhere. That slot
            must belong to no other sequence's context in the call (as every
            slot a `KVCache` hands out does).

    Returns:
        ``[batch, num_heads, head_dim]``, same dtype as ``query``.
    """
    device, query, slot_table, context_lens, kv_code = _decode_inputs(
        query, key_pool, value_pool, slot_table, context_lens, num_kv_groups, num_splits, k_scale, v_scale)
    batch, num_heads, head_dim = query.shape
    num_kv_heads = key_pool.shape[1]
    max_context = slot_table.shape[1]
    if (new_key is None) != (new_value is None):
        raise ValueError("give both new_key and new_value, or neither")
    if new_key is not None:
        want = (batch, num_kv_heads, head_dim)
        for name, t in (("new_key", new_key), ("new_value", new_value)):
            if tuple(t.shape) != want or t.dtype != query.dtype or t.device != query.device:
                raise ValueError(f"{name} must be {list(want)} {query.dtype} on {query.device}, "
                                 f"got {list(t.shape)} {t.dtype} on {t.device}")
        new_key, new_value = _last_dim_contiguous(new_key), _last_dim_contiguous(new_value)
        if new_key.stride() != new_value.stride():
            new_key, new_value = new_key.contiguous(), new_value.contiguous()

    lib = _native.load()
    need = _decode_workspace_bytes(batch, num_heads, num_kv_heads, head_dim, max_context, num_splits or 0,
                                   device.index or 0, block_kv)
    out = torch.empty_like(query)
    workspace = torch.empty(need, dtype=torch.uint8, device=device) if need else None
    status = lib.li_paged_decode_write(
        query.data_ptr(), query.stride(0), query.stride(1),
        key_pool.data_ptr(), value_pool.data_ptr(), key_pool.stride(0), key_pool.stride(1),
        slot_table.data_ptr(), slot_table.stride(0), max_context, context_lens.data_ptr(),
        new_key.data_ptr() if new_key is not None else None,
        new_value.data_ptr() if new_value is not None else None,
        new_key.stride(0) if new_key is not None else 0, new_key.stride(1) if new_key is not None else 0,
        key_pool.shape[0], None,
        out.data_ptr(), out.stride(0), out.stride(1),
        batch, num_heads, num_kv_heads, head_dim, float(scaling),
        num_splits or 0, block_kv,
        workspace.data_ptr() if workspace is not None else None, need,
        _native.dtype_code(query.dtype), kv_code, float(k_scale), float(v_scale),
        _flags(kernel), _native.stream_handle(device),
    )
    _native.check(status, "paged_decode")
    return out


def paged_decode_noalloc(
    query: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    slot_table: torch.Tensor,
    context_lens: torch.Tensor,
    scaling: float,
    num_kv_groups: int,
    block_kv: int = _BLOCK_KV,
    num_splits: int | None = None,
    *,
    out: torch.Tensor,
    kernel: str = "auto",
) -> torch.Tensor:
    """`paged_decode` through the entry point that allocates nothing
    (``li_paged_decode_noalloc``): the partials live in a device array the
    library holds, so the call needs no workspace. ``out`` (``[batch,
    num_heads, head_dim]``, the query's dtype, last axis contiguous) receives
    the result. Raises ValueError when the call needs more scratch than the
    library holds. Calls that overlap on one GPU share the scratch and race.
    No counterpart in the reference.
    """
    device, query, slot_table, context_lens, kv_code = _decode_inputs(
        query, key_pool, value_pool, slot_table, context_lens, num_kv_groups, num_splits, 1.0, 1.0)
    if kv_code != _native.dtype_code(query.dtype):
        raise ValueError("paged_decode_noalloc takes a pool of the query's dtype")
    if out.shape != query.shape or out.dtype != query.dtype or out.device != query.device or out.stride(-1) != 1:
        raise ValueError("out must match the query's shape, dtype and device, with a contiguous last axis")
    batch, num_heads, head_dim = query.shape
    lib = _native.load()
    status = lib.li_paged_decode_noalloc(
        query.data_ptr(), query.stride(0), query.stride(1),
        key_pool.data_ptr(), value_pool.data_ptr(), key_pool.stride(0), key_pool.stride(1),
        slot_table.data_ptr(), slot_table.stride(0), slot_table.shape[1],
        context_lens.data_ptr(), out.data_ptr(), out.stride(0), out.stride(1),
        batch, num_heads, key_pool.shape[1], head_dim, float(scaling),
        num_splits or 0, block_kv, _native.dtype_code(query.dtype), _flags(kernel),
        _native.stream_handle(device),
    )
    _native.check(status, "paged_decode_noalloc")
    return out


@functools.lru_cache(maxsize=4096)
def _prefill_workspace_bytes(batch: int, num_heads: int, num_kv_heads: int, head_dim: int, max_context: int,
                             device_index: int) -> int:
    """li_paged_prefill_plan's workspace size for one shape (host integers only; asked once per shape)."""
    need = _native.ctypes.c_size_t()
    status = _native.load().li_paged_prefill_plan(batch, num_heads, num_kv_heads, head_dim, max_context,
                                                  _compute_unit_count(device_index), _native.ctypes.byref(need))
    _native.check(status, "paged_prefill")
    return need.value


def paged_prefill(
    query: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    slot_table: torch.Tensor,
    context_lens: torch.Tensor,
    query_start_loc: torch.Tensor,
    max_query_len: int,
    scaling: float,
    num_kv_groups: int,
    block_kv: int = _PREFILL_BLOCK_KV,
    block_q: int = _PREFILL_BLOCK_Q,
    *,
    kernel: str = "auto",
    one_query_rows: bool | None = None,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Attend each sequence's chunk of queries over the KV its slots address, causally.

    Sequence ``i``'s queries are rows ``[query_start_loc[i], query_start_loc[i +
    1])`` of `query`, and they are the *last* positions of its context: the
    chunk's own K/V are already in the pool, written by the layer's payload just
    before this call (paged_kernels.py:821-882).

    Args:
        query: ``[total_queries, num_heads, head_dim]``, sequences end to end,
            any strides with the last axis contiguous.
        key_pool: this layer's flat key store, ``[num_slots, num_kv_heads, head_dim]``.
        value_pool: the matching value store.
        slot_table: ``[batch, max_context]`` physical slot per logical position.
        context_lens: ``[batch]`` tokens each sequence holds, its chunk included.
        query_start_loc: ``[batch + 1]`` int32 prefix sums of the chunk lengths.
        max_query_len: longest chunk, which sizes the grid and so is a host int.
        scaling: softmax scale, normally ``head_dim ** -0.5``.
        num_kv_groups: query heads per KV head.
        block_kv, block_q: tiles of the general-shape kernel.
        kernel: ``"auto"`` (MFMA where it applies) or ``"generic"``.
        one_query_rows: whether any sequence brings a single query (``None``:
            unknown). The MFMA path hands those to the balanced decode split
            inside the prefill launch (its first work-groups fold them, then
            join the chunks). ``False`` lets the prefill kernel
            fold every sequence as query blocks and skips the split. Either
            way the result is the same attention.
        k_scale, v_scale: the scales of an fp8 pool (see `paged_decode`).
        out: where to write the result (the query's shape and dtype, last
            axis contiguous, any other strides); a new tensor when None.

    Returns:
        ``[total_queries, num_heads, head_dim]`` (`out`, or a new tensor with
        the strides of `query`).
    """
    if key_pool.stride() != value_pool.stride():
        raise ValueError("key and value pools must be laid out identically")
    device = _require_device_tensors(query, key_pool, value_pool, slot_table, context_lens, query_start_loc)
    _check_attend_pools(key_pool, value_pool)
    _, num_heads, head_dim = query.shape
    kv_code = _kv_dtype_code(query, key_pool, k_scale, v_scale)
    if num_heads % num_kv_groups != 0 or num_heads // num_kv_groups != key_pool.shape[1]:
        raise ValueError(
            f"{num_heads} query heads in groups of {num_kv_groups} do not match {key_pool.shape[1]} KV heads"
        )
    if head_dim != key_pool.shape[2]:
        raise ValueError(f"query head_dim {head_dim} does not match the pool's {key_pool.shape[2]}")
    query = _last_dim_contiguous(query)
    slot_table = _as_index(slot_table, torch.int64)
    if slot_table.stride(-1) != 1:
        slot_table = slot_table.contiguous()
    context_lens = _as_index(context_lens, torch.int32).contiguous()
    query_start_loc = _as_index(query_start_loc, torch.int32).contiguous()
    batch = context_lens.shape[0]
    if query_start_loc.shape[0] != batch + 1:
        raise ValueError(f"query_start_loc has {query_start_loc.shape[0]} entries for {batch} sequences")
    num_kv_heads = key_pool.shape[1]
    max_context = slot_table.shape[1]

    lib = _native.load()
    need = _prefill_workspace_bytes(batch, num_heads, num_kv_heads, head_dim, max_context, device.index or 0)
    if out is None:
        out = torch.empty_like(query)
    elif (out.shape != query.shape or out.dtype != query.dtype or out.device != query.device
          or out.stride(-1) != 1):
        raise ValueError("out must match the query's shape, dtype and device, with a contiguous last axis")
    workspace = torch.empty(need, dtype=torch.uint8, device=device) if need else None
    status = lib.li_paged_prefill_ex(
        query.data_ptr(), query.stride(0), query.stride(1),
        key_pool.data_ptr(), value_pool.data_ptr(), key_pool.stride(0), key_pool.stride(1),
        slot_table.data_ptr(), slot_table.stride(0), max_context,
        context_lens.data_ptr(), query_start_loc.data_ptr(), batch, int(max_query_len),
        out.data_ptr(), out.stride(0), out.stride(1),
        num_heads, num_kv_heads, head_dim, float(scaling), block_q, block_kv,
        workspace.data_ptr() if workspace is not None else None, need,
        _native.dtype_code(query.dtype), kv_code, float(k_scale), float(v_scale),
        _flags(_prefill_kernel(kernel)) | (_native.LI_FLAG_PREFILL_ONLY if one_query_rows is False else 0),
        _native.stream_handle(device),
    )
    _native.check(status, "paged_prefill")
    return out
