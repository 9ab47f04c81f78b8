"""The KV block pool and the addresses the kernels read it by.

Layout and addressing are liteinfer's (liteinfer/cache/block_pool.py), kept
identical because the kernels, the scheduler and a captured decode graph all
depend on them:

* One pool serves every layer: keys and values are each
  ``[num_layers, num_blocks * block_size, num_kv_heads, head_dim]`` (:63),
  zero-initialised. A layer's view is a flat run of token *slots*
  ``[num_slots, num_kv_heads, head_dim]``, and token ``t`` of block ``b`` lives
  in slot ``b * block_size + t``. On MI355X the rows of one slot across all KV
  heads are one contiguous ``num_kv_heads * head_dim`` run (2 KiB at 8 x 128
  bf16), which the kernels read with 16-byte loads.
* Addresses are per token: a ``[B, W]`` int64 slot table, left-aligned, whose
  columns at or past a row's context length are never read.
"""

from __future__ import annotations

from collections.abc import Sequence
from typing import NamedTuple

import numpy as np
import torch


class BlockPoolExhaustedError(RuntimeError):
    """The pool cannot hold what was asked of it."""


CACHE_QUANT_FORMATS = (None, "fp8")


class BlockPool:
    """Fixed-size pool of KV blocks shared by all layers, with one free-list.

    ``cache_quant="fp8"`` stores K and V as OCP e4m3 (``torch.float8_e4m3fn``),
    one byte per element: each row is written as ``x / k_scale`` (``v_scale``
    for V) rounded to e4m3 and read back times the scale — the reference's
    planned storage-level quantisation (docs/roadmap.md section 2.5, behind a
    ``cache_quant`` flag). ``dtype`` stays the dtype K/V arrive and leave in.
    """

    def __init__(
        self,
        num_blocks: int,
        block_size: int,
        num_layers: int,
        num_kv_heads: int,
        head_dim: int,
        dtype: torch.dtype,
        device: torch.device,
        cache_quant: str | None = None,
        k_scale: float = 1.0,
        v_scale: float = 1.0,
    ) -> None:
        if cache_quant not in CACHE_QUANT_FORMATS:
            raise ValueError(f"cache_quant must be one of {CACHE_QUANT_FORMATS}, got {cache_quant!r}")
        if not (k_scale > 0 and v_scale > 0):
            raise ValueError(f"k_scale and v_scale must be > 0, got {k_scale}, {v_scale}")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.cache_quant = cache_quant
        self.k_scale = float(k_scale)
        self.v_scale = float(v_scale)
        storage = torch.float8_e4m3fn if cache_quant == "fp8" else dtype
        shape = (num_layers, num_blocks * block_size, num_kv_heads, head_dim)
        self._keys = torch.zeros(shape, dtype=storage, device=device)
        self._values = torch.zeros(shape, dtype=storage, device=device)
        self._free_blocks: list[int] = list(range(num_blocks))
        # Count of slot writes that named a slot outside the pool. The device
        # kernels skip such a write and add to this counter instead of raising.
        self.bad_slots = torch.zeros(1, dtype=torch.int32, device=device)

    @property
    def nbytes(self) -> int:
        """Device bytes held by keys and values together."""
        return 2 * self._keys.numel() * self._keys.element_size()

    @property
    def device(self) -> torch.device:
        return self._keys.device

    @property
    def num_free_blocks(self) -> int:
        return len(self._free_blocks)

    def allocate(self) -> int:
        """Pop a free block index; raises BlockPoolExhaustedError when none is left."""
        if not self._free_blocks:
            raise BlockPoolExhaustedError(
                f"KV block pool exhausted: all {self.num_blocks} blocks are in use. "
                "Increase num_gpu_blocks or reduce max_num_seqs / max_model_len."
            )
        return self._free_blocks.pop()

    def free(self, block_idx: int) -> None:
        self._free_blocks.append(block_idx)

    def check_slot_writes(self) -> None:
        """Raise IndexError if any slot write since the last check missed the pool.

        Reads a device counter, so it waits for the writes already queued;
        call it where the caller synchronises anyway, never under capture.
        """
        self.raise_if_missed(int(self.bad_slots.item()))

    def raise_if_missed(self, missed: int) -> None:
        """`check_slot_writes` on a count already read from the device counter."""
        if missed:
            self.bad_slots.zero_()
            raise IndexError(f"{missed} K/V slot writes named a slot outside the pool's "
                             f"{self.num_blocks * self.block_size} slots and were not stored")

    def slots(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        """This layer's flat key/value stores, ``[num_slots, num_kv_heads, head_dim]``."""
        return self._keys[layer_idx], self._values[layer_idx]


_copy_streams: dict[int, torch.cuda.Stream] = {}


def to_device(values, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    """`values` (nested lists or a numpy array) as a tensor on `device`, ready for the current stream.

    To a ROCm device the host copy goes through pinned memory with an
    asynchronous copy on a copy stream of its own, which the current stream
    then waits for: the host does not wait for the work already queued (a
    copy from pageable memory would), and the copy runs beside that work
    instead of after it, so an engine stages a step's addresses while the
    previous step still runs and the step starts without waiting for them.
    torch's pinned-memory cache keeps the staging buffer until the copy has
    read it; the result is marked as used by the current stream. Refused
    inside a graph capture: a captured copy would read the staging buffer
    again on every replay, after the cache has handed it out anew.
    """
    host = torch.from_numpy(values) if isinstance(values, np.ndarray) else torch.tensor(values, dtype=dtype)
    host = host.to(dtype)
    if device.type != "cuda":
        return host.to(device)
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("to_device: host values cannot be staged inside a graph capture; "
                           "copy them into the graph's static buffers before it")
    host = host.pin_memory()
    index = device.index if device.index is not None else torch.cuda.current_device()
    side = _copy_streams.get(index)
    if side is None:
        side = _copy_streams[index] = torch.cuda.Stream(device=index)  # default priority
    current = torch.cuda.current_stream(index)
    # `out` comes from the copy stream's own memory pool, whose blocks are
    # handed out again only once every stream marked as using them is done,
    # so the copy needs to wait for nothing the current stream has queued.
    with torch.cuda.stream(side):
        out = host.to(device, non_blocking=True)
    current.wait_stream(side)
    out.record_stream(current)
    return out


def _block_matrix(
    block_tables: Sequence[Sequence[int]], device: torch.device, *leading: Sequence[int]
) -> torch.Tensor:
    """Block tables padded with block 0 into one ``[B, len(leading) + max_blocks]`` int64 tensor.

    `leading` columns (one integer per sequence each) ride in front, so the
    whole batch crosses to the device in a single transfer (block_pool.py:103-121).
    """
    width = max(len(table) for table in block_tables)
    lead = len(leading)
    matrix = np.zeros((len(block_tables), lead + width), dtype=np.int64)
    for j, column in enumerate(leading):
        matrix[:, j] = column
    for i, table in enumerate(block_tables):
        matrix[i, lead:lead + len(table)] = table
    return to_device(matrix, torch.int64, device)


def _position_slots(blocks: torch.Tensor, width: int, block_size: int) -> torch.Tensor:
    """``[B, width]``: slot of logical position p = blocks[:, p // bs] * bs + p % bs (block_pool.py:124-132)."""
    positions = torch.arange(width, device=blocks.device)
    return blocks.index_select(1, positions // block_size) * block_size + positions % block_size


def slot_table(
    block_tables: Sequence[Sequence[int]],
    totals: Sequence[int],
    block_size: int,
    device: torch.device,
) -> torch.Tensor:
    """Each sequence's positions ``[0, totals[i])`` as pool slots, ``[B, max(totals)]`` (block_pool.py:135-148)."""
    return _position_slots(_block_matrix(block_tables, device), max(totals), block_size)


def newest_slots(
    block_tables: Sequence[Sequence[int]],
    positions: Sequence[int],
    block_size: int,
    device: torch.device,
) -> torch.Tensor:
    """The slot of one position per sequence, as ``[1, B]``, computed on the host (block_pool.py:151-170)."""
    slots = []
    for table, position in zip(block_tables, positions, strict=True):
        block, offset = divmod(position, block_size)
        slots.append(table[block] * block_size + offset)
    return to_device([slots], torch.long, device)


class PackedAddresses(NamedTuple):
    """Every address a packed pass needs (block_pool.py:173-188)."""

    slots: torch.Tensor
    """``[1, total]`` slot each token of the run is written to."""
    positions: torch.Tensor
    """``[1, total]`` logical position of each token (what RoPE reads)."""
    query_start_loc: torch.Tensor
    """``[B + 1]`` int32 prefix sums of the counts."""
    slot_table: torch.Tensor
    """``[B, max(start + count)]`` slots of each sequence's whole context."""
    context_lens: torch.Tensor
    """``[B]`` int32 start + count."""


def packed_addresses(
    block_tables: Sequence[Sequence[int]],
    starts: Sequence[int],
    counts: Sequence[int],
    block_size: int,
    device: torch.device,
) -> PackedAddresses:
    """Addresses of a pass where sequence i brings positions ``[starts[i], starts[i] + counts[i])``.

    One transfer carries the counts, starts and block tables; everything else
    is derived on the device (block_pool.py:191-223).
    """
    moved = _block_matrix(block_tables, device, counts, starts)
    count, start, blocks = moved[:, 0], moved[:, 1], moved[:, 2:]
    total = sum(counts)
    run_ends = torch.cumsum(count, 0)
    owner = torch.repeat_interleave(torch.arange(len(counts), device=device), count, output_size=total)
    offset_in_run = torch.arange(total, device=device) - (run_ends - count)[owner]
    positions = start[owner] + offset_in_run
    widest = max(s + c for s, c in zip(starts, counts, strict=True))
    table = _position_slots(blocks, widest, block_size)
    return PackedAddresses(
        slots=table[owner, positions].unsqueeze(0),
        positions=positions.unsqueeze(0),
        query_start_loc=torch.cat([run_ends.new_zeros(1), run_ends]).to(torch.int32),
        slot_table=table,
        context_lens=(start + count).to(torch.int32),
    )
