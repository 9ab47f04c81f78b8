"""Paged KV cache: the block pool, its addressing, and the per-pass payloads."""

from liteinfer_amd.cache.block_pool import (
    BlockPool,
    BlockPoolExhaustedError,
    PackedAddresses,
    newest_slots,
    packed_addresses,
    slot_table,
)
from liteinfer_amd.cache.kv_cache import KVCache, KVPayload

__all__ = [
    "BlockPool",
    "BlockPoolExhaustedError",
    "KVCache",
    "KVPayload",
    "PackedAddresses",
    "newest_slots",
    "packed_addresses",
    "slot_table",
]
