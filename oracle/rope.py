"""Rotary position embedding as liteinfer computes it — TEST INFRASTRUCTURE ONLY.

Restates `_rotate_half` / `_apply_rotary_pos_emb`
(liteinfer/models/llama.py:79-98): ``x * cos + rotate_half(x) * sin`` with
``rotate_half(x) = cat(-x[..., D/2:], x[..., :D/2])``, evaluated as the
reference's separate torch ops evaluate it — each product and the sum is
rounded to the tensor dtype (bf16 / fp16 round-to-nearest-even, fp32 IEEE).
Arrays are float32 numpy arrays holding values of the named dtype, or float64
for the exact (unrounded) rotation.
"""

from __future__ import annotations

import numpy as np

from oracle.addressing import scatter


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to `dtype` ("f32", "bf16", "f16"), returned as float32."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f32":
        return x
    if dtype == "f16":
        with np.errstate(over="ignore"):  # beyond fp16's range: inf, as torch gives
            return x.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
        return (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    raise ValueError(f"unknown dtype {dtype!r}")


def rotate_half(x: np.ndarray) -> np.ndarray:
    half = x.shape[-1] // 2
    return np.concatenate((-x[..., half:], x[..., :half]), axis=-1)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, dtype: str) -> np.ndarray:
    """``x * cos + rotate_half(x) * sin`` with the reference's roundings.

    ``dtype="f64"`` computes it exactly in float64 (no rounding).
    """
    if dtype == "f64":
        x, cos, sin = (np.asarray(a, dtype=np.float64) for a in (x, cos, sin))
        return x * cos + rotate_half(x) * sin
    x, cos, sin = (np.asarray(a, dtype=np.float32) for a in (x, cos, sin))
    a = round_to(x * cos, dtype)
    b = round_to(rotate_half(x) * sin, dtype)
    return round_to(a + b, dtype)


def rope_kv_write(q, k, v, cos, sin, slots, key_pool, value_pool, dtype: str):
    """q, k, v ``[B, H, T, D]``; cos / sin ``[B or 1, T, D]``.

    Returns (rotated q, key pool, value pool): the pools as copies with the
    rotated k and the unchanged v stored at `slots` (batch-major).
    """
    c = np.asarray(cos)[:, None]
    s = np.asarray(sin)[:, None]
    q_out = rope(q, c, s, dtype)
    k_out = rope(k, c, s, dtype)
    kp, vp = scatter(key_pool, value_pool, np.asarray(slots).reshape(-1), k_out, np.asarray(v, dtype=np.float32))
    return q_out, kp, vp
