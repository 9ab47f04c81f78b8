"""The minimal engine's fused elementwise ops on a ROCm device (`li_add_rms_norm`, `li_silu_mul`).

Same results as the model's torch ops (liteinfer/models/llama.py:34-48,
:101-116) up to the order of the fp32 sum of squares and the exponential's
last bit; one launch each instead of a chain of torch kernels. Refuse what
they do not serve (ValueError); the model keeps its torch ops for CPU tensors.
"""

from __future__ import annotations

import torch

from liteinfer_amd import _native


def _rows(t: torch.Tensor, name: str) -> tuple[int, int]:
    if t.dim() < 1 or t.stride(-1) != 1:
        raise ValueError(f"{name} must have a contiguous last axis")
    flat = t.reshape(-1, t.shape[-1])
    if flat.data_ptr() != t.data_ptr() or (flat.shape[0] > 1 and t.dim() > 2 and not t.is_contiguous()):
        raise ValueError(f"{name} rows must be evenly strided")
    return flat.shape[0], (flat.stride(0) if flat.shape[0] > 1 else t.shape[-1])


def add_rms_norm(h: torch.Tensor, weight: torch.Tensor, eps: float, delta: torch.Tensor | None = None) -> torch.Tensor:
    """``h += delta`` in place (when given), then RMSNorm of h times `weight`; returns the normalised rows."""
    if h.dtype not in (torch.bfloat16, torch.float16) or weight.dtype != h.dtype or weight.shape != h.shape[-1:]:
        raise ValueError("add_rms_norm takes bf16 / f16 rows and a weight of their width and dtype")
    if delta is not None and (delta.shape != h.shape or delta.dtype != h.dtype):
        raise ValueError("delta must match h")
    rows, h_s = _rows(h, "h")
    d_s = _rows(delta, "delta")[1] if delta is not None else 0
    out = torch.empty(h.shape, dtype=h.dtype, device=h.device)
    status = _native.load().li_add_rms_norm(
        h.data_ptr(), delta.data_ptr() if delta is not None else None, weight.contiguous().data_ptr(),
        out.data_ptr(), rows, h.shape[-1], h_s, d_s, h.shape[-1], float(eps), _native.dtype_code(h.dtype),
        _native.stream_handle(h.device))
    _native.check(status, "add_rms_norm")
    return out


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """``silu(gate) * up`` of the fused projection's halves ``gate_up = [gate | up]``."""
    if gate_up.dtype not in (torch.bfloat16, torch.float16) or gate_up.shape[-1] % 2:
        raise ValueError("silu_mul takes bf16 / f16 rows of an even width")
    ffn = gate_up.shape[-1] // 2
    rows, gu_s = _rows(gate_up, "gate_up")
    out = torch.empty(*gate_up.shape[:-1], ffn, dtype=gate_up.dtype, device=gate_up.device)
    status = _native.load().li_silu_mul(gate_up.data_ptr(), out.data_ptr(), rows, ffn, gu_s, ffn,
                                        _native.dtype_code(gate_up.dtype), _native.stream_handle(gate_up.device))
    _native.check(status, "silu_mul")
    return out
