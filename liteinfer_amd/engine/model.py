"""A random-initialised Llama-architecture model over the paged HIP path.

The end-to-end configuration (Llama-3-8B architecture: 32 layers, hidden 4096,
32 / 8 heads, head_dim 128, FFN 14336, vocab 128256, bf16) needs a model that
calls this build's attention the way liteinfer's `LlamaForCausalLM` does
(liteinfer/models/llama.py:34-270). No checkpoint can be fetched here, so the
weights are seeded random normals (std 0.02) — the arithmetic per token, and so
the throughput, is that of the real model.

Per layer: RMSNorm in fp32 (llama.py:34-48), one fused q/k/v projection (the
reference's three `nn.Linear`s stacked, the same products), RoPE and the KV
slot-write in one HIP launch (`payload.update_rotated`, the fused form of
llama.py:155-160), `paged_attention` (llama.py:161), the output projection,
RMSNorm and the SiLU-gated MLP (llama.py:101-112) with gate and up stacked.
Projections are torch GEMMs (hipBLASLt); attention, RoPE and the slot-write are
this library's kernels.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from liteinfer_amd.attention import paged_attention


@dataclass(frozen=True)
class LlamaShape:
    hidden_size: int = 4096
    num_layers: int = 32
    num_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 14336
    vocab_size: int = 128256
    rms_norm_eps: float = 1e-5
    rope_theta: float = 500000.0

    @property
    def groups(self) -> int:
        return self.num_heads // self.num_kv_heads


LLAMA_3_8B = LlamaShape()


class _Layer:
    def __init__(self, shape: LlamaShape, gen: torch.Generator, device, dtype, std: float) -> None:
        h, d = shape.hidden_size, shape.head_dim
        qkv_out = (shape.num_heads + 2 * shape.num_kv_heads) * d

        def w(out_f, in_f):
            return (torch.randn(out_f, in_f, generator=gen, device=device, dtype=torch.float32) * std).to(dtype)

        self.attn_norm = torch.ones(h, device=device, dtype=dtype)
        self.w_qkv = w(qkv_out, h)
        self.w_o = w(h, shape.num_heads * d)
        self.mlp_norm = torch.ones(h, device=device, dtype=dtype)
        self.w_gate_up = w(2 * shape.intermediate_size, h)
        self.w_down = w(h, shape.intermediate_size)


class RandomLlama:
    """Seeded random weights of a Llama architecture; `forward` mirrors LlamaForCausalLM.forward."""

    def __init__(self, shape: LlamaShape = LLAMA_3_8B, device="cuda", dtype=torch.bfloat16, seed: int = 0,
                 std: float = 0.02) -> None:
        self.shape = shape
        self.device = torch.device(device)
        self.dtype = dtype
        gen = torch.Generator(device=self.device).manual_seed(seed)
        self.embed = (torch.randn(shape.vocab_size, shape.hidden_size, generator=gen, device=self.device,
                                  dtype=torch.float32) * std).to(dtype)
        self.layers = [_Layer(shape, gen, self.device, dtype, std) for _ in range(shape.num_layers)]
        self.final_norm = torch.ones(shape.hidden_size, device=self.device, dtype=dtype)
        self.lm_head = (torch.randn(shape.vocab_size, shape.hidden_size, generator=gen, device=self.device,
                                    dtype=torch.float32) * std).to(dtype)
        # 16-bit models on the GPU run the residual adds, RMSNorms and SiLU
        # gate as fused HIP kernels (engine/ops.py); fp32 models (the exact
        # references of the engine tests) keep the torch ops.
        self._fused_ops = None
        if (self.device.type == "cuda" and dtype in (torch.bfloat16, torch.float16)
                and shape.hidden_size % 8 == 0 and shape.hidden_size <= 8192 and shape.intermediate_size % 8 == 0):
            from liteinfer_amd.engine import ops

            self._fused_ops = ops
        d = shape.head_dim
        # The "default" rope type: no frequency scaling (llama.py:62-67).
        self.inv_freq = 1.0 / (shape.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float32, device=self.device) / d))
        self.scaling = d ** -0.5

    def parameter_bytes(self) -> int:
        tensors = [self.embed, self.lm_head, self.final_norm]
        for layer in self.layers:
            tensors += [layer.attn_norm, layer.w_qkv, layer.w_o, layer.mlp_norm, layer.w_gate_up, layer.w_down]
        return sum(t.numel() * t.element_size() for t in tensors)

    def _rms_norm(self, x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
        """fp32 RMSNorm, cast back before the weight (llama.py:42-48)."""
        xf = x.to(torch.float32)
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.shape.rms_norm_eps)
        return weight * xf.to(x.dtype)

    def _rotary(self, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """cos / sin ``[B, T, D]`` in the model dtype, computed in fp32 (llama.py:70-78)."""
        freqs = positions[..., None].to(torch.float32) * self.inv_freq
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(self.dtype), emb.sin().to(self.dtype)

    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor, payload,
                logits_positions: torch.Tensor | None = None) -> torch.Tensor:
        """Logits of the selected rows.

        input_ids / positions: ``[B, T]`` (``[1, T]`` for a packed pass,
        ``[B, 1]`` for a decode step). `payload` is a KV payload
        (`KVCache.make_packed_payload` / `make_decode_payload`).
        `logits_positions` picks rows of a packed pass (each sequence's last
        token); ``None`` takes the last position of every batch row.
        """
        s = self.shape
        batch, tokens = input_ids.shape
        h = F.embedding(input_ids, self.embed)
        cos, sin = self._rotary(positions)
        nq, nkv = s.num_heads, s.num_kv_heads
        fused = self._fused_ops
        delta = None  # the MLP output not yet added to the residual stream
        for idx, layer in enumerate(self.layers):
            if fused:
                x = fused.add_rms_norm(h, layer.attn_norm, s.rms_norm_eps, delta)
            else:
                x = self._rms_norm(h, layer.attn_norm)
            qkv = F.linear(x, layer.w_qkv).view(batch, tokens, nq + 2 * nkv, s.head_dim)
            q = qkv[:, :, :nq].transpose(1, 2)
            k = qkv[:, :, nq:nq + nkv].transpose(1, 2)
            v = qkv[:, :, nq + nkv:].transpose(1, 2)
            q, kv = payload.update_rotated(q, k, v, cos, sin, idx)
            attn = paged_attention(q, kv, self.scaling, s.groups)
            attn = attn.transpose(1, 2).reshape(batch, tokens, nq * s.head_dim)
            if fused:
                x = fused.add_rms_norm(h, layer.mlp_norm, s.rms_norm_eps, F.linear(attn, layer.w_o))
                delta = F.linear(fused.silu_mul(F.linear(x, layer.w_gate_up)), layer.w_down)
            else:
                h = h + F.linear(attn, layer.w_o)
                x = self._rms_norm(h, layer.mlp_norm)
                gate, up = F.linear(x, layer.w_gate_up).chunk(2, dim=-1)
                h = h + F.linear(F.silu(gate) * up, layer.w_down)
        if fused:
            h = fused.add_rms_norm(h, self.final_norm, s.rms_norm_eps, delta)
        else:
            h = self._rms_norm(h, self.final_norm)
        rows = h[0, logits_positions] if logits_positions is not None else h[:, -1]
        return F.linear(rows, self.lm_head)
