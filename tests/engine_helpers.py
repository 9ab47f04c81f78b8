"""Shared pieces of the engine tests: a dense reference forward, prompts, and a logits recorder."""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from liteinfer_amd.engine.llm import LLM
from liteinfer_amd.engine.model import RandomLlama


def dense_logits(model: RandomLlama, tokens: list[int], dtype: torch.dtype | None = None) -> torch.Tensor:
    """Last-position logits of a cache-free forward over the whole sequence.

    `dtype` None computes in the model's dtype (attention scores in fp32);
    torch.float32 runs the same weights, widened exactly, entirely in fp32.
    """
    s = model.shape
    dt = dtype or model.dtype
    W = lambda w: w.to(dt)
    ids = torch.tensor([tokens], device=model.device)
    t = len(tokens)
    h = F.embedding(ids, W(model.embed))
    pos = torch.arange(t, device=model.device)[None]
    freqs = pos[..., None].float() * model.inv_freq
    emb = torch.cat((freqs, freqs), -1)
    cos, sin = emb.cos().to(dt)[:, None], emb.sin().to(dt)[:, None]

    def rot(x):
        half = x.shape[-1] // 2
        return x * cos + torch.cat((-x[..., half:], x[..., :half]), -1) * sin

    def norm(x, w):
        xf = x.float()
        return W(w) * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + s.rms_norm_eps)).to(x.dtype)

    mask = torch.ones(t, t, dtype=torch.bool, device=model.device).tril()
    for layer in model.layers:
        x = norm(h, layer.attn_norm)
        qkv = F.linear(x, W(layer.w_qkv)).view(1, t, s.num_heads + 2 * s.num_kv_heads, s.head_dim)
        q = rot(qkv[:, :, :s.num_heads].transpose(1, 2)).float()
        k = rot(qkv[:, :, s.num_heads:s.num_heads + s.num_kv_heads].transpose(1, 2)).float()
        v = qkv[:, :, s.num_heads + s.num_kv_heads:].transpose(1, 2).float()
        k = k.repeat_interleave(s.groups, dim=1)
        v = v.repeat_interleave(s.groups, dim=1)
        scores = (q @ k.transpose(-1, -2)) / math.sqrt(s.head_dim)
        attn = scores.masked_fill(~mask, float("-inf")).softmax(-1) @ v
        attn = attn.to(dt).transpose(1, 2).reshape(1, t, -1)
        h = h + F.linear(attn, W(layer.w_o))
        x = norm(h, layer.mlp_norm)
        gate, up = F.linear(x, W(layer.w_gate_up)).chunk(2, -1)
        h = h + F.linear(F.silu(gate) * up, W(layer.w_down))
    h = norm(h, model.final_norm)
    return F.linear(h[0, -1], W(model.lm_head))


def random_prompts(n, lo, hi, vocab, seed=0):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (n,), generator=g).tolist()
    return [torch.randint(0, vocab, (m,), generator=g).tolist() for m in lens]


def record_logits(llm: LLM) -> list[tuple[list[str], torch.Tensor]]:
    """Make `llm` keep, for every step, the request ids it samples and those rows' logits (fp32 copies)."""
    steps: list[tuple[list[str], torch.Tensor]] = []
    execute = llm.runner.execute

    def recording(seqs, num_tokens, pending=None):
        logits = execute(seqs, num_tokens, pending)
        rows = [i for i, s in enumerate(seqs) if s.num_computed_tokens == len(s)]
        if rows:
            picked = logits.index_select(0, torch.tensor(rows, device=logits.device)).float()
            steps.append(([seqs[i].request_id for i in rows], picked))
        return logits

    llm.runner.execute = recording
    return steps


def sampled_logits(steps, request_id: str) -> list[torch.Tensor]:
    """The logits each generated token of `request_id` was taken from, in order."""
    return [logits[ids.index(request_id)] for ids, logits in steps if request_id in ids]


def check_tracks_dense(model: RandomLlama, prompt: list[int], out: list[int], engine_logits: list[torch.Tensor],
                       slack: float = 2.0, tokens: int | None = None) -> list[tuple[float, float]]:
    """The engine against exact arithmetic, for each of the first `tokens` generated tokens.

    The reference is the same weights run entirely in fp32. The engine's
    logits error must be within `slack` times the error of a plain dense
    forward in the model's dtype (what that dtype's rounding costs anyway),
    and the token it picked must score within twice its own error of the
    fp32 maximum (a different token only where rounding can tie them).
    Returns the (engine, dense) max-abs errors per token.
    """
    seq = list(prompt)
    errors = []
    for i, tok in enumerate(out[: tokens or len(out)]):
        exact = dense_logits(model, seq, torch.float32).float()
        plain = dense_logits(model, seq).float()
        got = engine_logits[i].to(exact.device)
        err = (got - exact).abs().max().item()
        ref_err = (plain - exact).abs().max().item()
        errors.append((err, ref_err))
        assert torch.isfinite(got).all()
        assert err <= slack * ref_err + 1e-6, (i, err, ref_err)
        assert exact[tok].item() >= exact.max().item() - 2 * err, (i, tok, int(exact.argmax()), err)
        seq.append(tok)
    return errors
