"""The minimal engine generates what a dense, cache-free forward of the same model generates.

A small Llama-shaped model runs through the engine (continuous batching,
chunked prefill, packed passes with decode rows, captured decode graphs, the
fused RoPE + slot-write, paged decode and prefill) and through a plain torch
forward over each whole sequence with causal attention (the textbook
definition the reference's model computes, liteinfer/models/llama.py:34-270);
greedy continuations must agree token for token in fp32, and the first step's
logits must agree within bf16 rounding in bf16.
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from liteinfer_amd.engine.llm import LLM, EngineConfig
from liteinfer_amd.engine.model import LlamaShape, RandomLlama

pytestmark = pytest.mark.gpu

TINY = LlamaShape(hidden_size=512, num_layers=2, num_heads=8, num_kv_heads=2, head_dim=64,
                  intermediate_size=1024, vocab_size=1000)


def _dense_logits(model: RandomLlama, tokens: list[int]) -> torch.Tensor:
    """Last-position logits of a cache-free forward over the whole sequence."""
    s = model.shape
    ids = torch.tensor([tokens], device=model.device)
    t = len(tokens)
    h = F.embedding(ids, model.embed)
    pos = torch.arange(t, device=model.device)[None]
    freqs = pos[..., None].float() * model.inv_freq
    emb = torch.cat((freqs, freqs), -1)
    cos, sin = emb.cos().to(model.dtype)[:, None], emb.sin().to(model.dtype)[:, None]

    def rot(x):
        half = x.shape[-1] // 2
        return x * cos + torch.cat((-x[..., half:], x[..., :half]), -1) * sin

    def norm(x, w):
        xf = x.float()
        return w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + s.rms_norm_eps)).to(x.dtype)

    mask = torch.ones(t, t, dtype=torch.bool, device=model.device).tril()
    for layer in model.layers:
        x = norm(h, layer.attn_norm)
        qkv = F.linear(x, layer.w_qkv).view(1, t, s.num_heads + 2 * s.num_kv_heads, s.head_dim)
        q = rot(qkv[:, :, :s.num_heads].transpose(1, 2)).float()
        k = rot(qkv[:, :, s.num_heads:s.num_heads + s.num_kv_heads].transpose(1, 2)).float()
        v = qkv[:, :, s.num_heads + s.num_kv_heads:].transpose(1, 2).float()
        k = k.repeat_interleave(s.groups, dim=1)
        v = v.repeat_interleave(s.groups, dim=1)
        scores = (q @ k.transpose(-1, -2)) / math.sqrt(s.head_dim)
        attn = scores.masked_fill(~mask, float("-inf")).softmax(-1) @ v
        attn = attn.to(model.dtype).transpose(1, 2).reshape(1, t, -1)
        h = h + F.linear(attn, layer.w_o)
        x = norm(h, layer.mlp_norm)
        gate, up = F.linear(x, layer.w_gate_up).chunk(2, -1)
        h = h + F.linear(F.silu(gate) * up, layer.w_down)
    h = norm(h, model.final_norm)
    return F.linear(h[0, -1], model.lm_head)


def _prompts(n, lo, hi, vocab, seed=0):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (n,), generator=g).tolist()
    return [torch.randint(0, vocab, (m,), generator=g).tolist() for m in lens]


@pytest.mark.parametrize("use_graphs", [True, False])
def test_greedy_outputs_match_a_dense_forward_fp32(use_graphs):
    model = RandomLlama(TINY, dtype=torch.float32, seed=1, std=0.05)
    config = EngineConfig(max_num_seqs=4, max_model_len=256, max_num_batched_tokens=48, num_gpu_blocks=128,
                          use_graphs=use_graphs)
    prompts = _prompts(6, 5, 70, TINY.vocab_size)  # more requests than slots, prompts longer than the budget
    outputs, stats = LLM(model, config).generate(prompts, max_tokens=6)
    assert stats.output_tokens == 36 and stats.decode_steps > 0
    for prompt, out in zip(prompts, outputs):
        seq = list(prompt)
        for tok in out:
            want = int(_dense_logits(model, seq).argmax())
            assert tok == want
            seq.append(tok)


def test_bf16_engine_logits_track_the_dense_forward():
    model = RandomLlama(TINY, dtype=torch.bfloat16, seed=2, std=0.05)
    config = EngineConfig(max_num_seqs=8, max_model_len=512, max_num_batched_tokens=256, num_gpu_blocks=256)
    llm = LLM(model, config)
    prompts = _prompts(5, 40, 200, TINY.vocab_size, seed=3)
    outputs, _ = llm.generate(prompts, max_tokens=3)
    for prompt, out in zip(prompts, outputs):
        want = _dense_logits(model, prompt).float()
        assert int(want.argmax()) == out[0] or want.topk(2).values.diff().abs().item() < 0.05


TINY128 = LlamaShape(hidden_size=512, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=128,
                     intermediate_size=1024, vocab_size=1000)


@pytest.mark.parametrize("use_graphs", [True, False])
def test_fp8_cache_engine_logits_track_the_dense_forward(use_graphs):
    """The engine over an fp8 (e4m3) KV cache: its first tokens follow the dense bf16 forward,
    up to near-ties the cache's rounding may flip."""
    model = RandomLlama(TINY128, dtype=torch.bfloat16, seed=4, std=0.05)
    config = EngineConfig(max_num_seqs=8, max_model_len=512, max_num_batched_tokens=256, num_gpu_blocks=256,
                          use_graphs=use_graphs, cache_quant="fp8", k_scale=0.5, v_scale=0.5)
    llm = LLM(model, config)
    assert llm.cache.pool.cache_quant == "fp8"
    prompts = _prompts(5, 40, 200, TINY128.vocab_size, seed=5)
    outputs, stats = llm.generate(prompts, max_tokens=3)
    assert stats.output_tokens == 15
    for prompt, out in zip(prompts, outputs):
        want = _dense_logits(model, prompt).float()
        assert int(want.argmax()) == out[0] or want.topk(2).values.diff().abs().item() < 0.1
