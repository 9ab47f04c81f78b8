"""The generate loop's bookkeeping on the CPU: step n + 1 staged before step n's tokens are read
back (their ids gathered on the device side from the pending argmax), chunked prompts, seats
freed and refilled, decode rows inside packed passes. The layer's attention here is the
reference's eager attention over the same paged cache (the HIP kernels need a ROCm device;
their parity is the GPU tests'); the answer is a cache-free dense forward's greedy tokens."""

from __future__ import annotations

import pytest
import torch

import liteinfer_amd.engine.model as model_module
from liteinfer_amd.attention import eager_attention
from liteinfer_amd.engine.llm import LLM, EngineConfig
from liteinfer_amd.engine.model import LlamaShape, RandomLlama
from tests.engine_helpers import dense_logits, random_prompts

SHAPE = LlamaShape(hidden_size=128, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=32,
                   intermediate_size=256, vocab_size=300, rms_norm_eps=1e-5, rope_theta=10000.0)


@pytest.fixture
def eager_layers(monkeypatch):
    monkeypatch.setattr(model_module, "paged_attention", eager_attention)


def _dense_greedy(model, prompt, n):
    seq = list(prompt)
    for _ in range(n):
        seq.append(int(dense_logits(model, seq, torch.float32).argmax()))
    return seq[len(prompt):]


@pytest.mark.parametrize(("max_num_seqs", "budget"), [(4, 64), (2, 16), (3, 7)])
def test_pipelined_loop_matches_dense_greedy_decoding(eager_layers, max_num_seqs, budget):
    model = RandomLlama(SHAPE, dtype=torch.float32, seed=3, std=0.08, device="cpu")
    config = EngineConfig(max_num_seqs=max_num_seqs, max_model_len=128, max_num_batched_tokens=budget,
                          num_gpu_blocks=64, use_graphs=False)
    prompts = random_prompts(5, 3, 40, SHAPE.vocab_size, seed=max_num_seqs + budget)
    outputs, stats = LLM(model, config).generate_ids(prompts, max_tokens=6)
    assert stats.output_tokens == 30 and stats.logits_finite
    for prompt, out in zip(prompts, outputs):
        assert out == _dense_greedy(model, prompt, 6)
