"""Config 5 at its real geometry: `LLM.generate` over a random-initialised Llama-3-8B-architecture model.

A bounded slice of the bench's workload (64 of its 256 requests, 64 of its
256 output tokens, the same prompt-length distribution) so the test runs in
about a minute: every request ends with exactly `max_tokens` tokens from
finite logits, the captured-graph decode produces the same tokens as eager
launches, and the first tokens follow a dense cache-free forward of the same
weights (the reference's end-to-end check, tests/e2e/test_llama_gpu.py:140-218,
without its Hugging Face checkpoint, which this build cannot load).
"""

from __future__ import annotations

import pytest
import torch

from liteinfer_amd.engine import e2e
from liteinfer_amd.engine.llm import LLM, EngineConfig
from liteinfer_amd.engine.model import LLAMA_3_8B, RandomLlama
from tests.engine_helpers import check_tracks_dense, record_logits, sampled_logits

pytestmark = pytest.mark.gpu

REQUESTS, OUTPUT_TOKENS = 64, 64


@pytest.fixture(scope="module")
def model():
    m = RandomLlama(LLAMA_3_8B, seed=0)
    yield m
    del m
    torch.cuda.empty_cache()


def _config(use_graphs: bool) -> EngineConfig:
    # Budget above the prompts' total, so every request is prefilled in the
    # first step and all decode steps run the full batch of 64 (a captured
    # width): graph and eager then see the same shapes.
    return EngineConfig(max_num_seqs=REQUESTS, max_model_len=e2e.PROMPT_CLIP[1] + OUTPUT_TOKENS,
                        max_num_batched_tokens=65536, num_gpu_blocks=4096, use_graphs=use_graphs)


def _generate(model, use_graphs):
    llm = LLM(model, _config(use_graphs))
    steps = record_logits(llm)
    prompts = e2e.prompts(seed=0, n=REQUESTS)
    assert sum(len(p) for p in prompts) <= 65536
    outputs, stats = llm.generate_ids(prompts, max_tokens=OUTPUT_TOKENS)
    del llm
    torch.cuda.empty_cache()
    return prompts, outputs, stats, steps


def test_c5_graph_and_eager_decode_agree_and_track_the_dense_forward(model):
    prompts, graph_out, stats, steps = _generate(model, use_graphs=True)
    print(f"prompt tokens {stats.prompt_tokens}, steps {stats.steps}, decode steps {stats.decode_steps}", flush=True)
    assert stats.output_tokens == REQUESTS * OUTPUT_TOKENS and stats.logits_finite
    assert all(len(out) == OUTPUT_TOKENS for out in graph_out)
    assert all(0 <= t < LLAMA_3_8B.vocab_size for out in graph_out for t in out)
    assert stats.decode_steps == OUTPUT_TOKENS - 1
    assert all(bool(torch.isfinite(logits).all()) for _, logits in steps)

    _, eager_out, eager_stats, eager_steps = _generate(model, use_graphs=False)
    assert eager_stats.output_tokens == REQUESTS * OUTPUT_TOKENS
    assert all(bool(torch.isfinite(logits).all()) for _, logits in eager_steps)
    assert eager_out == graph_out

    for i in range(3):
        errors = check_tracks_dense(model, prompts[i], graph_out[i], sampled_logits(steps, f"req-{i}"), tokens=2)
        print(f"request {i}: (engine, dense bf16) max-abs logit error vs fp32: {errors}", flush=True)
