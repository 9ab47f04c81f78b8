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

import pytest
import torch

from liteinfer_amd.engine.llm import LLM, EngineConfig
from liteinfer_amd.engine.model import LlamaShape, RandomLlama
from tests.engine_helpers import dense_logits as _dense_logits
from tests.engine_helpers import random_prompts as _prompts
from tests.engine_helpers import check_tracks_dense, record_logits, sampled_logits

pytestmark = pytest.mark.gpu

TINY = LlamaShape(hidden_size=512, num_layers=2, num_heads=8, num_kv_heads=2, head_dim=64,
                  intermediate_size=1024, vocab_size=1000)


@pytest.mark.parametrize("use_graphs", [True, False])
def test_greedy_outputs_match_a_dense_forward_fp32(use_graphs):
    model = RandomLlama(TINY, dtype=torch.float32, seed=1, std=0.05)
    config = EngineConfig(max_num_seqs=4, max_model_len=256, max_num_batched_tokens=48, num_gpu_blocks=128,
                          use_graphs=use_graphs)
    prompts = _prompts(6, 5, 70, TINY.vocab_size)  # more requests than slots, prompts longer than the budget
    outputs, stats = LLM(model, config).generate_ids(prompts, max_tokens=6)
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
    steps = record_logits(llm)
    prompts = _prompts(5, 40, 200, TINY.vocab_size, seed=3)
    outputs, _ = llm.generate_ids(prompts, max_tokens=3)
    for i, (prompt, out) in enumerate(zip(prompts, outputs)):
        assert len(out) == 3
        print(check_tracks_dense(model, prompt, out, sampled_logits(steps, f"req-{i}")))


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
    steps = record_logits(llm)
    prompts = _prompts(5, 40, 200, TINY128.vocab_size, seed=5)
    outputs, stats = llm.generate_ids(prompts, max_tokens=3)
    assert stats.output_tokens == 15
    for i, (prompt, out) in enumerate(zip(prompts, outputs)):
        # e4m3 keeps 3 mantissa bits to bf16's 7: its rounding of the cached
        # K/V is up to 16x coarser than the dense bf16 forward's.
        print(check_tracks_dense(model, prompt, out, sampled_logits(steps, f"req-{i}"), slack=16.0))


def test_a_failed_step_frees_the_batch_blocks_and_the_llm_runs_again():
    """A step that raises (here: the slot-write check) leaves no sequence
    holding cache blocks; the next generate runs on the whole pool."""
    model = RandomLlama(TINY, dtype=torch.bfloat16, seed=4, std=0.05)
    config = EngineConfig(max_num_seqs=4, max_model_len=256, max_num_batched_tokens=64, num_gpu_blocks=64)
    llm = LLM(model, config)
    pool = llm.cache.pool
    free0 = pool.num_free_blocks
    check = pool.raise_if_missed
    calls = []

    def failing(missed):
        # the loop's per-step check of the missed-write count read back with a step's tokens
        calls.append(1)
        if len(calls) == 2:
            raise IndexError("1 K/V slot writes named a slot outside the pool")
        check(missed)

    pool.raise_if_missed = failing
    prompts = _prompts(6, 5, 70, TINY.vocab_size, seed=5)
    with pytest.raises(IndexError):
        llm.generate_ids(prompts, max_tokens=4)
    assert len(calls) == 2
    assert pool.num_free_blocks == free0
    pool.raise_if_missed = check
    outputs, _ = llm.generate_ids(prompts, max_tokens=4)
    assert [len(o) for o in outputs] == [4] * 6
    assert pool.num_free_blocks == free0


def test_text_prompts_round_trip_through_the_tokenizer(tmp_path):
    """LLM.generate(prompts, SamplingParams) as the reference's (liteinfer/llm.py:49-55): text in,
    RequestOutputs out, the same tokens as the token-id loop, the text their decoding."""
    from liteinfer_amd.engine.outputs import SamplingParams
    from liteinfer_amd.engine.tokenizer import Tokenizer, make_wordlevel

    make_wordlevel(TINY.vocab_size, tmp_path)
    tok = Tokenizer(tmp_path)
    model = RandomLlama(TINY, dtype=torch.bfloat16, seed=6, std=0.05)
    config = EngineConfig(max_num_seqs=4, max_model_len=256, max_num_batched_tokens=64, num_gpu_blocks=128)
    ids = _prompts(5, 3, 40, TINY.vocab_size, seed=7)
    texts = [" ".join(f"tok{t}" for t in p) for p in ids]
    llm = LLM(model, config, tokenizer=tok)
    results = llm.generate(texts, SamplingParams(temperature=0.0, max_tokens=5, ignore_eos=True))
    want, _ = LLM(model, config).generate_ids(ids, max_tokens=5)
    assert [r.token_ids for r in results] == want
    assert [r.prompt for r in results] == texts
    assert all(r.text == tok.decode(r.token_ids) and r.finish_reason == "length" for r in results)
    assert llm.stats is not None and llm.stats.output_tokens == 25
    with pytest.raises(ValueError, match="greedily"):
        llm.generate(texts[:1], SamplingParams(temperature=0.7))
