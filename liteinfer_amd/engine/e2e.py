"""The end-to-end configuration: `LLM.generate` over a random-initialised
Llama-3-8B-architecture model with the HIP `paged` attention.

256 requests of random token ids, prompt lengths lognormal with median 512
(sigma 0.7) clipped to [16, 4096], 256 greedy output tokens each (fixed
length: no EOS), continuous batching over at most 256 sequences with chunked
prefill under a token budget. The prompts are rendered as text (token id i
is the word ``tok<i>`` of a local word-level tokenizer) and go through
`LLM.generate(prompts, SamplingParams)`, which encodes them, generates and
decodes the outputs. The timed region is that one call; model initialisation
and the capture of every decode graph width come before it.
"""

from __future__ import annotations

import math
import tempfile
import time

import numpy as np

from liteinfer_amd.engine.llm import LLM, EngineConfig
from liteinfer_amd.engine.model import LLAMA_3_8B, RandomLlama
from liteinfer_amd.engine.outputs import SamplingParams
from liteinfer_amd.engine.tokenizer import Tokenizer, make_wordlevel

NUM_REQUESTS = 256
OUTPUT_TOKENS = 256
PROMPT_MEDIAN = 512
PROMPT_SIGMA = 0.7
PROMPT_CLIP = (16, 4096)


def prompts(seed: int = 0, n: int = NUM_REQUESTS, vocab: int = LLAMA_3_8B.vocab_size) -> list[list[int]]:
    rng = np.random.default_rng(seed)
    lens = np.clip(np.round(rng.lognormal(math.log(PROMPT_MEDIAN), PROMPT_SIGMA, size=n)), *PROMPT_CLIP).astype(int)
    return [rng.integers(0, vocab, size=int(m)).tolist() for m in lens]


def run(seed: int = 0, config: EngineConfig | None = None, num_requests: int = NUM_REQUESTS,
        output_tokens: int = OUTPUT_TOKENS, cache_quant: str | None = None) -> dict:
    config = config or EngineConfig(max_num_seqs=256, max_model_len=PROMPT_CLIP[1] + OUTPUT_TOKENS,
                                    max_num_batched_tokens=8192, num_gpu_blocks=32768, cache_quant=cache_quant)
    model = RandomLlama(LLAMA_3_8B, seed=seed)
    with tempfile.TemporaryDirectory(prefix="liteinfer_amd_tok_") as tok_dir:
        make_wordlevel(model.shape.vocab_size, tok_dir)
        tokenizer = Tokenizer(tok_dir)
    llm = LLM(model, config, tokenizer=tokenizer)
    # warm-up: kernels, allocator, and every decode graph width
    llm.generate_ids(prompts(seed + 1, n=8), max_tokens=4)
    if llm.runner.graphs is not None:
        llm.runner.graphs.capture_all()
    reqs = prompts(seed, n=num_requests)
    texts = [" ".join(f"tok{t}" for t in p) for p in reqs]
    params = SamplingParams(temperature=0.0, max_tokens=output_tokens, min_tokens=output_tokens, ignore_eos=True)
    t0 = time.perf_counter()
    results = llm.generate(texts, params)
    wall = time.perf_counter() - t0
    stats = llm.stats
    outputs = [r.token_ids for r in results]
    vocab = model.shape.vocab_size
    return {
        # the whole generate call: encoding, the engine loop, decoding
        "output_tok_per_s": round(stats.output_tokens / wall, 1),
        "total_tok_per_s": round((stats.output_tokens + stats.prompt_tokens) / wall, 1),
        "wall_s": round(wall, 3),
        "engine_loop_s": round(stats.wall_s, 3),
        "requests": num_requests,
        "prompt_tokens": stats.prompt_tokens,
        "output_tokens": stats.output_tokens,
        "steps": stats.steps,
        "decode_steps": stats.decode_steps,
        "model": "Llama-3-8B architecture, random init (std 0.02), bf16",
        "max_num_seqs": config.max_num_seqs,
        "max_num_batched_tokens": config.max_num_batched_tokens,
        "decode_graphs": config.use_graphs,
        "kv_cache": config.cache_quant or "bf16",
        "parameter_bytes": model.parameter_bytes(),
        # properties of the timed run's output, checked after the clock stops
        "every_request_full_length": all(len(o) == output_tokens for o in outputs),
        "tokens_in_vocab": all(0 <= t < vocab for o in outputs for t in o),
        "sampled_logits_finite": stats.logits_finite,
        "distinct_tokens": len({t for o in outputs for t in o}),
        "prompts_round_trip": all(r.prompt == t for r, t in zip(results, texts)) and [
            tokenizer.encode(t) for t in texts[:8]] == reqs[:8],
        "texts_decode_the_tokens": all(r.text == tokenizer.decode(r.token_ids) for r in results),
    }


if __name__ == "__main__":
    import json

    print(json.dumps(run()))
