"""The generate loop (liteinfer/llm.py `LLM.generate` over the engine core), greedy:
each step schedules, runs one forward, samples the argmax for every sequence
whose prompt is complete, and retires sequences that reached their
`max_tokens` (stop strings and EOS do not apply: the end-to-end configuration
fixes every output at its length).

`generate(prompts, sampling_params)` takes text and returns `RequestOutput`s
through a local tokenizer, as the reference's `LLM.generate` does;
`generate_ids` is the same loop on token ids, with the step statistics.
"""

from __future__ import annotations

import time
from dataclasses import dataclass

import torch

from liteinfer_amd.cache.block_pool import BlockPool
from liteinfer_amd.cache.kv_cache import KVCache
from liteinfer_amd.engine.model import RandomLlama
from liteinfer_amd.engine.outputs import RequestOutput, SamplingParams
from liteinfer_amd.engine.runner import ModelRunner
from liteinfer_amd.engine.scheduler import Scheduler, Sequence, SequenceStatus
from liteinfer_amd.engine.tokenizer import Tokenizer


@dataclass
class EngineConfig:
    max_num_seqs: int = 256
    max_model_len: int = 4352
    max_num_batched_tokens: int = 8192
    num_gpu_blocks: int = 24576
    block_size: int = 16
    use_graphs: bool = True
    cache_quant: str | None = None
    """None (the model dtype) or "fp8": K/V stored as e4m3 with `k_scale` / `v_scale`."""
    k_scale: float = 1.0
    v_scale: float = 1.0


@dataclass
class GenerateStats:
    wall_s: float
    steps: int
    decode_steps: int
    prompt_tokens: int
    output_tokens: int
    logits_finite: bool = True
    """Every logit row the step sampled from was finite."""

    @property
    def output_tokens_per_s(self) -> float:
        return self.output_tokens / self.wall_s


class LLM:
    def __init__(self, model: RandomLlama, config: EngineConfig = EngineConfig(),
                 tokenizer: Tokenizer | None = None) -> None:
        s = model.shape
        self.config = config
        self.model = model
        self.tokenizer = tokenizer
        self.stats: GenerateStats | None = None  # the last generate call's step statistics
        pool = BlockPool(num_blocks=config.num_gpu_blocks, block_size=config.block_size, num_layers=s.num_layers,
                         num_kv_heads=s.num_kv_heads, head_dim=s.head_dim, dtype=model.dtype, device=model.device,
                         cache_quant=config.cache_quant, k_scale=config.k_scale, v_scale=config.v_scale)
        self.cache = KVCache(pool)
        self.runner = ModelRunner(model, self.cache, config.max_num_seqs, config.max_model_len, config.use_graphs)
        self.scheduler = Scheduler(config.max_num_seqs, config.max_num_batched_tokens)

    def generate(self, prompts: str | list[str], sampling_params: SamplingParams | None = None) -> list[RequestOutput]:
        """Completions of text prompts, in the order given (liteinfer/llm.py:49-55).

        Greedy and fixed-length: `sampling_params` must ask for temperature 0
        with no top-p / top-k / stop strings, and every output runs to
        `max_tokens` (the tokenizer has no end-of-sequence token).
        """
        if self.tokenizer is None:
            raise ValueError("this LLM has no tokenizer: pass one, or call generate_ids with token ids")
        params = sampling_params or SamplingParams(temperature=0.0)
        if not params.greedy or params.top_p != 1.0 or params.top_k != -1 or params.stop or params.stop_token_ids:
            raise ValueError("this engine samples greedily: temperature 0, no top-p / top-k / stop conditions")
        texts = [prompts] if isinstance(prompts, str) else list(prompts)
        ids = [self.tokenizer.encode(t) for t in texts]
        for i, p in enumerate(ids):
            if not p:
                raise ValueError(f"prompt {i} encodes to no tokens")
        outputs, stats = self.generate_ids(ids, params.max_tokens)
        self.stats = stats
        return [RequestOutput(f"req-{i}", text, self.tokenizer.decode(out), out, "length")
                for i, (text, out) in enumerate(zip(texts, outputs))]

    def generate_ids(self, prompts: list[list[int]], max_tokens: int) -> tuple[list[list[int]], GenerateStats]:
        """Greedy continuation of every token-id prompt to exactly `max_tokens` tokens."""
        seqs = []
        for i, p in enumerate(prompts):
            if len(p) + max_tokens > self.config.max_model_len:
                raise ValueError(f"request {i}: {len(p)} + {max_tokens} tokens exceed max_model_len")
            seq = Sequence(f"req-{i}", list(p), max_tokens)
            seqs.append(seq)
            self.scheduler.add(seq)
        steps = decode_steps = 0
        # Finiteness of every sampled logit row, kept on the device (one
        # small reduction per step, read once at the end).
        finite = torch.ones((), dtype=torch.bool, device=self.model.device)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        try:
            while self.scheduler.has_unfinished():
                out = self.scheduler.schedule()
                counts = [out.num_scheduled_tokens[s.request_id] for s in out.seqs]
                logits = self.runner.execute(out.seqs, counts)
                steps += 1
                decode_steps += all(c == 1 for c in counts)
                sample = [i for i, s in enumerate(out.seqs) if s.num_computed_tokens == len(s)]
                if sample:
                    rows = torch.tensor(sample, device=logits.device)
                    picked = logits.index_select(0, rows)
                    finite &= torch.isfinite(picked).all()
                    tokens = picked.argmax(dim=-1).tolist()
                    self.cache.pool.check_slot_writes()
                    for i, tok in zip(sample, tokens):
                        seq = out.seqs[i]
                        seq.output_token_ids.append(int(tok))
                        if len(seq.output_token_ids) >= seq.max_tokens:
                            seq.status = SequenceStatus.FINISHED_LENGTH
                for seq in self.scheduler.remove_finished():
                    self.runner.release(seq)
        except BaseException:
            # A failed step (a slot write that missed the pool, a launch
            # error) leaves no sequence holding cache blocks: the LLM stays
            # usable for the next generate.
            for seq in self.scheduler.abort_all():
                self.runner.release(seq)
            raise
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        self.cache.pool.check_slot_writes()
        stats = GenerateStats(wall, steps, decode_steps, sum(len(p) for p in prompts),
                              sum(len(s.output_token_ids) for s in seqs), bool(finite))
        return [s.output_token_ids for s in seqs], stats
