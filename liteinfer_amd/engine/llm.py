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

from liteinfer_amd.cache.block_pool import BlockPool, to_device
from liteinfer_amd.cache.kv_cache import KVCache
from liteinfer_amd.engine.model import RandomLlama
from liteinfer_amd.engine.outputs import RequestOutput, SamplingParams
from liteinfer_amd.engine.runner import ModelRunner, PendingTokens
from liteinfer_amd.engine.scheduler import PENDING_TOKEN, Scheduler, Sequence, SequenceStatus
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
        by_id = {s.request_id: s for s in seqs}
        steps = decode_steps = 0
        # Finiteness of every sampled logit row, kept on the device (one
        # small reduction per step, read once at the end).
        finite = torch.ones((), dtype=torch.bool, device=self.model.device)
        # The last step's sampled tokens, still on the device: read back once
        # the next step is launched, so the host stages step n + 1 while the
        # GPU runs step n. Outputs end at a fixed length, so which sequences
        # run next never depends on a token's value; the ids the next step
        # feeds in are gathered on the device.
        pending: PendingTokens | None = None
        readback: tuple = ()
        self._sync()
        t0 = time.perf_counter()
        try:
            while self.scheduler.has_unfinished():
                out = self.scheduler.schedule()
                counts = [out.num_scheduled_tokens[s.request_id] for s in out.seqs]
                logits = self.runner.execute(out.seqs, counts, pending)
                if pending is not None:
                    self._read_back(pending, readback, by_id)
                    pending = None
                steps += 1
                decode_steps += all(c == 1 for c in counts)
                sample = [i for i, s in enumerate(out.seqs) if s.num_computed_tokens == len(s)]
                if sample:
                    if len(sample) == logits.shape[0]:
                        picked = logits
                    else:
                        picked = logits.index_select(0, to_device(sample, torch.long, logits.device))
                    finite &= torch.isfinite(picked).all()
                    tokens = picked.argmax(dim=-1)
                    index = {}
                    for k, i in enumerate(sample):
                        seq = out.seqs[i]
                        seq.output_token_ids.append(PENDING_TOKEN)
                        index[seq.request_id] = k
                        if len(seq.output_token_ids) >= seq.max_tokens:
                            seq.status = SequenceStatus.FINISHED_LENGTH
                    pending = PendingTokens(tokens, index)
                    readback = self._stage_read_back(tokens)
                for seq in self.scheduler.remove_finished():
                    self.runner.release(seq)
            if pending is not None:
                self._read_back(pending, readback, by_id)
                pending = None
        except BaseException:
            # A failed step (a slot write that missed the pool, a launch
            # error) leaves no sequence holding cache blocks: the LLM stays
            # usable for the next generate.
            for seq in self.scheduler.abort_all():
                self.runner.release(seq)
            raise
        self._sync()
        wall = time.perf_counter() - t0
        self.cache.pool.check_slot_writes()
        stats = GenerateStats(wall, steps, decode_steps, sum(len(p) for p in prompts),
                              sum(len(s.output_token_ids) for s in seqs), bool(finite))
        return [s.output_token_ids for s in seqs], stats

    def _sync(self) -> None:
        if self.model.device.type == "cuda":
            torch.cuda.synchronize()

    def _stage_read_back(self, tokens: torch.Tensor) -> tuple:
        """Queue the copies of a step's sampled tokens and of the pool's missed-write counter to the host.

        On a ROCm device they go into pinned memory behind the step's work,
        with an event after them: reading them waits for that step only, not
        for the next one, which is queued behind them by then.
        """
        bad = self.cache.pool.bad_slots
        if tokens.device.type != "cuda":
            return tokens, bad.clone(), None
        host = torch.empty(tokens.shape, dtype=tokens.dtype, pin_memory=True)
        host.copy_(tokens, non_blocking=True)
        missed = torch.empty(bad.shape, dtype=bad.dtype, pin_memory=True)
        missed.copy_(bad, non_blocking=True)
        done = torch.cuda.Event()
        done.record()
        return host, missed, done

    def _read_back(self, pending: PendingTokens, readback: tuple, by_id: dict[str, Sequence]) -> None:
        """Fill in a step's sampled tokens (waits for that step), and check the slot writes up to it."""
        host, missed, done = readback
        if done is not None:
            done.synchronize()
        tokens = host.tolist()
        self.cache.pool.raise_if_missed(int(missed[0]))
        for request_id, k in pending.index.items():
            out = by_id[request_id].output_token_ids
            if out[-1] != PENDING_TOKEN:
                raise RuntimeError(f"{request_id}: its newest output token is not the pending one")
            out[-1] = int(tokens[k])
