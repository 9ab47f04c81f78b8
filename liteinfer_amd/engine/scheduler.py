"""Continuous-batching scheduler with a token budget (liteinfer/engine/scheduler.py).

Every step spends a token budget. A running sequence is owed the rest of its
prompt while it prefills and one token while it decodes; the scheduler grants
each what it is owed clamped by what is left of the budget, running sequences
first in admission order, then admits waiting sequences into free slots
(``max_num_seqs``) while budget remains. A prompt larger than what is left is
chunked: it takes the rest of the budget and continues next step. No
preemption, as in the reference.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field
from enum import Enum


class SequenceStatus(str, Enum):
    WAITING = "waiting"
    RUNNING = "running"
    FINISHED_LENGTH = "finished_length"


@dataclass
class Sequence:
    """One request's token stream (liteinfer/engine/sequence.py:34-80, token ids only)."""

    request_id: str
    prompt_token_ids: list[int]
    max_tokens: int
    output_token_ids: list[int] = field(default_factory=list)
    status: SequenceStatus = SequenceStatus.WAITING
    num_computed_tokens: int = 0
    """Tokens whose K/V are in the cache; the next step computes the rest."""

    def __len__(self) -> int:
        return len(self.prompt_token_ids) + len(self.output_token_ids)

    @property
    def is_finished(self) -> bool:
        return self.status == SequenceStatus.FINISHED_LENGTH

    @property
    def num_uncomputed_tokens(self) -> int:
        return len(self) - self.num_computed_tokens

    def token_at(self, position: int) -> int:
        n = len(self.prompt_token_ids)
        return self.prompt_token_ids[position] if position < n else self.output_token_ids[position - n]


@dataclass
class SchedulerOutput:
    seqs: list[Sequence] = field(default_factory=list)
    num_scheduled_tokens: dict[str, int] = field(default_factory=dict)

    @property
    def is_empty(self) -> bool:
        return not self.seqs


class Scheduler:
    def __init__(self, max_num_seqs: int, token_budget: int) -> None:
        if max_num_seqs < 1 or token_budget < 1:
            raise ValueError("max_num_seqs and token_budget must be >= 1")
        self.max_num_seqs = max_num_seqs
        self.token_budget = token_budget
        self.waiting: deque[Sequence] = deque()
        self.running: list[Sequence] = []

    def add(self, seq: Sequence) -> None:
        seq.status = SequenceStatus.WAITING
        self.waiting.append(seq)

    def schedule(self) -> SchedulerOutput:
        out = SchedulerOutput()
        budget = self.token_budget
        for seq in self.running:
            if budget == 0:
                break
            if not seq.is_finished:
                budget -= self._grant(out, seq, budget)
        while budget > 0 and self.waiting and len(self.running) < self.max_num_seqs:
            seq = self.waiting.popleft()
            seq.status = SequenceStatus.RUNNING
            self.running.append(seq)
            budget -= self._grant(out, seq, budget)
        return out

    @staticmethod
    def _grant(out: SchedulerOutput, seq: Sequence, budget: int) -> int:
        num_tokens = min(seq.num_uncomputed_tokens, budget)
        assert num_tokens > 0, f"{seq.request_id} was scheduled with nothing to compute"
        out.seqs.append(seq)
        out.num_scheduled_tokens[seq.request_id] = num_tokens
        return num_tokens

    def remove_finished(self) -> list[Sequence]:
        finished = [s for s in self.running if s.is_finished]
        self.running = [s for s in self.running if not s.is_finished]
        return finished

    def has_unfinished(self) -> bool:
        return bool(self.waiting or self.running)
