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


# An output token sampled on the device and not read back yet (the generate
# loop reads a step's tokens while the next step runs, and fills them in).
PENDING_TOKEN = -1


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

    def take(self, seq: Sequence, tokens: int) -> None:
        """Put `tokens` of `seq`'s uncomputed tokens into this step."""
        self.seqs.append(seq)
        self.num_scheduled_tokens[seq.request_id] = tokens


class _Budget:
    """What is left of one step's token budget."""

    def __init__(self, tokens: int) -> None:
        self.left = tokens

    @property
    def spent(self) -> bool:
        return self.left == 0

    def draw(self, seq: Sequence) -> int:
        """Tokens granted to `seq` now: all it is owed, or what the budget still has."""
        owed = seq.num_uncomputed_tokens
        if owed <= 0:
            raise RuntimeError(f"{seq.request_id} has no uncomputed token to schedule")
        grant = min(owed, self.left)
        self.left -= grant
        return grant


class Scheduler:
    """Seats (``max_num_seqs``) and a per-step token budget, no preemption.

    A step serves the seated sequences first, oldest first, each with what it
    is owed or what the budget has left; then, while tokens and seats remain,
    seats the head of the waiting queue and serves it the same way. A prompt
    larger than what is left is cut there and resumes next step.
    """

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
        step = SchedulerOutput()
        budget = _Budget(self.token_budget)
        for seq in [s for s in self.running if not s.is_finished]:
            if budget.spent:
                break
            step.take(seq, budget.draw(seq))
        while not budget.spent and self.waiting and len(self.running) < self.max_num_seqs:
            seq = self._seat(self.waiting.popleft())
            step.take(seq, budget.draw(seq))
        return step

    def _seat(self, seq: Sequence) -> Sequence:
        seq.status = SequenceStatus.RUNNING
        self.running.append(seq)
        return seq

    def remove_finished(self) -> list[Sequence]:
        done, kept = [], []
        for seq in self.running:
            (done if seq.is_finished else kept).append(seq)
        self.running = kept
        return done

    def abort_all(self) -> list[Sequence]:
        """Drop every waiting and seated sequence (a failed step); returns them so their blocks can be freed."""
        dropped = [*self.running, *self.waiting]
        self.running, self.waiting = [], deque()
        return dropped

    def has_unfinished(self) -> bool:
        return len(self.waiting) + len(self.running) > 0
