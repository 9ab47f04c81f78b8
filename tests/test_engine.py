"""The engine's scheduler: the reference's token-budget rules (liteinfer/engine/scheduler.py)."""

import pytest

from liteinfer_amd.engine.scheduler import Scheduler, Sequence, SequenceStatus


def _seq(rid, prompt_len, max_tokens=4):
    return Sequence(rid, list(range(prompt_len)), max_tokens)


def test_prompts_are_granted_until_the_budget_runs_out_and_the_last_one_is_chunked():
    s = Scheduler(max_num_seqs=8, token_budget=100)
    for rid, n in (("a", 30), ("b", 50), ("c", 40)):
        s.add(_seq(rid, n))
    out = s.schedule()
    assert [q.request_id for q in out.seqs] == ["a", "b", "c"]
    assert out.num_scheduled_tokens == {"a": 30, "b": 50, "c": 20}


def test_running_sequences_are_served_before_waiting_ones():
    s = Scheduler(max_num_seqs=8, token_budget=10)
    a, b = _seq("a", 4), _seq("b", 20)
    s.add(a)
    s.add(b)
    out = s.schedule()
    assert out.num_scheduled_tokens == {"a": 4, "b": 6}
    a.num_computed_tokens, b.num_computed_tokens = 4, 6
    a.output_token_ids.append(7)  # a decodes next
    out = s.schedule()
    assert [q.request_id for q in out.seqs] == ["a", "b"]
    assert out.num_scheduled_tokens == {"a": 1, "b": 9}


def test_max_num_seqs_caps_admission():
    s = Scheduler(max_num_seqs=2, token_budget=1000)
    for i in range(5):
        s.add(_seq(f"r{i}", 3))
    out = s.schedule()
    assert len(out.seqs) == 2 and len(s.waiting) == 3


def test_finished_sequences_leave_and_free_their_slot():
    s = Scheduler(max_num_seqs=1, token_budget=16)
    a, b = _seq("a", 2), _seq("b", 2)
    s.add(a)
    s.add(b)
    s.schedule()
    a.status = SequenceStatus.FINISHED_LENGTH
    assert s.remove_finished() == [a]
    out = s.schedule()
    assert [q.request_id for q in out.seqs] == ["b"]
    assert s.has_unfinished()


def test_nonsense_configuration_is_refused():
    with pytest.raises(ValueError):
        Scheduler(max_num_seqs=0, token_budget=8)


def test_a_budget_exactly_spent_by_running_sequences_admits_no_one():
    """The seated sequences take the whole budget: nobody waiting is seated
    this step (the reference's `budget == 0` break), and a finished sequence
    in the running list is skipped, not served."""
    sched = Scheduler(max_num_seqs=4, token_budget=2)
    a, b, c = (Sequence(r, [1] * 3, max_tokens=5) for r in "abc")
    for s in (a, b):
        sched.add(s)
    first = sched.schedule()                       # a gets 2 of its 3 prompt tokens
    assert [s.request_id for s in first.seqs] == ["a"] and first.num_scheduled_tokens["a"] == 2
    a.num_computed_tokens = 2
    sched.add(c)
    second = sched.schedule()                      # a finishes its prompt (1), b starts (1)
    assert second.num_scheduled_tokens == {"a": 1, "b": 1}
    assert [s.request_id for s in sched.waiting] == ["c"]
    a.status = SequenceStatus.FINISHED_LENGTH
    b.num_computed_tokens = 1
    third = sched.schedule()                       # a skipped; b owes 2, the budget is spent
    assert third.num_scheduled_tokens == {"b": 2} and len(sched.waiting) == 1


def test_a_sequence_with_nothing_to_compute_is_an_error():
    sched = Scheduler(max_num_seqs=2, token_budget=8)
    s = Sequence("x", [1, 2], max_tokens=3)
    sched.add(s)
    sched.schedule()
    s.num_computed_tokens = len(s)
    with pytest.raises(RuntimeError, match="no uncomputed token"):
        sched.schedule()


def test_abort_all_returns_every_waiting_and_seated_sequence():
    s = Scheduler(max_num_seqs=2, token_budget=1000)
    seqs = [_seq(f"r{i}", 3) for i in range(5)]
    for q in seqs:
        s.add(q)
    s.schedule()
    dropped = s.abort_all()
    assert sorted(q.request_id for q in dropped) == [q.request_id for q in seqs]
    assert not s.has_unfinished() and s.schedule().seqs == []


def test_wordlevel_tokenizer_round_trips_token_ids(tmp_path):
    from liteinfer_amd.engine.tokenizer import Tokenizer, make_wordlevel

    make_wordlevel(1000, tmp_path)
    tok = Tokenizer(tmp_path)
    assert tok.vocab_size == 1000 and tok.eos_token_ids == ()
    ids = [0, 999, 17, 17, 500]
    text = " ".join(f"tok{i}" for i in ids)
    assert tok.encode(text) == ids
    assert tok.decode(ids) == text
    assert tok.encode("  tok3\ttok4\n") == [3, 4]


def test_tokenizer_reads_local_files_only(tmp_path):
    from liteinfer_amd.engine.tokenizer import Tokenizer

    with pytest.raises(FileNotFoundError):
        Tokenizer(tmp_path / "missing")


def test_sampling_params_checks_follow_the_reference():
    from liteinfer_amd.engine.outputs import SamplingParams

    assert SamplingParams(temperature=0.0).greedy
    for bad in ({"temperature": -1}, {"top_p": 0.0}, {"top_k": 0}, {"max_tokens": 0}, {"min_tokens": -1},
                {"max_tokens": 4, "min_tokens": 5}):
        with pytest.raises(ValueError):
            SamplingParams(**bad)
