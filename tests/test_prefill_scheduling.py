"""The reference's prefill-scheduling tests (bench/test_prefill_scheduling.py:44-213), restated on kvx's engine.

CPU only: a deterministic model runner (token = 10 * first prompt token + completion index) drives the
Scheduler and BlockManager restatements, so these pin the admission and chunking decisions that decide when
the copy path saves and restores blocks. The test that composes the policy with CPU restores
(:178-193) runs on a GPU pool in tests/test_gpu_engine.py.
"""

import pytest

from kvx.engine.llm_engine import EngineConfig, LLMEngine
from kvx.engine.sequence import SamplingParams


class DeterministicRunner:
    """bench/test_prefill_scheduling.py:15-22."""

    def __init__(self):
        self.calls = []

    def call(self, method, *args):
        if method == "exit":
            return None
        seqs, is_prefill = args
        self.calls.append((is_prefill, [(seq.seq_id, seq.num_scheduled_tokens) for seq in seqs]))
        return [10 * seq[0] + seq.num_completion_tokens for seq in seqs]


def engine_for(policy, budget=8, num_blocks=16, **config):
    return LLMEngine(DeterministicRunner(), max_num_seqs=4, max_num_batched_tokens=budget, eos=99,
                     kvcache_block_size=256, num_kvcache_blocks=num_blocks, prefill_policy=policy, **config)


def params(**kwargs):
    return SamplingParams(temperature=0, **kwargs)


def assert_pool_consistent(manager):
    free = list(manager.free_block_ids)
    assert len(free) == len(set(free)) and not set(free) & manager.used_block_ids
    assert set(free) | manager.used_block_ids == set(range(len(manager.blocks)))


def drain(engine, limit=2000):
    decisions, events = [], []
    while not engine.is_finished():
        assert len(decisions) < limit, "scheduler failed to make bounded progress"
        result = engine.step_with_events()
        decisions.append(engine.scheduler.last_schedule)
        events.extend(result.token_events)
        assert_pool_consistent(engine.scheduler.block_manager)
    assert not engine.scheduler.block_manager.used_block_ids
    return decisions, events


@pytest.mark.parametrize("policy", ["fixed", "decode_aware"])
def test_long_prefill_yields_to_decode_and_both_finish(policy):
    engine = engine_for(policy, prefill_chunk_size=4)
    active = engine.add_request([1], params(max_tokens=8))
    engine.step_with_events()
    incoming = engine.add_request([2] * 17, params(max_tokens=2))
    decisions, events = drain(engine)
    assert decisions[0].phase == "decode" and decisions[0].seq_ids == (active,)
    assert any(d.phase == "prefill" for d in decisions)
    for previous, current in zip(decisions, decisions[1:]):
        if previous.phase == "prefill" and current.decode_requests:
            assert current.phase == "decode"
    assert [e.output_index for e in events if e.seq_id == active] == list(range(1, 8))
    assert [e.output_index for e in events if e.seq_id == incoming] == [0, 1]
    assert all(d.scheduled_tokens <= d.prefill_budget for d in decisions if d.phase == "prefill")


def test_legacy_keeps_prefill_priority_for_comparison():
    engine = engine_for("legacy", budget=8, prefill_chunk_size=2)
    active = engine.add_request([1], params(max_tokens=4))
    engine.step_with_events()
    engine.add_request([2] * 17, params(max_tokens=1))
    assert [engine.step_with_events().num_tokens for _ in range(3)] == [8, 8, 1]
    assert engine.scheduler.running[0].seq_id == active
    assert engine.step_with_events().num_tokens == -1


@pytest.mark.parametrize("policy, hard_cap, expected", [("fixed", 50, 12), ("decode_aware", 50, 4),
                                                        ("fixed", 2, 2), ("decode_aware", 2, 2)])
def test_budget_accounts_for_decode_load_and_hard_token_cap(policy, hard_cap, expected):
    engine = engine_for(policy, budget=50, prefill_chunk_size=12, prefill_min_chunk_size=3)
    for value in (1, 2):
        engine.add_request([value], params(max_tokens=5))
    engine.step_with_events()
    engine.scheduler.max_num_batched_tokens = hard_cap
    engine.add_request([3] * 25, params(max_tokens=1))
    assert engine.step_with_events().num_tokens == -2
    result = engine.step_with_events()
    decision = engine.scheduler.last_schedule
    assert decision.decode_requests == 2
    assert decision.prefill_budget == result.num_tokens == expected
    assert result.token_events == []


def test_adaptive_budget_recovers_when_decode_load_disappears():
    engine = engine_for("decode_aware", budget=20, prefill_chunk_size=12, prefill_min_chunk_size=2)
    engine.add_request([1], params(max_tokens=3))
    engine.step_with_events()
    engine.add_request([2] * 25, params(max_tokens=1))
    assert [engine.step_with_events().num_tokens for _ in range(4)] == [-1, 6, -1, 12]  # the decoder finishes
    assert engine.scheduler.last_schedule.decode_requests == 0
    drain(engine)


@pytest.mark.parametrize("policy", ["fixed", "decode_aware"])
def test_decode_batches_rotate_when_resident_requests_exceed_batch_slots(policy):
    engine = engine_for(policy, prefill_chunk_size=12)
    ids = [engine.add_request([value], params(max_tokens=3)) for value in (1, 2, 3)]
    engine.step_with_events()
    engine.scheduler.max_num_seqs = 1
    assert [engine.step_with_events().token_events[0].seq_id for _ in range(6)] == ids + ids
    assert engine.is_finished()


@pytest.mark.parametrize("policy", ["legacy", "fixed", "decode_aware"])
def test_policy_preserves_outputs_and_token_indices_across_chunk_shapes(policy):
    engine = engine_for(policy, budget=8, prefill_chunk_size=3)
    ids = [engine.add_request([value] * length, params(max_tokens=3)) for value, length in ((1, 7), (2, 2), (3, 13))]
    _, events = drain(engine)
    for value, request_id in enumerate(ids, 1):
        observed = [e for e in events if e.seq_id == request_id]
        assert [e.output_index for e in observed] == [0, 1, 2]
        assert [e.token_id for e in observed] == [10 * value + i for i in range(3)]
        assert [e.finished for e in observed] == [False, False, True]


def test_partial_prefill_releases_reservations_for_decode_growth():
    engine = engine_for("fixed", budget=512, num_blocks=3, prefill_chunk_size=256)
    active = engine.add_request([1] * 255, params(max_tokens=4))
    engine.step_with_events()
    incoming = engine.add_request([2] * 257, params(max_tokens=1))
    assert engine.step_with_events().num_tokens == -1  # the pending token reaches a block boundary
    assert engine.step_with_events().num_tokens == 256
    partial = engine.scheduler.waiting[0]
    assert len(partial.block_table) == 2 and partial.num_cached_tokens == 256
    result = engine.step_with_events()  # must reclaim the partial prefill's blocks to grow the decoder
    assert result.num_tokens == -1 and result.token_events[0].seq_id == active
    assert not partial.block_table and partial.num_cached_tokens == 0
    decisions, events = drain(engine)
    assert any(e.seq_id == incoming and e.finished for e in events) and decisions


@pytest.mark.parametrize("policy", ["fixed", "decode_aware"])
def test_no_decode_work_means_consecutive_prefill_chunks_can_progress(policy):
    engine = engine_for(policy, prefill_chunk_size=2)
    request = engine.add_request([1] * 5, params(max_tokens=1))
    assert engine.step_with_events().token_events == []
    assert engine.step_with_events().token_events == []
    assert engine.step_with_events().outputs == [(request, [10])]
    assert engine.is_finished()


def test_failed_admission_does_not_advance_policy_phase(monkeypatch):
    engine = engine_for("fixed", prefill_chunk_size=4)
    engine.add_request([1], params(max_tokens=3))
    engine.step_with_events()
    engine.step_with_events()
    engine.add_request([2] * 5, params(max_tokens=1))
    previous = engine.scheduler.last_schedule

    def fail(*args):
        raise RuntimeError("copy failed")

    with monkeypatch.context() as patch:
        patch.setattr(engine.scheduler.block_manager, "allocate", fail)
        with pytest.raises(RuntimeError, match="copy failed"):
            engine.step_with_events()
    assert engine.scheduler.last_schedule is previous
    assert engine.step_with_events().num_tokens == 4  # the prefill is retried, not a decode
    drain(engine)


@pytest.mark.parametrize("kwargs, message", [
    ({"prefill_policy": "unknown"}, "prefill_policy"),
    ({"prefill_chunk_size": 0}, "prefill_chunk_size"),
    ({"prefill_chunk_size": True}, "prefill_chunk_size"),
    ({"prefill_chunk_size": 1.5}, "prefill_chunk_size"),
    ({"prefill_min_chunk_size": 0}, "prefill_min_chunk_size"),
    ({"prefill_chunk_size": 4, "prefill_min_chunk_size": 5}, "must not exceed"),
    ({"max_num_batched_tokens": 0}, "max_num_batched_tokens"),
    ({"max_num_seqs": 0}, "max_num_seqs"),
])
def test_config_rejects_invalid_policy_before_model_loading(kwargs, message):
    with pytest.raises(ValueError, match=message):
        EngineConfig(**kwargs)


def test_oversized_request_fails_explicitly_instead_of_spinning():
    engine = engine_for("fixed", num_blocks=1)
    engine.add_request([1] * 257, params(max_tokens=1))
    with pytest.raises(RuntimeError, match="GPU KV capacity"):
        engine.step_with_events()
