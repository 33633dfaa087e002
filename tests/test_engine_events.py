"""The reference's engine event-API tests (bench/test_engine_events.py:81-190), restated on kvx's LLMEngine.

CPU only: a scripted model runner (no KV pool, no copy engine) drives the
scheduler and BlockManager restatements; these pin the step / step_with_events
/ generate contract that the engine-side callers of the copy path rely on.
"""

from types import SimpleNamespace

import pytest

from kvx.engine.llm_engine import LLMEngine, TokenEvent
from kvx.engine.sequence import SamplingParams


class ScriptedRunner:
    """bench/test_engine_events.py:47-57."""

    def __init__(self, batches):
        self.batches = iter(batches)
        self.calls = []

    def call(self, method, *args):
        if method == "exit":
            return None
        seqs, is_prefill = args
        tokens = next(self.batches)
        assert len(tokens) == len(seqs)
        self.calls.append((is_prefill, [seq.seq_id for seq in seqs]))
        return tokens


def make_engine(batches, budget=8, num_blocks=16, **config):
    """bench/test_engine_events.py:60-74: a space-separated integer tokenizer."""
    tokenizer = SimpleNamespace(encode=lambda text: [int(t) for t in text.split()],
                                decode=lambda tokens: " ".join(map(str, tokens)))
    return LLMEngine(ScriptedRunner(batches), tokenizer, max_num_seqs=4, max_num_batched_tokens=budget, eos=99,
                     kvcache_block_size=256, num_kvcache_blocks=num_blocks, **config)


def params(**kwargs):
    return SamplingParams(temperature=0, **kwargs)


def test_add_request_returns_distinct_ids_for_text_and_token_prompts():
    engine = make_engine([])
    first = engine.add_request("1 2", params(max_tokens=2))
    second = engine.add_request([3, 4], params(max_tokens=2))
    queued = list(engine.scheduler.waiting)
    assert first != second
    assert [seq.seq_id for seq in queued] == [first, second]
    assert [seq.prompt_token_ids for seq in queued] == [[1, 2], [3, 4]]


def test_chunked_prefill_emits_only_actual_outputs_then_finishes_once():
    engine = make_engine([[90], [91], [10], [11]], budget=2)
    request_id = engine.add_request([1, 2, 3, 4, 5], params(max_tokens=2))
    for _ in range(2):
        chunk = engine.step_with_events()
        assert chunk.token_events == [] and chunk.outputs == [] and chunk.num_tokens == 2
    first = engine.step_with_events()
    assert first.token_events == [TokenEvent(request_id, 0, 10, False)]
    assert first.outputs == [] and first.num_tokens == 1
    last = engine.step_with_events()
    assert last.token_events == [TokenEvent(request_id, 1, 11, True)]
    assert last.outputs == [(request_id, [10, 11])] and last.num_tokens == -1
    assert engine.is_finished() and not engine.scheduler.block_manager.used_block_ids
    assert [prefill for prefill, _ in engine.model_runner.calls] == [True, True, True, False]


def test_batched_requests_keep_independent_indices_and_finish_states():
    engine = make_engine([[10, 20], [21], [22]])
    first = engine.add_request([1, 2], params(max_tokens=1))
    second = engine.add_request([3, 4], params(max_tokens=3))
    prefill = engine.step_with_events()
    assert prefill.token_events == [TokenEvent(first, 0, 10, True), TokenEvent(second, 0, 20, False)]
    assert prefill.outputs == [(first, [10])] and prefill.num_tokens == 4
    assert engine.step_with_events().token_events == [TokenEvent(second, 1, 21, False)]
    final = engine.step_with_events()
    assert final.token_events == [TokenEvent(second, 2, 22, True)]
    assert final.outputs == [(second, [20, 21, 22])]
    assert engine.is_finished()


@pytest.mark.parametrize("ignore_eos", [False, True])
def test_eos_event_respects_ignore_eos(ignore_eos):
    engine = make_engine([[99], [10]])
    request_id = engine.add_request([1], params(max_tokens=2, ignore_eos=ignore_eos))
    first = engine.step_with_events()
    assert first.token_events == [TokenEvent(request_id, 0, 99, not ignore_eos)]
    if ignore_eos:
        assert first.outputs == []
        final = engine.step_with_events()
        assert final.token_events == [TokenEvent(request_id, 1, 10, True)]
        assert final.outputs == [(request_id, [99, 10])]
    else:
        assert first.outputs == [(request_id, [99])]
    assert engine.is_finished() and not engine.scheduler.block_manager.used_block_ids


def test_step_and_event_api_share_progress_without_replaying_tokens():
    engine = make_engine([[10], [11], [12]])
    request_id = engine.add_request([1], params(max_tokens=3))
    assert engine.step_with_events().token_events == [TokenEvent(request_id, 0, 10, False)]
    assert engine.step() == ([], -1)
    final = engine.step_with_events()
    assert final.token_events == [TokenEvent(request_id, 2, 12, True)]
    assert final.outputs == [(request_id, [10, 11, 12])]
    assert len(engine.model_runner.calls) == 3


def test_legacy_step_still_returns_completed_outputs_and_signed_work():
    engine = make_engine([[10], [11]])
    request_id = engine.add_request([1, 2], params(max_tokens=2))
    assert engine.step() == ([], 2)
    assert engine.step() == ([(request_id, [10, 11])], -1)
    assert engine.is_finished()


def test_generate_preserves_output_order_and_matches_streamed_tokens():
    prompts = [[1], [2, 3]]
    sampling = params(max_tokens=2)
    generated = make_engine([[10, 20], [11, 21]]).generate(prompts, sampling, use_tqdm=False)
    assert generated == [{"text": "10 11", "token_ids": [10, 11]}, {"text": "20 21", "token_ids": [20, 21]}]
    streaming = make_engine([[10, 20], [11, 21]])
    request_ids = [streaming.add_request(prompt, sampling) for prompt in prompts]
    tokens = {request_id: [] for request_id in request_ids}
    while not streaming.is_finished():
        for event in streaming.step_with_events().token_events:
            assert event.output_index == len(tokens[event.seq_id])
            tokens[event.seq_id].append(event.token_id)
    assert [tokens[i] for i in request_ids] == [item["token_ids"] for item in generated]
