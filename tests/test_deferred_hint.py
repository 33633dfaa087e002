"""Prefetch hints kept while requests wait (LLMEngine.prefetch_prefix(..., defer=True)), on the CPU.

The scheduler starts a kept hint at the end of the prefill pass that admitted
the waiting requests, after their admission hooks and before the step's model
run, with a reserve of one block per running or partly prefilled request. The
immediate form keeps the reference's contract (nanovllm/engine/llm_engine.py:112-126):
nothing while a request waits.
"""

from types import SimpleNamespace

import pytest

from kvx.engine.llm_engine import LLMEngine
from kvx.engine.scheduler import Scheduler
from kvx.engine.sequence import SamplingParams, Sequence
from test_block_manager import BS, Entry, RecordingCache, consistent, cpu_only_prefix, params


def scheduler(num_blocks, budget=4096):
    Sequence.block_size = BS
    config = SimpleNamespace(max_num_seqs=4, max_num_batched_tokens=budget, eos=-1, kvcache_block_size=BS,
                             num_kvcache_blocks=num_blocks)
    sched = Scheduler(config)
    cache = RecordingCache(prefetch=True)
    sched.block_manager._cpu_prefix_cache = cache
    return sched, cache


def copies(cache):
    return [c for c in cache.calls if c[0] == "copy"]


def test_kept_hint_starts_after_the_admission_it_waited_for():
    sched, cache = scheduler(8)
    keys = cpu_only_prefix(sched.block_manager, cache, 2, token=1)
    current = Sequence([5] * 512 + [6], params())
    sched.add(current)
    sched.prefetch_hint = Sequence([1] * 512 + [7], params())
    seqs, is_prefill = sched.schedule()
    assert is_prefill and seqs == [current] and sched.prefetch_hint is None
    # The admission takes its three fresh blocks first; the hint's two restores follow, unwaited.
    assert len(current.block_table) == 3
    assert [(slot, wait) for _, slot, _, wait in copies(cache)] == [(0, False), (1, False)]
    restored = [block for _, _, block, _ in copies(cache)]
    assert not set(restored) & set(current.block_table)
    assert [sched.block_manager.hash_to_block_id[k] for k in keys] == restored
    assert cache._prefetched_blocks == 2
    consistent(sched.block_manager)


def test_kept_hint_waits_while_a_request_lacks_blocks():
    sched, cache = scheduler(4)
    cpu_only_prefix(sched.block_manager, cache, 2, token=1)
    first = Sequence([5] * 600, params())  # three blocks
    second = Sequence([6] * 600, params())  # three more: cannot be admitted beside the first
    sched.add(first)
    sched.add(second)
    hint = Sequence([1] * 512 + [7], params())
    sched.prefetch_hint = hint
    seqs, _ = sched.schedule()
    assert seqs == [first] and list(sched.waiting) == [second] and not second.block_table
    assert sched.prefetch_hint is hint and not copies(cache)  # kept: the waiting request needs the blocks
    consistent(sched.block_manager)


def test_kept_hint_reserves_a_block_for_a_chunked_request():
    sched, cache = scheduler(6, budget=256)
    cpu_only_prefix(sched.block_manager, cache, 3, token=1)
    chunked = Sequence([5] * 600, params())  # three blocks, prefilled 256 tokens a step
    sched.add(chunked)
    sched.prefetch_hint = Sequence([1] * 768 + [7], params())
    seqs, _ = sched.schedule()
    assert seqs == [chunked] and list(sched.waiting) == [chunked] and len(chunked.block_table) == 3
    # Three blocks are free; one stays for the chunked request's sampled token, two are restored.
    assert len(copies(cache)) == 2 and sched.prefetch_hint is None
    consistent(sched.block_manager)


def test_failing_hint_rewinds_the_pass_and_is_dropped():
    sched, cache = scheduler(8)
    cpu_only_prefix(sched.block_manager, cache, 2, token=1)
    current = Sequence([5] * 512 + [6], params())
    sched.add(current)
    sched.prefetch_hint = Sequence([1] * 512 + [7], params())
    cache.fail_copy_after = 0
    with pytest.raises(RuntimeError, match="restore failed"):
        sched.schedule()
    assert list(sched.waiting) == [current] and not current.block_table and not sched.running
    assert sched.prefetch_hint is None and not sched.block_manager.used_block_ids
    consistent(sched.block_manager)
    cache.fail_copy_after = None
    seqs, _ = sched.schedule()  # the retry admits the request; the dropped hint starts nothing
    assert seqs == [current] and not copies(cache)


class _Runner:
    """Just enough of a model runner for LLMEngine's constructor and step()."""

    def __init__(self, num_blocks):
        self.kv_cache = SimpleNamespace(shape=(2, 1, num_blocks, BS, 1, 4))
        self.block_size = BS
        self.world_size = 1

    def call(self, method, *args):
        if method == "run":
            return [3] * len(args[0])
        return None


def test_engine_keeps_a_deferred_hint_and_drops_an_immediate_one():
    engine = LLMEngine(_Runner(8), kvcache_block_size=BS, eos=-1)
    cache = RecordingCache(prefetch=True)
    engine.scheduler.block_manager._cpu_prefix_cache = cache
    cpu_only_prefix(engine.scheduler.block_manager, cache, 2, token=1)
    engine.add_request([5] * 300, params())
    assert engine.prefetch_prefix([1] * 600) == 0 and engine.scheduler.prefetch_hint is None
    assert engine.prefetch_prefix([1] * 600, defer=True) == 0
    assert engine.scheduler.prefetch_hint is not None and not copies(cache)
    engine.step()
    assert len(copies(cache)) == 2 and engine.scheduler.prefetch_hint is None
    assert engine.is_finished()
    # With nothing waiting the hint starts at once, deferred or not.
    hint = [1] * 512 + [2] * 10
    engine.scheduler.block_manager._last_prefetch = None
    assert engine.prefetch_prefix(hint, defer=True) == 0  # both CPU hits are now idle GPU hits
    consistent(engine.scheduler.block_manager)


def test_seeded_streams_with_deferred_hints_keep_the_pool_consistent():
    """Random arrivals, decode lengths and hints, deferred or not, through the real scheduler: after every step
    the free order and the references agree, every block in a table is referenced once per table, and a pass that
    started the kept hint left no request waiting without blocks."""
    import random

    for seed in range(40):
        rng = random.Random(seed)
        sched, cache = scheduler(rng.randint(6, 12), budget=rng.choice([256, 512, 2048]))
        manager = sched.block_manager
        docs = [[100 * d + i for i in range(rng.randint(1, 4))] for d in range(4)]
        for d, doc in enumerate(docs[:2]):  # some documents start as CPU-only prefixes
            h = -1
            for i, token in enumerate(doc):
                h = manager.compute_hash([token] * BS, h)
                cache.entries[h] = Entry(tuple([token] * BS), slot=10 * d + i)
        for step in range(50):
            for _ in range(rng.choice([0, 0, 1, 2])):
                doc = rng.choice(docs)
                tokens = [v for v in doc[:rng.randint(1, len(doc))] for _ in range(BS)] + [7] * rng.randint(1, 50)
                if len(tokens) // BS + 2 < len(manager.blocks):
                    sched.add(Sequence(tokens, SamplingParams(temperature=0, max_tokens=rng.randint(1, 4),
                                                              ignore_eos=True)))
            if rng.random() < 0.4:
                hint = rng.choice(docs)
                sched.prefetch_hint = Sequence([v for v in hint for _ in range(BS)] + [1], params())
            if sched.is_finished():
                continue
            hint = sched.prefetch_hint
            seqs, is_prefill = sched.schedule()
            if hint is not None and sched.prefetch_hint is None:  # the pass started the kept hint
                assert all(s.block_table for s in sched.waiting), (seed, step)
            sched.postprocess(seqs, [7] * len(seqs), is_prefill)
            consistent(manager)
            refs = {}
            for s in list(sched.running) + list(sched.waiting):
                for b in s.block_table:
                    refs[b] = refs.get(b, 0) + 1
            for b, n in refs.items():
                assert manager.blocks[b].ref_count == n, (seed, step, b)
