"""The block manager's cache hooks and admission logic, on the CPU with a recording cache double.

Restates the pure-Python parts of bench/test_cpu_cache_optimizations.py,
bench/test_cpu_prefix_cache.py and bench/test_automatic_cpu_cache.py: which
hook runs when, in which order, and how failures roll back.
"""

from dataclasses import dataclass

import pytest

from kvx.engine.block_manager import BlockManager, plan_split
from kvx.engine.sequence import SamplingParams, Sequence

BS = 256


@dataclass(frozen=True)
class Entry:
    token_ids: tuple
    slot: int


class RecordingCache:
    """Duck-typed CPU cache: records every hook the block manager calls."""

    def __init__(self, prefetch=False, hybrid=None):
        self.prefetch_enabled = prefetch
        self.hybrid = hybrid
        self._prefetched_blocks = 0
        self.entries: dict[int, Entry] = {}
        self.calls: list[tuple] = []
        self.fail_preserve = False
        self.fail_copy_after = None

    def _preserve_before_recycle(self, h):
        self.calls.append(("preserve_recycle", h))
        if self.fail_preserve:
            raise RuntimeError("preservation copy failed")

    def _preserve_on_release(self, h):
        self.calls.append(("preserve_release", h))

    def before_block_reuse(self, block_id):
        self.calls.append(("reuse", block_id))

    def before_block_use(self, block_id):
        self.calls.append(("use", block_id))

    def _entry_for(self, h, token_ids):
        e = self.entries.get(h)
        return e if e is not None and e.token_ids == tuple(token_ids) else None

    def _copy_entry(self, entry, block_id, wait=True):
        copies = [c for c in self.calls if c[0] == "copy"]
        if self.fail_copy_after is not None and len(copies) >= self.fail_copy_after:
            raise RuntimeError("restore failed")
        self.calls.append(("copy", entry.slot, block_id, wait))


def publish(manager, block_id, token, prefix=-1):
    tokens = [token] * BS
    h = manager.compute_hash(tokens, prefix)
    manager.blocks[block_id].update(h, tokens)
    manager.hash_to_block_id[h] = block_id
    return h


def consistent(manager):
    free = list(manager.free_block_ids)
    assert len(free) == len(set(free))
    assert set(free).isdisjoint(manager.used_block_ids)
    assert set(free) | manager.used_block_ids == set(range(len(manager.blocks)))
    assert all(manager.blocks[i].ref_count == 0 for i in free)


def params():
    return SamplingParams(temperature=0, max_tokens=1)


def test_plan_split_known_answers():
    # bench/test_cpu_cache_optimizations.py:47-52
    assert plan_split(8, 256, 1.0, 1 / 256, 0) == 4
    assert plan_split(8, 256, 1.0, 0, 0) == 8
    assert plan_split(8, 256, 0, 1, 0) == 0
    assert plan_split(0, 256, 1.0, 1.0, 1.0) == 0


def test_plan_split_matches_brute_force_minimum():
    for blocks in range(0, 12):
        for r, a, b in [(1.0, 1 / 256, 1e-6), (0.3, 2 / 256, 0), (2.0, 1e-4, 1e-7)]:
            costs = [max(k * BS * a + (k * BS) ** 2 * b, (blocks - k) * r) for k in range(blocks + 1)]
            assert plan_split(blocks, BS, r, a, b) == costs.index(min(costs))


def test_chained_hashes_depend_on_the_prefix():
    a = BlockManager.compute_hash([1] * BS)
    assert BlockManager.compute_hash([1] * BS) == a
    assert BlockManager.compute_hash([1] * BS, a) != a
    assert BlockManager.compute_hash([2] * BS, a) != BlockManager.compute_hash([2] * BS)


def test_block_hash_known_answers_and_the_reference_construction():
    """block_manager.py:67-73 streams the 8-byte prefix and np.array(token_ids).tobytes() into xxh64; the engine
    packs the int64 tokens with struct in one buffer. Golden values, then agreement on random blocks."""
    import random

    import numpy as np
    import xxhash

    def streamed(token_ids, prefix=-1):
        h = xxhash.xxh64()
        if prefix != -1:
            h.update(prefix.to_bytes(8, "little"))
        h.update(np.array(token_ids).tobytes())
        return h.intdigest()

    a = BlockManager.compute_hash([1] * BS)
    b = BlockManager.compute_hash(list(range(BS)), a)
    c = BlockManager.compute_hash([2**63 - 1, -1, 0, 151643], b)
    assert (a, b, c) == (18283542310692251843, 9163549530594832100, 16783557659952266248)
    rng = random.Random(3)
    prefix = -1
    for n in [BS, BS, 16, 1, 0, 255, 257, BS]:
        tokens = [rng.choice([rng.randrange(0, 200_000), rng.randrange(-2**63, 2**63)]) for _ in range(n)]
        got = BlockManager.compute_hash(tokens, prefix)
        assert got == streamed(tokens, prefix), (n, prefix)
        prefix = got
    # Token ids outside int64 are refused (numpy would hash a lone 2**63 as uint64; vocabularies are far smaller).
    with pytest.raises(Exception):
        BlockManager.compute_hash([2**63])


def test_mru_eviction_recycles_the_latest_release_tail_first():
    # bench/test_cpu_cache_optimizations.py:214-232
    manager = BlockManager(6, BS, "mru")
    seqs = []
    for token in (1, 2):
        seq = Sequence([token] * 512 + [9], params())
        manager.allocate(seq, 0)
        seq.num_cached_tokens, seq.num_scheduled_tokens = 0, len(seq)
        manager.hash_blocks(seq)
        seqs.append(seq)
    first, second = ([*seq.block_table] for seq in seqs)
    for seq in seqs:
        manager.deallocate(seq)
    order = [manager._allocate_block() for _ in range(4)]
    assert set(order[:2]) == {first[2], second[2]}
    assert order[2:] == [second[1], second[0]]
    with pytest.raises(ValueError):
        BlockManager(2, BS, "fifo")


@pytest.mark.parametrize("error", [RuntimeError, KeyboardInterrupt])
def test_hash_is_published_only_after_copy_and_failure_returns_block(error):
    # bench/test_cpu_prefix_cache.py:83-103
    manager = BlockManager(2, BS)
    publish(manager, 0, 1)
    restored_key = manager.compute_hash([5] * BS)
    called = []

    def copy_then_fail(block_id):
        assert restored_key not in manager.hash_to_block_id
        assert block_id in manager.used_block_ids and block_id not in manager.free_block_ids
        called.append(block_id)
        raise error("copy readiness failed")

    with pytest.raises(error, match="readiness"):
        manager.restore_cached_block(restored_key, [5] * BS, copy_then_fail)
    assert len(called) == 1 and restored_key not in manager.hash_to_block_id
    assert manager.blocks[called[0]].hash == -1 and not manager.used_block_ids
    consistent(manager)


def test_restore_validates_and_reuses_live_gpu_hits():
    manager = BlockManager(2, BS)
    key = publish(manager, 1, 3)
    with pytest.raises(ValueError, match="valid prefix hash"):
        manager.restore_cached_block(key, [3] * (BS - 1), lambda b: None)
    with pytest.raises(ValueError, match="conflicting token"):
        manager.restore_cached_block(key, [4] * BS, lambda b: None)
    assert manager.restore_cached_block(key, [3] * BS, lambda b: pytest.fail("no copy")) == 1
    manager.free_block_ids.clear()
    with pytest.raises(MemoryError, match="free KV blocks"):
        manager.restore_cached_block(manager.compute_hash([7] * BS), [7] * BS, lambda b: None)


def test_recycling_a_published_block_saves_it_first_then_orders_writes():
    manager = BlockManager(2, BS)
    cache = RecordingCache()
    manager._cpu_prefix_cache = cache
    key = publish(manager, 0, 1)
    assert manager._allocate_block() == 0
    assert cache.calls == [("preserve_recycle", key), ("reuse", 0)]
    assert key not in manager.hash_to_block_id
    # A restore destination is reserved without write ordering (block_manager.py:168).
    cache.calls.clear()
    h = manager.compute_hash([5] * BS)
    manager.restore_cached_block(h, [5] * BS, lambda b: cache.calls.append(("copy_to", b)))
    assert ("reuse", 1) not in cache.calls and cache.calls[0] == ("copy_to", 1)


def test_failed_preservation_does_not_pop_or_invalidate_victim():
    # bench/test_automatic_cpu_cache.py:172-189
    manager = BlockManager(2, BS)
    cache = RecordingCache()
    manager._cpu_prefix_cache = cache
    key = publish(manager, 1, 1)
    manager.free_block_ids.remove(1)
    manager.free_block_ids.appendleft(1)
    before = list(manager.free_block_ids)
    cache.fail_preserve = True
    with pytest.raises(RuntimeError, match="preservation"):
        manager._allocate_block()
    assert list(manager.free_block_ids) == before and manager.hash_to_block_id[key] == 1
    assert not manager.used_block_ids
    consistent(manager)


def cpu_only_prefix(manager, cache, blocks, token=1):
    """Chained prefix whose blocks exist only as CPU entries."""
    keys, h = [], -1
    for i in range(blocks):
        h = manager.compute_hash([token] * BS, h)
        cache.entries[h] = Entry(tuple([token] * BS), slot=i)
        keys.append(h)
    return keys


def test_admission_restores_cpu_hits_and_waits_for_them():
    manager = BlockManager(4, BS)
    cache = RecordingCache()
    manager._cpu_prefix_cache = cache
    keys = cpu_only_prefix(manager, cache, 2)
    seq = Sequence([1] * 512 + [5], params())
    assert manager.can_allocate(seq) == 2
    manager.allocate(seq, 2)
    copies = [c for c in cache.calls if c[0] == "copy"]
    assert [(slot, wait) for _, slot, _, wait in copies] == [(0, True), (1, True)]
    assert seq.num_cached_tokens == 512 and seq.restore_span is None
    assert [manager.hash_to_block_id[k] for k in keys] == seq.block_table[:2]
    manager.deallocate(seq)
    consistent(manager)


def test_split_admission_recomputes_the_head_and_defers_waits():
    # bench/test_cpu_cache_optimizations.py:148-204
    manager = BlockManager(5, BS)
    cache = RecordingCache(hybrid=(1.0, 1 / 256, 0))
    manager._cpu_prefix_cache = cache
    keys = cpu_only_prefix(manager, cache, 3)
    seq = Sequence([1] * 768 + [5] * 10, params())
    manager.allocate(seq, manager.can_allocate(seq))
    copies = [c for c in cache.calls if c[0] == "copy"]
    assert [(slot, wait) for _, slot, _, wait in copies] == [(1, False), (2, False)]
    assert seq.num_cached_tokens == 0 and seq.restore_span == (256, 768)
    assert keys[0] not in manager.hash_to_block_id  # the head is recomputed, not restored
    seq.num_cached_tokens = 256
    cache.calls.clear()
    manager.finish_restore_span(seq)
    assert cache.calls == [("use", seq.block_table[1]), ("use", seq.block_table[2])]
    assert seq.num_cached_tokens == 768 and seq.restore_span is None
    manager.deallocate(seq)
    consistent(manager)


def test_preempting_a_split_admission_resets_its_span():
    manager = BlockManager(4, BS)
    cache = RecordingCache(hybrid=(1.0, 1 / 256, 0))
    manager._cpu_prefix_cache = cache
    cpu_only_prefix(manager, cache, 2)
    seq = Sequence([1] * 512 + [5], params())
    manager.allocate(seq, manager.can_allocate(seq))
    assert seq.restore_span == (256, 512) and seq.num_cached_tokens == 0
    manager.deallocate(seq)
    assert seq.restore_span is None and not manager.used_block_ids
    consistent(manager)


def test_free_recompute_restores_nothing():
    manager = BlockManager(4, BS)
    cache = RecordingCache(hybrid=(1.0, 0, 0))
    manager._cpu_prefix_cache = cache
    cpu_only_prefix(manager, cache, 2)
    seq = Sequence([1] * 512 + [5], params())
    manager.allocate(seq, manager.can_allocate(seq))
    assert not [c for c in cache.calls if c[0] == "copy"] and seq.num_cached_tokens == 0


def test_restore_failure_during_admission_releases_everything():
    manager = BlockManager(4, BS)
    cache = RecordingCache()
    cache.fail_copy_after = 1
    manager._cpu_prefix_cache = cache
    cpu_only_prefix(manager, cache, 2)
    seq = Sequence([1] * 512 + [5], params())
    with pytest.raises(RuntimeError, match="restore failed"):
        manager.allocate(seq, 2)
    assert not seq.block_table and not manager.used_block_ids
    consistent(manager)


def test_all_gpu_hits_are_protected_before_any_cpu_restore():
    # bench/test_automatic_cpu_cache.py:78-106, with the adversarial free-list order.
    manager = BlockManager(3, BS)
    cache = RecordingCache()
    manager._cpu_prefix_cache = cache
    first = manager.compute_hash([1] * BS)
    cache.entries[first] = Entry(tuple([1] * BS), slot=0)
    second = publish(manager, 1, 2, first)
    manager.free_block_ids.clear()
    manager.free_block_ids.extend([1, 0, 2])  # the GPU hit is the first recyclable slot
    seq = Sequence([1] * 256 + [2] * 256 + [3], params())
    manager.allocate(seq, manager.can_allocate(seq))
    assert seq.block_table[1] == 1 and manager.hash_to_block_id[second] == 1
    assert ("preserve_recycle", second) not in cache.calls
    consistent(manager)


def test_prefetch_uses_spare_blocks_once_and_marks_them_pending():
    manager = BlockManager(4, BS)
    cache = RecordingCache(prefetch=True)
    manager._cpu_prefix_cache = cache
    keys = cpu_only_prefix(manager, cache, 2)
    seq = Sequence([1] * 512 + [7], params())
    assert manager.prefetch(seq, reserve=1) == 2
    assert manager.prefetch(seq, reserve=1) == 0  # nothing changed: throttled
    copies = [c for c in cache.calls if c[0] == "copy"]
    assert all(wait is False for *_, wait in copies) and cache._prefetched_blocks == 2
    assert all(k in manager.hash_to_block_id for k in keys)
    # LRU keeps the prefetched blocks from recycling by their place: the back of the free order.
    assert list(manager.free_block_ids)[-2:] == [manager.hash_to_block_id[k] for k in keys]
    consistent(manager)
    cache.prefetch_enabled = False
    assert manager.prefetch(Sequence([1] * 600, params())) == 0


def test_lookup_does_not_mutate_and_memoises_hashes(monkeypatch):
    manager = BlockManager(2, BS)
    cache = RecordingCache()
    manager._cpu_prefix_cache = cache
    cpu_only_prefix(manager, cache, 2)
    seq = Sequence([1] * 513, params())
    before = (list(manager.free_block_ids), dict(manager.hash_to_block_id))
    assert manager.can_allocate(seq) == -1  # three blocks needed, two exist
    assert (list(manager.free_block_ids), manager.hash_to_block_id) == before and not cache.calls
    calls = []
    original = manager.compute_hash
    monkeypatch.setattr(manager, "compute_hash", lambda *a: calls.append(a) or original(*a))
    manager.can_allocate(seq)
    assert calls == []


def test_resume_allocation_failure_releases_partial_blocks():
    # bench/test_automatic_cpu_cache.py:273-287
    manager = BlockManager(2, BS)
    cache = RecordingCache()
    manager._cpu_prefix_cache = cache
    publish(manager, 1, 9)
    manager.free_block_ids.clear()
    manager.free_block_ids.extend([0, 1])
    cache.fail_preserve = True
    seq = Sequence([1] * 257, params())
    seq.append_token(10)
    with pytest.raises(RuntimeError, match="preservation"):
        manager.allocate_for_resume(seq, 257)
    assert not seq.block_table and seq.num_cached_tokens == 0 and not manager.used_block_ids
    consistent(manager)
