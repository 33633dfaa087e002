"""The reference's engine-level CPU-tier tests, restated on a ROCm pool over libkvx.

Each test names the reference test it restates (bench/test_cpu_prefix_cache.py,
bench/test_automatic_cpu_cache.py, bench/test_cpu_cache_optimizations.py). The
reference runs these on CPU pools with torch copies; here every save and
restore goes through the copy engine's kernels, DMAs and events, and the
scripted model's KV writes (where enabled) through store_kvcache. Failure
injection patches the cache's copy seams (_save_to_slot / _restore_from_slot)
instead of torch.Tensor.copy_, since no torch copy is on the path.
"""

from collections import deque
from contextlib import nullcontext

import pytest
import torch

from engine_fixtures import (BS, assert_pool_consistent, block_bytes, cached_engine, completed_prefix,
                             finite_prefix, new_cache, overwrite_prefix, params, pool_of, slow_copies, step,
                             write_scheduled_kv)
from kvx.engine.cpu_prefix_cache import CPUBlockCache, CPUCacheFullError
from kvx.engine.sequence import Sequence

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, params=["batched", "per_block"])
def copy_calls(request, monkeypatch):
    """Every test runs twice: with kvx's block manager handing its loops' copies to the engine in batches
    (CPUBlockCache.coalesce), and with one engine call per block, the call pattern of the reference's
    unmodified BlockManager (block_manager.py:97-137, 202-237, 266-336), which has no coalesce()."""
    if request.param == "per_block":
        monkeypatch.setattr(CPUBlockCache, "coalesce", lambda self: nullcontext())
    return request.param


# -- bench/test_cpu_prefix_cache.py ---------------------------------------------

def test_round_trip_survives_recycling_and_reduces_next_turn_prefill(gpu):
    engine, manager, key = completed_prefix(gpu, [[90], [91], [12]])
    source_id = manager.hash_to_block_id[key]
    expected = block_bytes(engine, source_id)
    cache = new_cache(engine)
    assert cache.save_block(key)
    assert key in cache and len(cache) == 1
    assert cache.bytes_used == cache.block_bytes == cache.max_bytes
    overwrite_prefix(engine)
    assert key not in manager.hash_to_block_id
    pool_of(engine).fill_(-7)
    destination_id = cache.restore_block(key)
    assert destination_id != source_id
    assert torch.equal(block_bytes(engine, destination_id), expected)
    assert manager.blocks[destination_id].ref_count == 0
    assert_pool_consistent(manager)
    request_id = engine.add_request([1] * 257 + [10, 11] + [2] * 10, params(max_tokens=1))
    result = step(engine)
    assert result.num_tokens == 13  # 269 prompt positions minus the restored 256
    assert result.outputs == [(request_id, [12])]
    assert not manager.used_block_ids
    assert_pool_consistent(manager)


def test_failed_restore_keeps_cpu_copy_and_retry_is_byte_exact(gpu, monkeypatch):
    engine, manager, key = completed_prefix(gpu, [[90], [91]])
    cache = new_cache(engine)
    expected = block_bytes(engine, manager.hash_to_block_id[key])
    cache.save_block(key)
    overwrite_prefix(engine)

    def fail_copy(slot, block_id, wait):
        pool_of(engine)[:, :, block_id].fill_(0)
        raise RuntimeError("injected copy failure")

    with monkeypatch.context() as patch:
        patch.setattr(cache, "_restore_from_slot", fail_copy)
        with pytest.raises(RuntimeError, match="injected"):
            cache.restore_block(key)
    assert key in cache and cache.bytes_used == cache.block_bytes
    assert key not in manager.hash_to_block_id
    assert_pool_consistent(manager)
    restored = cache.restore_block(key)
    assert torch.equal(block_bytes(engine, restored), expected)


def test_failed_save_does_not_publish_or_consume_budget(gpu, monkeypatch):
    engine, manager, key = completed_prefix(gpu)
    cache = new_cache(engine)
    mapping = manager.hash_to_block_id.copy()

    def fail_copy(*args, **kwargs):
        raise RuntimeError("host allocation/copy failed")

    with monkeypatch.context() as patch:
        patch.setattr(cache, "_save_to_slot", fail_copy)
        with pytest.raises(RuntimeError, match="host allocation/copy"):
            cache.save_block(key)
    assert len(cache) == cache.bytes_used == 0
    assert manager.hash_to_block_id == mapping
    assert_pool_consistent(manager)
    assert cache.save_block(key)


def test_budget_deduplication_and_explicit_discard(gpu):
    engine, manager, key = completed_prefix(gpu, [[90], [91]])
    cache = new_cache(engine)
    assert cache.save_block(key)
    assert not cache.save_block(key)
    overwrite_prefix(engine)
    assert not cache.save_block(key)  # the CPU copy survives the GPU miss
    engine.model_runner.batches = iter([[92]])
    engine.add_request([6] * 257, params(max_tokens=1))
    step(engine)
    other = manager.compute_hash([6] * BS)
    with pytest.raises(MemoryError, match="budget"):
        cache.save_block(other)
    assert cache.bytes_used == cache.block_bytes and other not in cache
    assert cache.discard(key) and not cache.discard(key)
    assert cache.bytes_used == 0
    assert cache.save_block(other)
    cache.clear()
    assert cache.bytes_used == len(cache) == 0
    assert other in manager.hash_to_block_id


def test_budget_smaller_than_one_block_rejects_before_allocating(gpu, monkeypatch):
    engine, _, key = completed_prefix(gpu)
    cache = engine.create_cpu_prefix_cache(max_bytes=1)

    def fail_allocation(*args, **kwargs):
        raise AssertionError("budget check must precede host allocation")

    monkeypatch.setattr(torch, "empty", fail_allocation)
    with pytest.raises(CPUCacheFullError, match="budget"):
        cache.save_block(key)
    assert cache.bytes_used == 0


def test_restore_without_space_preserves_active_request_and_cpu_entry(gpu):
    engine, manager, key = completed_prefix(gpu, [[90], [91]])
    cache = new_cache(engine)
    cache.save_block(key)
    engine.add_request([3] * 257, params(max_tokens=2))
    step(engine)
    before = manager.used_block_ids.copy()
    assert not manager.free_block_ids and key not in manager.hash_to_block_id
    with pytest.raises(MemoryError, match="free KV blocks"):
        cache.restore_block(key)
    assert manager.used_block_ids == before and key in cache
    assert_pool_consistent(manager)
    step(engine)
    assert cache.restore_block(key) in manager.hash_to_block_id.values()
    assert_pool_consistent(manager)


def test_existing_live_gpu_hit_is_not_overwritten_or_referenced_again(gpu, monkeypatch):
    engine = cached_engine(gpu, [[10]], num_blocks=2)
    engine.add_request([1] * 257, params(max_tokens=2))
    step(engine)
    manager = engine.scheduler.block_manager
    key = manager.compute_hash([1] * BS)
    cache = new_cache(engine)
    cache.save_block(key)
    block_id = manager.hash_to_block_id[key]
    references = manager.blocks[block_id].ref_count

    def fail_copy(*args, **kwargs):
        raise AssertionError("GPU hit must not be copied over")

    monkeypatch.setattr(cache, "_restore_from_slot", fail_copy)
    assert cache.restore_block(key) == block_id
    assert manager.blocks[block_id].ref_count == references
    assert not manager.free_block_ids
    assert_pool_consistent(manager)


def test_restore_chained_prefix_blocks_preserves_ancestry(gpu):
    engine = cached_engine(gpu, [[10], [90], [11]], budget=768, num_blocks=3)
    manager = engine.scheduler.block_manager
    original = [1] * 256 + [2] * 256 + [3]
    engine.add_request(original, params(max_tokens=1))
    step(engine)
    first = manager.compute_hash([1] * BS)
    second = manager.compute_hash([2] * BS, first)
    cache = new_cache(engine, blocks=2)
    cache.save_block(first)
    cache.save_block(second)
    engine.add_request([8] * 513, params(max_tokens=1))
    step(engine)
    assert first not in manager.hash_to_block_id and second not in manager.hash_to_block_id
    cache.restore_block(first)
    cache.restore_block(second)
    engine.add_request(original + [9] * 10, params(max_tokens=1))
    assert step(engine).num_tokens == 11
    assert_pool_consistent(manager)


def test_rejects_unknown_and_unpublished_partial_blocks(gpu):
    engine, manager, key = completed_prefix(gpu)
    cache = new_cache(engine)
    with pytest.raises(KeyError):
        cache.save_block(-1)
    with pytest.raises(KeyError):
        cache.restore_block(key)
    block = manager.blocks[manager.hash_to_block_id[key]]
    block.token_ids = block.token_ids[:-1]
    with pytest.raises(ValueError, match="full prefix block"):
        cache.save_block(key)
    assert len(cache) == 0


def test_conflicting_gpu_token_metadata_is_not_silently_reused(gpu):
    engine, manager, key = completed_prefix(gpu)
    cache = new_cache(engine)
    cache.save_block(key)
    manager.blocks[manager.hash_to_block_id[key]].token_ids = [7] * BS
    with pytest.raises(ValueError, match="conflicting token"):
        cache.save_block(key)
    with pytest.raises(ValueError, match="conflicting token"):
        cache.restore_block(key)
    assert cache.bytes_used == cache.block_bytes


def test_close_releases_pool_references_and_engine_exit_closes_cache(gpu):
    engine, _, key = completed_prefix(gpu)
    cache = new_cache(engine)
    cache.save_block(key)
    with pytest.raises(RuntimeError, match="already has"):
        new_cache(engine)
    cache.close()
    cache.close()
    assert cache.closed and cache.bytes_used == 0 and cache._manager is None
    with pytest.raises(RuntimeError, match="closed"):
        cache.save_block(key)
    with pytest.raises(RuntimeError, match="closed"):
        cache.restore_block(key)
    replacement = new_cache(engine)
    replacement.save_block(key)
    engine.exit()
    assert replacement.closed and replacement.bytes_used == 0
    assert engine.model_runner.calls[-1] == "exit"


def test_discarded_slots_are_reused_without_new_host_allocation(gpu, monkeypatch):
    engine, manager, key = completed_prefix(gpu, [[90], [91]])
    cache = new_cache(engine)
    assert cache.reserved_bytes == 0
    assert cache.save_block(key)
    assert cache.reserved_bytes == cache.block_bytes
    overwrite_prefix(engine)
    other = manager.compute_hash([3] * BS)
    assert cache.discard(key)

    def fail_allocation(*args, **kwargs):
        raise AssertionError("a free slot must be reused")

    monkeypatch.setattr(torch, "empty", fail_allocation)
    assert cache.save_block(other)
    assert cache.reserved_bytes == cache.bytes_used == cache.block_bytes


def test_preallocated_multi_slab_slots_round_trip_byte_exact(gpu, monkeypatch):
    import kvx.engine.cpu_prefix_cache as module

    monkeypatch.setattr(module, "_SLAB_CHUNK_BYTES", 1)
    engine, manager, key = completed_prefix(gpu, [[90], [91]])
    pool = pool_of(engine)
    cache = engine.create_cpu_prefix_cache(max_bytes=3 * pool[:, :, 0].numel() * pool.element_size(),
                                           preallocate=True)
    assert len(cache._slabs) == 3 and cache.reserved_bytes == 3 * cache.block_bytes
    expected = {key: block_bytes(engine, manager.hash_to_block_id[key])}
    cache.save_block(key)
    overwrite_prefix(engine)
    other = manager.compute_hash([3] * BS)
    expected[other] = block_bytes(engine, manager.hash_to_block_id[other])
    cache.save_block(other)
    assert cache._entries[key].slot != cache._entries[other].slot
    for prefix_hash, data in expected.items():
        manager.hash_to_block_id.pop(prefix_hash, None)
        restored = cache.restore_block(prefix_hash)
        assert torch.equal(block_bytes(engine, restored), data)


@pytest.mark.parametrize("bad_budget", [0, -1, 1.5, True])
def test_invalid_budget_is_rejected_before_creating_cache(gpu, bad_budget):
    """bench/test_cpu_prefix_cache.py:255-260."""
    engine, _, _ = completed_prefix(gpu)
    with pytest.raises(ValueError, match="positive integer"):
        engine.create_cpu_prefix_cache(bad_budget)
    assert engine._cpu_prefix_cache is None


def test_tp_and_layout_mismatch_are_rejected(gpu):
    """bench/test_cpu_prefix_cache.py:263-272."""
    engine, _, _ = completed_prefix(gpu)
    engine.model_runner.world_size = 2
    with pytest.raises(NotImplementedError, match="TP=1"):
        new_cache(engine)
    engine.model_runner.world_size = 1
    engine.model_runner.block_size = 128
    with pytest.raises(ValueError, match="layout"):
        new_cache(engine)


def test_save_on_release_requires_automatic_mode(gpu):
    """bench/test_cpu_prefix_cache.py:349-353."""
    engine, _, _ = completed_prefix(gpu)
    with pytest.raises(ValueError, match="automatic"):
        engine.create_cpu_prefix_cache(max_bytes=1 << 20, save_on_release=True)
    assert engine._cpu_prefix_cache is None


# -- bench/test_automatic_cpu_cache.py --------------------------------------------

def automatic_cache(engine, blocks=2, **kwargs):
    return new_cache(engine, blocks=blocks, automatic=True, **kwargs)


def test_automatic_save_restore_and_next_turn_without_manual_calls(gpu):
    engine, manager, key = completed_prefix(gpu, [[90], [91], [12]])
    source = manager.hash_to_block_id[key]
    expected = block_bytes(engine, source)
    cache = automatic_cache(engine, blocks=1)
    write_scheduled_kv(engine)
    for prompt in ([3] * 257, [4]):
        engine.add_request(prompt, params(max_tokens=1))
        step(engine)
    assert key not in manager.hash_to_block_id and key in cache
    engine.add_request([1] * 257 + [10, 11] + [2] * 10, params(max_tokens=1))
    assert step(engine).num_tokens == 13
    target = manager.hash_to_block_id[key]
    assert target != source
    assert torch.equal(block_bytes(engine, target), expected)
    assert cache.stats == {"saved_blocks": 1, "restored_blocks": 1, "budget_skips": 1}
    assert not manager.used_block_ids
    assert_pool_consistent(manager)


@pytest.mark.parametrize("cpu_logical", [0, 1])
def test_all_gpu_hits_are_protected_before_any_cpu_restore(gpu, cpu_logical):
    engine = cached_engine(gpu, [[10], [90], [11]], budget=768, num_blocks=3)
    manager = engine.scheduler.block_manager
    original = [1] * 256 + [2] * 256 + [3]
    engine.add_request(original, params(max_tokens=1))
    step(engine)
    first = manager.compute_hash([1] * BS)
    second = manager.compute_hash([2] * BS, first)
    keys = [first, second]
    victim = manager.hash_to_block_id[keys[cpu_logical]]
    gpu_hit = manager.hash_to_block_id[keys[1 - cpu_logical]]
    cache = automatic_cache(engine, blocks=1)
    write_scheduled_kv(engine)
    tail = next(i for i in manager.free_block_ids if i not in (victim, gpu_hit))
    manager.free_block_ids = deque([victim, gpu_hit, tail])
    engine.add_request([9], params(max_tokens=1))
    step(engine)
    assert keys[cpu_logical] in cache
    assert manager.free_block_ids[0] == gpu_hit
    expected = block_bytes(engine, gpu_hit)
    engine.add_request(original + [8] * 10, params(max_tokens=1))
    assert step(engine).num_tokens == 11
    assert manager.hash_to_block_id[keys[1 - cpu_logical]] == gpu_hit
    assert torch.equal(block_bytes(engine, gpu_hit), expected)
    assert cache.stats["restored_blocks"] == 1
    assert_pool_consistent(manager)


def test_cpu_hit_waits_for_capacity_without_mutating_pool_during_lookup(gpu):
    engine, manager, key = completed_prefix(gpu, [[90], [91], [12]])
    cache = automatic_cache(engine, blocks=1)
    write_scheduled_kv(engine)
    engine.add_request([3] * 257, params(max_tokens=2))
    step(engine)
    engine.add_request([1] * 257 + [10, 11] + [2] * 10, params(max_tokens=1))
    waiting = engine.scheduler.waiting[0]
    before = (manager.used_block_ids.copy(), manager.hash_to_block_id.copy(), cache.stats)
    assert key in cache and not manager.free_block_ids
    assert manager.can_allocate(waiting) == -1
    assert (manager.used_block_ids, manager.hash_to_block_id, cache.stats) == before
    assert not waiting.block_table
    assert step(engine).num_tokens == -1  # the running decode completes
    assert step(engine).num_tokens == 13
    assert cache.stats["restored_blocks"] == 1
    assert_pool_consistent(manager)


def test_full_cpu_budget_falls_back_to_recomputation(gpu):
    engine, manager, key = completed_prefix(gpu, [[90], [91], [12]])
    cache = engine.create_cpu_prefix_cache(max_bytes=1, automatic=True)
    for prompt in ([3] * 257, [4]):
        engine.add_request(prompt, params(max_tokens=1))
        step(engine)
    assert key not in cache and key not in manager.hash_to_block_id
    engine.add_request([1] * 257 + [10, 11] + [2] * 10, params(max_tokens=1))
    assert step(engine).num_tokens == 269
    assert cache.stats["budget_skips"] >= 1
    assert cache.stats["saved_blocks"] == cache.stats["restored_blocks"] == 0
    assert_pool_consistent(manager)


def test_gpu_hits_are_shared_with_active_requests_without_cpu_copy(gpu):
    """bench/test_automatic_cpu_cache.py:142-155."""
    engine = cached_engine(gpu, [[10], [20]], budget=512, num_blocks=3)
    manager = engine.scheduler.block_manager
    cache = automatic_cache(engine)
    first_id = engine.add_request([1] * 257, params(max_tokens=3))
    step(engine)
    first = engine.scheduler.running[0]
    block_id = manager.hash_to_block_id[manager.compute_hash([1] * BS)]
    engine.add_request([1] * 257 + [10] + [2] * 10, params(max_tokens=1))
    assert step(engine).num_tokens == 12
    assert first.seq_id == first_id and manager.blocks[block_id].ref_count == 1
    assert cache.stats == {"saved_blocks": 0, "restored_blocks": 0, "budget_skips": 0}
    assert_pool_consistent(manager)


def test_resume_allocation_failure_releases_partially_reserved_blocks(gpu, monkeypatch):
    """bench/test_automatic_cpu_cache.py:273-287, with the real cache (tests/test_block_manager.py has a fake)."""
    engine, manager, _ = completed_prefix(gpu)
    cache = automatic_cache(engine)
    seq = Sequence([1] * 257, params(max_tokens=3))
    seq.append_token(10)

    def fail(*args):
        raise RuntimeError("preservation failed")

    monkeypatch.setattr(cache, "save_block", fail)
    with pytest.raises(RuntimeError, match="preservation failed"):
        manager.allocate_for_resume(seq, 257)
    assert not seq.block_table and seq.num_cached_tokens == 0
    assert not manager.used_block_ids
    assert_pool_consistent(manager)


def test_failed_later_admission_keeps_already_prefilled_chunks(gpu, monkeypatch):
    """bench/test_automatic_cpu_cache.py:290-326."""
    engine = cached_engine(gpu, [[20], [90], [91], [92], [10], [13, 14]], budget=512, num_blocks=5)
    manager = engine.scheduler.block_manager
    engine.add_request([3] * 257, params(max_tokens=1))
    step(engine)
    cache = automatic_cache(engine, blocks=2)
    key = manager.compute_hash([3] * BS)
    cache.save_block(key)
    engine.add_request([9] * 1025, params(max_tokens=1))
    for _ in range(3):
        step(engine)
    assert key not in manager.hash_to_block_id
    first_id = engine.add_request([1] * 513, params(max_tokens=1))
    second_id = engine.add_request([3] * 257, params(max_tokens=1))
    step(engine)  # the first request's first 512 tokens are prefilled
    first = engine.scheduler.waiting[0]
    blocks = first.block_table.copy()
    assert first.num_cached_tokens == 512

    def fail(*args, **kwargs):
        raise RuntimeError("restore failed")

    with monkeypatch.context() as patch:
        patch.setattr(cache, "_copy_entry", fail)
        with pytest.raises(RuntimeError, match="restore failed"):
            step(engine)
    assert [seq.seq_id for seq in engine.scheduler.waiting] == [first_id, second_id]
    assert not engine.scheduler.running
    assert first.block_table == blocks and first.num_cached_tokens == 512 and first.num_scheduled_tokens == 0
    assert manager.used_block_ids == set(blocks)
    assert_pool_consistent(manager)
    result = step(engine)
    assert result.num_tokens == 2
    assert result.outputs == [(first_id, [13]), (second_id, [14])]
    assert not manager.used_block_ids


def test_cpu_hits_do_not_make_an_oversized_active_request_fit(gpu):
    """bench/test_automatic_cpu_cache.py:329-340."""
    engine, manager, key = completed_prefix(gpu, [[90], [91]])
    cache = automatic_cache(engine, blocks=1)
    for prompt in ([3] * 257, [4]):
        engine.add_request(prompt, params(max_tokens=1))
        step(engine)
    assert key in cache and key not in manager.hash_to_block_id
    seq = Sequence([1] * 513, params(max_tokens=1))
    before = (list(manager.free_block_ids), cache.stats)
    assert manager.can_allocate(seq) == -1  # three GPU blocks needed, the pool has two
    assert (list(manager.free_block_ids), cache.stats) == before
    assert not seq.block_table


def test_repeated_admission_checks_do_not_rehash_a_waiting_prompt(gpu, monkeypatch):
    """bench/test_automatic_cpu_cache.py:391-404."""
    engine, manager, key = completed_prefix(gpu, [[90], [91]])
    cache = automatic_cache(engine, blocks=1)
    for prompt in ([3] * 257, [4]):
        engine.add_request(prompt, params(max_tokens=1))
        step(engine)
    assert key in cache and key not in manager.hash_to_block_id
    seq = Sequence([1] * 257, params(max_tokens=1))
    assert manager.can_allocate(seq) == 1
    calls = []
    original = manager.compute_hash
    monkeypatch.setattr(manager, "compute_hash", lambda *a: calls.append(a) or original(*a))
    assert manager.can_allocate(seq) == 1
    assert calls == []


def test_close_detaches_automatic_hooks(gpu):
    engine, manager, key = completed_prefix(gpu, [[90], [91], [12]])
    cache = automatic_cache(engine)
    assert cache.automatic
    cache.close()
    assert not cache.automatic and manager._cpu_prefix_cache is None
    for prompt in ([3] * 257, [4]):
        engine.add_request(prompt, params(max_tokens=1))
        step(engine)
    engine.add_request([1] * 257 + [10, 11] + [2] * 10, params(max_tokens=1))
    assert step(engine).num_tokens == 269
    assert cache.stats["saved_blocks"] == 0


def test_prefill_batch_restore_failure_rolls_back_all_admissions(gpu, monkeypatch):
    engine = cached_engine(gpu, [[10], [20], [90], [13, 14]], budget=1024, num_blocks=4)
    manager = engine.scheduler.block_manager
    engine.add_request([1] * 257, params(max_tokens=1))
    step(engine)
    cache = automatic_cache(engine, blocks=2)
    first = manager.compute_hash([1] * BS)
    cache.save_block(first)
    engine.add_request([3] * 257, params(max_tokens=1))
    step(engine)
    second = manager.compute_hash([3] * BS)
    cache.save_block(second)
    engine.add_request([9] * 769, params(max_tokens=1))
    step(engine)
    assert first not in manager.hash_to_block_id and second not in manager.hash_to_block_id
    ids = [engine.add_request([value] * 257, params(max_tokens=1)) for value in (1, 3)]
    calls = []
    original = cache._copy_entry

    def fail_second(entry, block_id, wait=True):
        calls.append(block_id)
        if len(calls) == 2:
            pool_of(engine)[:, :, block_id].fill_(0)
            raise RuntimeError("restore failed")
        original(entry, block_id, wait)

    with monkeypatch.context() as patch:
        patch.setattr(cache, "_copy_entry", fail_second)
        with pytest.raises(RuntimeError, match="restore failed"):
            step(engine)
    assert [seq.seq_id for seq in engine.scheduler.waiting] == ids
    assert not engine.scheduler.running and not manager.used_block_ids
    assert all(not seq.block_table and seq.num_cached_tokens == seq.num_scheduled_tokens == 0
               for seq in engine.scheduler.waiting)
    assert len([c for c in engine.model_runner.calls if c != "exit"]) == 3
    assert_pool_consistent(manager)
    result = step(engine)
    assert result.num_tokens == 2  # one uncached tail token per 257-token prompt
    assert result.outputs == [(ids[0], [13]), (ids[1], [14])]
    assert_pool_consistent(manager)


def test_decode_growth_failure_restores_queue_and_tail_reservations(gpu, monkeypatch):
    engine = cached_engine(gpu, [[80], [81], [10, 20], [11, 21]], budget=512, num_blocks=4)
    manager = engine.scheduler.block_manager
    for value in (7, 8):
        engine.add_request([value] * 256, params(max_tokens=1))
        step(engine)
    cache = automatic_cache(engine, blocks=2)
    ids = [engine.add_request([value] * 256, params(max_tokens=2)) for value in (1, 2)]
    step(engine)
    before = manager.used_block_ids.copy()
    original = cache.save_block
    count = 0

    def fail_second(key):
        nonlocal count
        count += 1
        if count == 2:
            raise RuntimeError("preservation failed")
        return original(key)

    with monkeypatch.context() as patch:
        patch.setattr(cache, "save_block", fail_second)
        with pytest.raises(RuntimeError, match="preservation failed"):
            step(engine)
    assert [seq.seq_id for seq in engine.scheduler.running] == ids
    assert manager.used_block_ids == before
    assert all(len(seq.block_table) == 1 and seq.num_scheduled_tokens == 0 for seq in engine.scheduler.running)
    assert_pool_consistent(manager)
    assert step(engine).outputs == [(ids[0], [10, 11]), (ids[1], [20, 21])]
    assert not manager.used_block_ids
    assert_pool_consistent(manager)


@pytest.mark.parametrize("slow", [False, True])
def test_save_on_release_saves_idle_blocks_before_recycling_overwrites_them(gpu, slow):
    engine = cached_engine(gpu, [[10], [11], [90], [12]], num_blocks=2)
    pool = pool_of(engine)
    manager = engine.scheduler.block_manager
    size = pool[:, :, 0].numel() * pool.element_size()
    cache = engine.create_cpu_prefix_cache(max_bytes=size, automatic=True, save_on_release=True)
    if slow:
        slow_copies(cache)
    write_scheduled_kv(engine)
    engine.add_request([1] * 257, params(max_tokens=2))
    step(engine)
    engine.add_request([3] * 257, params(max_tokens=1))
    step(engine)  # [3] waits for blocks while [1] decodes, then [1] releases
    key = manager.compute_hash([1] * BS)
    assert key in cache and key in manager.hash_to_block_id
    assert cache.stats["saved_blocks"] == 1
    expected = block_bytes(engine, manager.hash_to_block_id[key])
    step(engine)  # admitting [3] recycles the source block: the pending save must win
    assert engine.is_finished() and key not in manager.hash_to_block_id
    engine.add_request([1] * 257 + [10, 11] + [2] * 10, params(max_tokens=1))
    assert step(engine).num_tokens == 13
    target = manager.hash_to_block_id[key]
    assert torch.equal(block_bytes(engine, target), expected)
    assert cache.stats["saved_blocks"] == cache.stats["restored_blocks"] == 1
    assert not manager.used_block_ids
    assert_pool_consistent(manager)


def test_save_on_release_waits_for_blocked_admission(gpu):
    engine = cached_engine(gpu, [[10], [11]], num_blocks=4)
    pool = pool_of(engine)
    size = pool[:, :, 0].numel() * pool.element_size()
    cache = engine.create_cpu_prefix_cache(max_bytes=size, automatic=True, save_on_release=True)
    engine.add_request([1] * 257, params(max_tokens=2))
    step(engine)
    step(engine)
    assert engine.is_finished() and cache.stats["saved_blocks"] == 0


@pytest.mark.parametrize("slow", [False, True])
def test_prefetch_restores_blocked_waiting_hits_while_others_decode(gpu, slow):
    engine = cached_engine(gpu, [[10], [20], [21], [22], [30]], num_blocks=4)
    pool = pool_of(engine)
    manager = engine.scheduler.block_manager
    size = pool[:, :, 0].numel() * pool.element_size()
    cache = engine.create_cpu_prefix_cache(max_bytes=2 * size, automatic=True, prefetch=True)
    if slow:
        slow_copies(cache)
    write_scheduled_kv(engine)
    engine.add_request([1] * 257, params(max_tokens=1))
    step(engine)
    key = manager.compute_hash([1] * BS)
    source = manager.hash_to_block_id[key]
    expected = block_bytes(engine, source)
    cache.save_block(key)
    cache.synchronize()  # zero_() below bypasses the allocator's ordering
    del manager.hash_to_block_id[key]
    manager.blocks[source].hash, manager.blocks[source].token_ids = -1, []
    pool[:, :, source].zero_()
    engine.add_request([3] * 257, params(max_tokens=3))
    step(engine)  # the running request holds 2 of 4 blocks
    waiting = engine.add_request([1] * 256 + [5] * 300, params(max_tokens=1))
    step(engine)  # needs 3 blocks; one spare block prefetches its hit
    assert key in manager.hash_to_block_id and cache.prefetched_blocks == 1
    assert [seq.seq_id for seq in engine.scheduler.waiting] == [waiting]
    step(engine)
    result = step(engine)
    assert result.num_tokens == 300  # admitted with the prefetched block as a GPU hit
    target = manager.hash_to_block_id[key]
    assert torch.equal(block_bytes(engine, target), expected)
    assert cache.stats["restored_blocks"] == 1
    assert not manager.used_block_ids
    assert_pool_consistent(manager)


# -- bench/test_cpu_cache_optimizations.py --------------------------------------

def test_fp8_payload_is_smaller_and_restores_within_quantization_error(gpu):
    engine, manager, (key,) = finite_prefix(gpu, [[90], [91]])
    pool = pool_of(engine)
    source = pool[:, :, manager.hash_to_block_id[key]].float().cpu().clone()
    bf16_bytes = pool[:, :, 0].numel() * pool.element_size()
    cache = engine.create_cpu_prefix_cache(max_bytes=4 * bf16_bytes, fp8=True)
    numel = pool[:, :, 0].numel()
    assert cache.block_bytes == numel + numel // pool.shape[-1] * pool.element_size()
    assert cache.save_block(key)
    overwrite_prefix(engine)
    assert key not in manager.hash_to_block_id
    target = cache.restore_block(key)
    cache.synchronize()
    restored = pool[:, :, target].float().cpu()
    bound = source.abs().amax(-1, keepdim=True) / 16
    assert torch.all((restored - source).abs() <= bound)
    assert cache.stats["restored_blocks"] == 1


def split_stream_cache(gpu):
    engine, manager, (key,) = finite_prefix(gpu, [[90], [91], [92], [93]], num_blocks=3)
    pool = pool_of(engine)
    size = pool[:, :, 0].numel() * pool.element_size()
    cache = engine.create_cpu_prefix_cache(max_bytes=size, split_streams=True, preallocate=True)
    assert cache._restore_stream is not cache._copy_stream
    for slab in cache._slab_memory:
        slab.fill_(0xAB)
    return engine, manager, key, pool, cache


def forget_gpu_copy(manager, key):
    block_id = manager.hash_to_block_id.pop(key)
    manager.blocks[block_id].hash, manager.blocks[block_id].token_ids = -1, []
    return block_id


@pytest.mark.parametrize("slow", [False, True])
def test_split_streams_restore_waits_for_its_save(gpu, slow):
    engine, manager, key, pool, cache = split_stream_cache(gpu)
    if slow:
        slow_copies(cache, ["_save_to_slot"])
    expected = block_bytes(engine, manager.hash_to_block_id[key])
    assert cache.save_block(key)
    forget_gpu_copy(manager, key)
    target = cache.restore_block(key)
    cache.synchronize()
    assert torch.equal(block_bytes(engine, target), expected)


@pytest.mark.parametrize("slow", [False, True])
def test_split_streams_slot_reuse_waits_for_pending_restore(gpu, slow):
    engine, manager, key, pool, cache = split_stream_cache(gpu)
    expected = block_bytes(engine, manager.hash_to_block_id[key])
    assert cache.save_block(key)
    cache.synchronize()
    forget_gpu_copy(manager, key)
    if slow:
        slow_copies(cache, ["_restore_from_slot"])
    entry = cache._entries[key]
    target = manager.restore_cached_block(
        key, entry.token_ids, lambda block_id: cache._copy_entry(entry, block_id, wait=False))
    assert cache.discard(key)
    other = next(i for i in range(len(manager.blocks)) if i != target)
    pool[:, :, other].fill_(7)
    manager.blocks[other].update(12345, [2] * BS)
    manager.hash_to_block_id[12345] = other
    assert cache.save_block(12345)  # reuses the slot the restore is still reading
    cache.synchronize()
    assert torch.equal(block_bytes(engine, target), expected)
    assert torch.equal(cache._slot_view(0)[0].view(torch.uint8), block_bytes(engine, other))


def drop_gpu_copies(cache, manager, pool, keys):
    for key in keys:
        cache.save_block(key)
    cache.synchronize()
    for key in keys:
        block_id = manager.hash_to_block_id.pop(key)
        manager.blocks[block_id].hash, manager.blocks[block_id].token_ids = -1, []
        pool[:, :, block_id].zero_()


@pytest.mark.parametrize("slow", [False, True])
def test_split_admission_recomputes_head_while_restoring_tail(gpu, slow):
    engine, manager, keys = finite_prefix(gpu, [[90], [91], [92]], blocks=3, num_blocks=5)
    pool = pool_of(engine)
    size = pool[:, :, 0].numel() * pool.element_size()
    expected = [block_bytes(engine, manager.hash_to_block_id[key]) for key in keys]
    cache = engine.create_cpu_prefix_cache(max_bytes=3 * size, automatic=True)
    cache.hybrid = (1.0, 1 / 256, 0)
    drop_gpu_copies(cache, manager, pool, keys)
    if slow:
        slow_copies(cache)
    write_scheduled_kv(engine)
    request = engine.add_request([1] * 768 + [5] * 10, params(max_tokens=1))
    head = step(engine)
    seq = next(seq for seq in engine.scheduler.waiting if seq.seq_id == request)
    assert head.num_tokens == 256 and seq.restore_span is None and seq.num_cached_tokens == 768
    assert cache.stats["restored_blocks"] == 2
    assert torch.equal(block_bytes(engine, seq.block_table[1]), expected[1])
    assert torch.equal(block_bytes(engine, seq.block_table[2]), expected[2])
    assert manager.hash_to_block_id[keys[0]] == seq.block_table[0]
    tail = step(engine)
    assert tail.num_tokens == 10 and tail.outputs
    assert engine.is_finished() and not manager.used_block_ids
    assert_pool_consistent(manager)


def test_prefetch_hint_restores_cpu_hits_into_free_blocks(gpu):
    engine, manager, keys = finite_prefix(gpu, blocks=2, num_blocks=4)
    pool = pool_of(engine)
    size = pool[:, :, 0].numel() * pool.element_size()
    expected = [block_bytes(engine, manager.hash_to_block_id[key]) for key in keys]
    cache = engine.create_cpu_prefix_cache(max_bytes=2 * size, automatic=True, prefetch=True)
    drop_gpu_copies(cache, manager, pool, keys)
    hint = Sequence([1] * 512 + [7], params(max_tokens=1))
    assert engine.prefetch_prefix(hint) == 2
    assert engine.prefetch_prefix(hint) == 0  # nothing changed: throttled
    cache.synchronize()
    for key, payload in zip(keys, expected):
        assert torch.equal(block_bytes(engine, manager.hash_to_block_id[key]), payload)
    engine.add_request([9], params(max_tokens=1))
    assert engine.prefetch_prefix([1] * 600) == 0  # never while a request waits
    assert_pool_consistent(manager)


def test_later_requests_join_the_step_of_a_split_admission_head(gpu):
    engine, manager, keys = finite_prefix(gpu, [[90, 91], [92]], blocks=3, num_blocks=6)
    pool = pool_of(engine)
    size = pool[:, :, 0].numel() * pool.element_size()
    cache = engine.create_cpu_prefix_cache(max_bytes=3 * size, automatic=True)
    cache.hybrid = (1.0, 1 / 256, 0)
    drop_gpu_copies(cache, manager, pool, keys)
    split = engine.add_request([1] * 768 + [5] * 10, params(max_tokens=1))
    short = engine.add_request([8] * 10, params(max_tokens=1))
    first = step(engine)
    assert first.num_tokens == 256 + 10
    assert [seq.seq_id for seq in engine.scheduler.waiting] == [split]
    assert first.outputs == [(short, [91])]  # the split head samples nothing yet; the short request finishes
    assert step(engine).num_tokens == 10
    assert engine.is_finished()
    assert_pool_consistent(manager)


def test_split_admission_that_recomputes_everything_uses_no_restore(gpu):
    """bench/test_cpu_cache_optimizations.py:178-189."""
    engine, manager, keys = finite_prefix(gpu, [[90], [91]], blocks=2, num_blocks=4)
    pool = pool_of(engine)
    size = pool[:, :, 0].numel() * pool.element_size()
    cache = engine.create_cpu_prefix_cache(max_bytes=2 * size, automatic=True)
    cache.hybrid = (1.0, 0, 0)  # recompute is free
    drop_gpu_copies(cache, manager, pool, keys)
    request = engine.add_request([1] * 512 + [5], params(max_tokens=1))
    step(engine)
    seq = next(seq for seq in engine.scheduler.waiting if seq.seq_id == request)
    assert seq.num_cached_tokens == 512 and seq.restore_span is None  # computed, not skipped
    assert cache.stats["restored_blocks"] == 0


def test_hybrid_requires_automatic_cache(gpu):
    """bench/test_cpu_cache_optimizations.py:207-211."""
    engine, _, _ = finite_prefix(gpu)
    cache = engine.create_cpu_prefix_cache(max_bytes=1 << 20)
    with pytest.raises(ValueError, match="automatic"):
        cache.hybrid = (1.0, 0, 0)


# -- bench/test_prefill_scheduling.py --------------------------------------------

@pytest.mark.parametrize("fp8", [False, True])
def test_cpu_restoration_and_prefill_budget_compose(gpu, fp8):
    """bench/test_prefill_scheduling.py:178-193: a CPU hit admitted under a small
    prefill token budget is restored once, then its uncached tail is prefilled in
    budget-sized chunks. The restored block also holds the saved bytes (BF16
    byte-exact, FP8 within the reference's per-row bound). The reference sets the
    budget through its chunked prefill policy; here it is the batch token budget."""
    engine = cached_engine(gpu, [[10], [90], [91], [92], [12]], budget=512, num_blocks=2)
    manager = engine.scheduler.block_manager
    engine.add_request([1] * 257, params(max_tokens=1))
    step(engine)
    key = manager.compute_hash([1] * BS)
    pool = pool_of(engine)
    before = pool[:, :, manager.hash_to_block_id[key]].clone()
    size = pool[:, :, 0].numel() * pool.element_size()
    cache = engine.create_cpu_prefix_cache(size, automatic=True, fp8=fp8)
    for value, length in ((3, 257), (4, 1)):
        engine.add_request([value] * length, params(max_tokens=1))
        step(engine)
    assert key not in manager.hash_to_block_id and key in cache
    engine.scheduler.max_num_batched_tokens = 8
    engine.add_request([1] * 269, params(max_tokens=1))
    assert step(engine).num_tokens == 8
    assert cache.stats["restored_blocks"] == 1
    torch.cuda.synchronize(pool.device)
    after = pool[:, :, manager.hash_to_block_id[key]]
    if fp8:
        row_amax = before.float().abs().amax(dim=-1, keepdim=True)
        assert bool(((after.float() - before.float()).abs() <= row_amax / 16).all())
    else:
        assert torch.equal(after.view(torch.int16), before.view(torch.int16))
    assert step(engine).num_tokens == 5
    assert engine.is_finished()
    assert_pool_consistent(manager)
