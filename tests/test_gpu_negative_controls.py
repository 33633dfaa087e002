"""Negative controls for the copy engine's ordering rules.

Each test drops exactly one rule (kvx_cache_set_debug) in a scenario where a
delay kernel on one copy stream lets the unordered access overtake the other,
and asserts that the bytes come out wrong in at least one of a few attempts.
The same scenarios pass with every rule in place (the last tests here), as do
the matching positive tests (test_gpu_cache.py, test_gpu_engine.py), so these
show those tests would catch a missing wait.
The reference claims such controls (README.md:114-117) but commits none.
"""

from collections import deque
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from helpers import u8
from kvx import _lib, ops
from kvx.engine.block_manager import BlockManager
from kvx.engine.cpu_prefix_cache import CPUBlockCache

pytestmark = pytest.mark.gpu
BS = 256


def pool_with_bytes(device, blocks):
    pool = torch.empty((2, 2, blocks, BS, 1, 4), dtype=torch.bfloat16, device=device)
    raw = torch.arange(pool.numel() * 2, device=device).remainder(251).to(torch.uint8)
    pool.view(torch.uint8).copy_(raw.view(pool.view(torch.uint8).shape))
    return pool


def publish(manager, block_id, token):
    tokens = [token] * BS
    h = manager.compute_hash(tokens)
    manager.blocks[block_id].update(h, tokens)
    manager.hash_to_block_id[h] = block_id
    return h


def forget(manager, key):
    block_id = manager.hash_to_block_id.pop(key)
    manager.blocks[block_id].hash, manager.blocks[block_id].token_ids = -1, []


def cache_for(pool, manager, blocks, **kwargs):
    size = pool[:, :, 0].numel() * pool.element_size()
    runner = SimpleNamespace(world_size=1, block_size=BS, kv_cache=pool)
    return CPUBlockCache(runner, manager, blocks * size, **kwargs)


def delay(stream, device):
    ops.sleep(20_000, stream=stream, device=device)


def block(pool, b):
    torch.cuda.synchronize()
    return u8(pool[:, :, b])


# The HIP runtime maps every stream onto one of the process's few hardware
# queues, and a delay kernel holds up everything queued behind it on its
# queue. When the two streams of a scenario share a queue, the unordered
# access runs in queue order and the race stays hidden. Each scenario
# therefore runs on fresh caches, whose streams come from the next torch pool
# slots, until one attempt shows the race; the control requires that one does.
ATTEMPTS = 6


def shows_race(scenario, *args):
    return any(scenario(*args) for _ in range(ATTEMPTS))


def restore_without_save_wait(gpu, debug=_lib.DEBUG_SKIP_SAVE_WAIT):
    pool = pool_with_bytes(gpu, 3)
    manager = BlockManager(3, BS)
    key = publish(manager, 0, 1)
    cache = cache_for(pool, manager, 1, split_streams=True, preallocate=True)
    cache._slab_memory[0].fill_(0xAB)
    expected = block(pool, 0)
    cache._engine.set_debug(debug)
    delay(cache._copy_stream, gpu)
    assert cache.save_block(key)
    forget(manager, key)
    manager.free_block_ids = deque([1, 2, 0])  # restore into a block no save is pending on
    target = cache.restore_block(key)
    cache.synchronize()
    assert target == 1
    got = block(pool, target)
    cache.close()
    if np.array_equal(got, expected):
        return False
    assert np.all(got == 0xAB)  # it copied the poison
    return True


def test_restore_reads_a_poisoned_slot_without_the_save_wait(gpu):
    assert shows_race(restore_without_save_wait, gpu)


def reuse_without_reuse_wait(gpu, compute, debug=_lib.DEBUG_SKIP_REUSE_WAIT):
    """One save delayed on the copy stream, then a compute-stream write with the reuse wait dropped."""
    pool = pool_with_bytes(gpu, 2)
    manager = BlockManager(2, BS)
    key = publish(manager, 1, 1)
    with torch.cuda.stream(compute):
        cache = cache_for(pool, manager, 1)
        expected = block(pool, 1)
        cache._engine.set_debug(debug)
        delay(cache._copy_stream, gpu)
        assert cache.save_block(key)
        forget(manager, key)
        cache.before_block_reuse(1)  # no longer waits for the save
        pool.fill_(-7)
        target = cache.restore_block(key)
        cache.synchronize()
        corrupted = not np.array_equal(block(pool, target), expected)
    cache.close()
    return corrupted


def test_compute_overwrites_a_block_before_its_save_without_the_reuse_wait(gpu):
    # The compute stream matters here too: torch's default stream first, then pool streams.
    candidates = [torch.cuda.default_stream(gpu)] + [torch.cuda.Stream(gpu) for _ in range(ATTEMPTS - 1)]
    assert any(reuse_without_reuse_wait(gpu, s) for s in candidates)


def restore_without_victim_wait(gpu, debug=_lib.DEBUG_SKIP_VICTIM_WAIT):
    pool = pool_with_bytes(gpu, 2)
    manager = BlockManager(2, BS)
    victim_key = publish(manager, 0, 3)
    key = publish(manager, 1, 4)
    cache = cache_for(pool, manager, 2, automatic=True, split_streams=True)
    victim_bytes = block(pool, 0)
    assert cache.save_block(key)
    cache.synchronize()
    forget(manager, key)
    cache._engine.set_debug(debug)
    original = cache._save_to_slot

    def slow_save(block_id, slot):
        delay(cache._copy_stream, gpu)
        original(block_id, slot)

    cache._save_to_slot = slow_save
    entry = cache._entries[key]
    target = manager.restore_cached_block(key, entry.token_ids,
                                          lambda b: cache._copy_entry(entry, b, wait=False))
    assert target == 0 and victim_key in cache
    cache.synchronize()
    corrupted = not np.array_equal(u8(cache._entries[victim_key].kv), victim_bytes)
    cache.close()
    return corrupted


def test_restore_overwrites_a_victim_before_its_save_without_the_victim_wait(gpu):
    assert shows_race(restore_without_victim_wait, gpu)


def save_without_slot_read_wait(gpu, debug=_lib.DEBUG_SKIP_SLOT_READ_WAIT):
    pool = pool_with_bytes(gpu, 3)
    manager = BlockManager(3, BS)
    key_a = publish(manager, 0, 5)
    cache = cache_for(pool, manager, 1, automatic=True, split_streams=True)
    expected = block(pool, 0)
    assert cache.save_block(key_a)
    cache.synchronize()
    forget(manager, key_a)
    cache._engine.set_debug(debug)
    entry = cache._entries[key_a]
    manager.free_block_ids = deque([2, 0, 1])
    delay(cache._restore_stream, gpu)
    # A prefetch restore (the compute stream does not wait for it) still reading slot 0 ...
    target = manager.restore_cached_block(key_a, entry.token_ids,
                                          lambda b: cache._copy_entry(entry, b, wait=False))
    assert target == 2
    # ... when its entry is dropped and another block's save reuses the slot.
    assert cache.discard(key_a)
    key_b = publish(manager, 1, 6)
    assert cache.save_block(key_b)
    assert cache._entries[key_b].slot == entry.slot
    cache.synchronize()
    got = block(pool, target)
    cache.close()
    return not np.array_equal(got, expected)


def test_save_overwrites_a_slot_a_prefetch_still_reads_without_the_slot_read_wait(gpu):
    assert shows_race(save_without_slot_read_wait, gpu)


def test_chunked_recycle_overwrites_victims_before_their_save_without_the_victim_wait(gpu):
    from test_gpu_cache import chunked_recycle

    assert shows_race(lambda device: not chunked_recycle(device, _lib.DEBUG_SKIP_VICTIM_WAIT), gpu)


def test_a_prefetch_overwrites_a_later_waited_restore_without_the_overwrite_wait(gpu):
    from test_gpu_cache import waited_restore_over_prefetch

    assert shows_race(lambda device: not waited_restore_over_prefetch(device, _lib.DEBUG_SKIP_OVERWRITE_WAIT), gpu)


def test_a_save_overwrites_a_slot_another_callers_stream_still_reads_without_the_slot_read_wait(gpu):
    from test_gpu_cache import slot_reuse_across_caller_streams

    assert shows_race(lambda device: not slot_reuse_across_caller_streams(device, _lib.DEBUG_SKIP_SLOT_READ_WAIT), gpu)


@pytest.mark.parametrize("scenario", [restore_without_save_wait, restore_without_victim_wait,
                                      save_without_slot_read_wait], ids=lambda f: f.__name__)
def test_each_scenario_keeps_its_bytes_with_every_rule_in_place(gpu, scenario):
    # The same scenarios with no rule dropped: no attempt may show a race.
    assert not any(scenario(gpu, 0) for _ in range(ATTEMPTS))


def test_the_reuse_scenario_keeps_its_bytes_with_every_rule_in_place(gpu):
    candidates = [torch.cuda.default_stream(gpu)] + [torch.cuda.Stream(gpu) for _ in range(ATTEMPTS - 1)]
    assert not any(reuse_without_reuse_wait(gpu, s, 0) for s in candidates)


@pytest.mark.parametrize("scenario", ["chunked_recycle", "waited_restore_over_prefetch",
                                      "slot_reuse_across_caller_streams"])
def test_the_engine_level_scenarios_keep_their_bytes_with_every_rule_in_place(gpu, scenario):
    # As often as their controls run them, each time on fresh streams.
    import test_gpu_cache

    assert all(getattr(test_gpu_cache, scenario)(gpu) for _ in range(ATTEMPTS))
