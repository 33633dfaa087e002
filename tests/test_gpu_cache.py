"""CPUBlockCache over libkvx's copy engine, restating the reference's cache tests on a ROCm pool.

Sources: bench/test_cpu_prefix_cache.py, bench/test_cpu_cache_optimizations.py and
bench/test_automatic_cpu_cache.py. The reference drives these through its engine
with a scripted model; here the block manager is driven directly (publishing
blocks as a finished prefill would), which exercises the same cache hooks.
Ordering is stressed the reference's way: a delay kernel queued on a copy
stream before each copy (test_automatic_cpu_cache.py:37-51) and pinned slabs
poisoned with 0xAB (test_cpu_cache_optimizations.py:83-86).
"""

from collections import deque
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from helpers import bf16_bits, u8
from kvx import ops
from kvx.engine.block_manager import BlockManager
from kvx.engine.cpu_prefix_cache import CPUBlockCache, CPUCacheFullError
from oracle import kvx_oracle as oracle

pytestmark = pytest.mark.gpu

BS = 256
DELAY_US = 20_000  # about torch.cuda._sleep(20_000_000) at ~1 GHz


def make_pool(device, num_blocks, layers=2, heads=1, hd=4, pattern="bytes"):
    """The reference fixtures' pool (2, 2, NB, 256, 1, 4) (test_engine_handoff.py:16)."""
    pool = torch.empty((2, layers, num_blocks, BS, heads, hd), dtype=torch.bfloat16, device=device)
    if pattern == "bytes":  # every bit pattern, NaNs included (test_cpu_prefix_cache.py:15-18)
        raw = torch.arange(pool.numel() * 2, device=device).remainder(256).to(torch.uint8)
        pool.view(torch.uint8).copy_(raw.view(pool.view(torch.uint8).shape))
    else:  # finite values for FP8
        g = torch.Generator(device=device).manual_seed(num_blocks)
        pool.copy_(torch.randn(pool.shape, generator=g, device=device))
    return pool


def publish(manager: BlockManager, block_id: int, token: int, prefix: int = -1) -> int:
    """Mark a GPU block as a finished, published full prefix block; return its hash."""
    tokens = [token] * manager.block_size
    h = manager.compute_hash(tokens, prefix)
    manager.blocks[block_id].update(h, tokens)
    manager.hash_to_block_id[h] = block_id
    return h


def forget(manager: BlockManager, key: int) -> int:
    """Unpublish a GPU block without touching its bytes or ordering (test_cpu_cache_optimizations.py:90-94)."""
    block_id = manager.hash_to_block_id.pop(key)
    manager.blocks[block_id].hash, manager.blocks[block_id].token_ids = -1, []
    return block_id


def block_bytes(pool, block_id):
    torch.cuda.synchronize()
    return u8(pool[:, :, block_id])


def new_cache(pool, manager, blocks=1, **kwargs):
    runner = SimpleNamespace(world_size=1, block_size=BS, kv_cache=pool)
    bf16_block = pool[:, :, 0].numel() * pool.element_size()
    if kwargs.get("fp8"):
        rows = pool[:, :, 0].numel() // pool.shape[-1]
        size = pool[:, :, 0].numel() + rows * (kwargs.get("scale_dtype") or pool.dtype).itemsize
    else:
        size = bf16_block
    return CPUBlockCache(runner, manager, blocks * size, **kwargs)


def slow_copies(cache, names=("_save_to_slot", "_restore_from_slot")):
    """Queue a delay on the copy stream before each copy so a missing wait corrupts bytes."""
    streams = {"_save_to_slot": cache._copy_stream, "_restore_from_slot": cache._restore_stream}
    for name in names:
        original = getattr(cache, name)

        def delayed(*args, _original=original, _stream=streams[name], **kwargs):
            ops.sleep(DELAY_US, stream=_stream, device=cache._cache.device)
            return _original(*args, **kwargs)

        setattr(cache, name, delayed)


@pytest.mark.parametrize("slow", [False, True])
def test_round_trip_is_byte_exact_and_survives_pool_overwrite(gpu, slow):
    pool = make_pool(gpu, 4)
    manager = BlockManager(4, BS)
    key = publish(manager, 1, 1)
    expected = block_bytes(pool, 1)
    cache = new_cache(pool, manager)
    if slow:
        slow_copies(cache)
    assert cache.save_block(key)
    assert key in cache and len(cache) == 1
    assert cache.bytes_used == cache.block_bytes == cache.max_bytes
    forget(manager, key)
    # Overwrite the pool on the compute stream; before_block_reuse orders it after the save.
    cache.before_block_reuse(1)
    pool.fill_(-7)
    target = cache.restore_block(key)
    assert np.array_equal(block_bytes(pool, target), expected)
    assert manager.blocks[target].ref_count == 0 and manager.hash_to_block_id[key] == target
    cache.close()


@pytest.mark.parametrize("scale_dtype", [None, torch.float32])
def test_fp8_entry_is_bit_exact_and_restores_within_the_reference_bound(gpu, scale_dtype):
    pool = make_pool(gpu, 3, layers=2, heads=8, hd=128, pattern="normal")
    manager = BlockManager(3, BS)
    key = publish(manager, 2, 5)
    source = pool[:, :, 2].float().cpu()
    host_pool = bf16_bits(pool)
    cache = new_cache(pool, manager, blocks=4, fp8=True, scale_dtype=scale_dtype)
    numel = pool[:, :, 0].numel()
    sdtype = scale_dtype or pool.dtype
    assert cache.block_bytes == numel + numel // pool.shape[-1] * sdtype.itemsize  # (:64)
    assert cache.save_block(key)
    cache.synchronize()
    entry = cache._entries[key]
    codes, scales = oracle.save_block_fp8(host_pool, 2, sdtype == torch.float32)
    assert np.array_equal(u8(entry.kv), codes) and np.array_equal(u8(entry.scale), scales.view(np.uint8))
    forget(manager, key)
    cache.before_block_reuse(2)
    pool[:, :, 2].zero_()
    target = cache.restore_block(key)
    cache.synchronize()
    restored = pool[:, :, target].float().cpu()
    bound = source.abs().amax(-1, keepdim=True) / 16  # test_cpu_cache_optimizations.py:71-73
    assert torch.all((restored - source).abs() <= bound)
    assert np.array_equal(bf16_bits(pool[:, :, target]), oracle.dequantize(codes, scales, sdtype == torch.float32))
    assert cache.stats["restored_blocks"] == 1


def split_cache(pool, manager, **kwargs):
    cache = new_cache(pool, manager, split_streams=True, preallocate=True, **kwargs)
    assert cache._restore_stream is not cache._copy_stream
    for slab in cache._slab_memory:
        slab.fill_(0xAB)
    return cache


@pytest.mark.parametrize("slow", [False, True])
def test_split_streams_restore_waits_for_its_save(gpu, slow):
    pool = make_pool(gpu, 3)
    manager = BlockManager(3, BS)
    key = publish(manager, 0, 1)
    cache = split_cache(pool, manager)
    if slow:
        slow_copies(cache, ["_save_to_slot"])  # a fast restore would overtake a missing wait
    expected = block_bytes(pool, 0)
    assert cache.save_block(key)
    forget(manager, key)
    target = cache.restore_block(key)
    cache.synchronize()
    assert np.array_equal(block_bytes(pool, target), expected)


@pytest.mark.parametrize("slow", [False, True])
def test_split_streams_slot_reuse_waits_for_pending_restore(gpu, slow):
    pool = make_pool(gpu, 3)
    manager = BlockManager(3, BS)
    key = publish(manager, 0, 1)
    cache = split_cache(pool, manager)
    expected = block_bytes(pool, 0)
    assert cache.save_block(key)
    cache.synchronize()
    forget(manager, key)
    if slow:
        slow_copies(cache, ["_restore_from_slot"])  # a fast save would overwrite the slot first
    entry = cache._entries[key]
    target = manager.restore_cached_block(key, entry.token_ids,
                                          lambda block_id: cache._copy_entry(entry, block_id, wait=False))
    assert cache.discard(key)
    other = next(i for i in range(3) if i != target)
    pool[:, :, other].fill_(7)
    other_key = publish(manager, other, 2)
    assert cache.save_block(other_key)  # reuses the slot the restore may still read
    cache.synchronize()
    assert np.array_equal(block_bytes(pool, target), expected)
    assert np.array_equal(u8(cache._slot_view(0)[0]), block_bytes(pool, other))


def test_restore_into_a_recycled_victim_waits_for_the_victims_save(gpu):
    # A prefetch-style restore allocates without write ordering
    # (block_manager.py:168); if that recycles a published victim, the victim's
    # save was queued just before. The copy engine orders the restore's writes
    # after that save, so both the saved victim and the restored block are intact.
    pool = make_pool(gpu, 2)
    manager = BlockManager(2, BS)
    victim_key = publish(manager, 0, 3)
    key = publish(manager, 1, 4)
    cache = new_cache(pool, manager, blocks=2, automatic=True, split_streams=True)
    victim_bytes, expected = block_bytes(pool, 0), block_bytes(pool, 1)
    assert cache.save_block(key)
    cache.synchronize()
    forget(manager, key)
    assert list(manager.free_block_ids) == [0, 1]  # block 0 (the victim) recycles first
    slow_copies(cache, ["_save_to_slot"])
    entry = cache._entries[key]
    target = manager.restore_cached_block(key, entry.token_ids,
                                          lambda block_id: cache._copy_entry(entry, block_id, wait=False))
    assert target == 0 and victim_key in cache
    cache.before_block_use(target)
    cache.synchronize()
    assert np.array_equal(block_bytes(pool, 0), expected)
    victim = cache._entries[victim_key]
    assert np.array_equal(u8(victim.kv), victim_bytes)


def test_budget_rules_dedup_discard_and_slot_reuse(gpu):
    pool = make_pool(gpu, 3)
    manager = BlockManager(3, BS)
    key = publish(manager, 0, 1)
    other = publish(manager, 1, 2)
    cache = new_cache(pool, manager)
    assert cache.reserved_bytes == 0
    assert cache.save_block(key)
    assert not cache.save_block(key)
    assert cache.reserved_bytes == cache.block_bytes
    with pytest.raises(CPUCacheFullError, match="budget"):
        cache.save_block(other)
    assert cache.discard(key) and not cache.discard(key)
    assert cache.save_block(other)  # reuses the freed slot
    assert cache.reserved_bytes == cache.bytes_used == cache.block_bytes
    with pytest.raises(KeyError):
        cache.save_block(-1)
    cache.clear()
    assert cache.bytes_used == len(cache) == 0 and other in manager.hash_to_block_id
    cache.close()
    cache.close()
    assert cache.closed
    with pytest.raises(RuntimeError, match="closed"):
        cache.save_block(key)


def test_preallocated_multi_slab_slots_round_trip(gpu, monkeypatch):
    import kvx.engine.cpu_prefix_cache as module

    monkeypatch.setattr(module, "_SLAB_CHUNK_BYTES", 1)
    pool = make_pool(gpu, 4)
    manager = BlockManager(4, BS)
    keys = [publish(manager, b, 10 + b) for b in range(3)]
    expected = {k: block_bytes(pool, manager.hash_to_block_id[k]) for k in keys}
    cache = new_cache(pool, manager, blocks=3, preallocate=True)
    assert len(cache._slabs) == 3 and cache.reserved_bytes == 3 * cache.block_bytes
    for k in keys:
        cache.save_block(k)
    assert len({cache._entries[k].slot for k in keys}) == 3
    cache.synchronize()
    for k in keys:
        forget(manager, k)
    cache.before_block_reuse(0)
    pool.fill_(0)
    for k in keys:
        restored = cache.restore_block(k)
        assert np.array_equal(block_bytes(pool, restored), expected[k])


def test_measure_restore_time_is_positive(gpu):
    pool = make_pool(gpu, 2, layers=2, heads=8, hd=128, pattern="normal")
    cache = new_cache(pool, BlockManager(2, BS), fp8=True)
    seconds = cache.measure_restore_s_per_block(repeats=4)
    assert 0 < seconds < 1


def test_every_split_cache_gets_copy_streams_that_run_concurrently(gpu):
    # Torch's pool streams map round-robin onto the process's hardware queues; without
    # the concurrency check every other cache's save and restore streams shared one
    # queue and ran one after the other.
    pool = make_pool(gpu, 2)
    compute = torch.cuda.current_stream(gpu)
    for _ in range(6):
        cache = new_cache(pool, BlockManager(2, BS), split_streams=True)
        engine = cache._engine
        assert engine.streams_concurrent
        streams = {engine.save_stream.cuda_stream, engine.restore_stream.cuda_stream, compute.cuda_stream}
        assert len(streams) == 3
        cache.close()
    single = new_cache(pool, BlockManager(2, BS))
    assert single._engine.streams_concurrent and single._engine.save_stream == single._engine.restore_stream
    single.close()


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_byte_copy_mode_round_trips_pools_of_other_dtypes(gpu, dtype):
    # BF16 storage mode is a byte copy (cpu_prefix_cache.py:319, 386), so any pool dtype works; FP8 needs bf16.
    pool = torch.empty((2, 2, 3, BS, 1, 4), dtype=dtype, device=gpu)
    raw = torch.arange(pool.numel() * pool.element_size(), device=gpu).remainder(256).to(torch.uint8)
    pool.view(torch.uint8).copy_(raw.view(pool.view(torch.uint8).shape))
    manager = BlockManager(3, BS)
    keys = [publish(manager, b, b + 1) for b in (0, 2)]
    expected = {k: block_bytes(pool, b) for k, b in zip(keys, (0, 2))}
    cache = new_cache(pool, manager, blocks=2)
    assert cache.block_bytes == pool[:, :, 0].numel() * pool.element_size()
    for k in keys:
        assert cache.save_block(k)
    cache.synchronize()
    for k in keys:
        manager.hash_to_block_id.pop(k)
    pool.fill_(0)
    for k in keys:
        assert np.array_equal(block_bytes(pool, cache.restore_block(k)), expected[k])
    cache.close()
    with pytest.raises(NotImplementedError, match="bfloat16 pool"):
        new_cache(pool, BlockManager(3, BS), fp8=True)


def test_save_of_a_block_waits_for_its_pending_restore(gpu):
    # A prefetched block whose CPU entry was dropped can be saved again before
    # its first use; the save must read the restored bytes, not the old ones.
    pool = make_pool(gpu, 3)
    manager = BlockManager(3, BS)
    key = publish(manager, 0, 1)
    cache = new_cache(pool, manager, blocks=2, split_streams=True)
    expected = block_bytes(pool, 0)
    assert cache.save_block(key)
    cache.synchronize()
    forget(manager, key)
    pool[:, :, 2].fill_(0)
    manager.free_block_ids = deque([2, 0, 1])
    entry = cache._entries[key]
    ops.sleep(DELAY_US, stream=cache._restore_stream, device=gpu)
    target = manager.restore_cached_block(key, entry.token_ids, lambda b: cache._copy_entry(entry, b, wait=False))
    assert target == 2
    assert cache.discard(key)
    cache._free_slots.remove(entry.slot)  # the new save takes the other slot, so only the new rule orders it
    cache._free_slots.insert(0, entry.slot)
    assert cache.save_block(key)
    assert cache._entries[key].slot != entry.slot
    cache.synchronize()
    assert np.array_equal(u8(cache._entries[key].kv), expected)
    assert np.array_equal(block_bytes(pool, 2), expected)
    cache.close()


def test_coalesced_restores_land_before_dependent_work(gpu):
    pool = make_pool(gpu, 6)
    manager = BlockManager(6, BS)
    keys = [publish(manager, b, 20 + b) for b in range(3)]
    expected = {k: block_bytes(pool, b) for b, k in enumerate(keys)}
    cache = new_cache(pool, manager, blocks=3, split_streams=True)
    for k in keys:
        assert cache.save_block(k)
    cache.synchronize()
    for k in keys:
        forget(manager, k)
    pool.fill_(0)
    slow_copies(cache)
    entries = [cache._entries[k] for k in keys]
    with cache.coalesce():
        cache._copy_entry(entries[0], 3)  # wait=True: compute waits when the block ends
        cache._copy_entry(entries[1], 4, wait=False)
        assert len(cache._batcher.restores) == 2  # held back
        # A save of a queued block flushes first and reads the restored bytes.
        manager.blocks[4].update(keys[1], [21] * BS)
        manager.hash_to_block_id[keys[1]] = 4
        cache.discard(keys[1])
        assert cache.save_block(keys[1]) and not cache._batcher.restores
        cache._copy_entry(entries[2], 5, wait=False)
    assert not cache._batcher.restores
    copy = pool[:, :, 3].clone()  # compute-stream work after the block sees the restored bytes
    cache.before_block_use(5)
    copy5 = pool[:, :, 5].clone()
    cache.synchronize()
    assert np.array_equal(u8(copy), expected[keys[0]])
    assert np.array_equal(u8(copy5), expected[keys[2]])
    assert np.array_equal(u8(cache._entries[keys[1]].kv), expected[keys[1]])
    cache.close()


def test_coalesced_saves_and_reuse_waits_keep_victims_intact(gpu):
    pool = make_pool(gpu, 4)
    manager = BlockManager(4, BS)
    keys = [publish(manager, b, 40 + b) for b in range(2)]
    expected = {k: block_bytes(pool, b) for b, k in enumerate(keys)}
    cache = new_cache(pool, manager, blocks=3, split_streams=True)
    slow_copies(cache)
    with cache.coalesce():
        for b, k in enumerate(keys):
            assert cache.save_block(k)
            cache.before_block_reuse(b)  # recycling the victim: deferred behind the held-back save
        assert len(cache._batcher.saves) == 2 and cache._batcher.reuse == [0, 1]
        # A second save into a slot a held-back save writes flushes first.
        slot = cache._entries[keys[1]].slot
        cache.discard(keys[1])
        assert cache._free_slots[-1] == slot
        keys.append(publish(manager, 2, 42))
        expected[keys[2]] = block_bytes(pool, 2)
        assert cache.save_block(keys[2]) and not cache._batcher.reuse
        cache.before_block_reuse(2)
        assert cache._batcher.reuse == [2]
    pool[:, :, 0:3].fill_(-1)  # compute overwrites the victims after the block
    cache.synchronize()
    for k in (keys[0], keys[2]):
        assert np.array_equal(u8(cache._entries[k].kv), expected[k]), k
    cache.close()


def test_engine_rejects_two_copies_into_one_destination(gpu):
    pool = make_pool(gpu, 4)
    manager = BlockManager(4, BS)
    keys = [publish(manager, b, 60 + b) for b in range(2)]
    expected = block_bytes(pool, 0)
    cache = new_cache(pool, manager, blocks=2, split_streams=True)
    for k in keys:
        assert cache.save_block(k)
    slots = [cache._entries[k].slot for k in keys]
    engine, compute = cache._engine, cache._compute_stream()
    with pytest.raises(ValueError, match="slot appears twice"):
        engine.save([2, 3], [slots[0], slots[0]], compute)
    with pytest.raises(ValueError, match="block appears twice"):
        engine.restore(slots, [3, 3], True, compute)
    # Rejected calls queue nothing: the cache keeps working.
    engine.restore(slots[:1], [3], True, compute)
    cache.synchronize()
    assert np.array_equal(block_bytes(pool, 3), expected)
    cache.close()


@pytest.mark.parametrize("caller_busy", [False, True])
@pytest.mark.parametrize("heads,hd", [(8, 128), (4, 64), (2, 256)])
@pytest.mark.parametrize("fmt,scale_dtype", [(ops.FORMAT_FP8, torch.float32), (ops.FORMAT_FP8, torch.bfloat16),
                                             (ops.FORMAT_RAW, None)])
def test_engine_saves_of_every_path_write_the_oracle_bytes(gpu, fmt, scale_dtype, heads, hd, caller_busy):
    # Calls of 1-2 blocks issued while the caller's stream is busy are written to the host slots by a capped grid
    # of save workgroups that stride over the tiles; other calls go through staging and a copy. 48-token blocks
    # of 3 layers do not divide evenly among the striding workgroups.
    from kvx.engine.cpu_prefix_cache import _CopyEngine

    g = torch.Generator(device=gpu).manual_seed(11)
    pool = (torch.randn((2, 3, 9, 48, heads, hd), generator=g, device=gpu) * 3).to(torch.bfloat16)
    layout = ops.pool_layout(pool, scale_dtype)
    engine = _CopyEngine(pool, layout, fmt, split=True)
    try:
        stride = engine.entry_stride
        slab = torch.full((8 * stride,), 0xA5, dtype=torch.uint8, pin_memory=True)
        staging = [torch.empty(4 * stride, dtype=torch.uint8, device=gpu) for _ in range(2)]
        engine.add_slab(slab, 8)
        engine.set_staging(*staging, 4)
        compute = torch.cuda.current_stream(gpu).cuda_stream
        calls = [([7], [0]), ([2, 5], [1, 2]), ([0, 8, 3], [3, 4, 5]), ([1, 6], [7, 6])]
        for blocks, slots in calls:
            if caller_busy:
                ops.sleep(2000, device=gpu)  # on the caller's (current) stream
            engine.save(blocks, slots, compute)
        engine.synchronize()
        host_pool = bf16_bits(pool)
        entries = slab.numpy().reshape(8, stride)
        for blocks, slots in calls:
            for b, slot in zip(blocks, slots):
                got = entries[slot]
                if fmt == ops.FORMAT_RAW:
                    want = np.ascontiguousarray(host_pool[:, :, b]).view(np.uint8).ravel()
                    assert np.array_equal(got[:want.size], want), (b, slot)
                    continue
                codes, scales = oracle.save_block_fp8(host_pool, b, scale_dtype == torch.float32)
                offset = engine.scale_offset
                assert np.array_equal(got[:codes.size], codes.ravel()), (b, slot)
                assert np.array_equal(got[offset:offset + scales.nbytes], scales.view(np.uint8).ravel()), (b, slot)
        assert engine.counters()["saved_blocks"] == 8
    finally:
        engine.close()


@pytest.mark.parametrize("heads,hd", [(8, 128), (4, 64), (2, 256)])
@pytest.mark.parametrize("fmt,scale_dtype", [(ops.FORMAT_FP8, torch.float32), (ops.FORMAT_FP8, torch.bfloat16),
                                             (ops.FORMAT_RAW, None)])
def test_engine_restores_of_every_path_write_the_oracle_bytes(gpu, fmt, scale_dtype, heads, hd):
    # With no save in flight, waited restores of 1-2 blocks are read from the host slots by a capped grid of
    # restore workgroups; 3+ blocks, and restores nobody waits for, go through staging and a copy. 50-token
    # blocks leave a ragged last tile in every plane.
    from kvx.engine.cpu_prefix_cache import _CopyEngine

    g = torch.Generator(device=gpu).manual_seed(12)
    pool = (torch.randn((2, 3, 9, 50, heads, hd), generator=g, device=gpu) * 3).to(torch.bfloat16)
    layout = ops.pool_layout(pool, scale_dtype)
    engine = _CopyEngine(pool, layout, fmt, split=True)
    try:
        stride = engine.entry_stride
        slab = torch.full((8 * stride,), 0xA5, dtype=torch.uint8, pin_memory=True)
        staging = [torch.empty(4 * stride, dtype=torch.uint8, device=gpu) for _ in range(2)]
        engine.add_slab(slab, 8)
        engine.set_staging(*staging, 4)
        compute = torch.cuda.current_stream(gpu).cuda_stream
        sources = [7, 2, 5, 0, 8, 3, 6, 1]  # slot i holds block sources[i]
        engine.save(sources, list(range(8)), compute)
        engine.synchronize()
        host_pool = bf16_bits(pool)
        fp32 = scale_dtype == torch.float32
        calls = [([0], [4], True), ([1, 2], [7, 0], True), ([3, 4, 5], [1, 2, 3], True), ([6], [5], False),
                 ([7], [6], True)]
        for slots, blocks, wait in calls:
            engine.restore(slots, blocks, wait, compute)
        engine.synchronize()
        after = bf16_bits(pool)
        for slots, blocks, _ in calls:
            for slot, d in zip(slots, blocks):
                b = sources[slot]
                if fmt == ops.FORMAT_RAW:
                    expect = host_pool[:, :, b]
                else:
                    codes, scales = oracle.save_block_fp8(host_pool, b, fp32)
                    expect = oracle.dequantize(codes, scales, fp32)
                assert np.array_equal(after[:, :, d], expect), (slot, b, d)
        assert np.array_equal(after[:, :, 8], host_pool[:, :, 8])  # never a destination
        assert engine.counters()["restored_blocks"] == 8
    finally:
        engine.close()


@pytest.mark.parametrize("ending", ["synchronize", "close"])
def test_waited_restores_on_the_callers_stream_finish_before_synchronize_and_close_return(gpu, ending):
    # A waited one-block restore with no save in flight reads its host slot from the caller's stream. Queued
    # behind a delay there, it is still pending when synchronize() or close() is called; once either returns,
    # the slot's pinned memory may be overwritten (or released and reused) without touching the restore.
    from kvx.engine.cpu_prefix_cache import _CopyEngine

    g = torch.Generator(device=gpu).manual_seed(21)
    pool = torch.randn((2, 4, 4, BS, 8, 128), generator=g, device=gpu).to(torch.bfloat16)
    layout = ops.pool_layout(pool, torch.float32)
    engine = _CopyEngine(pool, layout, ops.FORMAT_FP8, split=True)
    stride = engine.entry_stride
    slab = torch.empty(2 * stride, dtype=torch.uint8, pin_memory=True)
    staging = [torch.empty(2 * stride, dtype=torch.uint8, device=gpu) for _ in range(2)]
    engine.add_slab(slab, 2)
    engine.set_staging(*staging, 2)
    caller = torch.cuda.current_stream(gpu)
    try:
        engine.save([1], [0], caller.cuda_stream)
        engine.synchronize()
        codes, scales = oracle.save_block_fp8(bf16_bits(pool), 1, True)
        ops.sleep(DELAY_US, stream=caller, device=gpu)
        engine.restore([0], [3], True, caller.cuda_stream)
        getattr(engine, ending)()
        slab.fill_(0x7F)  # e4m3 NaN codes: a restore still reading the slot would land them
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(pool[:, :, 3]), oracle.dequantize(codes, scales, True))
    finally:
        engine.close()


def chunked_recycle(gpu, debug: int = 0) -> bool:
    """An admission under memory pressure, batched; True if every byte comes out right.

    12 victims are saved through a 4-entry staging (three chunks, each read
    by its own kernel), then 12 entries are restored into those same blocks,
    waited for. The saves are delayed, so every restore copy is ready long
    before the save kernels run: each restore chunk must still wait for the
    kernel that read its destinations, or it overwrites a victim unsaved.
    `debug` drops ordering rules (kvx._lib.DEBUG_*) for the negative control.
    """
    from kvx.engine.cpu_prefix_cache import _CopyEngine

    g = torch.Generator(device=gpu).manual_seed(31)
    pool = torch.randn((2, 2, 24, BS, 8, 128), generator=g, device=gpu).to(torch.bfloat16)
    layout = ops.pool_layout(pool, torch.float32)
    engine = _CopyEngine(pool, layout, ops.FORMAT_FP8, split=True)
    try:
        stride, offset = engine.entry_stride, engine.scale_offset
        slab = torch.full((24 * stride,), 0xAB, dtype=torch.uint8, pin_memory=True)
        staging = [torch.empty(4 * stride, dtype=torch.uint8, device=gpu) for _ in range(2)]
        engine.add_slab(slab, 24)
        engine.set_staging(*staging, 4)
        compute = torch.cuda.current_stream(gpu).cuda_stream
        victims, others = list(range(12)), list(range(12, 24))
        engine.save(others, others, compute)  # slots 12..23: entries of blocks 12..23
        engine.synchronize()
        before = bf16_bits(pool)
        engine.set_debug(debug)
        ops.sleep(DELAY_US, stream=engine.save_stream, device=gpu)
        engine.save(victims, victims, compute)
        engine.restore(others, victims, True, compute)
        engine.synchronize()
        torch.cuda.synchronize()
        entries = slab.view(24, stride).numpy()
        after = bf16_bits(pool)
        for v, o in zip(victims, others):
            codes, scales = oracle.save_block_fp8(before, v, True)
            if not (np.array_equal(entries[v, :codes.size], codes.ravel())
                    and np.array_equal(entries[v, offset:offset + scales.nbytes], scales.view(np.uint8).ravel())):
                return False  # the victim was saved after a restore overwrote it
            restored_codes, restored_scales = oracle.save_block_fp8(before, o, True)
            if not np.array_equal(after[:, :, v], oracle.dequantize(restored_codes, restored_scales, True)):
                return False
        return np.array_equal(after[:, :, 12:], before[:, :, 12:])
    finally:
        engine.close()


def test_restores_into_victims_of_a_chunked_save_wait_for_each_chunk_kernel(gpu):
    assert chunked_recycle(gpu)


def waited_restore_over_prefetch(gpu, debug: int = 0) -> bool:
    """A prefetched block recycled before its first use; True if the later, waited restore lands last.

    restore_cached_block reserves its destination without write ordering
    (block_manager.py:168), so a waited restore can target a block whose
    prefetch (wait=False, restore stream) is still delayed. The waited restore
    of one block, with no save in flight, is read by the kernel from the host
    slot on the caller's stream: it must wait for the prefetch, or the
    prefetch overwrites it. `debug` drops ordering rules for the negative control.
    """
    from kvx.engine.cpu_prefix_cache import _CopyEngine

    g = torch.Generator(device=gpu).manual_seed(41)
    pool = torch.randn((2, 2, 4, BS, 8, 128), generator=g, device=gpu).to(torch.bfloat16)
    layout = ops.pool_layout(pool)
    engine = _CopyEngine(pool, layout, ops.FORMAT_RAW, split=True)
    try:
        stride = engine.entry_stride
        slab = torch.empty(2 * stride, dtype=torch.uint8, pin_memory=True)
        staging = [torch.empty(2 * stride, dtype=torch.uint8, device=gpu) for _ in range(2)]
        engine.add_slab(slab, 2)
        engine.set_staging(*staging, 2)
        compute = torch.cuda.current_stream(gpu).cuda_stream
        engine.save([0, 1], [0, 1], compute)
        engine.synchronize()
        expected = bf16_bits(pool[:, :, 1])
        engine.set_debug(debug)
        ops.sleep(DELAY_US, stream=engine.restore_stream, device=gpu)
        engine.restore([0], [2], False, compute)  # the prefetch, held up on the restore stream
        engine.restore([1], [2], True, compute)   # the waited restore into the same block
        engine.synchronize()
        torch.cuda.synchronize()
        return np.array_equal(bf16_bits(pool[:, :, 2]), expected)
    finally:
        engine.close()


def test_a_waited_restore_into_a_block_still_being_prefetched_lands_last(gpu):
    assert waited_restore_over_prefetch(gpu)


def slot_reuse_across_caller_streams(gpu, debug: int = 0) -> bool:
    """One copy stream; True if a save into a slot waits for a kernel-read restore queued from another stream.

    A waited one-block restore with no save in flight is read by the kernel
    from its slot on the caller's stream, here a side stream A held up by a
    delay. The slot is then reused by a save issued from the idle current
    stream B. The save's wait for B does not cover A, so it must wait for the
    slot's last read itself. `debug` drops ordering rules for the negative control.
    """
    from kvx.engine.cpu_prefix_cache import _CopyEngine

    g = torch.Generator(device=gpu).manual_seed(43)
    pool = torch.randn((2, 2, 4, BS, 8, 128), generator=g, device=gpu).to(torch.bfloat16)
    engine = _CopyEngine(pool, ops.pool_layout(pool), ops.FORMAT_RAW, split=False)
    try:
        stride = engine.entry_stride
        slab = torch.empty(2 * stride, dtype=torch.uint8, pin_memory=True)
        staging = torch.empty(2 * stride, dtype=torch.uint8, device=gpu)
        engine.add_slab(slab, 2)
        engine.set_staging(staging, staging, 2)
        current = torch.cuda.current_stream(gpu)
        engine.save([0], [0], current.cuda_stream)
        engine.synchronize()
        expected = bf16_bits(pool[:, :, 0])
        engine.set_debug(debug)
        side = torch.cuda.Stream(gpu)
        ops.sleep(DELAY_US, stream=side, device=gpu)
        engine.restore([0], [1], True, side.cuda_stream)  # read by the kernel on the side stream
        engine.save([2], [0], current.cuda_stream)        # the slot, reused from the idle current stream
        engine.synchronize()
        torch.cuda.synchronize()
        return np.array_equal(bf16_bits(pool[:, :, 1]), expected)
    finally:
        engine.close()


def test_a_save_waits_for_a_kernel_read_restore_queued_from_another_callers_stream(gpu):
    assert slot_reuse_across_caller_streams(gpu)


def test_split_streams_refuse_overlapping_staging(gpu):
    from kvx.engine.cpu_prefix_cache import _CopyEngine

    pool = torch.zeros((2, 2, 4, BS, 8, 128), dtype=torch.bfloat16, device=gpu)
    layout = ops.pool_layout(pool, torch.float32)
    engine = _CopyEngine(pool, layout, ops.FORMAT_FP8, split=True)
    try:
        stride = engine.entry_stride
        buffer = torch.empty(3 * stride, dtype=torch.uint8, device=gpu)
        for save, restore in ((buffer, buffer), (buffer[:2 * stride], buffer[stride:])):
            with pytest.raises(ValueError, match="do not overlap"):
                engine.set_staging(save, restore, 2)
        engine.set_staging(buffer[:stride], buffer[stride:2 * stride], 1)  # adjacent is fine
    finally:
        engine.close()


def test_replacing_split_staging_orders_both_copy_streams(gpu):
    """New staging areas on a split-stream cache: each copy stream waits for the other's queued work, so an
    area one stream still uses can become the other's. Unchanged areas queue no wait."""
    from kvx.engine.cpu_prefix_cache import _CopyEngine

    pool = torch.zeros((2, 2, 4, BS, 8, 128), dtype=torch.bfloat16, device=gpu)
    engine = _CopyEngine(pool, ops.pool_layout(pool, torch.float32), ops.FORMAT_FP8, split=True)
    try:
        a, b = (torch.empty(engine.entry_stride, dtype=torch.uint8, device=gpu) for _ in range(2))
        engine.set_staging(a, b, 1)
        waits = engine.counters()["stream_waits"]
        engine.set_staging(a, b, 1)
        assert engine.counters()["stream_waits"] == waits
        for stream in (engine.save_stream, engine.restore_stream):
            ops.sleep(20_000, stream=stream, device=gpu)
        engine.set_staging(b, a, 1)  # swapped while both streams have work queued
        assert engine.counters()["stream_waits"] == waits + 2
        engine.synchronize()
    finally:
        engine.close()


def test_copy_streams_that_cannot_run_side_by_side_warn_and_still_copy(gpu, monkeypatch):
    from kvx.engine import cpu_prefix_cache

    monkeypatch.setattr(cpu_prefix_cache, "_run_side_by_side", lambda a, b, device: False)
    pool = make_pool(gpu, 4)
    manager = BlockManager(4, BS)
    keys = [publish(manager, b, 40 + b) for b in (0, 1, 2)]
    expected = {k: block_bytes(pool, b) for k, b in zip(keys, (0, 1, 2))}
    with pytest.warns(RuntimeWarning, match="serialise"):
        cache = new_cache(pool, manager, blocks=3, split_streams=True)
    assert not cache.streams_concurrent and cache.copy_stats["streams_concurrent"] is False
    for k in keys:
        assert cache.save_block(k)
    cache.synchronize()
    for k in keys:
        manager.hash_to_block_id.pop(k)
    pool.fill_(0)
    with cache.coalesce():  # three restores in one engine call: staged, one DMA
        targets = {k: cache.restore_block(k) for k in keys}
    for k in keys:
        assert np.array_equal(block_bytes(pool, targets[k]), expected[k])
    stats = cache.copy_stats
    assert stats["d2h_copies"] >= 1 and stats["d2h_bytes"] >= 3 * cache.block_bytes
    assert stats["h2d_copies"] >= 1 and stats["h2d_bytes"] >= 3 * cache.block_bytes
    assert cache.stats == {"saved_blocks": 3, "restored_blocks": 3, "budget_skips": 0}
    cache.close()


def test_a_failed_batch_withdraws_the_metadata_it_published(gpu, monkeypatch):
    pool = make_pool(gpu, 6)
    manager = BlockManager(6, BS)
    keys = [publish(manager, b, 70 + b) for b in range(2)]
    expected = block_bytes(pool, 0)
    cache = new_cache(pool, manager, blocks=3, split_streams=True)
    assert cache.save_block(keys[0])
    cache.synchronize()
    forget(manager, keys[0])  # only the CPU copy of keys[0] remains

    def broken(*args):
        raise RuntimeError("hipErrorLaunchFailure")

    engine_restore = cache._engine.restore
    monkeypatch.setattr(cache._engine, "restore", broken)
    with pytest.raises(RuntimeError, match="LaunchFailure"):
        with cache.coalesce():
            assert cache.save_block(keys[1])  # published now, issued at the end of the block
            target = cache.restore_block(keys[0])  # published now, issued at the end of the block
            assert keys[1] in cache._entries and manager.hash_to_block_id.get(keys[0]) == target
    # Neither the save nor the restore may be trusted: both are withdrawn.
    assert keys[1] not in cache._entries
    assert keys[0] not in manager.hash_to_block_id and manager.blocks[target].hash == -1
    assert keys[0] in cache._entries  # the CPU copy that was already saved stays for a retry
    monkeypatch.setattr(cache._engine, "restore", engine_restore)
    again = cache.restore_block(keys[0])
    cache.synchronize()
    assert np.array_equal(block_bytes(pool, again), expected)
    cache.close()
