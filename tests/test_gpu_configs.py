"""Parity at the benchmark configurations' full sizes (Qwen3-0.6B / Qwen3-8B KV geometry).

Config 1: FP8 save of 16 seeded blocks of a [2,28,512,256,8,128] pool, restore into 16 other seeded blocks.
Config 2: FP8 save (fp32 scales) of 128 seeded blocks of the Student-t Qwen3-8B pool [2,36,320,256,8,128] to
          pinned host slots through the copy engine, restore into 128 other seeded blocks.
Config 3: BF16 byte-exact save of 200 scattered Qwen3-8B blocks to pinned host slots and restore into a seeded
          permutation of free blocks that overlaps the sources; hybrid admission of a 32,768-token prefix that
          restores only its tail.
Config 4: ragged continuous-batch store_kvcache (16 sequences, strided V, -1 padding) over all 36 layers while FP8
          saves of 64 evicted blocks run on the save stream.
Every FP8 block is checked bit-exactly against the oracle (payload, scales and the restored bytes), in chunks
of blocks so host memory stays bounded; every BF16 block and every store_kvcache layer byte-exactly.
"""

from collections import deque
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from helpers import bf16_bits, u8
from kvx import ops
from kvx.engine.block_manager import BlockManager, plan_split
from kvx.engine.cpu_prefix_cache import CPUBlockCache
from kvx.engine.sequence import SamplingParams, Sequence
from workloads import QWEN3_0_6B, QWEN3_8B, block_selection, fill_normal, fill_student_t
from oracle import kvx_oracle as oracle

pytestmark = pytest.mark.gpu
BS = 256


def random_bits_pool(shape, device, seed):
    """Every bf16 bit pattern, NaNs included."""
    pool = torch.empty(shape, dtype=torch.bfloat16, device=device)
    g = torch.Generator(device=device).manual_seed(seed)
    pool.view(torch.int16).random_(-32768, 32768, generator=g)
    return pool


def publish(manager, block_id, tokens, prefix=-1):
    h = manager.compute_hash(tokens, prefix)
    manager.blocks[block_id].update(h, list(tokens))
    manager.hash_to_block_id[h] = block_id
    return h


def forget(manager, key):
    block_id = manager.hash_to_block_id.pop(key)
    manager.blocks[block_id].hash, manager.blocks[block_id].token_ids = -1, []


def runner_for(pool):
    return SimpleNamespace(world_size=1, block_size=BS, kv_cache=pool)


def same_bytes(a: torch.Tensor, b: torch.Tensor) -> bool:
    return torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16))


def check_fp8_entries(sources: torch.Tensor, entries: np.ndarray, restored: torch.Tensor, layout, offset: int,
                      fp32: bool, label: str, chunk: int = 16):
    """Every block i: entries[i] holds the oracle's codes and scales of sources[:, :, i], and restored[:, :, i]
    the oracle's dequantisation of them (bit-exact); also the reference's acceptance bound |delta| <= amax/16.

    sources/restored: [2, L, n, BS, H, hd] device tensors; entries: [n, entry_stride] uint8 host entries.
    """
    n = sources.shape[2]
    rows = layout.planes * layout.plane_rows
    sbytes = 4 if fp32 else 2
    for lo in range(0, n, chunk):
        hi = min(n, lo + chunk)
        src = bf16_bits(sources[:, :, lo:hi].transpose(0, 2).transpose(1, 2))  # [blocks, 2, L, BS, H, hd]
        got = bf16_bits(restored[:, :, lo:hi].transpose(0, 2).transpose(1, 2))
        codes, scales = oracle.quantize(src, fp32)
        back = oracle.dequantize(codes, scales, fp32)
        for j, i in enumerate(range(lo, hi)):
            assert np.array_equal(entries[i, :codes[j].size], codes[j].ravel()), f"{label}: payload of block {i}"
            assert np.array_equal(entries[i, offset:offset + rows * sbytes], scales[j].view(np.uint8).ravel()), \
                f"{label}: scales of block {i}"
            assert np.array_equal(got[j], back[j]), f"{label}: restored block {i}"
        s = sources[:, :, lo:hi].float()
        assert torch.all((restored[:, :, lo:hi].float() - s).abs() <= s.abs().amax(-1, keepdim=True) / 16), label


def test_config1_fp8_round_trip_of_16_blocks(gpu):
    pool = torch.empty(QWEN3_0_6B.shape, dtype=torch.bfloat16, device=gpu)
    fill_normal(pool, seed=0)
    order = block_selection(QWEN3_0_6B.num_blocks, 32, seed=1)
    sources, dests = order[:16], order[16:]
    layout = ops.pool_layout(pool, torch.float32)
    logical, offset, stride = ops.entry_layout(layout, ops.FORMAT_FP8)
    staging = torch.empty(16 * stride, dtype=torch.uint8, device=gpu)
    entries = [staging.data_ptr() + i * stride for i in range(16)]
    source_copy = pool[:, :, sources].clone()
    others = sorted(set(range(QWEN3_0_6B.num_blocks)) - set(dests))
    canary = pool[:, :, others].clone()
    ops.save_blocks(pool, sources, entries, ops.FORMAT_FP8, torch.float32)
    ops.restore_blocks(pool, dests, entries, ops.FORMAT_FP8, torch.float32)
    torch.cuda.synchronize()
    check_fp8_entries(source_copy, u8(staging).reshape(16, stride), pool[:, :, dests], layout, offset, True,
                      "config 1")
    assert same_bytes(pool[:, :, others], canary)


@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.bfloat16])
def test_config2_fp8_128_blocks_through_pinned_slots(gpu, scale_dtype):
    from kvx.engine.cpu_prefix_cache import _CopyEngine

    pool = torch.empty(QWEN3_8B.shape, dtype=torch.bfloat16, device=gpu)
    fill_student_t(pool, seed=0)  # bf16(0.5 t4), 4 seeded x20 outlier channels per (kv, layer, head)
    order = block_selection(QWEN3_8B.num_blocks, 256, seed=1)
    sources, dests = order[:128], order[128:]
    fp32 = scale_dtype == torch.float32
    layout = ops.pool_layout(pool, scale_dtype)
    engine = _CopyEngine(pool, layout, ops.FORMAT_FP8, split=True)
    try:
        stride, offset = engine.entry_stride, engine.scale_offset
        slab = torch.full((128 * stride,), 0xAB, dtype=torch.uint8, pin_memory=True)
        staging = [torch.empty(32 * stride, dtype=torch.uint8, device=gpu) for _ in range(2)]
        engine.add_slab(slab, 128)
        engine.set_staging(*staging, 32)
        compute = torch.cuda.current_stream(gpu).cuda_stream
        source_copy = pool[:, :, sources].clone()
        others = sorted(set(range(QWEN3_8B.num_blocks)) - set(dests))
        canary = pool[:, :, others].clone()
        engine.save(sources, list(range(128)), compute)
        engine.restore(list(range(128)), dests, False, compute)
        engine.before_block_use(dests[0], compute)  # (all 128 share one restore event)
        engine.synchronize()
        torch.cuda.synchronize()
        check_fp8_entries(source_copy, slab.view(128, stride).numpy(), pool[:, :, dests], layout, offset, fp32,
                          f"config 2, {scale_dtype} scales")
        assert same_bytes(pool[:, :, others], canary)  # no block outside the destinations was written
    finally:
        engine.close()


def test_config3_bf16_200_blocks_into_permuted_free_blocks(gpu):
    pool = random_bits_pool(QWEN3_8B.shape, gpu, seed=0)
    manager = BlockManager(QWEN3_8B.num_blocks, BS)
    sources = block_selection(QWEN3_8B.num_blocks, 200, seed=1)
    keys = [publish(manager, b, [1000 + i] * BS) for i, b in enumerate(sources)]
    originals = pool[:, :, sources].clone()
    block_bytes = pool[:, :, 0].numel() * pool.element_size()
    cache = CPUBlockCache(runner_for(pool), manager, 200 * block_bytes, split_streams=True)
    for key in keys:
        assert cache.save_block(key)
    for key in keys:
        forget(manager, key)
    # Restores recycle blocks in a seeded order that overlaps the sources:
    # each write must wait for the pending save that still reads its block.
    manager.free_block_ids = deque(block_selection(QWEN3_8B.num_blocks, QWEN3_8B.num_blocks, seed=2))
    targets = [cache.restore_block(key) for key in keys]
    assert len(set(targets)) == 200 and set(targets) & set(sources)
    cache.synchronize()
    for i, t in enumerate(targets):
        assert same_bytes(pool[:, :, t], originals[:, :, i]), f"block {sources[i]} -> {t}"
    entry = cache._entries[keys[5]]
    assert np.array_equal(u8(entry.kv), u8(originals[:, :, 5]))  # host slot layout == block bytes
    cache.close()


def test_config3_hybrid_admission_restores_only_the_tail(gpu):
    pool = random_bits_pool(QWEN3_8B.shape, gpu, seed=3)
    manager = BlockManager(QWEN3_8B.num_blocks, BS)
    sources = block_selection(QWEN3_8B.num_blocks, 128, seed=4)
    tokens = [t for i in range(128) for t in [2000 + i] * BS]  # a 32,768-token prefix
    keys, h = [], -1
    for i, b in enumerate(sources):
        h = publish(manager, b, tokens[i * BS:(i + 1) * BS], h)
        keys.append(h)
    originals = pool[:, :, sources].clone()
    block_bytes = pool[:, :, 0].numel() * pool.element_size()
    cache = CPUBlockCache(runner_for(pool), manager, 128 * block_bytes, automatic=True, split_streams=True)
    for key in keys:
        cache.save_block(key)
    cache.synchronize()
    for key in keys:
        forget(manager, key)
    pool.view(torch.int16).fill_(0x5A5A)  # canary: blocks the admission must not write
    # Equal per-block cost at k = 13: recompute(13 blocks) = restore(115 blocks).
    cache.hybrid = (1.0, 115 / (13 * BS), 0.0)
    seq = Sequence(tokens + [7], SamplingParams(temperature=0, max_tokens=1))
    assert manager.can_allocate(seq) == 128
    manager.allocate(seq, 128)
    assert seq.restore_span == (13 * BS, 128 * BS) and seq.num_cached_tokens == 0
    assert cache.stats["restored_blocks"] == 115
    seq.num_cached_tokens = 13 * BS  # the head was prefilled
    manager.finish_restore_span(seq)
    cache.synchronize()
    canary = torch.full_like(pool[:, :, 0], 0).view(torch.int16).fill_(0x5A5A)
    for i in range(13):
        assert torch.equal(pool[:, :, seq.block_table[i]].view(torch.int16), canary), f"head block {i} written"
    for i in range(13, 128):
        assert same_bytes(pool[:, :, seq.block_table[i]], originals[:, :, i]), f"tail block {i}"
    manager.deallocate(seq)
    cache.close()


def test_hybrid_split_follows_the_measured_restore_cost(gpu):
    """The calibration loop of bench/agent_replay.py:387-391: measure, set hybrid, admit."""
    pool = random_bits_pool(QWEN3_8B.shape, gpu, seed=11)
    manager = BlockManager(QWEN3_8B.num_blocks, BS)
    n = 128
    sources = block_selection(QWEN3_8B.num_blocks, n, seed=12)
    tokens = [t for i in range(n) for t in [3000 + i] * BS]
    keys, h = [], -1
    for i, b in enumerate(sources):
        h = publish(manager, b, tokens[i * BS:(i + 1) * BS], h)
        keys.append(h)
    originals = pool[:, :, sources].clone()
    block_bytes = pool[:, :, 0].numel() * pool.element_size()
    cache = CPUBlockCache(runner_for(pool), manager, n * block_bytes, automatic=True, split_streams=True)
    restore_s = cache.measure_restore_s_per_block()
    # One BF16 block over a PCIe 5.0 x16 link: about 0.6-0.7 ms.
    assert 0.3e-3 < restore_s < 3e-3, restore_s
    cache.hybrid = (restore_s, 6.87e-6, 9.3e-10)  # recompute costs: agent_replay.py:283-286 defaults
    split = plan_split(n, BS, *cache.hybrid)
    assert 0 < split < n
    for key in keys:
        cache.save_block(key)
    cache.synchronize()
    for key in keys:
        forget(manager, key)
    seq = Sequence(tokens + [7], SamplingParams(temperature=0, max_tokens=1))
    manager.allocate(seq, manager.can_allocate(seq))
    assert seq.restore_span == (split * BS, n * BS)
    assert cache.stats["restored_blocks"] == n - split
    seq.num_cached_tokens = split * BS
    manager.finish_restore_span(seq)
    cache.synchronize()
    for i in range(split, n):
        assert same_bytes(pool[:, :, seq.block_table[i]], originals[:, :, i]), f"tail block {i}"
    manager.deallocate(seq)
    cache.close()


def test_config4_ragged_store_kvcache_with_concurrent_fp8_saves(gpu):
    shape = QWEN3_8B.shape
    _, layers, nb, bs, heads, hd = shape
    pool = torch.empty(shape, dtype=torch.bfloat16, device=gpu)
    fill_student_t(pool, seed=5)
    evicted = block_selection(nb, 64, seed=6)
    rng = np.random.default_rng(7)
    lengths = rng.integers(1, 8193, size=16)
    free_slots = np.array([b * bs + i for b in range(nb) if b not in set(evicted) for i in range(bs)])
    if lengths.sum() > free_slots.size:  # cap the batch to the slots outside the evicted blocks
        lengths = np.maximum(1, lengths * free_slots.size // lengths.sum())
    cu_seqlens = np.concatenate([[0], np.cumsum(lengths)])
    total = int(cu_seqlens[-1])
    padded = -(-total // 256) * 256  # graph-style padding with -1 slots
    slots = np.full(padded, -1, dtype=np.int32)
    slots[:total] = rng.permutation(free_slots)[:total]
    g = torch.Generator(device=gpu).manual_seed(8)
    qkv = torch.randn((padded, (32 + 2 * heads) * hd), generator=g, device=gpu).to(torch.bfloat16)
    key = qkv[:, 32 * hd:(32 + heads) * hd].contiguous().view(padded, heads, hd)
    value = qkv[:, (32 + heads) * hd:].view(padded, heads, hd)
    assert value.stride(0) == 6144
    mapping = torch.from_numpy(slots).to(gpu)

    manager = BlockManager(nb, bs)
    keys = [publish(manager, b, [3000 + i] * bs) for i, b in enumerate(evicted)]
    evicted_before = pool[:, :, evicted].clone()
    block_bytes = pool[:, :, 0].numel() + pool[:, :, 0].numel() // hd * 4
    cache = CPUBlockCache(runner_for(pool), manager, 64 * block_bytes, split_streams=True, fp8=True,
                          scale_dtype=torch.float32)
    before = [bf16_bits(pool[0, l]).reshape(-1, heads * hd) for l in (0, layers - 1)]
    for k in keys:  # queued on the save stream
        cache.save_block(k)
    for layer in range(layers):  # meanwhile, the compute stream writes the batch's KV
        ops.store_kvcache(key, value, pool[0, layer], pool[1, layer], mapping)
    cache.synchronize()
    torch.cuda.synchronize()
    valid = slots >= 0
    rows = torch.from_numpy(slots[valid].astype(np.int64)).to(gpu)
    for layer in range(layers):
        assert torch.equal(pool[0, layer].view(-1, heads * hd)[rows], key.view(padded, -1)[torch.from_numpy(valid).to(gpu)])
        assert torch.equal(pool[1, layer].view(-1, heads * hd)[rows],
                           value.reshape(padded, -1)[torch.from_numpy(valid).to(gpu)])
    for (layer, expect) in zip((0, layers - 1), before):
        oracle.store_kvcache(bf16_bits(key), bf16_bits(value), expect, expect.copy(), slots)
        assert np.array_equal(bf16_bits(pool[0, layer]).reshape(-1, heads * hd), expect)
    assert torch.equal(pool[:, :, evicted], evicted_before)  # the batch never touches evicted blocks
    for lo in range(0, 64, 16):  # every saved entry, bit-exact
        codes, scales = oracle.quantize(bf16_bits(evicted_before[:, :, lo:lo + 16].transpose(0, 2).transpose(1, 2)),
                                        True)
        for j in range(16):
            entry = cache._entries[keys[lo + j]]
            assert np.array_equal(u8(entry.kv), codes[j]), f"payload of evicted block {lo + j}"
            assert np.array_equal(u8(entry.scale), scales[j].view(np.uint8)), f"scales of evicted block {lo + j}"
    cache.close()
