"""Scripted-model engine fixtures for the restated reference tests.

ScriptedRunner follows bench/test_engine_events.py:47-57 (scripted token
batches) and cached_engine bench/test_engine_handoff.py:11-20 (a
(2, 2, NB, 256, 1, 4) bf16 pool of arange % 251). With write_kv=True the runner
also writes every scheduled token's K/V (the value of the request's first
token, as bench/test_automatic_cpu_cache.py:19-34 emulates) into the pool
through kvx.ops.store_kvcache and the engine's slot mapping, so the paged
write runs in the engine loop.
"""

from dataclasses import dataclass

import torch

from kvx import ops
from kvx.engine.block_manager import BlockManager
from kvx.engine.llm_engine import LLMEngine
from kvx.engine.sequence import SamplingParams
from kvx.engine.slot_mapping import decode_slot_mapping, prefill_slot_mapping, upload

BS = 256


@dataclass
class Step:
    """engine.step()'s (outputs, num_tokens) by name."""

    outputs: list
    num_tokens: int


def step(engine) -> Step:
    return Step(*engine.step())


class ScriptedRunner:
    def __init__(self, batches, pool):
        self.batches = iter(batches)
        self.calls = []
        self.kv_cache = pool
        self.world_size = 1
        self.block_size = BS
        self.write_kv = False

    def call(self, method, *args):
        if method == "exit":
            self.calls.append("exit")
            return None
        assert method == "run"
        seqs, is_prefill = args
        tokens = next(self.batches)
        assert len(tokens) == len(seqs)
        self.calls.append((is_prefill, [seq.seq_id for seq in seqs]))
        if self.write_kv:
            self._write(seqs, is_prefill)
        return tokens

    def _write(self, seqs, is_prefill):
        pool = self.kv_cache
        if is_prefill:
            slots = prefill_slot_mapping(seqs, BS)
            values = [seq[0] for seq in seqs for _ in range(seq.num_scheduled_tokens)]
        else:
            slots = decode_slot_mapping(seqs, BS)
            values = [seq[0] for seq in seqs]
        if not len(slots):
            return
        heads, hd = pool.shape[4], pool.shape[5]
        rows = torch.tensor(values, dtype=torch.float32, device=pool.device)
        kv = rows[:, None, None].expand(len(values), heads, hd).to(pool.dtype).contiguous()
        mapping = upload(slots, pool.device)
        for layer in range(pool.shape[1]):
            ops.store_kvcache(kv, kv, pool[0, layer], pool[1, layer], mapping)


def params(**kwargs):
    return SamplingParams(temperature=0, **kwargs)


def cached_engine(device, batches, budget=512, num_blocks=16, **config):
    pool = torch.arange(2 * 2 * num_blocks * BS * 4, device=device).remainder(251).to(torch.bfloat16)
    pool = pool.reshape(2, 2, num_blocks, BS, 1, 4)
    runner = ScriptedRunner(batches, pool)
    return LLMEngine(runner, max_num_seqs=4, max_num_batched_tokens=budget, eos=99, kvcache_block_size=BS,
                     num_kvcache_blocks=num_blocks, **config)


def pool_of(engine):
    return engine.model_runner.kv_cache


def block_bytes(engine, block_id):
    pool = pool_of(engine)
    torch.cuda.synchronize(pool.device)
    return pool[:, :, block_id].contiguous().cpu().view(torch.uint8).clone()


def completed_prefix(device, extra_batches=()):
    """A finished 257-token request whose first block is an idle published GPU hit
    (bench/test_cpu_prefix_cache.py:12-26); the pool holds every byte pattern, NaNs included."""
    engine = cached_engine(device, [[10], [11], *extra_batches], num_blocks=2)
    pool = pool_of(engine)
    raw = torch.arange(pool.numel() * 2, dtype=torch.int64, device=device).remainder(256).to(torch.uint8)
    pool.view(torch.uint8).copy_(raw.view(pool.view(torch.uint8).shape))
    engine.add_request([1] * 257, params(max_tokens=2))
    step(engine)
    step(engine)
    manager = engine.scheduler.block_manager
    key = manager.compute_hash([1] * BS)
    assert engine.is_finished() and key in manager.hash_to_block_id
    assert not manager.used_block_ids
    return engine, manager, key


def finite_prefix(device, batches=(), blocks=1, num_blocks=2):
    """A finished request whose `blocks` full blocks are idle GPU hits, finite KV
    (bench/test_cpu_cache_optimizations.py:26-40)."""
    steps = -(-(BS * blocks + 1) // 512) + 1
    engine = cached_engine(device, [[90]] * steps + [*batches], num_blocks=num_blocks)
    engine.add_request([1] * (BS * blocks + 1), params(max_tokens=2))
    while not engine.is_finished():
        step(engine)
    manager = engine.scheduler.block_manager
    keys, h = [], -1
    for _ in range(blocks):
        h = manager.compute_hash([1] * BS, h)
        keys.append(h)
    assert all(key in manager.hash_to_block_id for key in keys)
    return engine, manager, keys


def new_cache(engine, blocks=1, **kwargs):
    pool = pool_of(engine)
    size = pool[:, :, 0].numel() * pool.element_size()
    return engine.create_cpu_prefix_cache(max_bytes=blocks * size, **kwargs)


def overwrite_prefix(engine):
    """bench/test_cpu_prefix_cache.py:35-40."""
    engine.add_request([3] * 257, params(max_tokens=1))
    step(engine)
    engine.add_request([4], params(max_tokens=1))
    step(engine)


def assert_pool_consistent(manager: BlockManager):
    free = list(manager.free_block_ids)
    assert len(free) == len(set(free))
    assert set(free).isdisjoint(manager.used_block_ids)
    assert set(free) | manager.used_block_ids == set(range(len(manager.blocks)))
    assert all(manager.blocks[i].ref_count == 0 for i in free)


def write_scheduled_kv(engine):
    engine.model_runner.write_kv = True


def slow_copies(cache, names=("_save_to_slot", "_restore_from_slot"), microseconds=20_000):
    """bench/test_automatic_cpu_cache.py:37-51 with the copy engine's streams and kvx's delay kernel."""
    streams = {"_save_to_slot": cache._copy_stream, "_restore_from_slot": cache._restore_stream}
    for name in names:
        original = getattr(cache, name)

        def delayed(*args, _original=original, _stream=streams[name], **kwargs):
            ops.sleep(microseconds, stream=_stream, device=cache._cache.device)
            return _original(*args, **kwargs)

        setattr(cache, name, delayed)
