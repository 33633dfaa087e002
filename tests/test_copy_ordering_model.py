"""Ordering of saves, restores and block reuse under every interleaving a seeded scheduler finds (CPU only).

Random caller sequences (tests/copy_scenarios.py: admissions, prefetches, uses, release-time saves,
discards) go through the real `_CopyBatcher` into a model of libkvx's copy engine
(tests/copy_model.py), whose streams run in orders chosen at random within the waits the engine
queued. Every read on the caller's stream, and every block and live slot at the end, must equal what a
sequential execution gives. Both stream modes, staging of 1 to 128 entries, batched and one call per
block, with and without kernel-read restores.

The negative controls show that the sequences reach every ordering rule. Dropping one rule
(kvx_cache_set_debug's flags), or flushing held-back copies in a wrong order, makes some seed fail.
"""

import random

import pytest

from copy_model import (COMPUTE, SKIP_OVERWRITE_WAIT, SKIP_REUSE_WAIT, SKIP_SAVE_WAIT, SKIP_SLOT_READ_WAIT,
                        SKIP_VICTIM_WAIT, Device, Memory, ModelEngine)
from copy_scenarios import Caller, NoAllocSaves
from kvx.engine.cpu_prefix_cache import _CopyBatcher

BLOCKS, SLOTS, ROUNDS = 12, 10, 60


class ModelBackend:
    def __init__(self, seed: int, split: bool, staging: int, kernel_reads: bool = True, debug: int = 0,
                 batcher=_CopyBatcher, noalloc: bool = False):
        self.dev = Device(random.Random(seed * 7919 + 1), (COMPUTE, "caller 2", "save", "restore"))
        self.current = COMPUTE
        self.mem = Memory(BLOCKS, SLOTS)
        self.engine = ModelEngine(self.dev, self.mem, split, staging, kernel_reads, debug)
        engine = self.engine
        if noalloc:
            engine = NoAllocSaves(self.engine, lambda ids, slots, compute: self.engine.save(ids, slots, compute, True),
                                  self.engine.static_entries)
        self.batcher = batcher(engine, lambda: self.current)

    def switch_stream(self):
        new = "caller 2" if self.current == COMPUTE else COMPUTE
        self.dev.wait(new, self.dev.record(self.current))
        self.current = new

    def write(self, block, value):
        def op():
            self.mem.blocks[block] = value

        self.dev.run(self.current, op)

    def read(self, block):
        box = []
        self.dev.run(self.current, lambda: box.append(self.mem.blocks[block]))
        return box

    def value(self, token):
        return token[0]

    def between(self):
        self.dev.advance(6)

    def sync(self):
        self.dev.drain()

    def block_value(self, block):
        return self.mem.blocks[block]

    def slot_value(self, slot):
        return self.mem.slots[slot]


def run(seed, split, staging, batched=True, kernel_reads=True, debug=0, batcher=_CopyBatcher, noalloc=False,
        switch_streams=False):
    backend = ModelBackend(seed, split, staging, kernel_reads, debug, batcher, noalloc)
    caller = Caller(random.Random(seed), backend, BLOCKS, SLOTS, batched=batched, switch_streams=switch_streams)
    caller.run(ROUNDS)
    return caller.check(), caller, backend


MODES = [(split, staging, batched, reads)
         for split in (True, False) for staging in (1, 2, 3, 128)
         for batched in (True, False) for reads in (True, False)]


@pytest.mark.parametrize("split,staging,batched,kernel_reads", MODES)
def test_every_interleaving_found_gives_the_sequential_result(split, staging, batched, kernel_reads):
    paths = set()
    for seed in range(40):
        bad, caller, backend = run(seed, split, staging, batched, kernel_reads)
        assert not bad, f"seed {seed}: {bad[:5]}\n" + "\n".join(caller.log[-40:])
        paths.update(backend.engine.calls)
    # The sequences reach the engine's paths: staged saves and restores, kernel-written saves, and
    # kernel-read restores where they are allowed.
    assert ("save", "staged") in paths and ("restore", "staged") in paths and ("save", "direct") in paths
    assert (("restore", "direct") in paths) == kernel_reads


@pytest.mark.parametrize("split,staging,batched", [(True, 1, True), (True, 3, False), (False, 2, True),
                                                   (False, 1, False)])
def test_allocation_free_saves_keep_the_sequential_result(split, staging, batched):
    # Saves of up to 4 blocks go through kvx_cache_save_noalloc's rules (static staging, one re-recorded event).
    paths = set()
    for seed in range(40):
        bad, caller, backend = run(seed, split, staging, batched, noalloc=True)
        assert not bad, f"seed {seed}: {bad[:5]}\n" + "\n".join(caller.log[-40:])
        paths.update(backend.engine.calls)
    assert ("save", "staged", "fixed") in paths and ("save", "direct", "fixed") in paths


@pytest.mark.parametrize("split,staging,batched", [(True, 2, True), (True, 1, False), (False, 3, True),
                                                   (False, 1, False)])
def test_caller_stream_switches_keep_the_sequential_result(split, staging, batched):
    # The caller moves between two streams, each switch ordered after the previous stream (as torch code does):
    # kernel-read restores and waits land on either stream, saves reuse slots those restores read.
    for seed in range(40):
        bad, caller, _ = run(seed, split, staging, batched, switch_streams=True)
        assert not bad, f"seed {seed}: {bad[:5]}\n" + "\n".join(caller.log[-40:])


def fails_somewhere(seeds=60, **kwargs) -> bool:
    for split in (True, False):
        for staging in (1, 3):
            for batched in (True, False):
                for seed in range(seeds):
                    bad, _, _ = run(seed, split, staging, batched, **kwargs)
                    if bad:
                        return True
    return False


@pytest.mark.parametrize("flag", [SKIP_SAVE_WAIT, SKIP_SLOT_READ_WAIT, SKIP_REUSE_WAIT, SKIP_VICTIM_WAIT,
                                  SKIP_OVERWRITE_WAIT])
def test_dropping_any_ordering_rule_is_caught(flag):
    assert fails_somewhere(debug=flag)


@pytest.mark.parametrize("split", [True, False])
def test_a_waited_restore_into_a_block_still_being_prefetched_lands_last(split):
    # restore_cached_block recycles a prefetched block before its first use, without write ordering
    # (block_manager.py:168), and restores into it with wait=True: a kernel-read restore on the caller's
    # stream must still follow the prefetch queued on the restore stream.
    wrong = 0
    for seed in range(100):
        dev = Device(random.Random(seed), (COMPUTE, "save", "restore"))
        mem = Memory(4, 4)
        mem.slots[:2] = ["prefetched", "restored"]
        engine = ModelEngine(dev, mem, split, 2)
        engine.restore([0], [2], False, COMPUTE)
        engine.restore([1], [2], True, COMPUTE)
        assert engine.calls[-1] == ("restore", "direct")
        dev.drain()
        wrong += mem.blocks[2] != "restored"
    assert wrong == 0


def test_a_save_waits_for_a_kernel_read_restore_queued_from_another_callers_stream():
    # One copy stream. A waited one-block restore, read by the kernel from its slot, is queued on caller stream A
    # behind other work; the slot is then discarded and a save into it issued from caller stream B, which is idle.
    # The save's wait for B covers nothing A holds, so it must wait for the slot's last read itself.
    wrong = 0
    for seed in range(100):
        dev = Device(random.Random(seed), (COMPUTE, "other", "save"))
        mem = Memory(4, 2)
        mem.slots[0] = "entry"
        engine = ModelEngine(dev, mem, False, 2)
        dev.run(COMPUTE, lambda: None)  # A is busy
        engine.restore([0], [1], True, COMPUTE)
        assert engine.calls[-1] == ("restore", "direct")
        engine.save([2], [0], "other")
        dev.drain()
        wrong += mem.blocks[1] != "entry"
    assert wrong == 0


class RestoresFirst(_CopyBatcher):
    """A wrong flush order: held-back restores before the saves of the victims they overwrite."""

    def flush(self):
        saves, self.saves, self.save_slots = self.saves, [], set()
        reuse, self.reuse = self.reuse, []
        restores, self.restores = self.restores, []
        self.restore_blocks, self.restore_slots = set(), set()
        compute = self._compute()
        for slot, block, wait in restores:
            self.engine.restore([slot], [block], wait, compute)
        if saves:
            self.engine.save([b for b, _ in saves], [s for _, s in saves], compute)
        for block in reuse:
            self.engine.before_block_reuse(block, compute)


def test_a_batcher_that_restores_before_saving_is_caught():
    assert fails_somewhere(batcher=RestoresFirst)
