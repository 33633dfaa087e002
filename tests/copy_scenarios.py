"""Seeded caller sequences for the copy engine: what the block manager and the CPU tier ask of it.

`Caller` drives a `_CopyBatcher` (and through it a copy engine) and the caller's stream the way kvx's
BlockManager and CPUBlockCache do with the reference's hooks (block_manager.py:97-137, 145-183, 202-237,
266-336; cpu_prefix_cache.py:334-363, 370-398):
- admission, inside coalesce(): each block of the request is a recycled victim. Its value is saved
  first when the CPU tier does not hold it yet, then before_block_reuse; the block is either fresh or
  restores a CPU entry (wait=True; wait=False for a split admission's restored span, read later after
  before_block_use). After the block, the caller's stream writes the fresh blocks and reads the
  restored ones;
- prefetch, inside coalesce(): victims saved, then restores with wait=False into them, without
  before_block_reuse (block_manager.py:168 reserves blocks without write ordering);
- restore_block (restore_cached_block, block_manager.py:145-183): a victim saved if needed, then a
  restore with wait=True into it, without before_block_reuse, then a read;
- use: before_block_use, then the caller's stream reads the block;
- release-time saves of blocks that stay on the GPU (deallocate, inside coalesce());
- discards of CPU entries: the slot can be reused by the next save while a restore still reads it;
- with `switch_streams=True`, a change of the caller's current stream between actions, the new one first
  waiting for the old one, as a correct torch program switches streams (the engine then sees copies and
  waits issued for different caller streams).
With `batched=False` nothing is coalesced, as with the reference's BlockManager (one engine call per
block). The caller records what a sequential execution gives: every read of the caller's stream and the
final value of every block and live slot. `check()` compares them with what the backend observed.

A backend provides `batcher`, `write(block, value)` and `read(block) -> token` on the caller's stream,
`value(token)` after `sync()`, `between()` (host time between calls), `block_value` / `slot_value`
after `sync()`, and `switch_stream()` if streams are switched. Values are the integers 1, 2, 3, ...
"""

import random


class Caller:
    def __init__(self, rng: random.Random, backend, num_blocks: int, num_slots: int, batched: bool = True,
                 max_request_blocks: int = 6, switch_streams: bool = False):
        self.rng, self.backend = rng, backend
        self.batched = batched
        self.switch_streams = switch_streams
        self.num_blocks = num_blocks
        self.max_request = max_request_blocks
        self.next_value = 1
        self.block = [0] * num_blocks        # expected value of each block
        self.prefetched = set()              # blocks restored with wait=False, not used since
        self.entries = {}                    # live slot -> expected value
        self.slot_of = {}                    # value -> a live slot holding it
        self.free_slots = list(range(num_slots))
        self.reads = []                      # (expected value, token, what)
        self.log = []                        # actions, for failure messages
        for b in range(num_blocks):
            self.block[b] = self._value()
            backend.write(b, self.block[b])
        backend.sync()

    # -- helpers -------------------------------------------------------------------------------

    def _value(self) -> int:
        v = self.next_value
        self.next_value += 1
        return v

    def _coalesce(self):
        if self.batched:
            return self.backend.batcher.coalesce()
        return _Nothing()

    def _save(self, b: int):
        """Saves block b's value unless the CPU tier holds it or the budget is spent (a budget skip)."""
        value = self.block[b]
        if value in self.slot_of or not self.free_slots:
            return
        slot = self.free_slots.pop(self.rng.randrange(len(self.free_slots)))
        self.backend.batcher.save(b, slot)
        self.entries[slot] = value
        self.slot_of[value] = slot
        self.log.append(f"save {b} -> slot {slot} (value {value})")

    def _victims(self, k: int) -> list[int]:
        return self.rng.sample(range(self.num_blocks), k)

    def _read(self, b: int, what: str):
        self.reads.append((self.block[b], self.backend.read(b), f"{what}: block {b}"))
        self.log.append(f"read {b} (expect {self.block[b]})")

    # -- actions ---------------------------------------------------------------------------------

    def admission(self):
        blocks = self._victims(self.rng.randint(1, self.max_request))
        fresh, restored, later = [], [], []
        split = self.rng.random() < 0.25
        with self._coalesce():
            for b in blocks:
                if self.rng.random() < 0.7:
                    self._save(b)
                self.backend.batcher.before_block_reuse(b)
                self.prefetched.discard(b)
                self.log.append(f"reuse {b}")
                if self.entries and self.rng.random() < 0.6:
                    slot = self.rng.choice(list(self.entries))
                    wait = not split
                    self.backend.batcher.restore(slot, b, wait)
                    self.block[b] = self.entries[slot]
                    (restored if wait else later).append(b)
                    self.log.append(f"restore slot {slot} -> {b} wait={wait} (value {self.block[b]})")
                else:
                    fresh.append(b)
        self.backend.between()
        for b in fresh:
            self.block[b] = self._value()
            self.backend.write(b, self.block[b])
            self.log.append(f"write {b} = {self.block[b]}")
        for b in restored:
            self._read(b, "admission restore")
        for b in later:
            self.backend.batcher.before_block_use(b)
            self._read(b, "split admission restore")

    def prefetch(self):
        if not self.entries:
            return
        blocks = self._victims(self.rng.randint(1, self.max_request))
        with self._coalesce():
            for b in blocks:
                if self.rng.random() < 0.7:
                    self._save(b)
                slot = self.rng.choice(list(self.entries))
                self.backend.batcher.restore(slot, b, False)
                self.block[b] = self.entries[slot]
                self.prefetched.add(b)
                self.log.append(f"prefetch slot {slot} -> {b} (value {self.block[b]})")

    def restore_block(self):
        if not self.entries:
            return
        # The least recently used victims of a pool under pressure include prefetched blocks not used yet.
        pool = sorted(self.prefetched) if self.prefetched and self.rng.random() < 0.5 else range(self.num_blocks)
        b = self.rng.choice(list(pool))
        with self._coalesce():
            self._save(b)
            slot = self.rng.choice(list(self.entries))
            self.backend.batcher.restore(slot, b, True)
            self.block[b] = self.entries[slot]
            self.prefetched.discard(b)
            self.log.append(f"restore_block slot {slot} -> {b} (value {self.block[b]})")
        self._read(b, "restore_block")

    def use(self):
        pool = sorted(self.prefetched) if self.prefetched and self.rng.random() < 0.8 else range(self.num_blocks)
        b = self.rng.choice(list(pool))
        self.backend.batcher.before_block_use(b)
        self.prefetched.discard(b)
        self._read(b, "use")

    def release(self):
        with self._coalesce():
            for b in self._victims(self.rng.randint(1, 3)):
                self._save(b)

    def discard(self):
        if not self.entries:
            return
        slot = self.rng.choice(list(self.entries))
        value = self.entries.pop(slot)
        if self.slot_of.get(value) == slot:
            del self.slot_of[value]
        self.free_slots.append(slot)
        self.log.append(f"discard slot {slot}")

    def switch_stream(self):
        self.backend.switch_stream()
        self.log.append("switch stream")

    ACTIONS = (("admission", 4), ("prefetch", 2), ("restore_block", 2), ("use", 3), ("release", 2), ("discard", 2))

    def run(self, rounds: int):
        actions = self.ACTIONS + ((("switch_stream", 2),) if self.switch_streams else ())
        names, weights = zip(*actions)
        for _ in range(rounds):
            getattr(self, self.rng.choices(names, weights)[0])()
            self.backend.between()

    # -- verdict ----------------------------------------------------------------------------------

    def check(self) -> list[str]:
        """Every mismatch between the sequential expectation and what the backend observed."""
        self.backend.sync()
        bad = []
        for expected, token, what in self.reads:
            got = self.backend.value(token)
            if got != expected:
                bad.append(f"{what} read {got}, expected {expected}")
        for b, expected in enumerate(self.block):
            got = self.backend.block_value(b)
            if got != expected:
                bad.append(f"block {b} ends as {got}, expected {expected}")
        for slot, expected in self.entries.items():
            got = self.backend.slot_value(slot)
            if got != expected:
                bad.append(f"slot {slot} ends as {got}, expected {expected}")
        return bad


class NoAllocSaves:
    """An engine whose saves of up to `fits` blocks go through the allocation-free entry point.

    `save_noalloc(block_ids, slots, compute)` is that entry point; larger saves, and everything else, go to
    `engine` as usual, so sequences mix both kinds of save.
    """

    def __init__(self, engine, save_noalloc, fits: int):
        self.engine, self._save_noalloc, self.fits = engine, save_noalloc, fits

    def save(self, block_ids, slots, compute):
        if len(block_ids) <= self.fits:
            self._save_noalloc(block_ids, slots, compute)
        else:
            self.engine.save(block_ids, slots, compute)

    def __getattr__(self, name):
        return getattr(self.engine, name)


class _Nothing:
    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False
