"""Continuous-batching scheduler: the caller whose admissions trigger restores, saves and prefetches.

Each step is one homogeneous batch: prefill if any waiting request can be
admitted, else decode; if decode preempted everything, prefill is tried
once more (nanovllm/engine/scheduler.py:44-81, its default policy).

Prefill admits waiting requests in order within a token budget. Only the
first request of a batch may be chunked; a split (hybrid) admission
schedules its head only, and requests behind it may join the batch while its
restored span copies. A waiting request that does not fit sets
`block_manager.admission_blocked` (which arms save-on-release in the CPU
tier) and prefetches its CPU hits into spare blocks, keeping one block per
running request for decode growth (:101-107).

Decode gives each running request one token and a new block when it crosses
a block boundary, preempting the newest running request (or itself) when no
block is free.

A failure anywhere in a prefill or decode pass (a copy that raises) undoes
the whole pass: queues, request fields and the blocks the pass took are as
before, so the step can be retried (:130-141, 172-180).
"""

from collections import deque

from kvx.engine.block_manager import BlockManager
from kvx.engine.sequence import Sequence, SequenceStatus


class _PrefillUndo:
    """What a prefill pass changed, for restoring it if the pass raises."""

    def __init__(self, scheduler: "Scheduler"):
        self.scheduler = scheduler
        self.waiting = list(scheduler.waiting)
        self.touched: list[tuple[Sequence, int, int, SequenceStatus, bool]] = []
        self.promoted: list[Sequence] = []

    def note(self, seq: Sequence):
        self.touched.append((seq, seq.num_cached_tokens, seq.num_scheduled_tokens, seq.status,
                             bool(seq.block_table)))

    def restore(self):
        manager = self.scheduler.block_manager
        for seq, cached, scheduled, status, had_blocks in reversed(self.touched):
            if seq.block_table and not had_blocks:
                manager.deallocate(seq)
            seq.num_cached_tokens, seq.num_scheduled_tokens, seq.status = cached, scheduled, status
        for seq in self.promoted:
            self.scheduler.running.remove(seq)
        self.scheduler.waiting.clear()
        self.scheduler.waiting.extend(self.waiting)


class Scheduler:
    """Queues and batching over one BlockManager.

    `config` provides max_num_seqs, max_num_batched_tokens, eos,
    kvcache_block_size, num_kvcache_blocks and optionally kv_eviction
    ("lru" by default), as the reference's Config does.
    """

    def __init__(self, config):
        self.max_num_seqs = config.max_num_seqs
        self.max_num_batched_tokens = config.max_num_batched_tokens
        self.eos = config.eos
        self.block_size = config.kvcache_block_size
        self.block_manager = BlockManager(config.num_kvcache_blocks, config.kvcache_block_size,
                                          getattr(config, "kv_eviction", "lru"))
        self.waiting: deque[Sequence] = deque()
        self.running: deque[Sequence] = deque()

    def is_finished(self) -> bool:
        return not self.waiting and not self.running

    def add(self, seq: Sequence):
        self.waiting.append(seq)

    def schedule(self) -> tuple[list[Sequence], bool]:
        """The next batch and whether it is a prefill."""
        self.block_manager.admission_blocked = False
        for is_prefill, make in ((True, self._prefill_batch), (False, self._decode_batch),
                                 (True, self._prefill_batch)):
            batch = make()
            if batch:
                return batch, is_prefill
        raise RuntimeError("no request can progress: check GPU KV capacity and request lengths")

    def _prefill_batch(self) -> list[Sequence]:
        budget = self.max_num_batched_tokens
        manager = self.block_manager
        batch: list[Sequence] = []
        used = 0
        undo = _PrefillUndo(self)
        try:
            i = 0  # requests before i are split admissions whose head is already in this batch
            while i < len(self.waiting) and len(batch) < self.max_num_seqs and used < budget:
                seq = self.waiting[i]
                undo.note(seq)
                cached_blocks = None
                if seq.block_table:  # a chunked prefill, or a split head, continues
                    new_tokens = seq.num_tokens - seq.num_cached_tokens
                else:
                    cached_blocks = manager.can_allocate(seq)
                    if cached_blocks < 0:
                        manager.admission_blocked = True
                        manager.prefetch(seq, reserve=len(self.running))
                        break
                    new_tokens = seq.num_tokens - cached_blocks * self.block_size
                room = budget - used
                if batch and new_tokens > room:
                    break
                if cached_blocks is not None:
                    manager.allocate(seq, cached_blocks)
                stop = seq.restore_span[0] if seq.restore_span else seq.num_tokens
                seq.num_scheduled_tokens = min(stop - seq.num_cached_tokens, room)
                used += seq.num_scheduled_tokens
                batch.append(seq)
                reached = seq.num_cached_tokens + seq.num_scheduled_tokens
                if reached == seq.num_tokens:
                    seq.status = SequenceStatus.RUNNING
                    del self.waiting[i]
                    undo.promoted.append(seq)
                    self.running.append(seq)
                elif seq.restore_span and reached == seq.restore_span[0]:
                    i += 1
                else:
                    break  # chunked: it stays at the head of the queue
        except BaseException:
            undo.restore()
            raise
        return batch

    def _decode_batch(self) -> list[Sequence]:
        manager = self.block_manager
        batch: list[Sequence] = []
        before: list[tuple[Sequence, int, int, bool]] = []  # state of each request this pass grew
        try:
            while self.running and len(batch) < self.max_num_seqs:
                seq = self.running.popleft()
                while seq is not None and not manager.can_append(seq):
                    if self.running:
                        self.preempt(self.running.pop())
                    else:
                        self.preempt(seq)
                        seq = None
                if seq is None:
                    continue
                before.append((seq, len(seq.block_table), seq.num_scheduled_tokens, seq.is_prefill))
                seq.num_scheduled_tokens = 1
                seq.is_prefill = False
                manager.may_append(seq)
                batch.append(seq)
        except BaseException:
            for seq, length, scheduled, was_prefill in reversed(before):
                for block_id in reversed(seq.block_table[length:]):
                    manager._release_block(block_id)
                del seq.block_table[length:]
                seq.num_scheduled_tokens, seq.is_prefill = scheduled, was_prefill
            self.running.extendleft(reversed([seq for seq, *_ in before]))
            raise
        self.running.extendleft(reversed(batch))
        return batch

    def preempt(self, seq: Sequence):
        """Back to the front of the waiting queue without its KV (it is recomputed or hit again)."""
        seq.status = SequenceStatus.WAITING
        seq.is_prefill = True
        self.block_manager.deallocate(seq)
        self.waiting.appendleft(seq)

    def postprocess(self, seqs: list[Sequence], token_ids: list[int], is_prefill: bool):
        """After the model ran: publish filled blocks, advance, append sampled tokens, retire finished requests."""
        manager = self.block_manager
        for seq, token_id in zip(seqs, token_ids):
            manager.hash_blocks(seq)
            seq.num_cached_tokens += seq.num_scheduled_tokens
            seq.num_scheduled_tokens = 0
            if seq.restore_span and seq.num_cached_tokens == seq.restore_span[0]:
                manager.finish_restore_span(seq)
            if is_prefill and seq.num_cached_tokens < seq.num_tokens:
                continue  # a chunk or a split head: no token is sampled yet
            seq.append_token(token_id)
            hit_eos = not seq.ignore_eos and token_id == self.eos
            if hit_eos or seq.num_completion_tokens == seq.max_tokens:
                seq.status = SequenceStatus.FINISHED
                manager.deallocate(seq)
                self.running.remove(seq)
