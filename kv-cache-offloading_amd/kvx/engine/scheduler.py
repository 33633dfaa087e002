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

A client hint kept for later (`prefetch_hint`, set by
LLMEngine.prefetch_prefix(..., defer=True) while requests wait) is started
at the end of the first prefill pass after which no waiting request lacks
blocks: the step's admissions have taken theirs, and the model has not run
yet, so the hint's restores overlap the step's compute. The reference
starts hints only between steps (nanovllm/engine/llm_engine.py:112-126),
where a hint given while a request waits is dropped and its restores begin
after that request's compute.

Decode gives each running request one token and a new block when it crosses
a block boundary, preempting the newest running request (or itself) when no
block is free.

A pass records the inverse of each change it makes (an undo log). If
anything in it raises (a copy, a save of a recycled block), the log is
replayed newest first, so queues, request fields and the blocks the pass
took are as before and the step can be retried (:130-141, 172-180).
Preemptions and prefetches are not undone; they leave a consistent state.
"""

from collections import deque
from collections.abc import Callable

from kvx.engine.block_manager import BlockManager
from kvx.engine.sequence import Sequence, SequenceStatus


class _UndoLog:
    """Inverse operations of one scheduling pass, replayed newest first by rewind()."""

    def __init__(self):
        self._inverse: list[Callable[[], None]] = []

    def push(self, inverse: Callable[[], None]):
        self._inverse.append(inverse)

    def remember(self, obj, *names: str):
        """Restore these attributes of `obj` to their current values on rewind."""
        old = {name: getattr(obj, name) for name in names}
        self.push(lambda: [setattr(obj, name, value) for name, value in old.items()])

    def assign(self, obj, **fields):
        """Set attributes of `obj`, remembering their previous values."""
        self.remember(obj, *fields)
        for name, value in fields.items():
            setattr(obj, name, value)

    def rewind(self):
        while self._inverse:
            self._inverse.pop()()


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
        self.prefetch_hint: Sequence | None = None

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

    # -- prefill --------------------------------------------------------------------

    def _tokens_to_prefill(self, seq: Sequence) -> tuple[int, int | None] | None:
        """(tokens the request still has to prefill, cached blocks to admit it with), or None if it cannot be
        admitted now.

        A request without blocks is looked up (its cached prefix is skipped);
        one that has blocks continues a chunked prefill or a split head (no
        admission: None for the cached blocks).
        """
        if seq.block_table:
            return seq.num_tokens - seq.num_cached_tokens, None
        cached_blocks = self.block_manager.can_allocate(seq)
        if cached_blocks < 0:
            return None
        return seq.num_tokens - cached_blocks * self.block_size, cached_blocks

    def _prefill_batch(self) -> list[Sequence]:
        manager = self.block_manager
        log = _UndoLog()
        batch: list[Sequence] = []
        room = self.max_num_batched_tokens
        try:
            # Iterate over a snapshot: requests promoted to running leave the
            # queue, split heads stay in it while later requests join.
            for seq in list(self.waiting):
                if not room or len(batch) == self.max_num_seqs:
                    break
                log.remember(seq, "num_cached_tokens", "num_scheduled_tokens", "status")
                fit = self._tokens_to_prefill(seq)
                if fit is None:
                    manager.admission_blocked = True
                    manager.prefetch(seq, reserve=len(self.running))
                    break
                needed, cached_blocks = fit
                if batch and needed > room:
                    break  # only the first request of a batch may be chunked
                if cached_blocks is not None:
                    manager.allocate(seq, cached_blocks)
                    log.push(lambda seq=seq: manager.deallocate(seq))
                end = seq.restore_span[0] if seq.restore_span else seq.num_tokens
                seq.num_scheduled_tokens = min(end - seq.num_cached_tokens, room)
                room -= seq.num_scheduled_tokens
                batch.append(seq)
                reached = seq.num_cached_tokens + seq.num_scheduled_tokens
                if reached == seq.num_tokens:
                    self._promote(seq, log)
                elif not (seq.restore_span and reached == seq.restore_span[0]):
                    break  # chunked: it stays at the head of the queue
            if batch and self.prefetch_hint is not None:
                self._start_hint()
        except BaseException:
            log.rewind()
            raise
        return batch

    def _start_hint(self):
        """One attempt at the kept hint, once every waiting request holds its blocks; the hint is then dropped.

        Requests that are still waiting here continue a chunked prefill or a
        split head; each keeps a block, as running ones do, for the token it
        samples. A failing copy raises out of the pass, which then rewinds
        its admissions.
        """
        if any(not seq.block_table for seq in self.waiting):
            return  # a request still needs blocks: the hint must not take them
        hint, self.prefetch_hint = self.prefetch_hint, None
        self.block_manager.prefetch(hint, reserve=len(self.running) + len(self.waiting))

    def _promote(self, seq: Sequence, log: _UndoLog):
        """The request's whole prompt is in this batch: it moves from waiting to running."""
        position = self.waiting.index(seq)
        del self.waiting[position]
        self.running.append(seq)
        seq.status = SequenceStatus.RUNNING

        def undo():
            self.running.remove(seq)
            self.waiting.insert(position, seq)

        log.push(undo)

    # -- decode -----------------------------------------------------------------------

    def _make_room(self, seq: Sequence) -> bool:
        """Preempt the newest running requests until `seq` can grow; False if `seq` itself had to go."""
        manager = self.block_manager
        while not manager.can_append(seq):
            if not self.running:
                self.preempt(seq)
                return False
            self.preempt(self.running.pop())
        return True

    def _decode_batch(self) -> list[Sequence]:
        manager = self.block_manager
        log = _UndoLog()
        batch: list[Sequence] = []
        popped: list[Sequence] = []
        try:
            while self.running and len(batch) < self.max_num_seqs:
                seq = self.running.popleft()
                popped.append(seq)
                if not self._make_room(seq):
                    continue
                log.assign(seq, num_scheduled_tokens=1, is_prefill=False)
                length = len(seq.block_table)
                log.push(lambda seq=seq, length=length: self._shrink(seq, length))
                manager.may_append(seq)
                batch.append(seq)
        except BaseException:
            log.rewind()
            # Requests taken off the queue go back to its front in order, unless preempted.
            self.running.extendleft(reversed([seq for seq in popped if seq.status is not SequenceStatus.WAITING]))
            raise
        self.running.extendleft(reversed(batch))
        return batch

    def _shrink(self, seq: Sequence, length: int):
        """Give back the blocks `seq` gained beyond its first `length`."""
        for block_id in reversed(seq.block_table[length:]):
            self.block_manager._release_block(block_id)
        del seq.block_table[length:]

    def preempt(self, seq: Sequence):
        """Back to the front of the waiting queue without its KV (it is recomputed or hit again)."""
        seq.status = SequenceStatus.WAITING
        seq.is_prefill = True
        self.block_manager.deallocate(seq)
        self.waiting.appendleft(seq)

    # -- after the model ran ---------------------------------------------------------------

    def postprocess(self, seqs: list[Sequence], token_ids: list[int], is_prefill: bool):
        """Publish filled blocks, advance, append sampled tokens and retire finished requests."""
        for seq, token_id in zip(seqs, token_ids):
            self._advance(seq)
            if is_prefill and seq.num_cached_tokens < seq.num_tokens:
                continue  # a chunk or a split head: no token is sampled yet
            self._sample(seq, token_id)

    def _advance(self, seq: Sequence):
        """The step's tokens now have KV: publish the blocks they fill, and skip a restored span once reached."""
        manager = self.block_manager
        manager.hash_blocks(seq)
        seq.num_cached_tokens += seq.num_scheduled_tokens
        seq.num_scheduled_tokens = 0
        if seq.restore_span and seq.num_cached_tokens == seq.restore_span[0]:
            manager.finish_restore_span(seq)

    def _sample(self, seq: Sequence, token_id: int):
        seq.append_token(token_id)
        stop = token_id == self.eos and not seq.ignore_eos
        if stop or seq.num_completion_tokens == seq.max_tokens:
            seq.status = SequenceStatus.FINISHED
            self.block_manager.deallocate(seq)
            self.running.remove(seq)
