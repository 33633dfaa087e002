"""Continuous-batching scheduler: the caller that triggers saves, restores and prefetches.

Behaviour follows nanovllm/engine/scheduler.py (line citations below): legacy
or chunk-budgeted prefill policies, chunked prefill of the head request,
split (hybrid) admissions whose head joins later requests, decode with
preemption, and full rollback when a copy fails mid-batch. Admission blocking
is what arms save-on-release and prefetch in the block manager.
"""

from collections import deque
from dataclasses import dataclass

from kvx.engine.block_manager import BlockManager
from kvx.engine.sequence import Sequence, SequenceStatus

PREFILL_POLICIES = ("legacy", "fixed", "decode_aware")


def validate_scheduling_options(policy, chunk_size, min_chunk_size, batch_tokens, batch_seqs):
    """nanovllm/config.py:8-20."""
    if policy not in PREFILL_POLICIES:
        raise ValueError(f"prefill_policy must be one of {PREFILL_POLICIES}")
    for name, value in (("prefill_chunk_size", chunk_size), ("prefill_min_chunk_size", min_chunk_size),
                        ("max_num_batched_tokens", batch_tokens), ("max_num_seqs", batch_seqs)):
        if type(value) is not int or value < 1:
            raise ValueError(f"{name} must be a positive integer")
    if min_chunk_size > chunk_size:
        raise ValueError("prefill_min_chunk_size must not exceed prefill_chunk_size")


@dataclass(frozen=True)
class ScheduleDecision:
    policy: str
    phase: str
    prefill_budget: int
    decode_requests: int  # runnable decoders before admission/preemption
    scheduled_tokens: int
    seq_ids: tuple[int, ...]


class Scheduler:

    def __init__(self, config):
        self.max_num_seqs = config.max_num_seqs
        self.max_num_batched_tokens = config.max_num_batched_tokens
        self.prefill_policy = getattr(config, "prefill_policy", "legacy")
        self.prefill_chunk_size = getattr(config, "prefill_chunk_size", 512)
        self.prefill_min_chunk_size = getattr(config, "prefill_min_chunk_size", 1)
        validate_scheduling_options(self.prefill_policy, self.prefill_chunk_size, self.prefill_min_chunk_size,
                                    self.max_num_batched_tokens, self.max_num_seqs)
        self.last_schedule: ScheduleDecision | None = None
        self.eos = config.eos
        self.block_size = config.kvcache_block_size
        self.block_manager = BlockManager(config.num_kvcache_blocks, config.kvcache_block_size,
                                          getattr(config, "kv_eviction", "lru"))
        self.waiting: deque[Sequence] = deque()
        self.running: deque[Sequence] = deque()

    def is_finished(self):
        return not self.waiting and not self.running

    def add(self, seq: Sequence):
        self.waiting.append(seq)

    def _decision(self, phase, budget, decode_requests, seqs):
        self.last_schedule = ScheduleDecision(self.prefill_policy, phase, budget, decode_requests,
                                              sum(seq.num_scheduled_tokens for seq in seqs),
                                              tuple(seq.seq_id for seq in seqs))

    def schedule(self) -> tuple[list[Sequence], bool]:
        """One homogeneous prefill or decode batch (scheduler.py:44-81).

        Non-legacy policies cap prefill at a chunk budget and alternate
        phases: after a prefill batch, runnable decoders go first.
        """
        decode_requests = len(self.running)
        budget = self.max_num_batched_tokens
        self.block_manager.admission_blocked = False
        if self.prefill_policy != "legacy":
            chunk = self.prefill_chunk_size
            if self.prefill_policy == "decode_aware":
                chunk = max(self.prefill_min_chunk_size, chunk // (1 + decode_requests))
            budget = min(budget, chunk)
        decode_due = (self.prefill_policy != "legacy" and self.running and self.last_schedule is not None
                      and self.last_schedule.phase == "prefill")
        for is_prefill in ((False, True) if decode_due else (True, False)):
            seqs = self._schedule_prefill(budget) if is_prefill else self._schedule_decode()
            if seqs:
                self._decision("prefill" if is_prefill else "decode", budget, decode_requests, seqs)
                return seqs, is_prefill
        # Decode may have preempted everything, making a blocked prefill admissible.
        seqs = self._schedule_prefill(budget)
        if seqs:
            self._decision("prefill", budget, decode_requests, seqs)
            return seqs, True
        raise RuntimeError("no request can progress: check GPU KV capacity and request lengths")

    def _schedule_prefill(self, budget: int) -> list[Sequence]:
        """Admit and chunk waiting requests (scheduler.py:83-143); a failure restores every request."""
        scheduled: list[Sequence] = []
        batched = 0
        saved_state = []
        removed = []
        original_waiting = list(self.waiting)
        i = 0  # requests before i are split admissions whose head is already scheduled
        try:
            while i < len(self.waiting) and len(scheduled) < self.max_num_seqs:
                seq = self.waiting[i]
                remaining = budget - batched
                if remaining == 0:
                    break
                saved_state.append((seq, seq.num_cached_tokens, seq.num_scheduled_tokens, seq.status,
                                    bool(seq.block_table)))
                if not seq.block_table:
                    cached_blocks = self.block_manager.can_allocate(seq)
                    if cached_blocks == -1:
                        # Spend the wait restoring its CPU hits into spare blocks.
                        self.block_manager.admission_blocked = True
                        self.block_manager.prefetch(seq, reserve=len(self.running))
                        break
                    num_tokens = seq.num_tokens - cached_blocks * self.block_size
                else:
                    num_tokens = seq.num_tokens - seq.num_cached_tokens
                if remaining < num_tokens and scheduled:  # only the first request may be chunked
                    break
                if not seq.block_table:
                    self.block_manager.allocate(seq, cached_blocks)
                # A split admission prefills only up to its restore span first.
                end = seq.restore_span[0] if seq.restore_span else seq.num_tokens
                seq.num_scheduled_tokens = min(end - seq.num_cached_tokens, remaining)
                batched += seq.num_scheduled_tokens
                scheduled.append(seq)
                if seq.num_cached_tokens + seq.num_scheduled_tokens == seq.num_tokens:
                    seq.status = SequenceStatus.RUNNING
                    del self.waiting[i]
                    removed.append(seq)
                    self.running.append(seq)
                elif seq.restore_span and seq.num_cached_tokens + seq.num_scheduled_tokens == seq.restore_span[0]:
                    i += 1  # head fully scheduled; it stays queued while later requests join
                else:
                    break  # a chunked prefill stays at the head of the queue
        except BaseException:
            for seq, cached, sched, status, had_blocks in reversed(saved_state):
                if not had_blocks and seq.block_table:
                    self.block_manager.deallocate(seq)
                seq.num_cached_tokens, seq.num_scheduled_tokens, seq.status = cached, sched, status
            for seq in removed:
                self.running.remove(seq)
            self.waiting.clear()
            self.waiting.extend(original_waiting)
            raise
        return scheduled

    def _schedule_decode(self) -> list[Sequence]:
        """One token for each runnable request, preempting when blocks run out (scheduler.py:145-186)."""
        scheduled: list[Sequence] = []
        saved_state = []
        try:
            while self.running and len(scheduled) < self.max_num_seqs:
                seq = self.running.popleft()
                while not self.block_manager.can_append(seq):
                    # Reclaim interleaved partial prefills before evicting live decoders.
                    partial = next((item for item in reversed(self.waiting) if item.block_table), None)
                    if self.prefill_policy != "legacy" and partial is not None:
                        self.block_manager.deallocate(partial)
                        continue
                    if self.running:
                        self.preempt(self.running.pop())
                    else:
                        self.preempt(seq)
                        break
                else:
                    saved_state.append((seq, len(seq.block_table), seq.num_scheduled_tokens, seq.is_prefill))
                    seq.num_scheduled_tokens = 1
                    seq.is_prefill = False
                    self.block_manager.may_append(seq)
                    scheduled.append(seq)
        except BaseException:
            for seq, old_length, sched, is_prefill in reversed(saved_state):
                for block_id in reversed(seq.block_table[old_length:]):
                    self.block_manager._release_block(block_id)
                del seq.block_table[old_length:]
                seq.num_scheduled_tokens, seq.is_prefill = sched, is_prefill
            self.running.extendleft(reversed([seq for seq, *_ in saved_state]))
            raise
        if self.prefill_policy == "legacy":
            self.running.extendleft(reversed(scheduled))
        else:
            self.running.extend(scheduled)  # more residents than batch slots all get decode time
        return scheduled

    def preempt(self, seq: Sequence):
        seq.status = SequenceStatus.WAITING
        seq.is_prefill = True
        self.block_manager.deallocate(seq)
        self.waiting.appendleft(seq)

    def postprocess(self, seqs: list[Sequence], token_ids: list[int], is_prefill: bool):
        """Publish completed blocks, advance caches, append tokens, retire finished requests (:194-207)."""
        for seq, token_id in zip(seqs, token_ids):
            self.block_manager.hash_blocks(seq)
            seq.num_cached_tokens += seq.num_scheduled_tokens
            seq.num_scheduled_tokens = 0
            if seq.restore_span and seq.num_cached_tokens == seq.restore_span[0]:
                self.block_manager.finish_restore_span(seq)
            if is_prefill and seq.num_cached_tokens < seq.num_tokens:
                continue
            seq.append_token(token_id)
            if (not seq.ignore_eos and token_id == self.eos) or seq.num_completion_tokens == seq.max_tokens:
                seq.status = SequenceStatus.FINISHED
                self.block_manager.deallocate(seq)
                self.running.remove(seq)
