"""Uncompressed KV handoff of a running request between engines (TP=1).

Same snapshot format and semantics as nanovllm/engine/kv_handoff.py: the
payload holds the written tokens only, in logical order, on the CPU, as
[K/V, layer, token, KV head, head dim]. The gather (export) and scatter
(import) run as libkvx token-copy kernels instead of index_select + per-block
copy_; the payload lives in pinned host memory, which the kernels read and
write across the host link directly.
"""

from dataclasses import dataclass

import torch

from kvx import ops
from kvx.engine.handoff_timing import PhaseTimer
from kvx.engine.sequence import SamplingParams, Sequence, SequenceStatus


@dataclass
class KVSnapshot:
    token_ids: list[int]
    num_prompt_tokens: int
    num_cached_tokens: int
    block_size: int
    temperature: float
    max_tokens: int
    ignore_eos: bool
    kv: torch.Tensor  # [K/V, layer, written token, KV head, head dim], CPU

    @property
    def payload_bytes(self):
        return self.kv.numel() * self.kv.element_size()


def export_kv(runner, seq: Sequence) -> KVSnapshot:
    """Snapshot a running request between steps (kv_handoff.py:34-59).

    Timed phases (handoff_timing): gather_blocks allocates the pinned payload,
    pack queues the gather kernel that packs the blocks' written tokens into
    it, and copy_to_host waits for that kernel, whose writes cross the host link.
    """
    if runner.world_size != 1:
        raise NotImplementedError("KV handoff currently requires tensor_parallel_size=1")
    if seq.status != SequenceStatus.RUNNING or seq.num_scheduled_tokens:
        raise ValueError("export requires a running sequence between steps")
    count = seq.num_cached_tokens
    if count <= 0 or count != len(seq) - 1:
        raise ValueError("export requires exactly one pending, uncached token")
    num_blocks = -(-count // runner.block_size)
    timer = PhaseTimer("export_kv", seq_id=seq.seq_id, num_tokens=count, num_blocks=num_blocks)
    pool = runner.kv_cache
    with timer.phase("gather_blocks"):
        if len(seq.block_table) < num_blocks:
            raise ValueError("sequence is missing KV blocks")
        # The gather kernel writes the pinned host payload itself (one pass over the
        # host link, 54 GB/s on MI355X for a 32K-token Qwen3-8B request, against
        # 4.1 GB/s for a device gather followed by a pageable .cpu() copy).
        payload = torch.empty((2, pool.shape[1], count, *pool.shape[-2:]), dtype=pool.dtype, pin_memory=True)
    with timer.phase("pack"):
        ops.gather_tokens(pool, seq.block_table[:num_blocks], count, payload)
    with timer.phase("copy_to_host"):
        torch.cuda.current_stream(pool.device).synchronize()
    timer.finish(payload_bytes=payload.numel() * payload.element_size())
    return KVSnapshot(seq.token_ids.copy(), seq.num_prompt_tokens, count, runner.block_size, seq.temperature,
                      seq.max_tokens, seq.ignore_eos, payload)


def verify_imported_kv(runner, seq: Sequence, snapshot: KVSnapshot) -> bool:
    """Byte-compare the imported blocks with the snapshot, one block at a time (kv_handoff.py:62-77)."""
    pool = runner.kv_cache
    for logical, physical in enumerate(seq.block_table):
        start = logical * runner.block_size
        end = min(start + runner.block_size, snapshot.num_cached_tokens)
        if end <= start:
            break
        actual = pool[:, :, physical, :end - start].cpu()
        expected = snapshot.kv[:, :, start:end]
        if not torch.equal(actual.view(torch.uint8), expected.contiguous().view(torch.uint8)):
            return False
    return True


def import_kv(runner, block_manager, snapshot: KVSnapshot) -> Sequence:
    """Allocate fresh blocks and rebuild a decode-ready sequence (kv_handoff.py:80-135).

    Failure after allocation releases the blocks; prefix hashes are published
    only after the scatter is queued. Timed phases (handoff_timing) as the
    reference's; copy_to_device only copies a payload that is not pinned (a
    pinned one is read in place by the scatter kernel, queued in scatter_blocks).
    """
    if runner.world_size != 1:
        raise NotImplementedError("KV handoff currently requires tensor_parallel_size=1")
    timer = PhaseTimer("import_kv", num_cached_tokens=snapshot.num_cached_tokens,
                       num_tokens=len(snapshot.token_ids))
    seq = None
    try:
        with timer.phase("validate"):
            pool = runner.kv_cache
            expected = (2, pool.shape[1], snapshot.num_cached_tokens, *pool.shape[-2:])
            if (snapshot.block_size != runner.block_size or block_manager.block_size != runner.block_size
                    or tuple(snapshot.kv.shape) != expected or snapshot.kv.dtype != pool.dtype
                    or snapshot.kv.device.type != "cpu"):
                raise ValueError("snapshot layout, dtype or block size does not match this worker")
            if (not 0 < snapshot.num_prompt_tokens < len(snapshot.token_ids)
                    or snapshot.num_cached_tokens != len(snapshot.token_ids) - 1
                    or len(snapshot.token_ids) - snapshot.num_prompt_tokens >= snapshot.max_tokens):
                raise ValueError("snapshot must contain an unfinished completion and one uncached token")
        with timer.phase("rebuild_sequence"):
            seq = Sequence(snapshot.token_ids[:snapshot.num_prompt_tokens],
                           SamplingParams(temperature=snapshot.temperature, max_tokens=snapshot.max_tokens,
                                          ignore_eos=snapshot.ignore_eos))
            for token in snapshot.token_ids[snapshot.num_prompt_tokens:]:
                seq.append_token(token)
        with timer.phase("allocate_blocks"):
            block_manager.allocate_for_resume(seq, snapshot.num_cached_tokens)
        with timer.phase("copy_to_device"):
            # A pinned payload (what export_kv produces) is read by the scatter kernel in place, so it must stay
            # unchanged until the stream has run the scatter (resume_request synchronizes); others are copied first.
            payload = snapshot.kv
            if not (payload.is_pinned() and payload.is_contiguous()):
                payload = payload.to(device=pool.device).contiguous()
        with timer.phase("scatter_blocks"):
            ops.scatter_tokens(pool, seq.block_table, snapshot.num_cached_tokens, payload)
        with timer.phase("publish_cache"):
            # Prefix metadata becomes valid only once the payload's copy is queued.
            seq.num_cached_tokens = 0
            seq.num_scheduled_tokens = snapshot.num_cached_tokens
            block_manager.hash_blocks(seq)
            seq.num_scheduled_tokens = 0
            seq.num_cached_tokens = snapshot.num_cached_tokens
            seq.status = SequenceStatus.RUNNING
            seq.is_prefill = False
        timer.finish(payload_bytes=lambda: snapshot.payload_bytes, num_blocks=lambda: len(seq.block_table))
        return seq
    except BaseException as error:
        timer.abort(error)
        if seq is not None:
            block_manager.deallocate(seq)
        raise
