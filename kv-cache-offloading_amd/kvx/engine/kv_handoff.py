"""KV handoff: move a running request, with its KV, from one engine to another (TP=1).

A KVSnapshot holds a request's tokens and sampling limits and the KV of
every token but the pending last one, in logical token order, in pinned host
memory. Two payload formats:

- BF16 (the reference's, nanovllm/engine/kv_handoff.py:17-59): `kv` is
  [2, L, T, H, hd] in the pool dtype; import reproduces the pool bytes exactly.
- FP8: `kv` is float8_e4m3fn [2, L, T, H, hd] and `scale` [2, L, T, H, 1]
  (bfloat16 or float32): exactly fp8_quantize of the BF16 payload
  (nanovllm/engine/cpu_prefix_cache.py:20-24), 0.51-0.52x its bytes.
  Import writes fp8_dequantize of it, as a restore from the CPU tier does.

Export runs one token-gather kernel per 128 blocks that writes the pinned
payload across the host link itself (quantising on the way for FP8) and
waits for it. Import copies the payload into device memory with one DMA per
tensor, then scatters it (dequantising for FP8) into freshly allocated
blocks; it returns after those copies finish, so the caller may free or
reuse the snapshot immediately.
"""

from dataclasses import dataclass

import torch

from kvx import ops
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
    kv: torch.Tensor  # [K/V, layer, token, KV head, head dim], pinned host memory
    scale: torch.Tensor | None = None  # FP8 only: [K/V, layer, token, KV head, 1]

    @property
    def fp8(self) -> bool:
        return self.kv.dtype == torch.float8_e4m3fn

    @property
    def payload_bytes(self) -> int:
        total = self.kv.numel() * self.kv.element_size()
        if self.scale is not None:
            total += self.scale.numel() * self.scale.element_size()
        return total


def _require_tp1(runner):
    if runner.world_size != 1:
        raise NotImplementedError("KV handoff currently requires tensor_parallel_size=1")


def export_kv(runner, seq: Sequence, *, fp8: bool = False, scale_dtype: torch.dtype = torch.float32) -> KVSnapshot:
    """Snapshot a running request between steps (kv_handoff.py:34-59); fp8=True sends FP8 codes and scales."""
    _require_tp1(runner)
    if seq.status is not SequenceStatus.RUNNING or seq.num_scheduled_tokens:
        raise ValueError("export requires a running sequence between steps")
    count = seq.num_cached_tokens
    if count <= 0 or count != len(seq) - 1:
        raise ValueError("export requires exactly one pending, uncached token")
    blocks = -(-count // runner.block_size)
    if len(seq.block_table) < blocks:
        raise ValueError("sequence is missing KV blocks")
    pool = runner.kv_cache
    shape = (2, pool.shape[1], count, *pool.shape[-2:])
    table = seq.block_table[:blocks]
    scale = None
    if fp8:
        if scale_dtype not in ops.SCALE_DTYPES:
            raise ValueError("FP8 scales must be bfloat16 or float32")
        kv = torch.empty(shape, dtype=torch.float8_e4m3fn, pin_memory=True)
        scale = torch.empty((*shape[:-1], 1), dtype=scale_dtype, pin_memory=True)
        ops.gather_tokens_fp8(pool, table, count, kv, scale)
    else:
        kv = torch.empty(shape, dtype=pool.dtype, pin_memory=True)
        ops.gather_tokens(pool, table, count, kv)
    torch.cuda.current_stream(pool.device).synchronize()
    return KVSnapshot(list(seq.token_ids), seq.num_prompt_tokens, count, runner.block_size, seq.temperature,
                      seq.max_tokens, seq.ignore_eos, kv, scale)


def _check_snapshot(runner, block_manager, snapshot: KVSnapshot):
    pool = runner.kv_cache
    shape = (2, pool.shape[1], snapshot.num_cached_tokens, *pool.shape[-2:])
    if snapshot.fp8:
        payload_ok = (snapshot.scale is not None and tuple(snapshot.scale.shape) == (*shape[:-1], 1)
                      and snapshot.scale.dtype in ops.SCALE_DTYPES and snapshot.scale.device.type == "cpu")
    else:
        payload_ok = snapshot.kv.dtype == pool.dtype and snapshot.scale is None
    if (not payload_ok or snapshot.block_size != runner.block_size or block_manager.block_size != runner.block_size
            or tuple(snapshot.kv.shape) != shape or snapshot.kv.device.type != "cpu"):
        raise ValueError("snapshot layout, dtype or block size does not match this worker")
    tokens = len(snapshot.token_ids)
    if (not 0 < snapshot.num_prompt_tokens < tokens or snapshot.num_cached_tokens != tokens - 1
            or tokens - snapshot.num_prompt_tokens >= snapshot.max_tokens):
        raise ValueError("snapshot must contain an unfinished completion and one uncached token")


def _to_device(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    return t.contiguous().to(device, non_blocking=t.is_pinned())


def import_kv(runner, block_manager, snapshot: KVSnapshot) -> Sequence:
    """Allocate fresh blocks, copy the snapshot's KV into them and return a decode-ready request (:80-135).

    The blocks' prefix hashes are published once the copies are queued; if
    anything fails after allocation the blocks are released. Returns after
    the copies completed (the snapshot is no longer read).
    """
    _require_tp1(runner)
    _check_snapshot(runner, block_manager, snapshot)
    params = SamplingParams(temperature=snapshot.temperature, max_tokens=snapshot.max_tokens,
                            ignore_eos=snapshot.ignore_eos)
    seq = Sequence.resumed(snapshot.token_ids, snapshot.num_prompt_tokens, params)
    block_manager.allocate_for_resume(seq, snapshot.num_cached_tokens)
    pool = runner.kv_cache
    count = snapshot.num_cached_tokens
    try:
        kv = _to_device(snapshot.kv, pool.device)
        if snapshot.fp8:
            ops.scatter_tokens_fp8(pool, seq.block_table, count, kv, _to_device(snapshot.scale, pool.device))
        else:
            ops.scatter_tokens(pool, seq.block_table, count, kv)
        seq.num_cached_tokens, seq.num_scheduled_tokens = 0, count
        block_manager.hash_blocks(seq)
        seq.num_cached_tokens, seq.num_scheduled_tokens = count, 0
        seq.status = SequenceStatus.RUNNING
        seq.is_prefill = False
        torch.cuda.current_stream(pool.device).synchronize()
    except BaseException:
        block_manager.deallocate(seq)
        raise
    return seq


def verify_imported_kv(runner, seq: Sequence, snapshot: KVSnapshot) -> bool:
    """Whether the request's blocks hold the snapshot's KV: its bytes (BF16) or their FP8 round trip (kv_handoff.py:62-77).

    The comparison runs on the device: the request's tokens are gathered out
    of its blocks and compared with the snapshot (dequantised for FP8).
    """
    pool = runner.kv_cache
    count = snapshot.num_cached_tokens
    if len(seq.block_table) < -(-count // runner.block_size):
        return False
    actual = torch.empty((2, pool.shape[1], count, *pool.shape[-2:]), dtype=pool.dtype, device=pool.device)
    ops.gather_tokens(pool, seq.block_table, count, actual)
    if snapshot.fp8:
        expected = torch.empty_like(actual)
        ops.fp8_dequantize(_to_device(snapshot.kv, pool.device), _to_device(snapshot.scale, pool.device), expected)
    else:
        expected = _to_device(snapshot.kv, pool.device)
    return torch.equal(actual.view(torch.uint8), expected.view(torch.uint8))
