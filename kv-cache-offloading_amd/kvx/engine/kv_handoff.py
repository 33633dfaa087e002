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

Both directions move the payload a group of (K/V, layer) planes at a time
through two device staging buffers of at most 256 MiB each. A plane group is one contiguous
range of the payload, so each group is one DMA per tensor.
- Export gathers a group's tokens into staging (quantising for FP8), then
  copies it to the pinned payload. D2H DMA ran at ~57 GB/s on MI355X's PCIe
  Gen5 x16 link; a gather kernel writing the pinned payload itself reached
  54.5 GB/s for BF16 and 51.9 for FP8.
- Import copies a group into staging, then scatters it (dequantising for
  FP8) into freshly allocated blocks. No device buffer the size of the
  payload is needed.
Two staging buffers alternate, so one group's kernel overlaps the DMA of
the previous one.
Both return once the copies have finished, so the caller may free or reuse
the snapshot (or read the exported one) at once.
"""

from dataclasses import dataclass

import torch

from kvx import ops
from kvx.engine.sequence import SamplingParams, Sequence, SequenceStatus


_STAGING_BYTES = 256 << 20


def _plane_groups(pool: torch.Tensor, count: int, kv_dtype: torch.dtype, scale_dtype: torch.dtype | None):
    """(first, end) plane ranges whose tokens' payload (and scales) fit the staging, at least one plane each."""
    heads, hd = pool.shape[-2:]
    row = hd * torch.empty(0, dtype=kv_dtype).element_size()
    if scale_dtype is not None:
        row += torch.empty(0, dtype=scale_dtype).element_size()
    planes = 2 * pool.shape[1]
    group = max(1, min(planes, _STAGING_BYTES // max(1, count * heads * row)))
    return [(first, min(planes, first + group)) for first in range(0, planes, group)]


def copy_tokens(to_host: bool, pool: torch.Tensor, table, count: int, kv: torch.Tensor, scale=None):
    """Copies the first `count` tokens of the blocks `table` to (to_host) or from a host payload, a plane group at a time.

    `kv` is [2, L, count, H, hd] in the pool dtype, or float8_e4m3fn with
    `scale` [2, L, count, H, 1] (bfloat16 or float32); export writes pinned
    memory. Two staging buffers alternate: the gather or scatter kernels run
    on the current stream and the DMAs on a side stream, so one group's kernel
    overlaps the previous group's copy. Returns once the copies have finished.
    """
    heads, hd = pool.shape[-2:]
    groups = _plane_groups(pool, count, kv.dtype, scale.dtype if scale is not None else None)
    group = groups[0][1] - groups[0][0]
    device = pool.device
    kernels = torch.cuda.current_stream(device)
    dma = torch.cuda.Stream(device)
    stages = [torch.empty((group, count, heads, hd), dtype=kv.dtype, device=device) for _ in range(2)]
    host = kv.view(-1, count, heads, hd)
    if scale is not None:
        scale_stages = [torch.empty((group, count, heads, 1), dtype=scale.dtype, device=device) for _ in range(2)]
        host_scale = scale.view(-1, count, heads, 1)
    released = [None, None]  # per buffer: the event after the last work that read or wrote it
    dma.wait_stream(kernels)  # the pool's tokens, and the payload, are ready for the caller's queued work
    try:
        for i, (first, end) in enumerate(groups):
            n, k = end - first, i % 2
            stage = stages[k][:n]
            stage_scale = scale_stages[k][:n] if scale is not None else None
            if to_host:
                if released[k] is not None:
                    kernels.wait_event(released[k])  # its previous copy to the host has read it
                if scale is None:
                    ops.gather_tokens(pool, table, count, stage, planes=(first, end))
                else:
                    ops.gather_tokens_fp8(pool, table, count, stage, stage_scale, planes=(first, end))
                dma.wait_event(kernels.record_event())
                with torch.cuda.stream(dma):
                    host[first:end].copy_(stage, non_blocking=True)
                    if scale is not None:
                        host_scale[first:end].copy_(stage_scale, non_blocking=True)
                released[k] = dma.record_event()
            else:
                if released[k] is not None:
                    dma.wait_event(released[k])  # its previous scatter has read it
                with torch.cuda.stream(dma):
                    stage.copy_(host[first:end], non_blocking=True)
                    if scale is not None:
                        stage_scale.copy_(host_scale[first:end], non_blocking=True)
                kernels.wait_event(dma.record_event())
                if scale is None:
                    ops.scatter_tokens(pool, table, count, stage, planes=(first, end))
                else:
                    ops.scatter_tokens_fp8(pool, table, count, stage, stage_scale, planes=(first, end))
                released[k] = kernels.record_event()
    finally:
        # The staging is freed on return; later allocations on this stream must follow every DMA, also when
        # a call above raised.
        kernels.wait_stream(dma)
    kernels.synchronize()


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
    else:
        kv = torch.empty(shape, dtype=pool.dtype, pin_memory=True)
    copy_tokens(True, pool, table, count, kv, scale)
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

    The blocks' prefix hashes are published once the copies have finished;
    if anything fails after allocation the blocks are released. The snapshot
    is no longer read when this returns.
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
        scale = snapshot.scale.contiguous() if snapshot.fp8 else None
        copy_tokens(False, pool, seq.block_table, count, snapshot.kv.contiguous(), scale)
        seq.num_cached_tokens, seq.num_scheduled_tokens = 0, count
        block_manager.hash_blocks(seq)
        seq.num_cached_tokens, seq.num_scheduled_tokens = count, 0
        seq.status = SequenceStatus.RUNNING
        seq.is_prefill = False
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
