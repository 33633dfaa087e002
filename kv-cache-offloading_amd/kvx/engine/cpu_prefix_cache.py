"""Bounded pinned-host KV block store with optional automatic preservation.

Drop-in for CPUBlockCache of nanovllm/engine/cpu_prefix_cache.py: the same
constructor, properties, errors, budget and slot bookkeeping, and the same
duck-typed hooks the BlockManager calls. Data movement and its ordering run
in libkvx (include/kvx.h): a native copy engine queues work on a save stream
and, with split_streams=True, a separate restore stream (torch streams, as in
the reference); it gathers (and FP8-quantises) a pool block into device
staging with one kernel and moves it to its pinned host slot with one DMA,
and the reverse on restore. Per-block and per-slot events order save ->
restore -> slot reuse against the caller's current stream without host
synchronisation.

Call from the engine-owning thread between steps (no locking), as the
reference requires. The KV pool must be on a ROCm device: there is no
torch-op path for CPU-resident pools.
"""

import ctypes
import warnings
from collections import Counter
from contextlib import contextmanager
from dataclasses import dataclass
from math import prod

import torch

from kvx import _lib, ops
from kvx._lib import check, int32_array, lib
from kvx.engine.block_manager import BlockManager

# Pinned memory is allocated in chunks of about this size so one page-locking
# call covers many entries (cpu_prefix_cache.py:11-13).
_SLAB_CHUNK_BYTES = 1 << 30

# Device staging per copy stream: entries of one save/restore batch (55
# Qwen3-8B FP8 entries with fp32 scales). A batch larger than the staging is processed in
# chunks, and on one stream each chunk's kernel waits for the previous
# chunk's transfer; a larger staging reads more of a batch's blocks at once.
_STAGING_BYTES = 1 << 30
_MAX_BATCH = 128  # kMaxBatch in the library

# The codec operators live in this module in the reference (cpu_prefix_cache.py:20-28).
fp8_quantize = ops.fp8_quantize
fp8_dequantize = ops.fp8_dequantize


@dataclass(frozen=True)
class _CPUBlock:
    token_ids: tuple[int, ...]
    kv: torch.Tensor  # [K/V, layer, token, KV head, head dim], a slab slot view
    slot: int
    scale: torch.Tensor | None = None  # FP8 only: [K/V, layer, token, KV head, 1]
    saved: bool = False  # a save into `slot` was queued (its event lives in the copy engine)


class CPUCacheFullError(MemoryError):
    """save_block found the byte budget spent: no further entry fits."""


# Copy streams must run side by side with each other and with the compute
# stream. The HIP runtime maps every stream of a process onto one of a few
# hardware queues (four by default), and two streams on one queue execute in
# queue order: with such a pair, saves and restores of 2.5 GB each ran one
# after the other (55 GB/s in total instead of 94 GB/s full duplex on MI355X),
# and torch's pool handed out such pairs for every other cache (queues are
# assigned round-robin at a stream's first use, so every fourth pool stream
# shares the default stream's). A candidate stream is therefore accepted only
# after a bounded delay kernel on it overlaps one on each stream already chosen.
_PROBE_US = 200
_STREAM_CANDIDATES = 8


def _run_side_by_side(a: torch.cuda.Stream, b: torch.cuda.Stream, device: torch.device) -> bool:
    # A stream's first launch also creates its queue (milliseconds): warm both first.
    for stream in (a, b):
        ops.sleep(1, stream=stream, device=device)
        stream.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    start.record(a)
    b.wait_event(start)
    ends = []
    for stream in (a, b):
        ops.sleep(_PROBE_US, stream=stream, device=device)
        end = torch.cuda.Event(enable_timing=True)
        end.record(stream)
        ends.append(end)
    for end in ends:
        end.synchronize()
    return max(start.elapsed_time(end) for end in ends) < 1.5 * _PROBE_US / 1000


def _copy_streams(device: torch.device, count: int) -> tuple[list[torch.cuda.Stream], bool]:
    """`count` pool streams that run concurrently with the current stream and each other, if found."""
    chosen = [torch.cuda.current_stream(device)]
    concurrent = True
    for _ in range(count):
        for _ in range(_STREAM_CANDIDATES):
            candidate = torch.cuda.Stream(device)
            ok = all(_run_side_by_side(other, candidate, device) for other in chosen)
            if ok:
                break
        concurrent = concurrent and ok
        chosen.append(candidate)  # the last candidate still works, only serialised
    return chosen[1:], concurrent


class _CopyEngine:
    """Owner of one kvx_cache handle (events, slab/staging registry).

    The engine queues work on two torch streams it borrows, at default
    priority like the reference's (cpu_prefix_cache.py:110-113); torch keeps
    them alive, so torch work queued on them (events, host-allocator
    bookkeeping) never outlives its stream. The streams are chosen to run
    concurrently with the caller's stream and each other (_copy_streams).
    """

    def __init__(self, pool: torch.Tensor, layout, fmt: int, split: bool):
        self.layout, self.fmt = layout, fmt
        self.logical_bytes, self.scale_offset, self.entry_stride = ops.entry_layout(layout, fmt)
        streams, self.streams_concurrent = _copy_streams(pool.device, 2 if split else 1)
        if not self.streams_concurrent:
            warnings.warn(f"no {'pair of copy streams' if split else 'copy stream'} found that runs beside the "
                          "compute stream" + (" and each other" if split else "") + f" after {_STREAM_CANDIDATES} "
                          "candidates: copies and compute will serialise (saves and restores at about half the "
                          "duplex host-link rate)", RuntimeWarning, stacklevel=3)
        self.save_stream = streams[0]
        self.restore_stream = streams[-1]
        handle = ctypes.c_void_p()
        check(lib().kvx_cache_create(pool.data_ptr(), ctypes.byref(layout), fmt, self.save_stream.cuda_stream,
                                     self.restore_stream.cuda_stream, pool.device.index, ctypes.byref(handle)),
              "kvx_cache_create")
        self.handle = handle

    def set_staging(self, save: torch.Tensor, restore: torch.Tensor, entries: int):
        check(lib().kvx_cache_set_staging(self.handle, save.data_ptr(), restore.data_ptr(), entries), "staging")

    def add_slab(self, slab: torch.Tensor, count: int):
        check(lib().kvx_cache_add_slab(self.handle, slab.data_ptr(), count), "kvx_cache_add_slab")

    def save(self, block_ids, slots, compute: int):
        check(lib().kvx_cache_save(self.handle, int32_array(block_ids), int32_array(slots), len(block_ids),
                                   compute), "kvx_cache_save")

    def restore(self, slots, block_ids, wait: bool, compute: int):
        check(lib().kvx_cache_restore(self.handle, int32_array(slots), int32_array(block_ids), len(slots),
                                      int(wait), compute), "kvx_cache_restore")

    def before_block_reuse(self, block_id: int, compute: int):
        check(lib().kvx_cache_before_block_reuse(self.handle, block_id, compute), "before_block_reuse")

    def before_block_use(self, block_id: int, compute: int):
        check(lib().kvx_cache_before_block_use(self.handle, block_id, compute), "before_block_use")

    def synchronize(self):
        check(lib().kvx_cache_synchronize(self.handle), "kvx_cache_synchronize")

    def counters(self) -> dict[str, int]:
        vals = [ctypes.c_int64() for _ in range(3)]
        check(lib().kvx_cache_counters(self.handle, *map(ctypes.byref, vals)), "kvx_cache_counters")
        return dict(zip(("saved_blocks", "restored_blocks", "stream_waits"), (v.value for v in vals)))

    def dma_counters(self) -> dict[str, int]:
        """DMA transfers queued so far (each at most 64 MiB) and their bytes, per direction."""
        vals = [ctypes.c_int64() for _ in range(4)]
        check(lib().kvx_cache_dma_counters(self.handle, *map(ctypes.byref, vals)), "kvx_cache_dma_counters")
        return dict(zip(("d2h_copies", "d2h_bytes", "h2d_copies", "h2d_bytes"), (v.value for v in vals)))

    def set_debug(self, flags: int):
        """Negative controls for tests: drop ordering rules (kvx._lib.DEBUG_*); results become wrong."""
        check(lib().kvx_cache_set_debug(self.handle, flags), "kvx_cache_set_debug")

    def close(self):
        if self.handle:
            handle, self.handle = self.handle, None
            check(lib().kvx_cache_destroy(handle), "kvx_cache_destroy")


class _CopyBatcher:
    """Hands a cache's saves and restores to its copy engine, in batches inside coalesce().

    One engine call per block costs a cross-stream wait per block: on MI355X,
    with 128 calls queued, one-block restores ran at ~47 GB/s against ~55 GB/s
    for a batch, and one-block saves beside restores at ~83-86 GB/s against
    ~94. Batched saves are staged, and slowed concurrent bf16 matmuls by ~10%
    where one-block saves (written by a kernel) slowed them by 40-60%. Inside
    coalesce() saves, restores and before_block_reuse waits are held back. On
    exit:
      1. the saves go first, in one call, blocks that this flush restores
         into ahead of the others: the copy engine releases a saved block
         once its save kernel has read it, so restores into the first
         chunks can start while the later chunks still cross the link;
      2. the restores, one call per run of equal wait flags;
      3. the caller's stream waits for the blocks passed to
         before_block_reuse, except blocks restored into here: a restore
         waits for its destination's save itself, and the caller waits for
         the restore (wait=True, or before_block_use) before touching the
         block. Queued after the restores, these waits do not hold the
         restores back (a restore waits for work on the caller's stream).
    Restores with wait=True and before_block_reuse therefore take effect at
    the end of the block, so no work that reads or writes those blocks may be
    queued on the caller's stream inside it. Anything that must follow a
    held-back copy flushes
    first: a save of a block a held-back restore writes, a save into a slot a
    held-back restore reads or a held-back save writes, a restore into a block
    a held-back restore writes, before_block_use or before_block_reuse of a
    block with a held-back restore.

    Callers publish a held-back copy's metadata when they queue it. If a flush
    fails (the engine validates its arguments before queuing anything, so only
    a HIP error can), `on_failure(saves, restores)` gets every copy of that
    flush, whether or not it was issued, so the caller can withdraw them.
    """

    def __init__(self, engine, compute_stream, on_failure=None):
        self.engine = engine
        self._compute = compute_stream  # () -> the caller's current stream handle
        self._on_failure = on_failure
        self.depth = 0
        self.saves: list[tuple[int, int]] = []  # (block, slot)
        self.save_slots: set[int] = set()
        self.reuse: list[int] = []  # blocks whose before_block_reuse waits come after the copies
        self.restores: list[tuple[int, int, bool]] = []  # (slot, block, wait)
        self.restore_blocks: set[int] = set()
        self.restore_slots: set[int] = set()

    def save(self, block_id: int, slot: int):
        if block_id in self.restore_blocks or slot in self.restore_slots or slot in self.save_slots:
            self.flush()
        if self.depth:
            self.saves.append((block_id, slot))
            self.save_slots.add(slot)
            return
        self.engine.save([block_id], [slot], self._compute())

    def restore(self, slot: int, block_id: int, wait: bool):
        if block_id in self.restore_blocks:
            self.flush()
        if self.depth:
            self.restores.append((slot, block_id, wait))
            self.restore_blocks.add(block_id)
            self.restore_slots.add(slot)
            return
        self.engine.restore([slot], [block_id], wait, self._compute())

    def before_block_reuse(self, block_id: int):
        if block_id in self.restore_blocks:
            self.flush()
        if self.saves:
            self.reuse.append(block_id)
            return
        self.engine.before_block_reuse(block_id, self._compute())

    def before_block_use(self, block_id: int):
        if block_id in self.restore_blocks:
            self.flush()
        self.engine.before_block_use(block_id, self._compute())

    @contextmanager
    def coalesce(self):
        self.depth += 1
        try:
            yield
        finally:
            self.depth -= 1
            if not self.depth:
                self.flush()

    def flush(self):
        saves, self.saves, self.save_slots = self.saves, [], set()
        reuse, self.reuse = self.reuse, []
        restores, self.restores = self.restores, []
        self.restore_blocks, self.restore_slots = set(), set()
        try:
            compute = self._compute()
            destinations = {block for _, block, _ in restores}
            if saves:
                saves.sort(key=lambda save: save[0] not in destinations)  # stable: restore targets first
                self.engine.save([block for block, _ in saves], [slot for _, slot in saves], compute)
            start = 0
            while start < len(restores):
                end, wait = start, restores[start][2]
                while end < len(restores) and restores[end][2] == wait:
                    end += 1
                run = restores[start:end]
                self.engine.restore([slot for slot, _, _ in run], [block for _, block, _ in run], wait, compute)
                start = end
            for block_id in reuse:
                if block_id not in destinations:
                    self.engine.before_block_reuse(block_id, compute)
        except BaseException:
            if self._on_failure is not None and (saves or restores):
                self._on_failure(saves, restores)
            raise


def _checked_costs(costs) -> tuple[float, float, float]:
    """Hybrid admission costs (restore s/block, recompute s/token, recompute s/token^2), each >= 0."""
    if len(costs) != 3 or min(costs) < 0:
        raise ValueError("hybrid needs three nonnegative cost coefficients")
    return tuple(float(c) for c in costs)


def _checked_pool(runner, manager: BlockManager, max_bytes, automatic: bool, save_on_release: bool,
                  prefetch: bool, hybrid, fp8: bool, scale_dtype) -> torch.Tensor:
    """The runner's KV pool, once the cache's arguments fit it and this library (cpu_prefix_cache.py:76-91).

    Raises, in this order: a bad budget, tensor parallelism, automatic-only
    options without automatic=True, bad hybrid costs, a pool that does not
    match the block manager, and what libkvx cannot copy (a pool off the
    GPU, non-contiguous, or FP8 from a non-bf16 pool or with an unsupported
    scale dtype).
    """
    if type(max_bytes) is not int or max_bytes <= 0:
        raise ValueError("max_bytes must be a positive integer")
    if runner.world_size != 1:
        raise NotImplementedError("CPU prefix blocks currently require TP=1")
    if (save_on_release or prefetch or hybrid) and not automatic:
        raise ValueError("save_on_release, prefetch and hybrid require automatic=True")
    if hybrid is not None:
        _checked_costs(hybrid)
    pool = runner.kv_cache
    geometry_ok = (pool.ndim == 6 and pool.shape[0] == 2 and min(pool.shape) > 0
                   and pool.shape[2] == len(manager.blocks)
                   and pool.shape[3] == manager.block_size == runner.block_size)
    if not geometry_ok:
        raise ValueError("KV pool layout does not match the block manager")
    if pool.device.type != "cuda":
        raise ValueError("KV pool must be on a ROCm device (libkvx copies blocks with HIP kernels)")
    if not pool.is_contiguous():
        raise ValueError("KV pool must be contiguous")
    if fp8 and (pool.dtype != torch.bfloat16 or scale_dtype not in ops.SCALE_DTYPES):
        raise NotImplementedError("FP8 payloads need a bfloat16 pool and a bfloat16/float32 scale")
    return pool


class _HostSlots:
    """A cache's pinned host entries, registered with its copy engine.

    Slots are allocated a chunk at a time, ~1 GiB per page-locking call
    (never beyond `capacity`), and one chunk holds its entries back to back,
    `entry_stride` apart: the payload, then the scales at `scale_offset`, so
    one DMA moves a block. Free slots form a stack: a fresh chunk hands out
    its lowest slot first and a returned slot is the next one taken
    (cpu_prefix_cache.py:199-208). Typed views with the reference's slab
    shapes ([count, 2, L, BS, H, hd] payloads, [..., 1] scales) are kept per
    chunk.
    """

    def __init__(self, engine: _CopyEngine, capacity: int, entry_bytes: int, kv_shape, kv_dtype,
                 scale_shape, scale_dtype):
        self.engine = engine
        self.capacity = capacity
        self.entry_bytes = entry_bytes  # the budget's unit: payload plus scales
        self.kv_shape, self.kv_dtype = kv_shape, kv_dtype
        self.scale_shape, self.scale_dtype = scale_shape, scale_dtype
        self.memory: list[torch.Tensor] = []
        self.kv_views: list[torch.Tensor] = []
        self.scale_views: list[torch.Tensor] = []
        self.free: list[int] = []
        self.count = 0

    def _add_chunk(self):
        n = min(max(1, _SLAB_CHUNK_BYTES // self.entry_bytes), self.capacity - self.count)
        stride = self.engine.entry_stride
        memory = torch.empty(n * stride, dtype=torch.uint8, device="cpu", pin_memory=True)
        entries = memory.view(n, stride)
        kv_bytes = prod(self.kv_shape) * self.kv_dtype.itemsize
        self.kv_views.append(entries[:, :kv_bytes].view(self.kv_dtype).view(n, *self.kv_shape))
        if self.scale_shape is not None:
            at = self.engine.scale_offset
            nbytes = prod(self.scale_shape) * self.scale_dtype.itemsize
            self.scale_views.append(entries[:, at:at + nbytes].view(self.scale_dtype).view(n, *self.scale_shape))
        self.engine.add_slab(memory, n)
        self.memory.append(memory)
        self.free.extend(reversed(range(self.count, self.count + n)))
        self.count += n

    def take(self) -> int:
        if not self.free:
            self._add_chunk()
        return self.free.pop()

    def give_back(self, slot: int):
        self.free.append(slot)

    def reserve_all(self):
        while self.count < self.capacity:
            self._add_chunk()

    def view(self, slot: int) -> tuple[torch.Tensor, torch.Tensor | None]:
        """(payload, scale or None) of one slot, as views of its pinned entry."""
        base = 0
        for i, kv in enumerate(self.kv_views):
            if slot < base + len(kv):
                scale = self.scale_views[i][slot - base] if self.scale_views else None
                return kv[slot - base], scale
            base += len(kv)
        raise IndexError(slot)

    def release(self):
        for items in (self.memory, self.kv_views, self.scale_views, self.free):
            items.clear()
        self.count = 0


class CPUBlockCache:
    """A bounded store of KV blocks in pinned host memory, keyed by the engine's chained prefix hashes.

    The drop-in for cpu_prefix_cache.py:44-448: the same constructor
    options, properties, hooks, budget and errors. The budget counts entry
    bytes (FP8 payload plus scales, or the bf16 block), not Python metadata.
    A restored block is an ordinary idle GPU hit that can be recycled; its
    CPU entry stays until discard, clear or close.

    Options (each as the reference's): automatic attaches the cache to the
    block manager, which then saves published blocks it recycles and
    restores CPU hits on admission; save_on_release also saves a published
    block when its last owner releases it while an admission is blocked;
    prefetch lets the scheduler restore a blocked request's CPU hits into
    spare blocks in the background; split_streams gives restores their own
    stream, so saves and restores share the host link in both directions;
    fp8 stores float8_e4m3fn payloads with one scale per (token, KV head)
    row in `scale_dtype` (default: the pool dtype, as the reference); hybrid
    = (restore s/block, recompute s/token, recompute s/token^2) lets an
    admission recompute the head of a CPU-only prefix while its tail
    restores; preallocate pins the whole budget up front.

    Copies run in libkvx (see _CopyEngine and _CopyBatcher); call
    synchronize() before reading payloads on the host.
    """

    def __init__(self, runner, block_manager: BlockManager, max_bytes: int, *,
                 automatic: bool = False, save_on_release: bool = False, preallocate: bool = False,
                 prefetch: bool = False, split_streams: bool = False, fp8: bool = False,
                 hybrid: tuple[float, float, float] | None = None, scale_dtype: torch.dtype | None = None):
        pool = runner.kv_cache
        scale_dtype = pool.dtype if scale_dtype is None else scale_dtype
        pool = _checked_pool(runner, block_manager, max_bytes, automatic, save_on_release, prefetch, hybrid, fp8,
                             scale_dtype)
        self._hybrid = None if hybrid is None else _checked_costs(hybrid)
        self._fp8, self._scale_dtype = fp8, scale_dtype
        self._save_on_release, self._prefetch = save_on_release, prefetch
        self._cache, self._manager = pool, block_manager
        self._device_index = pool.device.index
        self._shape = (2, pool.shape[1], *pool.shape[3:])  # one block: [K/V, layer, token, KV head, head dim]
        self._max_bytes = max_bytes
        self._layout = ops.pool_layout(pool, scale_dtype if fp8 else None)
        self._engine = _CopyEngine(pool, self._layout, ops.FORMAT_FP8 if fp8 else ops.FORMAT_RAW, split_streams)
        entry_bytes = self._engine.logical_bytes  # kvx_entry_layout: payload plus scales, as the reference counts
        self._slots = _HostSlots(self._engine, max_bytes // entry_bytes, entry_bytes, self._shape,
                                 torch.float8_e4m3fn if fp8 else pool.dtype,
                                 (*self._shape[:-1], 1) if fp8 else None, scale_dtype)
        self._entries: dict[int, _CPUBlock] = {}
        self._counts = Counter()
        self._prefetched_blocks = 0  # the block manager adds its prefetches here
        self._copy_stream = self._engine.save_stream
        self._restore_stream = self._engine.restore_stream
        self._staging: list[torch.Tensor] = []
        self._batcher = _CopyBatcher(self._engine, self._compute_stream, self._withdraw_copies)
        if automatic:
            if block_manager._cpu_prefix_cache is not None:
                self._engine.close()
                raise RuntimeError("block manager already has an automatic CPU cache")
            block_manager._cpu_prefix_cache = self
        if preallocate:
            self._slots.reserve_all()

    # -- the reference's public surface (cpu_prefix_cache.py:133-197) -----------

    @property
    def max_bytes(self) -> int:
        return self._max_bytes

    @property
    def block_bytes(self) -> int:
        return self._slots.entry_bytes

    @property
    def bytes_used(self) -> int:
        return len(self._entries) * self._slots.entry_bytes

    @property
    def reserved_bytes(self) -> int:
        return self._slots.count * self._slots.entry_bytes

    @property
    def closed(self) -> bool:
        return self._cache is None

    @property
    def automatic(self) -> bool:
        return self._manager is not None and self._manager._cpu_prefix_cache is self

    @property
    def prefetch_enabled(self) -> bool:
        return self._prefetch

    @property
    def hybrid(self) -> tuple[float, float, float] | None:
        return self._hybrid

    @hybrid.setter
    def hybrid(self, costs: tuple[float, float, float] | None):
        """Set or clear the split-admission costs, e.g. from measure_restore_s_per_block()."""
        if costs is not None:
            if not self.automatic:
                raise ValueError("hybrid requires an automatic cache")
            costs = _checked_costs(costs)
        self._hybrid = costs

    @property
    def fp8(self) -> bool:
        return self._fp8

    @property
    def prefetched_blocks(self) -> int:
        return self._prefetched_blocks

    @property
    def stats(self) -> dict[str, int]:
        return {name: self._counts[name] for name in ("saved_blocks", "restored_blocks", "budget_skips")}

    @property
    def streams_concurrent(self) -> bool:
        """False if the copy streams found run serialised with the compute stream or each other (a warning said so)."""
        return self._engine.streams_concurrent

    @property
    def copy_stats(self) -> dict:
        """The copy engine's own figures, beside the reference's `stats` (whose keys its tests compare whole):
        whether the copy streams run concurrently, cross-stream waits queued, and DMA copies and bytes per
        direction."""
        self._require_open()
        out = {"streams_concurrent": self._engine.streams_concurrent,
               "stream_waits": self._engine.counters()["stream_waits"]}
        out.update(self._engine.dma_counters())
        return out

    def __len__(self):
        return len(self._entries)

    def __contains__(self, prefix_hash: int):
        return prefix_hash in self._entries

    def _require_open(self):
        if self.closed:
            raise RuntimeError("CPU prefix cache is closed")

    # Views the reference's tests inspect: typed payload slabs, the pinned
    # allocations, the free-slot stack and one slot's (payload, scale).

    @property
    def _slabs(self) -> list[torch.Tensor]:
        return self._slots.kv_views

    @property
    def _scale_slabs(self) -> list[torch.Tensor]:
        return self._slots.scale_views

    @property
    def _slab_memory(self) -> list[torch.Tensor]:
        return self._slots.memory

    @property
    def _free_slots(self) -> list[int]:
        return self._slots.free

    def _slot_view(self, slot: int) -> tuple[torch.Tensor, torch.Tensor | None]:
        return self._slots.view(slot)

    # -- device staging and the copy seams ---------------------------------

    def _ensure_staging(self):
        if self._staging:
            return
        stride = self._engine.entry_stride
        entries = max(1, min(_MAX_BATCH, _STAGING_BYTES // stride))
        device = self._cache.device
        save = torch.empty(entries * stride, dtype=torch.uint8, device=device)
        restore = save
        if self._restore_stream is not self._copy_stream:
            restore = torch.empty(entries * stride, dtype=torch.uint8, device=device)
        self._engine.set_staging(save, restore, entries)
        self._staging = [save, restore]

    def _compute_stream(self) -> int:
        # The raw handle: building a torch Stream object on every copy call cost a few microseconds each.
        return torch._C._cuda_getCurrentRawStream(self._device_index)

    def _save_to_slot(self, block_id: int, slot: int):
        """Queue pool block -> host slot on the save stream (the seam failure-injection tests patch)."""
        self._ensure_staging()
        self._batcher.save(block_id, slot)

    def _restore_from_slot(self, slot: int, block_id: int, wait: bool):
        """Queue host slot -> pool block on the restore stream."""
        self._ensure_staging()
        self._batcher.restore(slot, block_id, wait)

    def coalesce(self):
        """Batch the saves and restores issued inside a `with` block (see _CopyBatcher); used by the block
        manager's admission, prefetch and release loops."""
        return self._batcher.coalesce()

    def _withdraw_copies(self, saves, restores):
        """A batch of held-back copies failed to issue: drop the CPU entries its saves published and unpublish
        the GPU blocks its restores filled, so no metadata names bytes that may never have been copied."""
        slots = {slot for _, slot in saves}
        for prefix_hash in [h for h, e in self._entries.items() if e.slot in slots]:
            self._slots.give_back(self._entries.pop(prefix_hash).slot)
            self._counts["saved_blocks"] -= 1
        manager = self._manager
        for _, block_id, _ in restores:
            block = manager.blocks[block_id]
            if block.hash != -1 and manager.hash_to_block_id.get(block.hash) == block_id:
                del manager.hash_to_block_id[block.hash]
            block.hash, block.token_ids = -1, []
            self._counts["restored_blocks"] -= 1

    def synchronize(self):
        """Wait for every pending host<->device copy (needed before host reads)."""
        if not self.closed:
            self._batcher.flush()
            self._engine.synchronize()

    def measure_restore_s_per_block(self, repeats: int = 8) -> float:
        """Time this cache's restore path (H2D DMA plus FP8 dequantisation) on scratch buffers.

        Restores `repeats` zero entries into a one-block scratch pool through a
        scratch copy engine of the same format: one warm-up pass (kernels and
        clocks, as cpu_prefix_cache.py:245-268), then three timed passes whose
        median is returned in seconds per block. One timed pass lasts only a
        few milliseconds, and single passes measured on MI355X hosts
        occasionally took 2-8x as long as their neighbours.
        """
        self._require_open()
        device = self._cache.device
        scratch = torch.empty((2, self._shape[1], 1, *self._shape[2:]), dtype=self._cache.dtype, device=device)
        layout = ops.pool_layout(scratch, self._scale_dtype if self._fp8 else None)
        engine = _CopyEngine(scratch, layout, ops.FORMAT_FP8 if self._fp8 else ops.FORMAT_RAW, False)
        try:
            host = torch.zeros(repeats * engine.entry_stride, dtype=torch.uint8, pin_memory=True)
            staging = torch.empty(engine.entry_stride, dtype=torch.uint8, device=device)
            engine.add_slab(host, repeats)
            engine.set_staging(staging, staging, 1)
            stream = engine.restore_stream
            compute = torch.cuda.current_stream(device)
            passes = []
            for _ in range(4):
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                start.record(stream)
                for i in range(repeats):
                    engine.restore([i], [0], False, compute.cuda_stream)
                end.record(stream)
                end.synchronize()
                passes.append(start.elapsed_time(end) / 1000 / repeats)
            return sorted(passes[1:])[1]
        finally:
            engine.close()

    # -- saving -------------------------------------------------------------

    def _published_source(self, prefix_hash: int) -> tuple[int, tuple[int, ...]] | None:
        """(block id, tokens) of the full GPU block published under `prefix_hash`; None if no GPU block has
        the hash. A block holding the hash but not published with all its tokens cannot be a source."""
        block_id = self._manager.hash_to_block_id.get(prefix_hash)
        if block_id is None:
            return None
        block = self._manager.blocks[block_id]
        tokens = tuple(block.token_ids)
        if block.hash != prefix_hash or len(tokens) != self._manager.block_size:
            raise ValueError("source must be a published full prefix block")
        return block_id, tokens

    def save_block(self, prefix_hash: int) -> bool:
        """Copy a published full GPU block into a host slot; False if it is saved already (:275-332).

        Errors, before anything changes: KeyError if the hash is neither on
        the GPU nor saved, ValueError for an unpublished or partial source or
        a saved entry with other tokens, CPUCacheFullError when the budget
        is spent. If queueing the copy fails, the slot goes back and no
        entry appears.
        """
        self._require_open()
        saved = self._entries.get(prefix_hash)
        source = self._published_source(prefix_hash)
        if source is None:
            if saved is None:
                raise KeyError(f"GPU prefix block {prefix_hash} is not cached")
            return False
        block_id, tokens = source
        if saved is not None:
            if saved.token_ids != tokens:
                raise ValueError("prefix hash has conflicting token metadata")
            return False
        if len(self._entries) >= self._slots.capacity:
            raise CPUCacheFullError("CPU prefix cache payload budget exceeded")
        slot = self._slots.take()
        try:
            self._save_to_slot(block_id, slot)
        except BaseException:
            self._slots.give_back(slot)
            raise
        kv, scale = self._slots.view(slot)
        self._entries[prefix_hash] = _CPUBlock(tokens, kv, slot, scale, True)
        self._counts["saved_blocks"] += 1
        return True

    def _preserve(self, prefix_hash: int):
        """A save the block manager asks for: a spent budget is counted and skipped (:334-340); any other
        failure propagates, so device errors stay visible."""
        try:
            self.save_block(prefix_hash)
        except CPUCacheFullError:
            self._counts["budget_skips"] += 1

    def _preserve_before_recycle(self, prefix_hash: int):
        self._preserve(prefix_hash)

    def _preserve_on_release(self, prefix_hash: int):
        # Saved on release only while an admission waits for blocks: otherwise
        # the block probably stays a GPU hit and the D2H copy buys nothing.
        if self._save_on_release and self._manager.admission_blocked:
            self._preserve(prefix_hash)

    # -- restoring and ordering ---------------------------------------------

    def before_block_reuse(self, block_id: int):
        """Order later writes to a GPU block after its pending save and restore, without a host sync."""
        self._batcher.before_block_reuse(block_id)

    def before_block_use(self, block_id: int):
        """Order later reads of a prefetched GPU block after its restore."""
        self._batcher.before_block_use(block_id)

    def _entry_for(self, prefix_hash: int, token_ids):
        """The entry saved under `prefix_hash` for exactly these tokens, else None (a lookup, no side effects)."""
        saved = self._entries.get(prefix_hash)
        if saved is None or saved.token_ids != tuple(token_ids):
            return None
        return saved

    def _copy_entry(self, entry: _CPUBlock, block_id: int, wait: bool = True):
        """Restore `entry` into GPU block `block_id` (:370-398).

        With wait=True the current stream waits for the copy; otherwise the
        block stays pending until before_block_use/before_block_reuse.
        """
        self._require_open()
        self._restore_from_slot(entry.slot, block_id, wait)
        self._counts["restored_blocks"] += 1

    def restore_block(self, prefix_hash: int) -> int:
        """Restore a CPU hit into the pool and return its GPU block id (:400-414).

        An existing GPU hit is returned without a copy. If the copy fails,
        the destination is freed and stays unpublished, and the CPU entry is
        kept for a retry.
        """
        self._require_open()
        entry = self._entries[prefix_hash]
        return self._manager.restore_cached_block(
            prefix_hash, entry.token_ids, lambda block_id: self._copy_entry(entry, block_id))

    # -- releasing ----------------------------------------------------------

    def discard(self, prefix_hash: int) -> bool:
        """Drop one CPU entry (GPU state is untouched); False if none was saved under the hash.

        A later save into the freed slot is ordered after restores still
        reading it by the copy engine's per-slot events.
        """
        self._require_open()
        entry = self._entries.pop(prefix_hash, None)
        if entry is not None:
            self._slots.give_back(entry.slot)
        return entry is not None

    def clear(self):
        """Drop every CPU entry; the slots stay pinned for later saves."""
        for entry in self._entries.values():
            self._slots.give_back(entry.slot)
        self._entries.clear()

    def close(self):
        """Finish pending copies, detach from the block manager and release every host and device buffer.

        Idempotent; any later call but close raises RuntimeError.
        """
        if self.closed:
            return
        if self.automatic:
            self._manager._cpu_prefix_cache = None
        self.synchronize()
        self._entries.clear()
        self._engine.close()
        self._staging.clear()
        self._slots.release()
        self._cache = self._manager = None

    def __del__(self):
        engine = getattr(self, "_engine", None)
        if engine is not None and engine.handle:
            try:
                engine.close()
            except Exception:
                pass
