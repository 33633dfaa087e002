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

# Device staging per copy stream: entries of one save/restore batch.
_STAGING_BYTES = 256 << 20
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
    """The configured payload budget cannot admit another block."""


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

    def set_debug(self, flags: int):
        """Negative controls for tests: drop ordering rules (kvx._lib.DEBUG_*); results become wrong."""
        check(lib().kvx_cache_set_debug(self.handle, flags), "kvx_cache_set_debug")

    def reset_slabs(self):
        check(lib().kvx_cache_reset_slabs(self.handle), "kvx_cache_reset_slabs")

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
    coalesce() saves, restores and before_block_reuse waits
    are held back; on exit the saves go first (one call), then the caller's
    stream waits for the blocks passed to before_block_reuse, then the
    restores (one call per run of equal wait flags). Restores with wait=True
    and before_block_reuse therefore take effect at the end of the block, so
    no work that reads or writes those blocks may be queued on the caller's
    stream inside it. Anything that must follow a held-back copy flushes
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
        self.reuse: list[int] = []  # blocks whose before_block_reuse waits come after the saves
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
            if saves:
                self.engine.save([block for block, _ in saves], [slot for _, slot in saves], compute)
            for block_id in reuse:
                self.engine.before_block_reuse(block_id, compute)
            start = 0
            while start < len(restores):
                end, wait = start, restores[start][2]
                while end < len(restores) and restores[end][2] == wait:
                    end += 1
                run = restores[start:end]
                self.engine.restore([slot for slot, _, _ in run], [block for _, block, _ in run], wait, compute)
                start = end
        except BaseException:
            if self._on_failure is not None and (saves or restores):
                self._on_failure(saves, restores)
            raise


class CPUBlockCache:
    """One engine's bounded payload store, with optional automatic integration.

    Keys are the engine's chained prefix hashes, not physical block IDs. The
    byte budget covers tensor payloads (plus FP8 scales), not Python
    metadata. Restored GPU entries are recyclable, not pinned; the CPU copy
    survives until discard/clear/close. Behaviour of every option follows
    cpu_prefix_cache.py:44-70: save_on_release saves a published block when
    its last owner releases it while admission is blocked; prefetch restores
    a blocked request's CPU hits into spare blocks in the background; fp8
    stores float8_e4m3fn payloads with one scale per (token, KV head) row in
    `scale_dtype` (default: the pool dtype, as the reference); hybrid =
    (restore_s_per_block, recompute_s_per_token, recompute_s_per_token2)
    lets admission recompute a CPU-only prefix's head while its tail restores.
    Call synchronize() before reading payloads on the host.
    """

    def __init__(self, runner, block_manager: BlockManager, max_bytes: int, *,
                 automatic: bool = False, save_on_release: bool = False, preallocate: bool = False,
                 prefetch: bool = False, split_streams: bool = False, fp8: bool = False,
                 hybrid: tuple[float, float, float] | None = None, scale_dtype: torch.dtype | None = None):
        if type(max_bytes) is not int or max_bytes <= 0:
            raise ValueError("max_bytes must be a positive integer")
        if runner.world_size != 1:
            raise NotImplementedError("CPU prefix blocks currently require TP=1")
        if (save_on_release or prefetch or hybrid) and not automatic:
            raise ValueError("save_on_release, prefetch and hybrid require automatic=True")
        if hybrid is not None and (len(hybrid) != 3 or min(hybrid) < 0):
            raise ValueError("hybrid needs three nonnegative cost coefficients")
        cache = runner.kv_cache
        if (cache.ndim != 6 or cache.shape[0] != 2 or min(cache.shape) <= 0
                or cache.shape[2] != len(block_manager.blocks)
                or cache.shape[3] != block_manager.block_size
                or runner.block_size != block_manager.block_size):
            raise ValueError("KV pool layout does not match the block manager")
        if cache.device.type != "cuda":
            raise ValueError("KV pool must be on a ROCm device (libkvx copies blocks with HIP kernels)")
        if not cache.is_contiguous():
            raise ValueError("KV pool must be contiguous")
        scale_dtype = cache.dtype if scale_dtype is None else scale_dtype
        if fp8 and (cache.dtype != torch.bfloat16 or scale_dtype not in ops.SCALE_DTYPES):
            raise NotImplementedError("FP8 payloads need a bfloat16 pool and a bfloat16/float32 scale")
        self._cache = cache
        self._manager = block_manager
        self._shape = (2, cache.shape[1], *cache.shape[3:])
        self._fp8 = fp8
        self._dtype = torch.float8_e4m3fn if fp8 else cache.dtype
        self._scale_dtype = scale_dtype
        self._scale_shape = (*self._shape[:-1], 1)
        self._block_bytes = prod(self._shape) * self._dtype.itemsize
        if fp8:
            self._block_bytes += prod(self._scale_shape) * scale_dtype.itemsize
        self._max_bytes = max_bytes
        self._entries: dict[int, _CPUBlock] = {}
        self._capacity = max_bytes // self._block_bytes
        self._slabs: list[torch.Tensor] = []  # payload views [count, 2, L, BS, H, hd]
        self._scale_slabs: list[torch.Tensor] = []  # FP8 scale views [count, 2, L, BS, H, 1]
        self._slab_memory: list[torch.Tensor] = []  # the pinned allocations
        self._free_slots: list[int] = []
        self._num_slots = 0
        self._hybrid = hybrid
        self._save_on_release = save_on_release
        self._prefetch = prefetch
        self._prefetched_blocks = 0
        self._saved_blocks = 0
        self._restored_blocks = 0
        self._budget_skips = 0
        self._layout = ops.pool_layout(cache, scale_dtype if fp8 else None)
        fmt = ops.FORMAT_FP8 if fp8 else ops.FORMAT_RAW
        self._engine = _CopyEngine(cache, self._layout, fmt, split_streams)
        assert self._engine.logical_bytes == self._block_bytes
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
            while self._num_slots < self._capacity:
                self._grow()

    # -- properties (cpu_prefix_cache.py:133-193) --------------------------

    @property
    def max_bytes(self) -> int:
        return self._max_bytes

    @property
    def block_bytes(self) -> int:
        return self._block_bytes

    @property
    def bytes_used(self) -> int:
        return len(self._entries) * self._block_bytes

    @property
    def reserved_bytes(self) -> int:
        return self._num_slots * self._block_bytes

    @property
    def closed(self) -> bool:
        return self._cache is None

    @property
    def automatic(self) -> bool:
        return not self.closed and self._manager._cpu_prefix_cache is self

    @property
    def prefetch_enabled(self) -> bool:
        return self._prefetch

    @property
    def hybrid(self) -> tuple[float, float, float] | None:
        return self._hybrid

    @hybrid.setter
    def hybrid(self, costs: tuple[float, float, float] | None):
        """Set split-admission costs, e.g. after measure_restore_s_per_block()."""
        if costs is not None:
            if not self.automatic:
                raise ValueError("hybrid requires an automatic cache")
            if len(costs) != 3 or min(costs) < 0:
                raise ValueError("hybrid needs three nonnegative cost coefficients")
            costs = tuple(float(c) for c in costs)
        self._hybrid = costs

    @property
    def fp8(self) -> bool:
        return self._fp8

    @property
    def prefetched_blocks(self) -> int:
        return self._prefetched_blocks

    @property
    def stats(self) -> dict[str, int]:
        return {"saved_blocks": self._saved_blocks, "restored_blocks": self._restored_blocks,
                "budget_skips": self._budget_skips}

    def __len__(self):
        return len(self._entries)

    def __contains__(self, prefix_hash: int):
        return prefix_hash in self._entries

    def _require_open(self):
        if self.closed:
            raise RuntimeError("CPU prefix cache is closed")

    # -- host slabs and device staging -------------------------------------

    def _grow(self):
        """Pin one more chunk of slots (cpu_prefix_cache.py:199-208); LIFO free list, lowest slot first."""
        count = min(max(1, _SLAB_CHUNK_BYTES // self._block_bytes), self._capacity - self._num_slots)
        stride = self._engine.entry_stride
        memory = torch.empty(count * stride, dtype=torch.uint8, device="cpu", pin_memory=True)
        rows = memory.view(count, stride)
        payload_bytes = prod(self._shape) * self._dtype.itemsize
        payload = rows[:, :payload_bytes].view(self._dtype).view(count, *self._shape)
        scale = None
        if self._fp8:
            offset = self._engine.scale_offset
            nbytes = prod(self._scale_shape) * self._scale_dtype.itemsize
            scale = rows[:, offset:offset + nbytes].view(self._scale_dtype).view(count, *self._scale_shape)
        self._engine.add_slab(memory, count)
        self._slab_memory.append(memory)
        self._slabs.append(payload)
        if scale is not None:
            self._scale_slabs.append(scale)
        self._free_slots.extend(range(self._num_slots + count - 1, self._num_slots - 1, -1))
        self._num_slots += count

    def _slot_view(self, slot: int) -> tuple[torch.Tensor, torch.Tensor | None]:
        for i, slab in enumerate(self._slabs):
            if slot < len(slab):
                return slab[slot], self._scale_slabs[i][slot] if self._fp8 else None
            slot -= len(slab)
        raise IndexError(slot)

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
        return torch.cuda.current_stream(self._cache.device).cuda_stream

    # -- copies -------------------------------------------------------------

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

    def synchronize(self):
        """Wait for every pending host<->device copy (needed before host reads)."""
        if not self.closed:
            self._batcher.flush()
            self._engine.synchronize()

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
            self._free_slots.append(self._entries.pop(prefix_hash).slot)
            self._saved_blocks -= 1
        manager = self._manager
        for _, block_id, _ in restores:
            block = manager.blocks[block_id]
            if block.hash != -1 and manager.hash_to_block_id.get(block.hash) == block_id:
                del manager.hash_to_block_id[block.hash]
            block.hash, block.token_ids = -1, []
            self._restored_blocks -= 1

    def save_block(self, prefix_hash: int) -> bool:
        """Save a published full block; return False if already saved (cpu_prefix_cache.py:275-332).

        A full budget raises CPUCacheFullError before any allocation. A copy
        or allocation failure leaves CPU entries and GPU metadata unchanged.
        Partial tails cannot be saved.
        """
        self._require_open()
        entry = self._entries.get(prefix_hash)
        block_id = self._manager.hash_to_block_id.get(prefix_hash)
        if block_id is None:
            if entry is not None:
                return False
            raise KeyError(f"GPU prefix block {prefix_hash} is not cached")
        block = self._manager.blocks[block_id]
        tokens = tuple(block.token_ids)
        if block.hash != prefix_hash or len(tokens) != self._manager.block_size:
            raise ValueError("source must be a published full prefix block")
        if entry is not None:
            if entry.token_ids != tokens:
                raise ValueError("prefix hash has conflicting token metadata")
            return False
        if self.bytes_used + self.block_bytes > self.max_bytes:
            raise CPUCacheFullError("CPU prefix cache payload budget exceeded")
        if not self._free_slots:
            self._grow()
        slot = self._free_slots.pop()
        try:
            payload, scale = self._slot_view(slot)
            self._save_to_slot(block_id, slot)
        except BaseException:
            self._free_slots.append(slot)
            raise
        self._entries[prefix_hash] = _CPUBlock(tokens, payload, slot, scale, True)
        self._saved_blocks += 1
        return True

    def _preserve(self, prefix_hash: int):
        # Only a budget miss is an expected fallback; device and allocation
        # failures stay visible (cpu_prefix_cache.py:334-340).
        try:
            self.save_block(prefix_hash)
        except CPUCacheFullError:
            self._budget_skips += 1

    def _preserve_before_recycle(self, prefix_hash: int):
        self._preserve(prefix_hash)

    def _preserve_on_release(self, prefix_hash: int):
        # Only when a request is waiting for blocks: otherwise the block likely
        # stays a GPU hit and the D2H traffic would only delay later copies.
        if self._save_on_release and self._manager.admission_blocked:
            self._preserve(prefix_hash)

    def before_block_reuse(self, block_id: int):
        """Order later writes to a GPU block after its pending save and restore, without a host sync."""
        self._batcher.before_block_reuse(block_id)

    def before_block_use(self, block_id: int):
        """Order later reads of a prefetched GPU block after its restore."""
        self._batcher.before_block_use(block_id)

    def _entry_for(self, prefix_hash: int, token_ids):
        """Pure lookup used while planning admission."""
        entry = self._entries.get(prefix_hash)
        return entry if entry is not None and entry.token_ids == tuple(token_ids) else None

    def _copy_entry(self, entry: _CPUBlock, block_id: int, wait: bool = True):
        """Restore `entry` into GPU block `block_id` (cpu_prefix_cache.py:370-398).

        With wait=True the current stream waits for the copy; otherwise the
        block stays pending until before_block_use/before_block_reuse.
        """
        self._require_open()
        self._restore_from_slot(entry.slot, block_id, wait)
        self._restored_blocks += 1

    def restore_block(self, prefix_hash: int) -> int:
        """Restore a CPU hit; return the GPU cache's physical block ID (cpu_prefix_cache.py:400-414).

        GPU hits are reused without copying. On copy failure the destination
        is freed and the hash stays unpublished; the CPU entry remains for a
        retry.
        """
        self._require_open()
        entry = self._entries[prefix_hash]

        def copy_to_block(block_id):
            self._copy_entry(entry, block_id)

        return self._manager.restore_cached_block(prefix_hash, entry.token_ids, copy_to_block)

    def discard(self, prefix_hash: int) -> bool:
        """Release one CPU payload without changing GPU cache state.

        A later save into the freed slot is ordered after restores still
        reading it by the copy engine's per-slot events.
        """
        self._require_open()
        entry = self._entries.pop(prefix_hash, None)
        if entry is None:
            return False
        self._free_slots.append(entry.slot)
        return True

    def clear(self):
        for entry in self._entries.values():
            self._free_slots.append(entry.slot)
        self._entries.clear()

    def close(self):
        """Release payloads, streams and pool references; idempotent."""
        if self.closed:
            return
        if self.automatic:
            self._manager._cpu_prefix_cache = None
        self.synchronize()
        self.clear()
        self._engine.close()
        self._staging.clear()
        self._slabs.clear()
        self._scale_slabs.clear()
        self._slab_memory.clear()
        self._free_slots.clear()
        self._num_slots = 0
        self._cache = None
        self._manager = None

    def __del__(self):
        engine = getattr(self, "_engine", None)
        if engine is not None and engine.handle:
            try:
                engine.close()
            except Exception:
                pass
