"""Operator API of the KV-block copy path, backed by libkvx's HIP kernels.

These functions keep the reference's names, argument meaning and out-param
style (nanovllm/layers/attention.py:33-40, nanovllm/engine/cpu_prefix_cache.py:20-28)
and accept the same tensors. Work is queued on torch's current HIP stream of
the tensors' device. Tensors must live on a ROCm device: there is no CPU or
torch-op fallback, so a missing or unloadable libkvx raises.
"""

import ctypes
import threading
from math import prod

import numpy as np
import torch

from kvx import _lib
from kvx._lib import BlockLayout, check, int32_array, lib, uint64_array

FORMAT_RAW, FORMAT_FP8 = _lib.FORMAT_RAW, _lib.FORMAT_FP8
SCALE_DTYPES = {torch.bfloat16: _lib.SCALE_BF16, torch.float32: _lib.SCALE_FP32}

# Largest finite float8_e4m3fn magnitude (the codec's clamp bound).
FP8_MAX = 448.0


def _require_device(*tensors: torch.Tensor) -> torch.device:
    device = tensors[0].device
    for t in tensors:
        if t.device.type != "cuda":
            raise ValueError("kvx operators need tensors on a ROCm device (got %s)" % t.device)
        if t.device != device:
            raise ValueError("kvx operators need all tensors on one device")
    return device


def _stream(device: torch.device, stream=None) -> int:
    if stream is None:
        stream = torch.cuda.current_stream(device)
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


# Cache pairs already validated (dtype, contiguity, equal sizes, device), keyed by address, size, row width and
# dtype: a model binds one pair per layer for the engine's lifetime (model_runner.py:120-126), so each call
# after the first only repeats the checks that can change from call to call.
_store_caches: dict[tuple, tuple[int, int]] = {}
_STORE_CACHE_LIMIT = 4096


def _validate_store_caches(k_cache: torch.Tensor, v_cache: torch.Tensor, dtype: torch.dtype, row: int):
    if not (k_cache.dtype == v_cache.dtype == dtype):
        raise TypeError("key, value and caches must share one dtype")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()) or k_cache.numel() != v_cache.numel():
        raise ValueError("k_cache and v_cache must be equally sized contiguous slot arrays")
    device = _require_device(k_cache, v_cache)
    if len(_store_caches) >= _STORE_CACHE_LIMIT:
        _store_caches.clear()
    return k_cache.numel() // row, device.index


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping: torch.Tensor):
    """Slot-mapped paged KV write (nanovllm/layers/attention.py:33-40).

    key/value: [N, num_heads, head_dim] with contiguous rows (the row stride
    may differ, e.g. V is a view of a fused QKV output). k_cache/v_cache:
    contiguous [num_blocks, block_size, num_heads, head_dim] layer views of
    the pool. slot_mapping: int32 [N]; -1 (graph padding) skips a token, and
    so does any slot outside the cache. Capturable in a HIP graph.

    Every call makes the reference's four asserts. A cache pair is checked
    in full the first time it is seen; later calls with the same pair only
    check that it is still contiguous, and the inputs' shapes, dtypes and
    device.
    """
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == D and v_cache.stride(1) == D
    assert slot_mapping.numel() == N
    dtype = key.dtype
    k_ptr, v_ptr = k_cache.data_ptr(), v_cache.data_ptr()
    pair = (k_ptr, v_ptr, k_cache.numel(), v_cache.numel(), D, dtype)
    known = _store_caches.get(pair)
    if known is None or not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        known = _store_caches[pair] = _validate_store_caches(k_cache, v_cache, dtype, D)
    cache_slots, index = known
    if value.shape != key.shape:
        raise ValueError("key and value shapes differ")
    if value.dtype != dtype:
        raise TypeError("key, value and caches must share one dtype")
    if slot_mapping.dtype != torch.int32 or not slot_mapping.is_contiguous():
        raise TypeError("slot_mapping must be a contiguous int32 tensor")
    if key.get_device() != index or value.get_device() != index or slot_mapping.get_device() != index:
        _require_device(k_cache, key, value, slot_mapping)
        raise ValueError("kvx operators need all tensors on one device")
    if N == 0:
        return
    check(lib().kvx_store_kvcache(key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0), k_ptr, v_ptr,
                                  slot_mapping.data_ptr(), N, num_heads, head_dim, key.element_size(), cache_slots,
                                  torch._C._cuda_getCurrentRawStream(index)), "store_kvcache")


# ---------------------------------------------------------------------------
# Views as [planes][plane_rows][head_dim]

def _plane_views(t: torch.Tensor):
    """Yields (tensor, planes, plane_rows, plane_stride) covering `t` in row-major order.

    The rows (last dim) must be contiguous. A view whose leading dims do not
    collapse into one uniformly strided plane dimension is split along its
    first dim.
    """
    if t.stride(-1) != 1 and t.shape[-1] > 1:
        raise ValueError("the last dim (head_dim) must be contiguous")
    hd = t.shape[-1]
    sizes, strides = list(t.shape[:-1]), list(t.stride()[:-1])
    dims = [(s, st) for s, st in zip(sizes, strides) if s != 1]
    # Longest suffix of dims whose rows are packed back to back.
    rows, expect, k = 1, hd, len(dims)
    while k > 0 and dims[k - 1][1] == expect:
        rows *= dims[k - 1][0]
        expect *= dims[k - 1][0]
        k -= 1
    lead = dims[:k]
    collapsible = all(lead[i][1] == lead[i + 1][1] * lead[i + 1][0] for i in range(len(lead) - 1))
    if collapsible:
        planes = prod(s for s, _ in lead) if lead else 1
        plane_stride = lead[-1][1] if lead else rows * hd
        yield t, planes, rows, plane_stride
        return
    for i in range(t.shape[0]):
        yield from _plane_views(t[i])


def _check_codec(values: torch.Tensor, payload: torch.Tensor, scale: torch.Tensor):
    if values.dtype != torch.bfloat16:
        raise NotImplementedError("the FP8 codec supports bfloat16 KV values")
    if payload.dtype != torch.float8_e4m3fn or payload.shape != values.shape or not payload.is_contiguous():
        raise ValueError("payload must be a contiguous float8_e4m3fn tensor shaped like the values")
    if scale.dtype not in SCALE_DTYPES or not scale.is_contiguous() or \
            tuple(scale.shape) != (*values.shape[:-1], 1):
        raise ValueError("scale must be a contiguous bfloat16/float32 tensor shaped [..., 1]")


def _codec(save: bool, values: torch.Tensor, payload: torch.Tensor, scale: torch.Tensor):
    _check_codec(values, payload, scale)
    device = _require_device(values, payload, scale)
    if values.numel() == 0:
        return
    hd = values.shape[-1]
    stream = _stream(device)
    scale_bytes = scale.element_size()
    row = 0
    fn = lib().kvx_save_blocks if save else lib().kvx_restore_blocks
    for view, planes, rows, plane_stride in _plane_views(values):
        layout = BlockLayout(plane_stride, 0, planes, rows, hd, 1, 2, SCALE_DTYPES[scale.dtype])
        entry = payload.data_ptr() + row * hd
        scale_offset = scale.data_ptr() + row * scale_bytes - entry
        check(fn(view.data_ptr(), ctypes.byref(layout), FORMAT_FP8, int32_array([0]), uint64_array([entry]), 1,
                 scale_offset, stream), "fp8_quantize" if save else "fp8_dequantize")
        row += planes * rows


def fp8_quantize(source: torch.Tensor, payload: torch.Tensor, scale: torch.Tensor):
    """float8_e4m3fn payload with one scale (scale's dtype) per vector along the last dim.

    Same contract as nanovllm/engine/cpu_prefix_cache.py:20-24:
    scale = max(fp32(amax|x|) / 448, 1e-30) in scale's dtype, then
    payload = e4m3(clamp(fp32(x) / fp32(scale), -448, 448)). `source` may be a
    strided view (e.g. pool[:, :, block]); payload and scale are contiguous.
    """
    _codec(True, source, payload, scale)


def fp8_dequantize(payload: torch.Tensor, scale: torch.Tensor, target: torch.Tensor):
    """target = bf16(fp32(payload) * fp32(scale)) (nanovllm/engine/cpu_prefix_cache.py:27-28)."""
    _codec(False, target, payload, scale)


# ---------------------------------------------------------------------------
# Pool block lists

def pool_layout(pool: torch.Tensor, scale_dtype: torch.dtype | None = None) -> BlockLayout:
    """kvx_block_layout of a contiguous [2, L, NB, BS, H, hd] pool (model_runner.py:120)."""
    if pool.ndim != 6 or pool.shape[0] != 2 or not pool.is_contiguous():
        raise ValueError("pool must be a contiguous [2, layers, blocks, block_size, heads, head_dim] tensor")
    _, layers, nb, bs, heads, hd = pool.shape
    if scale_dtype is not None and scale_dtype not in SCALE_DTYPES:
        raise ValueError(f"FP8 scales must be bfloat16 or float32, not {scale_dtype}")
    # Without an explicit scale dtype, scales follow the pool dtype (the reference's default); pools of other
    # dtypes only use RAW entries, which carry no scales.
    scale = SCALE_DTYPES.get(scale_dtype if scale_dtype is not None else pool.dtype, _lib.SCALE_BF16)
    return BlockLayout(nb * bs * heads * hd, bs * heads * hd, 2 * layers, bs * heads, hd, nb,
                       pool.element_size(), scale)


def entry_layout(layout: BlockLayout, fmt: int) -> tuple[int, int, int]:
    """(logical bytes, scale offset, entry stride) of one host entry."""
    logical, offset, stride = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    check(lib().kvx_entry_layout(ctypes.byref(layout), fmt, ctypes.byref(logical), ctypes.byref(offset),
                                 ctypes.byref(stride)), "entry_layout")
    return logical.value, offset.value, stride.value


def save_blocks(pool: torch.Tensor, block_ids, entries, fmt: int, scale_dtype: torch.dtype | None = None,
                stream=None):
    """Queues save (gather [+ FP8 quantise]) of pool blocks into entry addresses."""
    layout = pool_layout(pool, scale_dtype)
    _, offset, _ = entry_layout(layout, fmt)
    ids, entries = list(block_ids), list(entries)
    if len(ids) != len(entries):
        raise ValueError("one entry per block")
    device = _require_device(pool)
    check(lib().kvx_save_blocks(pool.data_ptr(), ctypes.byref(layout), fmt, int32_array(ids),
                                uint64_array(entries), len(ids), offset, _stream(device, stream)), "save_blocks")


def restore_blocks(pool: torch.Tensor, block_ids, entries, fmt: int, scale_dtype: torch.dtype | None = None,
                   stream=None):
    """Queues restore ([FP8 dequantise +] scatter) of entry addresses into pool blocks."""
    layout = pool_layout(pool, scale_dtype)
    _, offset, _ = entry_layout(layout, fmt)
    ids, entries = list(block_ids), list(entries)
    if len(ids) != len(entries):
        raise ValueError("one entry per block")
    device = _require_device(pool)
    check(lib().kvx_restore_blocks(pool.data_ptr(), ctypes.byref(layout), fmt, int32_array(ids),
                                   uint64_array(entries), len(ids), offset, _stream(device, stream)),
          "restore_blocks")


# ---------------------------------------------------------------------------
# Step inputs: host-to-device uploads read by a kernel

class _PinnedRing:
    """Pinned host buffers that kvx_upload kernels read, used in turn.

    A buffer is rewritten only after the kernel that last read it has run
    (an event per buffer; the host waits only if the stream is that far
    behind). A buffer grows, to a power of two, when an array does not fit.
    """

    def __init__(self, count: int = 16):
        self.buffers: list[torch.Tensor | None] = [None] * count
        self.events: list[torch.cuda.Event | None] = [None] * count
        self.next = 0

    def stage(self, host: np.ndarray) -> tuple[torch.Tensor, int]:
        """(a pinned uint8 buffer holding `host`'s bytes, its slot); pass the slot to read_by after the launch."""
        i = self.next
        self.next = (i + 1) % len(self.buffers)
        if self.events[i] is not None:
            self.events[i].synchronize()
        nbytes = host.nbytes
        buf = self.buffers[i]
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(256, 1 << (nbytes - 1).bit_length()), dtype=torch.uint8, pin_memory=True)
            self.buffers[i] = buf
        buf[:nbytes].numpy()[:] = host.reshape(-1).view(np.uint8)
        return buf, i

    def read_by(self, i: int, stream: torch.cuda.Stream):
        event = self.events[i] or torch.cuda.Event()
        event.record(stream)
        self.events[i] = event


_rings: dict[int, _PinnedRing] = {}
_rings_lock = threading.Lock()


def upload(values: np.ndarray, device: torch.device, stream=None, out: torch.Tensor | None = None) -> torch.Tensor:
    """A device copy of a host array, read from pinned memory by a kernel on the current stream (kvx_upload).

    Replaces the pinned non-blocking copies of a step's inputs
    (nanovllm/engine/model_runner.py:169-173, 187-190): a DMA copy on the
    compute stream queues behind every host-to-device DMA already queued on
    the device, a restore stream's included, while the kernel does not. The
    host does not wait for the GPU, except when 16 uploads are still queued.
    `out` (a contiguous device tensor of the array's dtype and size, e.g. a
    captured graph's static input) receives the copy instead of a new tensor.
    `stream` is a torch.cuda.Stream of the device (default: its current stream).
    Eager only: later uploads rewrite the ring's buffers, so a captured graph
    would replay whatever they hold by then. Inside a graph, call kvx_upload
    with a pinned source the caller owns and rewrites between replays.
    """
    host = np.ascontiguousarray(values)
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError(f"upload needs a ROCm device (got {device})")
    index = device.index if device.index is not None else torch.cuda.current_device()
    device = torch.device("cuda", index)
    dtype = torch.from_numpy(host[:0]).dtype
    if out is None:
        out = torch.empty(host.shape, dtype=dtype, device=device)
    elif out.device != device or out.dtype != dtype or out.numel() != host.size or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous {dtype} tensor of {host.size} elements on {device}")
    if host.nbytes == 0:
        return out
    if host.nbytes > _lib.UPLOAD_MAX_BYTES:
        raise ValueError(f"upload of {host.nbytes} bytes exceeds {_lib.UPLOAD_MAX_BYTES}")
    if stream is not None and not isinstance(stream, torch.cuda.Stream):
        raise TypeError("stream must be a torch.cuda.Stream")
    with _rings_lock:
        ring = _rings.get(index)
        if ring is None:
            ring = _rings[index] = _PinnedRing()
        buf, slot = ring.stage(host)
        s = torch.cuda.current_stream(device) if stream is None else stream
        check(lib().kvx_upload(out.data_ptr(), buf.data_ptr(), host.nbytes, _stream(device, s)), "upload")
        ring.read_by(slot, s)
    return out


# ---------------------------------------------------------------------------
# Test hooks

def sleep(microseconds: int, stream=None, device=None):
    """Queues a bounded busy wait on `stream` (torch's current stream by default)."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    check(lib().kvx_sleep(_stream(device, stream), int(microseconds)), "sleep")


SELFTEST_FIELDS = ("e4m3_encode_mismatch", "bf16_round_mismatch", "nan_not_preserved", "division_mismatch",
                   "e4m3_decode_mismatch", "encode_inputs_2p20", "division_pairs_2p20", "decode_sweeps")


def selftest(device=None) -> dict[str, int]:
    """Runs libkvx's exhaustive device self-test; returns its counters by name."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    counters = torch.zeros(8, dtype=torch.int64, device=device)
    check(lib().kvx_selftest(counters.data_ptr(), _stream(device)), "selftest")
    return dict(zip(SELFTEST_FIELDS, counters.cpu().tolist()))


# ---------------------------------------------------------------------------
# Token-granular copies (KV handoff)

def _plane_range(pool: torch.Tensor, layout: BlockLayout, planes) -> tuple[int, BlockLayout, tuple]:
    """(pool address, layout, leading dense dims) of the pool's (K/V, layer) planes [first, end).

    Plane p is K/V half p // L, layer p % L; None means all 2L planes, whose
    dense buffers keep the [2, L, ...] shape. A plane range is the same
    layout with fewer planes, starting at the first one's address.
    """
    if planes is None:
        return pool.data_ptr(), layout, (2, pool.shape[1])
    first, end = planes
    if not 0 <= first < end <= layout.planes:
        raise ValueError(f"plane range [{first}, {end}) is not within the pool's {layout.planes} planes")
    sub = BlockLayout(*(getattr(layout, name) for name, _ in BlockLayout._fields_))
    sub.planes = end - first
    return pool.data_ptr() + first * layout.plane_stride * layout.elem_bytes, sub, (end - first,)


def _token_copy(gather: bool, pool: torch.Tensor, block_table, num_tokens: int, dense: torch.Tensor, stream=None,
                planes=None):
    if pool.ndim != 6:
        raise ValueError("pool must be [2, layers, blocks, block_size, heads, head_dim]")
    address, layout, lead = _plane_range(pool, pool_layout(pool), planes)
    expected = (*lead, num_tokens, *pool.shape[-2:])
    if tuple(dense.shape) != expected or dense.dtype != pool.dtype or not dense.is_contiguous():
        raise ValueError(f"dense buffer must be a contiguous {pool.dtype} tensor of shape {expected}")
    if dense.device.type == "cuda":
        _require_device(pool, dense)
    elif not dense.is_pinned():
        raise ValueError("a host buffer must be pinned (device-accessible)")
    device = _require_device(pool)
    table = list(block_table)
    fn = lib().kvx_gather_tokens if gather else lib().kvx_scatter_tokens
    check(fn(address, ctypes.byref(layout), int32_array(table), len(table), num_tokens * pool.shape[4],
             dense.data_ptr(), _stream(device, stream)),
          "gather_tokens" if gather else "scatter_tokens")


def gather_tokens(pool: torch.Tensor, block_table, num_tokens: int, out: torch.Tensor, stream=None, planes=None):
    """out[:, :, t] = pool[:, :, block_table[t // BS], t % BS] for t < num_tokens.

    `out` is [2, L, num_tokens, H, hd] (kv_handoff.py:46-55's packed payload),
    on the pool's device or in pinned host memory. With planes=(first, end),
    only those (K/V, layer) planes (plane p = K/V p // L, layer p % L) are
    copied, into an `out` of shape [end - first, num_tokens, H, hd].
    """
    _token_copy(True, pool, block_table, num_tokens, out, stream, planes)


def scatter_tokens(pool: torch.Tensor, block_table, num_tokens: int, src: torch.Tensor, stream=None, planes=None):
    """pool[:, :, block_table[t // BS], t % BS] = src[:, :, t] for t < num_tokens (kv_handoff.py:112-118).

    planes=(first, end) as for gather_tokens."""
    _token_copy(False, pool, block_table, num_tokens, src, stream, planes)


def _token_fp8(gather: bool, pool: torch.Tensor, block_table, num_tokens: int, payload: torch.Tensor,
               scale: torch.Tensor, stream=None, planes=None):
    if pool.ndim != 6 or pool.dtype != torch.bfloat16:
        raise ValueError("pool must be a bfloat16 [2, layers, blocks, block_size, heads, head_dim] tensor")
    if scale.dtype not in SCALE_DTYPES:
        raise ValueError("scale must be a bfloat16 or float32 tensor")
    address, layout, lead = _plane_range(pool, pool_layout(pool, scale.dtype), planes)
    shape = (*lead, num_tokens, *pool.shape[-2:])
    if tuple(payload.shape) != shape or payload.dtype != torch.float8_e4m3fn or not payload.is_contiguous():
        raise ValueError(f"payload must be a contiguous float8_e4m3fn tensor of shape {shape}")
    if (tuple(scale.shape) != (*shape[:-1], 1) or scale.dtype not in SCALE_DTYPES
            or not scale.is_contiguous()):
        raise ValueError(f"scale must be a contiguous bfloat16/float32 tensor of shape {(*shape[:-1], 1)}")
    for t in (payload, scale):
        if t.device.type == "cuda":
            _require_device(pool, t)
        elif not (gather and t.is_pinned()):
            raise ValueError("an FP8 gather may write pinned host memory; a scatter reads device memory")
    device = _require_device(pool)
    table = list(block_table)
    fn = lib().kvx_gather_tokens_fp8 if gather else lib().kvx_scatter_tokens_fp8
    check(fn(address, ctypes.byref(layout), int32_array(table), len(table), num_tokens * pool.shape[4],
             payload.data_ptr(), scale.data_ptr(), _stream(device, stream)),
          "gather_tokens_fp8" if gather else "scatter_tokens_fp8")


def gather_tokens_fp8(pool: torch.Tensor, block_table, num_tokens: int, payload: torch.Tensor, scale: torch.Tensor,
                      stream=None, planes=None):
    """fp8_quantize of gather_tokens' [2, L, num_tokens, H, hd] payload, without the BF16 intermediate.

    payload: float8_e4m3fn [2, L, num_tokens, H, hd]; scale: [2, L, num_tokens, H, 1] in bfloat16 or float32,
    both on the pool's device or in pinned host memory. planes=(first, end) as for gather_tokens: payload
    [end - first, num_tokens, H, hd] and scale [end - first, num_tokens, H, 1].
    """
    _token_fp8(True, pool, block_table, num_tokens, payload, scale, stream, planes)


def scatter_tokens_fp8(pool: torch.Tensor, block_table, num_tokens: int, payload: torch.Tensor, scale: torch.Tensor,
                       stream=None, planes=None):
    """pool[:, :, block_table[t // BS], t % BS] = fp8_dequantize(payload, scale)[:, :, t] (device tensors).

    planes=(first, end) as for gather_tokens_fp8."""
    _token_fp8(False, pool, block_table, num_tokens, payload, scale, stream, planes)
