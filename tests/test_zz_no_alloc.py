"""kvx_cache_save_noalloc through the C ABI: the same host-slot bytes as kvx_cache_save.

Two copy engines share one pool: one stages through attached device buffers
(kvx_cache_save), the other through the library's static array
(kvx_cache_save_noalloc). Both save the same blocks into their own poisoned
pinned slabs, in two calls in a row, the second with fewer blocks and a
refilled pool; every payload and scale byte must agree. A call beyond the
static array's capacity must fail before queuing anything. Allocation-free
saves of two caches with different save streams, alternating, each hold
their own blocks' bytes (the array is ordered per device), and a plain C
program that interposes the HIP runtime's allocation and creation calls sees
none of them during such saves.
"""

import ctypes
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from kvx import _lib, ops
from kvx._lib import check, int32_array, lib

pytestmark = pytest.mark.gpu

POISON = 0xAB


class Engine:
    """One kvx_cache over `pool` with its own streams, a poisoned pinned slab and, if `staged`, staging."""

    def __init__(self, pool, layout, fmt, slots, staged):
        device = pool.device
        self.streams = (torch.cuda.Stream(device), torch.cuda.Stream(device))
        self.handle = ctypes.c_void_p()
        check(lib().kvx_cache_create(pool.data_ptr(), ctypes.byref(layout), fmt, self.streams[0].cuda_stream,
                                     self.streams[1].cuda_stream, device.index, ctypes.byref(self.handle)),
              "kvx_cache_create")
        self.logical, self.offset, self.stride = ops.entry_layout(layout, fmt)
        self.slab = torch.full((slots * self.stride,), POISON, dtype=torch.uint8, pin_memory=True)
        check(lib().kvx_cache_add_slab(self.handle, self.slab.data_ptr(), slots), "kvx_cache_add_slab")
        self.staging = []
        if staged:
            self.staging = [torch.empty(4 * self.stride, dtype=torch.uint8, device=device) for _ in range(2)]
            check(lib().kvx_cache_set_staging(self.handle, self.staging[0].data_ptr(), self.staging[1].data_ptr(),
                                              4), "kvx_cache_set_staging")

    def entry(self, slot):
        return self.slab.numpy()[slot * self.stride:(slot + 1) * self.stride]

    def close(self):
        check(lib().kvx_cache_destroy(self.handle), "kvx_cache_destroy")


def fill(pool, seed):
    g = torch.Generator(device=pool.device).manual_seed(seed)
    t = torch.randn(pool.shape, generator=g, device=pool.device)
    t = t / torch.randn(pool.shape, generator=g, device=pool.device).abs().add_(0.25)  # heavy tails
    pool.copy_(t.to(pool.dtype))
    torch.cuda.synchronize(pool.device)


def data_ranges(layout, fmt, engine):
    """Byte ranges of an entry that carry data (payload, then scales for FP8)."""
    rows = layout.planes * layout.plane_rows
    if fmt == ops.FORMAT_RAW:
        return [(0, engine.logical)]
    scale_bytes = 2 if layout.scale_dtype == _lib.SCALE_BF16 else 4
    return [(0, rows * layout.head_dim), (engine.offset, engine.offset + rows * scale_bytes)]


CASES = [
    # (pool shape [2, L, NB, BS, H, hd], format, scale dtype, (block ids, slots) of the two calls)
    ((2, 2, 8, 256, 2, 128), ops.FORMAT_FP8, torch.float32, [([5, 1, 3], [0, 1, 2]), ([6], [3])]),
    ((2, 2, 8, 256, 2, 128), ops.FORMAT_FP8, torch.bfloat16, [([0, 7], [2, 0]), ([4], [1])]),
    ((2, 2, 8, 256, 2, 128), ops.FORMAT_RAW, None, [([2, 6, 1, 0], [3, 2, 1, 0]), ([5, 3], [4, 1])]),
    ((2, 2, 4, 256, 1, 4), ops.FORMAT_FP8, torch.float32, [([3, 0, 2], [0, 1, 2]), ([1], [0])]),
    ((2, 36, 8, 256, 8, 128), ops.FORMAT_FP8, torch.float32, [([7, 2, 4], [0, 1, 2]), ([1], [3])]),
]


@pytest.mark.parametrize("shape,fmt,scale_dtype,calls", CASES,
                         ids=["fp8-fp32", "fp8-bf16", "bf16", "fp8-hd4", "fp8-qwen3-8b"])
def test_noalloc_save_writes_the_bytes_of_the_staged_save(gpu, shape, fmt, scale_dtype, calls):
    pool = torch.empty(shape, dtype=torch.bfloat16, device=gpu)
    layout = ops.pool_layout(pool, scale_dtype)
    slots = 5
    staged = Engine(pool, layout, fmt, slots, staged=True)
    static = Engine(pool, layout, fmt, slots, staged=False)
    try:
        for seed, (ids, dest) in enumerate(calls):
            print(f"noalloc case {shape} fmt {fmt} scale {scale_dtype} call {seed}: blocks {ids} -> slots {dest}",
                  flush=True)
            fill(pool, seed)  # idle caller stream: both calls take the staged path
            compute = torch.cuda.current_stream(gpu).cuda_stream
            check(lib().kvx_cache_save(staged.handle, int32_array(ids), int32_array(dest), len(ids), compute),
                  "kvx_cache_save")
            check(lib().kvx_cache_save_noalloc(static.handle, int32_array(ids), int32_array(dest), len(ids),
                                               compute), "kvx_cache_save_noalloc")
            for engine in (staged, static):
                check(lib().kvx_cache_synchronize(engine.handle), "kvx_cache_synchronize")
            for slot in dest:
                for start, end in data_ranges(layout, fmt, staged):
                    want, got = staged.entry(slot)[start:end], static.entry(slot)[start:end]
                    assert not np.all(want == POISON), f"slot {slot} was not written"
                    assert np.array_equal(got, want), f"slot {slot} bytes [{start}, {end}) differ"
        # The slots no call named stay poisoned in both slabs.
        for slot in set(range(slots)) - {s for _, dest in calls for s in dest}:
            assert np.all(static.entry(slot) == POISON) and np.all(staged.entry(slot) == POISON)
    finally:
        staged.close()
        static.close()


def test_noalloc_save_rejects_more_blocks_than_its_static_staging_holds(gpu):
    pool = torch.zeros((2, 36, 8, 256, 8, 128), dtype=torch.bfloat16, device=gpu)
    layout = ops.pool_layout(pool, torch.float32)
    engine = Engine(pool, layout, ops.FORMAT_FP8, 4, staged=False)
    try:
        capacity = _lib.NOALLOC_SCRATCH_BYTES // engine.stride
        assert capacity == 3  # Qwen3-8B FP8 entries with fp32 scales
        compute = torch.cuda.current_stream(gpu).cuda_stream
        with pytest.raises(IndexError, match="exceed the static staging"):
            check(lib().kvx_cache_save_noalloc(engine.handle, int32_array([0, 1, 2, 3]), int32_array([0, 1, 2, 3]),
                                               4, compute), "kvx_cache_save_noalloc")
        check(lib().kvx_cache_synchronize(engine.handle), "kvx_cache_synchronize")
        assert np.all(engine.slab.numpy() == POISON)  # nothing was queued
        counters = [ctypes.c_int64() for _ in range(3)]
        check(lib().kvx_cache_counters(engine.handle, *map(ctypes.byref, counters)), "kvx_cache_counters")
        assert counters[0].value == 0
    finally:
        engine.close()


def test_noalloc_saves_of_two_caches_interleaved_hold_their_own_bytes(gpu):
    """Each static engine's save stream differs: without the per-device order, one engine's kernel would
    overwrite the array while the other's copies out of it are still queued."""
    pool = torch.empty((2, 36, 8, 256, 8, 128), dtype=torch.bfloat16, device=gpu)
    fill(pool, 11)
    layout = ops.pool_layout(pool, torch.float32)
    slots = 6
    staged = Engine(pool, layout, ops.FORMAT_FP8, slots, staged=True)
    statics = [Engine(pool, layout, ops.FORMAT_FP8, slots, staged=False) for _ in range(2)]
    try:
        compute = torch.cuda.current_stream(gpu).cuda_stream
        calls = [([0, 1, 2], [0, 1, 2]), ([3, 4, 5], [0, 1, 2]), ([6, 7, 0], [3, 4, 5]), ([1, 3, 5], [3, 4, 5])]
        for i, (ids, dest) in enumerate(calls):
            engine = statics[i % 2]
            print(f"interleaved noalloc call {i} on engine {i % 2}: blocks {ids} -> slots {dest}", flush=True)
            check(lib().kvx_cache_save_noalloc(engine.handle, int32_array(ids), int32_array(dest), len(ids),
                                               compute), "kvx_cache_save_noalloc")
        # The reference bytes: every block once, through attached staging.
        want = {}
        for base in range(0, 8, 4):
            ids = list(range(base, base + 4))
            check(lib().kvx_cache_save(staged.handle, int32_array(ids), int32_array(range(4)), 4, compute),
                  "kvx_cache_save")
            check(lib().kvx_cache_synchronize(staged.handle), "kvx_cache_synchronize")
            want.update({b: staged.entry(b - base).copy() for b in ids})
        for engine in statics:
            check(lib().kvx_cache_synchronize(engine.handle), "kvx_cache_synchronize")
        final = [{}, {}]
        for i, (ids, dest) in enumerate(calls):
            final[i % 2].update(zip(dest, ids))
        for e, engine in enumerate(statics):
            for slot, block in final[e].items():
                for start, end in data_ranges(layout, ops.FORMAT_FP8, engine):
                    assert np.array_equal(engine.entry(slot)[start:end], want[block][start:end]), \
                        f"engine {e} slot {slot} (block {block}) bytes [{start}, {end}) differ"
    finally:
        staged.close()
        for engine in statics:
            engine.close()


NOALLOC_CALLS = Path(__file__).resolve().parent / "c_abi" / "noalloc_calls"


def test_noalloc_saves_make_no_allocation_or_creation_call(gpu):
    assert NOALLOC_CALLS.exists(), "build() compiles tests/c_abi/noalloc_calls.c"
    print("noalloc_calls 5 400", flush=True)
    proc = subprocess.run([str(NOALLOC_CALLS), "5", "400"], capture_output=True, text=True, timeout=120)
    print(proc.stdout, proc.stderr, flush=True)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "0 allocation or creation calls" in proc.stdout and "0 mismatches" in proc.stdout
