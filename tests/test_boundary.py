"""The C ABI boundary on the CPU: the library loads, exports what include/kvx.h
declares, and rejects bad arguments before touching a device."""

import ctypes
import re
import subprocess
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

from kvx import _lib, ops
from kvx.engine.block_manager import BlockManager
from kvx.engine.cpu_prefix_cache import CPUBlockCache

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "kvx.h"


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"\b(kvx_[a-z0-9_]+)\s*\(", text)) - {"kvx_block_layout"}


def test_header_declarations_are_bound_and_exported():
    declared = declared_functions()
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)
    exported = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                              check=True).stdout
    names = {line.split()[-1] for line in exported.splitlines() if " T " in line}
    assert declared <= names, declared - names
    handle = _lib.lib()
    assert handle.kvx_abi_version() == _lib.ABI_VERSION
    assert all(hasattr(handle, name) for name in declared)


def test_block_layout_struct_matches_header():
    text = HEADER.read_text()
    body = text[text.index("typedef struct kvx_block_layout {"):text.index("} kvx_block_layout;")]
    fields = re.findall(r"int(\d+)_t\s+(\w+);", body)
    assert [(name, int(bits)) for bits, name in fields] == [
        (name, ctypes.sizeof(ctype) * 8) for name, ctype in _lib.BlockLayout._fields_]


QWEN3_8B_POOL = (2, 36, 320, 256, 8, 128)


def layout_for(shape, scale_dtype):
    _, layers, nb, bs, heads, hd = shape
    return _lib.BlockLayout(nb * bs * heads * hd, bs * heads * hd, 2 * layers, bs * heads, hd, nb, 2,
                            ops.SCALE_DTYPES[scale_dtype])


@pytest.mark.parametrize("fmt,scale_dtype,logical", [
    (ops.FORMAT_FP8, torch.float32, 19_464_192),   # 18,874,368 payload + 589,824 fp32 scales
    (ops.FORMAT_FP8, torch.bfloat16, 19_169_280),  # reference default: scales in the pool dtype
    (ops.FORMAT_RAW, torch.bfloat16, 37_748_736),  # BF16 block
])
def test_entry_sizes_match_the_reference_budget(fmt, scale_dtype, logical):
    got, offset, stride = ops.entry_layout(layout_for(QWEN3_8B_POOL, scale_dtype), fmt)
    assert got == logical
    assert stride % 256 == 0 and stride >= logical
    assert offset == (18_874_368 if fmt == ops.FORMAT_FP8 else 0)


def test_invalid_arguments_are_rejected_before_any_device_work():
    handle = _lib.lib()
    layout = layout_for(QWEN3_8B_POOL, torch.float32)
    ids = _lib.int32_array([320])
    entries = _lib.uint64_array([4096])
    with pytest.raises(IndexError, match="block id 320"):
        _lib.check(handle.kvx_save_blocks(4096, ctypes.byref(layout), ops.FORMAT_FP8, ids, entries, 1, 0, None))
    bad = layout_for(QWEN3_8B_POOL, torch.float32)
    bad.planes = 0
    with pytest.raises(ValueError, match="positive"):
        _lib.check(handle.kvx_restore_blocks(4096, ctypes.byref(bad), ops.FORMAT_FP8, ids, entries, 1, 0, None))
    with pytest.raises(ValueError, match="negative token count"):
        _lib.check(handle.kvx_store_kvcache(16, 0, 16, 0, 16, 16, 16, -1, 8, 128, 2, 10, None))
    fp8_fp16 = layout_for(QWEN3_8B_POOL, torch.float32)
    fp8_fp16.elem_bytes = 4
    with pytest.raises(NotImplementedError, match="bf16"):
        _lib.check(handle.kvx_save_blocks(4096, ctypes.byref(fp8_fp16), ops.FORMAT_FP8, ids, entries, 1, 0, None))
    out = ctypes.c_void_p()
    with pytest.raises(ValueError, match="aligned"):
        _lib.check(handle.kvx_cache_create(4097, ctypes.byref(layout), ops.FORMAT_FP8, 16, 16, 0, ctypes.byref(out)))
    with pytest.raises(ValueError, match="non-null streams"):
        _lib.check(handle.kvx_cache_create(4096, ctypes.byref(layout), ops.FORMAT_FP8, None, 16, 0, ctypes.byref(out)))
    assert out.value is None
    with pytest.raises(IndexError, match="sleep"):
        _lib.check(handle.kvx_sleep(None, -5))


def test_calls_that_would_write_one_destination_twice_are_rejected():
    # Validation runs before any device work, so these addresses are never touched.
    handle = _lib.lib()
    layout = layout_for(QWEN3_8B_POOL, torch.float32)
    _, scale_off, stride = ops.entry_layout(layout, ops.FORMAT_FP8)
    with pytest.raises(ValueError, match="appears twice in one restore"):
        _lib.check(handle.kvx_restore_blocks(4096, ctypes.byref(layout), ops.FORMAT_FP8, _lib.int32_array([3, 5, 3]),
                                             _lib.uint64_array([1 << 30, (1 << 30) + stride, (1 << 30) + 2 * stride]),
                                             3, scale_off, None))
    # Entries closer than one payload apart overlap.
    with pytest.raises(ValueError, match="overlap"):
        _lib.check(handle.kvx_save_blocks(4096, ctypes.byref(layout), ops.FORMAT_FP8, _lib.int32_array([3, 5]),
                                          _lib.uint64_array([1 << 30, (1 << 30) + stride // 2]), 2, scale_off, None))
    # One entry whose scales land inside its own payload.
    with pytest.raises(ValueError, match="overlap"):
        _lib.check(handle.kvx_save_blocks(4096, ctypes.byref(layout), ops.FORMAT_FP8, _lib.int32_array([3]),
                                          _lib.uint64_array([1 << 30]), 1, 1024, None))
    # Scales of entry 0 inside the payload of entry 1 (each entry's own ranges are disjoint).
    with pytest.raises(ValueError, match="overlap"):
        _lib.check(handle.kvx_save_blocks(4096, ctypes.byref(layout), ops.FORMAT_FP8, _lib.int32_array([3, 5]),
                                          _lib.uint64_array([1 << 30, (1 << 30) + 2 * stride]), 2, 2 * stride + 4096,
                                          None))
    raw = layout_for(QWEN3_8B_POOL, torch.bfloat16)
    with pytest.raises(ValueError, match="appears twice in one scatter"):
        _lib.check(handle.kvx_scatter_tokens(4096, ctypes.byref(raw), _lib.int32_array([7, 7]), 2, 2 * 256 * 8,
                                             1 << 30, None))


def test_operators_refuse_cpu_tensors_instead_of_falling_back():
    x = torch.zeros((4, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ROCm device"):
        ops.fp8_quantize(x, torch.empty(x.shape, dtype=torch.float8_e4m3fn), torch.empty((4, 1)))
    key = torch.zeros((2, 1, 4), dtype=torch.bfloat16)
    cache = torch.zeros((1, 4, 1, 4), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ROCm device"):
        ops.store_kvcache(key, key, cache, cache, torch.zeros(2, dtype=torch.int32))
    pool = torch.zeros((2, 2, 2, 256, 1, 4), dtype=torch.bfloat16)
    runner = SimpleNamespace(world_size=1, block_size=256, kv_cache=pool)
    with pytest.raises(ValueError, match="ROCm device"):
        CPUBlockCache(runner, BlockManager(2, 256), 1 << 20)


def test_cache_constructor_validates_like_the_reference():
    # Checks that precede any device use (cpu_prefix_cache.py:76-89).
    pool = torch.zeros((2, 2, 2, 256, 1, 4), dtype=torch.bfloat16)
    runner = SimpleNamespace(world_size=1, block_size=256, kv_cache=pool)
    manager = BlockManager(2, 256)
    for bad in (0, -1, 1.5, True):
        with pytest.raises(ValueError, match="positive integer"):
            CPUBlockCache(runner, manager, bad)
    with pytest.raises(ValueError, match="automatic"):
        CPUBlockCache(runner, manager, 1 << 20, save_on_release=True)
    with pytest.raises(ValueError, match="three nonnegative"):
        CPUBlockCache(runner, manager, 1 << 20, automatic=True, hybrid=(1.0, -1.0, 0.0))
    runner.world_size = 2
    with pytest.raises(NotImplementedError, match="TP=1"):
        CPUBlockCache(runner, manager, 1 << 20)
    runner.world_size, runner.block_size = 1, 128
    with pytest.raises(ValueError, match="layout"):
        CPUBlockCache(runner, manager, 1 << 20)


def test_pool_layout_rejects_unsupported_scale_dtypes():
    pool = torch.zeros((2, 2, 3, 4, 1, 8), dtype=torch.bfloat16)
    assert ops.pool_layout(pool).scale_dtype == _lib.SCALE_BF16
    assert ops.pool_layout(pool, torch.float32).scale_dtype == _lib.SCALE_FP32
    for bad in (torch.float16, torch.float8_e4m3fn, torch.int32):
        with pytest.raises(ValueError, match="bfloat16 or float32"):
            ops.pool_layout(pool, bad)
    raw = ops.pool_layout(pool.to(torch.float16))  # RAW-only pools keep a placeholder scale dtype
    assert (raw.planes, raw.plane_rows, raw.head_dim, raw.num_blocks) == (4, 4, 8, 3)


def test_a_missing_library_fails_loudly(monkeypatch):
    # No CPU or torch fallback exists: without libkvx every operator raises.
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", ROOT / "no-such-dir" / "libkvx.so")
    with pytest.raises(RuntimeError, match="libkvx is not built"):
        _lib.lib()
    layout = ops.pool_layout(torch.zeros((2, 1, 2, 4, 1, 8), dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="libkvx is not built"):
        ops.entry_layout(layout, ops.FORMAT_FP8)
