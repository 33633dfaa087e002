"""The C ABI boundary on the CPU: the library loads, exports what include/kvx.h
declares, and rejects bad arguments before touching a device."""

import ctypes
import re
import subprocess
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch
from hypothesis import example, given, settings, strategies as st

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


# -- layout and size validation: exact arithmetic against the library's answer ----------

_SPAN = 1 << 40
_INT32 = st.one_of(st.integers(-2, 300), st.integers(0, 2**31 - 1))
_INT64 = st.one_of(st.integers(-2, 1 << 20), st.integers(0, 2**63 - 1))


def _ceil256(n: int) -> int:
    return -(-n // 256) * 256


def _layout_accepted(fmt, planes, rows, hd, blocks, plane_stride, block_stride, elem, scale) -> bool:
    """What the library must accept, in Python integers (no overflow)."""
    if fmt not in (ops.FORMAT_RAW, ops.FORMAT_FP8) or min(planes, rows, hd, blocks) <= 0:
        return False
    if plane_stride < 0 or block_stride < 0 or (blocks > 1 and block_stride < rows * hd):
        return False
    if fmt == ops.FORMAT_FP8 and (elem != 2 or scale not in (0, 1)):
        return False
    if fmt == ops.FORMAT_RAW and elem not in (1, 2, 4, 8):
        return False
    if planes * rows * hd * elem > _SPAN:
        return False
    if ((blocks - 1) * block_stride + (planes - 1) * plane_stride + rows * hd) * elem > _SPAN:
        return False
    return 128 * planes * ((rows * hd * elem) // 16 + 1) <= 2**31 - 1


@settings(max_examples=600, deadline=None)
# Boundary cases random generation rarely reaches: a pool extent of exactly 2^40 bytes and one byte more,
# strides whose products overflow int64, and dimensions whose byte count wraps int64.
@example(fmt=ops.FORMAT_RAW, planes=1, rows=1, hd=16, blocks=2, plane_stride=0, block_stride=2**40 - 16, elem=1,
         scale=0)
@example(fmt=ops.FORMAT_RAW, planes=1, rows=1, hd=16, blocks=2, plane_stride=0, block_stride=2**40 - 15, elem=1,
         scale=0)
@example(fmt=ops.FORMAT_FP8, planes=72, rows=2048, hd=128, blocks=2, plane_stride=2**20, block_stride=2**62,
         elem=2, scale=1)
@example(fmt=ops.FORMAT_FP8, planes=2, rows=2048, hd=128, blocks=1, plane_stride=2**63 - 1, block_stride=0,
         elem=2, scale=0)
@example(fmt=ops.FORMAT_RAW, planes=1, rows=2**31 - 1, hd=2**31 - 1, blocks=1, plane_stride=0, block_stride=0,
         elem=8, scale=0)
@given(fmt=st.sampled_from([ops.FORMAT_RAW, ops.FORMAT_FP8, 7]), planes=_INT32, rows=_INT32, hd=_INT32,
       blocks=_INT32, plane_stride=_INT64, block_stride=_INT64, elem=st.sampled_from([1, 2, 3, 4, 8]),
       scale=st.sampled_from([0, 1, 5]))
def test_entry_layout_accepts_exactly_the_valid_layouts_and_sizes_them(fmt, planes, rows, hd, blocks, plane_stride,
                                                                       block_stride, elem, scale):
    layout = _lib.BlockLayout(plane_stride, block_stride, planes, rows, hd, blocks, elem, scale)
    logical, offset, stride = ctypes.c_int64(-1), ctypes.c_int64(-1), ctypes.c_int64(-1)
    rc = _lib.lib().kvx_entry_layout(ctypes.byref(layout), fmt, ctypes.byref(logical), ctypes.byref(offset),
                                     ctypes.byref(stride))
    accepted = _layout_accepted(fmt, planes, rows, hd, blocks, plane_stride, block_stride, elem, scale)
    assert (rc == 0) == accepted, (rc, _lib.lib().kvx_last_error())
    if not accepted:
        assert rc in (_lib.E_INVALID, _lib.E_UNSUPPORTED)
        return
    total_rows = planes * rows
    if fmt == ops.FORMAT_FP8:
        scale_bytes = total_rows * (2 if scale == 0 else 4)
        want = (total_rows * hd + scale_bytes, _ceil256(total_rows * hd), _ceil256(_ceil256(total_rows * hd)
                                                                                     + scale_bytes))
    else:
        want = (total_rows * hd * elem, 0, _ceil256(total_rows * hd * elem))
    assert (logical.value, offset.value, stride.value) == want


def test_spans_beyond_two_to_the_40_bytes_are_refused_before_any_device_work():
    # These addresses are never dereferenced: each call fails in its size checks.
    handle = _lib.lib()
    with pytest.raises(NotImplementedError, match="2\\^40"):
        _lib.check(handle.kvx_store_kvcache(16, 1 << 61, 16, 0, 16, 16, 16, 3, 8, 128, 2, 10, None))
    with pytest.raises(NotImplementedError, match="2\\^40"):
        _lib.check(handle.kvx_store_kvcache(16, 1024, 16, 1024, 16, 16, 16, 3, 8, 128, 2, 1 << 40, None))
    layout = layout_for(QWEN3_8B_POOL, torch.float32)
    table = _lib.int32_array([0])
    with pytest.raises(NotImplementedError, match="2\\^40"):
        _lib.check(handle.kvx_gather_tokens(4096, ctypes.byref(layout), table, 1, 1 << 50, 4096, None))
    with pytest.raises(NotImplementedError, match="2\\^40"):
        _lib.check(handle.kvx_gather_tokens_fp8(4096, ctypes.byref(layout), table, 1, 1 << 50, 4096, 8192, None))
    wide = layout_for(QWEN3_8B_POOL, torch.float32)
    wide.block_stride = 1 << 62
    with pytest.raises(NotImplementedError, match="2\\^40"):
        _lib.check(handle.kvx_restore_blocks(4096, ctypes.byref(wide), ops.FORMAT_FP8, table,
                                             _lib.uint64_array([4096]), 1, 0, None))


def test_upload_and_dma_counters_reject_bad_arguments_before_any_device_work():
    handle = _lib.lib()
    with pytest.raises(ValueError, match="negative byte count"):
        _lib.check(handle.kvx_upload(16, 16, -1, None))
    with pytest.raises(IndexError, match="largest upload"):
        _lib.check(handle.kvx_upload(16, 16, _lib.UPLOAD_MAX_BYTES + 1, None))
    with pytest.raises(ValueError, match="NULL"):
        _lib.check(handle.kvx_upload(0, 16, 64, None))
    _lib.check(handle.kvx_upload(0, 0, 0, None))  # nothing to copy: no pointer is looked at
    counts = [ctypes.c_int64() for _ in range(4)]
    with pytest.raises(ValueError, match="NULL cache"):
        _lib.check(handle.kvx_cache_dma_counters(None, *map(ctypes.byref, counts)))
