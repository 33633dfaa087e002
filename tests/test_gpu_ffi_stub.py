"""The maintainer-side ctypes binding (tests/kvx_ffi_stub.py) run against libkvx and checked with the oracle.

The stub binds the C ABI with ctypes alone, as nano-vllm would without the
kvx package: the paged write of nanovllm/layers/attention.py:33-40 and the
FP8 block codec of nanovllm/engine/cpu_prefix_cache.py:315-317, 383-386, with
entries in device memory and in pinned host memory, both scale formats.
"""

import importlib

import numpy as np
import pytest
import torch

from helpers import bf16_bits, bf16_tensor, finite_bf16_rows, u8
from kvx import _lib, ops
from oracle import kvx_oracle as oracle

pytestmark = pytest.mark.gpu

L, NB, BS, H, HD = 2, 5, 256, 2, 128


@pytest.fixture
def stub(gpu, monkeypatch):
    monkeypatch.setenv("KVX_LIBRARY", str(_lib.LIB_PATH))
    import kvx_ffi_stub

    return importlib.reload(kvx_ffi_stub)


def _pool(device, seed):
    rows = 2 * L * NB * BS * H
    return bf16_tensor(finite_bf16_rows(rows, HD, seed), device).reshape(2, L, NB, BS, H, HD)


def test_stub_store_kvcache_matches_the_oracle(stub, gpu):
    pool = _pool(gpu, 1)
    n = 700
    kv = bf16_tensor(finite_bf16_rows(2 * n * H, HD, 2), gpu).reshape(2, n, H, HD)
    rng = np.random.default_rng(3)
    slots = rng.permutation(NB * BS)[:n].astype(np.int32)
    slots[::7] = -1
    mapping = torch.from_numpy(slots).to(gpu)
    expect = bf16_bits(pool)
    key_bits, value_bits = bf16_bits(kv[0]), bf16_bits(kv[1])
    for layer in range(L):
        oracle.store_kvcache(key_bits, value_bits, expect[0, layer], expect[1, layer], slots)
        stub.store_kvcache(kv[0], kv[1], pool[0, layer], pool[1, layer], mapping)
    torch.cuda.synchronize(gpu)
    assert np.array_equal(bf16_bits(pool), expect)


def test_stub_store_kvcache_keeps_the_reference_asserts(stub, gpu):
    pool = _pool(gpu, 4)
    kv = torch.zeros(2, 3, H, HD, dtype=torch.bfloat16, device=gpu)
    mapping = torch.zeros(2, dtype=torch.int32, device=gpu)
    with pytest.raises(AssertionError):
        stub.store_kvcache(kv[0], kv[1], pool[0, 0], pool[1, 0], mapping)


@pytest.mark.parametrize("fp32_scales", [True, False], ids=["fp32-scales", "bf16-scales"])
@pytest.mark.parametrize("where", ["device", "pinned-host"])
def test_stub_fp8_block_round_trip_matches_the_oracle(stub, gpu, fp32_scales, where):
    pool = _pool(gpu, 5 + fp32_scales)
    stride, scale_offset = stub.entry_layout(pool, fp32_scales)
    _, expect_offset, expect_stride = ops.entry_layout(
        _lib.BlockLayout(NB * BS * H * HD, BS * H * HD, 2 * L, BS * H, HD, NB, 2,
                         _lib.SCALE_FP32 if fp32_scales else _lib.SCALE_BF16), ops.FORMAT_FP8)
    assert (stride, scale_offset) == (expect_stride, expect_offset)
    entries = torch.zeros(2, stride, dtype=torch.uint8,
                          **({"device": gpu} if where == "device" else {"pin_memory": True}))
    before = bf16_bits(pool)
    for i, block in enumerate((3, 0)):
        stub.save_fp8_block(pool, block, entries[i].data_ptr(), fp32_scales)
    torch.cuda.synchronize(gpu)
    staged = u8(entries)
    for i, (src, dst) in enumerate([(3, 1), (0, 4)]):
        codes, scales = oracle.save_block_fp8(before, src, fp32_scales)
        assert np.array_equal(staged[i, :codes.size], codes.ravel()), f"payload of block {src}"
        assert np.array_equal(staged[i, scale_offset:scale_offset + scales.nbytes], scales.view(np.uint8).ravel())
        stub.restore_fp8_block(pool, dst, entries[i].data_ptr(), fp32_scales)
        before[:, :, dst] = oracle.dequantize(codes, scales, fp32_scales)
    torch.cuda.synchronize(gpu)
    assert np.array_equal(bf16_bits(pool), before)


def test_stub_reports_a_rejected_block_id(stub, gpu):
    pool = _pool(gpu, 7)
    stride, _ = stub.entry_layout(pool)
    entry = torch.zeros(stride, dtype=torch.uint8, device=gpu)
    before = bf16_bits(pool)
    with pytest.raises(RuntimeError, match=r"\S"):
        stub.restore_fp8_block(pool, NB, entry.data_ptr())
    torch.cuda.synchronize(gpu)
    assert np.array_equal(bf16_bits(pool), before)
