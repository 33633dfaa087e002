"""The whole ctypes binding a nano-vllm maintainer adds to call libkvx without the kvx package.

Written as that maintainer's module (e.g. nanovllm/layers/kvx_ffi.py): torch
for tensors and streams, ctypes for the C ABI, nothing else. The library path
comes from KVX_LIBRARY. store_kvcache keeps the signature and asserts of
nanovllm/layers/attention.py:33-40; save_fp8_block / restore_fp8_block are the
FP8 codec copies of save_block and _copy_entry
(nanovllm/engine/cpu_prefix_cache.py:315-317, 383-386) for one block and one
device-accessible entry address (device memory or pinned host memory).
"""

import ctypes
import os

import torch  # first: libkvx binds to the HIP runtime torch loaded

_lib = ctypes.CDLL(os.environ["KVX_LIBRARY"])
_vp, _i32, _i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
FORMAT_FP8 = 1


class BlockLayout(ctypes.Structure):  # kvx_block_layout
    _fields_ = [("plane_stride", _i64), ("block_stride", _i64), ("planes", _i32), ("plane_rows", _i32),
                ("head_dim", _i32), ("num_blocks", _i32), ("elem_bytes", _i32), ("scale_dtype", _i32)]


_lib.kvx_last_error.restype = ctypes.c_char_p
_lib.kvx_store_kvcache.argtypes = [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i64, _vp]
_lib.kvx_entry_layout.argtypes = [ctypes.POINTER(BlockLayout), _i32, ctypes.POINTER(_i64),
                                  ctypes.POINTER(_i64), ctypes.POINTER(_i64)]
for _name in ("kvx_save_blocks", "kvx_restore_blocks"):
    getattr(_lib, _name).argtypes = [_vp, ctypes.POINTER(BlockLayout), _i32, ctypes.POINTER(_i32),
                                     ctypes.POINTER(ctypes.c_uint64), _i32, _i64, _vp]


def _check(rc):
    if rc:
        raise RuntimeError(_lib.kvx_last_error().decode())


def _stream():
    return torch.cuda.current_stream().cuda_stream


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping: torch.Tensor):
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == D and v_cache.stride(1) == D
    assert slot_mapping.numel() == N
    _check(_lib.kvx_store_kvcache(key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
                                  k_cache.data_ptr(), v_cache.data_ptr(), slot_mapping.data_ptr(), N,
                                  num_heads, head_dim, key.element_size(), k_cache.numel() // D, _stream()))


def _layout(pool: torch.Tensor, fp32_scales: bool) -> BlockLayout:
    _, L, NB, BS, H, hd = pool.shape
    return BlockLayout(NB * BS * H * hd, BS * H * hd, 2 * L, BS * H, hd, NB, pool.element_size(), int(fp32_scales))


def entry_layout(pool: torch.Tensor, fp32_scales: bool = True) -> tuple[int, int]:
    """(bytes one FP8 entry occupies, offset of its scales) for a [2, L, NB, BS, H, hd] pool."""
    logical, scale_offset, stride = _i64(), _i64(), _i64()
    _check(_lib.kvx_entry_layout(_layout(pool, fp32_scales), FORMAT_FP8, logical, scale_offset, stride))
    return stride.value, scale_offset.value


def _copy(name, pool, block_id, entry_ptr, fp32_scales):
    _, scale_offset = entry_layout(pool, fp32_scales)
    _check(getattr(_lib, name)(pool.data_ptr(), _layout(pool, fp32_scales), FORMAT_FP8, (_i32 * 1)(block_id),
                               (ctypes.c_uint64 * 1)(entry_ptr), 1, scale_offset, _stream()))


def save_fp8_block(pool: torch.Tensor, block_id: int, entry_ptr: int, fp32_scales: bool = True):
    _copy("kvx_save_blocks", pool, block_id, entry_ptr, fp32_scales)


def restore_fp8_block(pool: torch.Tensor, block_id: int, entry_ptr: int, fp32_scales: bool = True):
    _copy("kvx_restore_blocks", pool, block_id, entry_ptr, fp32_scales)
