"""ctypes binding of libkvx.so (the C ABI declared in include/kvx.h).

torch is imported first on purpose: libkvx links the HIP runtime by its
SONAME (libamdhip64.so.7), so loading it after torch binds it to the runtime
torch already loaded and streams/pointers from torch are valid in libkvx.
There is no fallback: if the library is missing or fails to load, every
entry point raises.
"""

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must precede the dlopen below)

LIB_PATH = Path(__file__).resolve().with_name("libkvx.so")
ABI_VERSION = 2

E_INVALID, E_RANGE, E_STATE, E_UNSUPPORTED = -1, -2, -3, -4
SCALE_BF16, SCALE_FP32 = 0, 1
FORMAT_RAW, FORMAT_FP8 = 0, 1
DEBUG_SKIP_SAVE_WAIT, DEBUG_SKIP_SLOT_READ_WAIT, DEBUG_SKIP_REUSE_WAIT, DEBUG_SKIP_VICTIM_WAIT = 1, 2, 4, 8
DEBUG_SKIP_OVERWRITE_WAIT = 16
NOALLOC_SCRATCH_BYTES = 64 << 20  # KVX_NOALLOC_SCRATCH_BYTES
UPLOAD_MAX_BYTES = 1 << 30  # KVX_UPLOAD_MAX_BYTES

_c_p = ctypes.c_void_p
_i32, _i64 = ctypes.c_int32, ctypes.c_int64


class BlockLayout(ctypes.Structure):
    """kvx_block_layout: a pool viewed as blocks of `planes` planes of `plane_rows` rows of `head_dim`."""

    _fields_ = [
        ("plane_stride", _i64),
        ("block_stride", _i64),
        ("planes", _i32),
        ("plane_rows", _i32),
        ("head_dim", _i32),
        ("num_blocks", _i32),
        ("elem_bytes", _i32),
        ("scale_dtype", _i32),
    ]

    def __repr__(self):
        return ("BlockLayout(" + ", ".join(f"{name}={getattr(self, name)}" for name, _ in self._fields_) + ")")


# name -> (restype, argtypes); every function declared in include/kvx.h.
SIGNATURES = {
    "kvx_entry_layout": (_i32, [ctypes.POINTER(BlockLayout), _i32, ctypes.POINTER(_i64), ctypes.POINTER(_i64),
                                ctypes.POINTER(_i64)]),
    "kvx_last_error": (ctypes.c_char_p, []),
    "kvx_abi_version": (_i32, []),
    "kvx_store_kvcache": (_i32, [_c_p, _i64, _c_p, _i64, _c_p, _c_p, _c_p, _i64, _i32, _i32, _i32, _i64, _c_p]),
    "kvx_save_blocks": (_i32, [_c_p, ctypes.POINTER(BlockLayout), _i32, ctypes.POINTER(_i32),
                               ctypes.POINTER(ctypes.c_uint64), _i32, _i64, _c_p]),
    "kvx_restore_blocks": (_i32, [_c_p, ctypes.POINTER(BlockLayout), _i32, ctypes.POINTER(_i32),
                                  ctypes.POINTER(ctypes.c_uint64), _i32, _i64, _c_p]),
    "kvx_gather_tokens": (_i32, [_c_p, ctypes.POINTER(BlockLayout), ctypes.POINTER(_i32), _i32, _i64, _c_p, _c_p]),
    "kvx_scatter_tokens": (_i32, [_c_p, ctypes.POINTER(BlockLayout), ctypes.POINTER(_i32), _i32, _i64, _c_p, _c_p]),
    "kvx_gather_tokens_fp8": (_i32, [_c_p, ctypes.POINTER(BlockLayout), ctypes.POINTER(_i32), _i32, _i64, _c_p, _c_p,
                                     _c_p]),
    "kvx_scatter_tokens_fp8": (_i32, [_c_p, ctypes.POINTER(BlockLayout), ctypes.POINTER(_i32), _i32, _i64, _c_p,
                                      _c_p, _c_p]),
    "kvx_cache_create": (_i32, [_c_p, ctypes.POINTER(BlockLayout), _i32, _c_p, _c_p, _i32, ctypes.POINTER(_c_p)]),
    "kvx_cache_destroy": (_i32, [_c_p]),
    "kvx_cache_set_staging": (_i32, [_c_p, _c_p, _c_p, _i32]),
    "kvx_cache_add_slab": (_i32, [_c_p, _c_p, _i32]),
    "kvx_cache_reset_slabs": (_i32, [_c_p]),
    "kvx_cache_streams": (_i32, [_c_p, ctypes.POINTER(_c_p), ctypes.POINTER(_c_p)]),
    "kvx_cache_save": (_i32, [_c_p, ctypes.POINTER(_i32), ctypes.POINTER(_i32), _i32, _c_p]),
    "kvx_cache_save_noalloc": (_i32, [_c_p, ctypes.POINTER(_i32), ctypes.POINTER(_i32), _i32, _c_p]),
    "kvx_cache_restore": (_i32, [_c_p, ctypes.POINTER(_i32), ctypes.POINTER(_i32), _i32, _i32, _c_p]),
    "kvx_cache_before_block_reuse": (_i32, [_c_p, _i32, _c_p]),
    "kvx_cache_before_block_use": (_i32, [_c_p, _i32, _c_p]),
    "kvx_cache_synchronize": (_i32, [_c_p]),
    "kvx_cache_counters": (_i32, [_c_p, ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "kvx_cache_dma_counters": (_i32, [_c_p, ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_i64),
                                      ctypes.POINTER(_i64)]),
    "kvx_cache_set_debug": (_i32, [_c_p, _i32]),
    "kvx_upload": (_i32, [_c_p, _c_p, _i64, _c_p]),
    "kvx_sleep": (_i32, [_c_p, _i64]),
    "kvx_selftest": (_i32, [_c_p, _c_p]),
}


class KvxError(RuntimeError):
    """A HIP failure reported by libkvx (code is the hipError_t value)."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


_lock = threading.Lock()
_lib = None


def lib() -> ctypes.CDLL:
    """The loaded libkvx, with argument types set. Raises if it is not built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(f"libkvx is not built ({LIB_PATH} missing): run "
                                       "python kv-cache-offloading_amd/build.py")
                handle = ctypes.CDLL(str(LIB_PATH))
                # The version first: a library of another version may lack symbols bound below.
                handle.kvx_abi_version.restype = _i32
                version = handle.kvx_abi_version()
                if version != ABI_VERSION:
                    raise RuntimeError(f"libkvx ABI {version} does not match the binding's {ABI_VERSION}: "
                                       "rebuild it with python kv-cache-offloading_amd/build.py")
                for name, (restype, argtypes) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = restype
                    fn.argtypes = argtypes
                _lib = handle
    return _lib


def check(rc: int, what: str = "libkvx"):
    """Raises the Python exception matching a non-zero libkvx return code."""
    if rc == 0:
        return
    message = f"{what}: {lib().kvx_last_error().decode(errors='replace')}"
    if rc == E_INVALID:
        raise ValueError(message)
    if rc == E_RANGE:
        raise IndexError(message)
    if rc == E_STATE:
        raise RuntimeError(message)
    if rc == E_UNSUPPORTED:
        raise NotImplementedError(message)
    raise KvxError(rc, message)


def int32_array(values) -> ctypes.Array:
    values = list(values)
    return (_i32 * len(values))(*values)


def uint64_array(values) -> ctypes.Array:
    values = list(values)
    return (ctypes.c_uint64 * len(values))(*values)
