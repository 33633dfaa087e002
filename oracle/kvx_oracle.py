"""Python face of the oracle: the C restatement (kvx_oracle.c) plus numpy closed forms.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's CPU baseline, to check libkvx against. Product code never imports it.

Everything here works on bit patterns held in numpy integer arrays (bf16 as
uint16, fp8 as uint8, fp32 scales as float32), so comparisons are bit-exact.
References (xxdydx/KV-Cache-Offloading):
  quantize / dequantize        nanovllm/engine/cpu_prefix_cache.py:20-28
  store_kvcache                nanovllm/layers/attention.py:21-30
  block gather / scatter       nanovllm/engine/cpu_prefix_cache.py:319, 386 on a
                               [2, L, NB, BS, H, hd] pool (model_runner.py:120)
"""

import ctypes
import os
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libkvx_oracle.so"
_THREADS = max(1, min(16, len(os.sched_getaffinity(0))))

_lib = None


def build():
    """Compiles libkvx_oracle.so with the Makefile beside this file."""
    subprocess.run(["make", "-s", "-C", str(HERE), "-B", "libkvx_oracle.so"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"oracle not built: run make -C {HERE}")
        handle = ctypes.CDLL(str(LIB_PATH))
        u8p, u16p, vp = ctypes.POINTER(ctypes.c_uint8), ctypes.POINTER(ctypes.c_uint16), ctypes.c_void_p
        handle.kvx_oracle_e4m3.argtypes, handle.kvx_oracle_e4m3.restype = [ctypes.c_float], ctypes.c_uint8
        handle.kvx_oracle_bf16.argtypes, handle.kvx_oracle_bf16.restype = [ctypes.c_float], ctypes.c_uint16
        handle.kvx_oracle_e4m3_decode.argtypes = [ctypes.c_uint8]
        handle.kvx_oracle_e4m3_decode.restype = ctypes.c_float
        handle.kvx_oracle_e4m3_range.argtypes = [ctypes.c_uint32, ctypes.c_uint32, u8p]
        handle.kvx_oracle_bf16_range.argtypes = [ctypes.c_uint32, ctypes.c_uint32, u16p]
        handle.kvx_oracle_quantize.argtypes = [u16p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, u8p, vp]
        handle.kvx_oracle_dequantize.argtypes = [u8p, vp, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, u16p]
        handle.kvx_oracle_fastdiv_mismatches.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
        handle.kvx_oracle_fastdiv_mismatches.restype = ctypes.c_int64
        _lib = handle
    return _lib


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def _split(total: int, parts: int):
    step = -(-total // parts)
    return [(i, min(step, total - i)) for i in range(0, total, step)]


# -- conversions ------------------------------------------------------------

def e4m3_of_bits(first: int, count: int) -> np.ndarray:
    """e4m3fn codes of the fp32 bit patterns [first, first + count)."""
    out = np.empty(count, dtype=np.uint8)
    with ThreadPoolExecutor(_THREADS) as pool:
        list(pool.map(lambda r: lib().kvx_oracle_e4m3_range(first + r[0], r[1], _ptr(out[r[0]:], ctypes.c_uint8)),
                      _split(count, _THREADS)))
    return out


def bf16_of_bits(first: int, count: int) -> np.ndarray:
    """bf16 bit patterns (RNE) of the fp32 bit patterns [first, first + count)."""
    out = np.empty(count, dtype=np.uint16)
    with ThreadPoolExecutor(_THREADS) as pool:
        list(pool.map(lambda r: lib().kvx_oracle_bf16_range(first + r[0], r[1], _ptr(out[r[0]:], ctypes.c_uint16)),
                      _split(count, _THREADS)))
    return out


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    return np.array([lib().kvx_oracle_e4m3_decode(int(c)) for c in codes.ravel()], dtype=np.float32).reshape(
        codes.shape)


def fastdiv_mismatches() -> int:
    """Pairs (bf16 significand, fp32 significand) where the kernels' division is not IEEE."""
    with ThreadPoolExecutor(_THREADS) as pool:
        return sum(pool.map(lambda r: lib().kvx_oracle_fastdiv_mismatches(r[0], r[1]), _split(1 << 23, _THREADS)))


# -- codec (cpu_prefix_cache.py:20-28) ---------------------------------------

def quantize(x_bits: np.ndarray, scale_fp32: bool) -> tuple[np.ndarray, np.ndarray]:
    """(codes uint8 [..., hd], scales [..., 1] as float32 or uint16 bf16 bits) of bf16 bits x."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    hd = x.shape[-1]
    rows = x.size // hd if hd else 0
    codes = np.empty(x.shape, dtype=np.uint8)
    scales = np.empty((*x.shape[:-1], 1), dtype=np.float32 if scale_fp32 else np.uint16)
    flat_x, flat_c, flat_s = x.reshape(rows, hd), codes.reshape(rows, hd), scales.reshape(rows)

    def run(r):
        lo, n = r
        lib().kvx_oracle_quantize(_ptr(flat_x[lo:], ctypes.c_uint16), n, hd, int(scale_fp32),
                                  _ptr(flat_c[lo:], ctypes.c_uint8), flat_s[lo:].ctypes.data)

    if rows:
        with ThreadPoolExecutor(_THREADS) as pool:
            list(pool.map(run, _split(rows, _THREADS)))
    return codes, scales


def dequantize(codes: np.ndarray, scales: np.ndarray, scale_fp32: bool) -> np.ndarray:
    """bf16 bits of fp32(code) * fp32(scale), rounded to nearest even."""
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    s = np.ascontiguousarray(scales, dtype=np.float32 if scale_fp32 else np.uint16)
    hd = c.shape[-1]
    rows = c.size // hd if hd else 0
    out = np.empty(c.shape, dtype=np.uint16)
    flat_c, flat_s, flat_o = c.reshape(rows, hd), s.reshape(rows), out.reshape(rows, hd)

    def run(r):
        lo, n = r
        lib().kvx_oracle_dequantize(_ptr(flat_c[lo:], ctypes.c_uint8), flat_s[lo:].ctypes.data, n, hd,
                                    int(scale_fp32), _ptr(flat_o[lo:], ctypes.c_uint16))

    if rows:
        with ThreadPoolExecutor(_THREADS) as pool:
            list(pool.map(run, _split(rows, _THREADS)))
    return out


# -- byte-copy closed forms ----------------------------------------------------

def store_kvcache(key: np.ndarray, value: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                  slot_mapping: np.ndarray):
    """In place: k_cache.reshape(-1, D)[s] = key[i].reshape(D) for each slot s = slot_mapping[i] != -1
    (attention.py:21-30); slots outside the cache write nothing, like libkvx."""
    n = key.shape[0]
    d = key[0].size if n else 0
    kc, vc = k_cache.reshape(-1, d), v_cache.reshape(-1, d)
    slots = np.asarray(slot_mapping, dtype=np.int64)
    ok = (slots >= 0) & (slots < kc.shape[0])
    kc[slots[ok]] = key.reshape(n, d)[ok]
    vc[slots[ok]] = value.reshape(n, d)[ok]


def gather_block(pool: np.ndarray, block_id: int) -> np.ndarray:
    """pool[:, :, block_id] as a contiguous [2, L, BS, H, hd] copy (cpu_prefix_cache.py:319)."""
    return np.ascontiguousarray(pool[:, :, block_id])


def scatter_block(pool: np.ndarray, block_id: int, payload: np.ndarray):
    """In place: pool[:, :, block_id] = payload (cpu_prefix_cache.py:386)."""
    pool[:, :, block_id] = payload


def save_block_fp8(pool_bits: np.ndarray, block_id: int, scale_fp32: bool):
    """FP8 entry (codes, scales) of pool block `block_id` (cpu_prefix_cache.py:315-317 via :225-234)."""
    return quantize(gather_block(pool_bits, block_id), scale_fp32)


def gather_tokens(pool: np.ndarray, table, count: int) -> np.ndarray:
    """[2, L, count, H, hd]: the first `count` tokens of the blocks `table` in order (kv_handoff.py:51-55,
    index_select over the block table, flattened, then sliced)."""
    table = list(table)
    picked = pool[:, :, table]
    return np.ascontiguousarray(picked.reshape(pool.shape[0], pool.shape[1], len(table) * pool.shape[3],
                                               *pool.shape[4:])[:, :, :count])


def scatter_tokens(pool: np.ndarray, table, dense: np.ndarray):
    """In place: the inverse of gather_tokens for dense's tokens (kv_handoff.py:112-118)."""
    count, bs = dense.shape[2], pool.shape[3]
    for i, block in enumerate(table):
        lo, hi = i * bs, min((i + 1) * bs, count)
        if lo >= hi:
            break
        pool[:, :, block, :hi - lo] = dense[:, :, lo:hi]
