"""Seeded caller sequences through the real copy engine on the GPU, checked against sequential execution.

The sequences of tests/copy_scenarios.py (admissions, prefetches, restore_block, uses, release-time
saves, discards) drive `_CopyBatcher` and libkvx's copy engine on a small pool. Each block holds one
repeated bf16 value, so a block or entry that mixes two writes, or holds a stale one, decodes to
nothing. Between calls, bounded delay kernels (0-2 ms) are queued at random on the save stream, the
restore stream or the caller's stream, so copies lag behind the caller's work, or the caller behind the
copies. Every read the caller's stream makes, and every block and live entry at the end, must hold what
a sequential execution gives. The CPU model (test_copy_ordering_model.py) explores the interleavings;
this runs the same sequences on the hardware, FP8 and BF16 entries, split streams and one copy stream,
batched and one call per block, with saves of up to 4 blocks through the allocation-free entry point
(kvx_cache_save_noalloc), and with the caller switching between two streams.
"""

import random

import numpy as np
import pytest
import torch

from copy_scenarios import Caller, NoAllocSaves
from kvx import _lib, ops
from kvx._lib import check, int32_array, lib
from kvx.engine.cpu_prefix_cache import _CopyBatcher, _CopyEngine

pytestmark = pytest.mark.gpu

BLOCKS, SLOTS, ROUNDS = 12, 10, 60
SHAPE = (2, 2, BLOCKS, 16, 2, 128)  # [K/V, layers, blocks, block size, heads, head_dim]
DELAYS_US = (0, 0, 0, 50, 300, 2000)


def bf16_bits_of(value: int, fp8: bool) -> int:
    """The bf16 bit pattern a block holding value id `value` repeats.

    FP8 entries need values their round trip returns exactly: powers of two within 2^-60..2^60, whose row
    scale is normal and whose codes are all +-448 (the sign alternates with the id)."""
    if fp8:
        sign = 0x8000 if value & 1 else 0
        exponent = (value >> 1) % 121 - 60
        return sign | (exponent + 127) << 7
    return 0x3C00 + value  # distinct finite positive bf16 values for ids below 17,000


class GpuBackend:
    def __init__(self, device, seed: int, fmt: int, split: bool, staging: int, noalloc: bool = False):
        self.device, self.fmt = device, fmt
        self.fp8 = fmt == ops.FORMAT_FP8
        self.rng = random.Random(seed * 104729 + 3)
        self.pool = torch.zeros(SHAPE, dtype=torch.bfloat16, device=device)
        layout = ops.pool_layout(self.pool, torch.float32 if self.fp8 else None)
        self.engine = _CopyEngine(self.pool, layout, fmt, split)
        self.stride = self.engine.entry_stride
        self.scale_offset = self.engine.scale_offset
        self.slab = torch.zeros(SLOTS * self.stride, dtype=torch.uint8, pin_memory=True)
        save = torch.empty(staging * self.stride, dtype=torch.uint8, device=device)
        restore = torch.empty_like(save) if split else save
        self.staging = (save, restore)
        self.engine.add_slab(self.slab, SLOTS)
        self.engine.set_staging(save, restore, staging)
        engine = self.engine
        if noalloc:
            assert _lib.NOALLOC_SCRATCH_BYTES // self.stride >= 4

            def save_noalloc(block_ids, slots, compute):
                check(lib().kvx_cache_save_noalloc(self.engine.handle, int32_array(block_ids), int32_array(slots),
                                                   len(block_ids), compute), "kvx_cache_save_noalloc")

            engine = NoAllocSaves(self.engine, save_noalloc, 4)
        self.batcher = _CopyBatcher(engine, lambda: torch.cuda.current_stream(device).cuda_stream)
        self.reads = torch.empty((ROUNDS * 8 + 8, *self.pool[:, :, 0].shape), dtype=torch.bfloat16, device=device)
        self.caller_streams = [torch.cuda.current_stream(device), torch.cuda.Stream(device)]
        self.n_reads = 0
        self.decode = {}  # bf16 bits -> value id

    def _bits(self, value: int) -> int:
        bits = bf16_bits_of(value, self.fp8)
        self.decode[bits] = value
        return bits

    def write(self, block, value):
        bits = np.array([self._bits(value)], dtype=np.uint16).view(np.int16)
        self.pool[:, :, block].fill_(torch.from_numpy(bits).view(torch.bfloat16).item())

    def read(self, block):
        i = self.n_reads
        assert i < len(self.reads), "more reads than the buffer holds"
        self.n_reads += 1
        self.reads[i].copy_(self.pool[:, :, block])
        return i

    def switch_stream(self):
        current = torch.cuda.current_stream(self.device)
        new = self.caller_streams[1] if current == self.caller_streams[0] else self.caller_streams[0]
        new.wait_stream(current)
        torch.cuda.set_stream(new)

    def between(self):
        if self.rng.random() < 0.5:
            streams = (self.engine.save_stream, self.engine.restore_stream, torch.cuda.current_stream(self.device))
            ops.sleep(self.rng.choice(DELAYS_US), stream=self.rng.choice(streams), device=self.device)

    def sync(self):
        self.engine.synchronize()
        torch.cuda.synchronize(self.device)

    def _decode(self, tensor) -> object:
        bits = np.unique(tensor.view(torch.int16).cpu().numpy().astype(np.uint16))
        if len(bits) != 1:
            return f"a mix of {len(bits)} values"
        return self.decode.get(int(bits[0]), f"bits {int(bits[0]):#06x}")

    def value(self, token):
        return self._decode(self.reads[token])

    def block_value(self, block):
        return self._decode(self.pool[:, :, block])

    def slot_value(self, slot):
        entry = self.slab[slot * self.stride:(slot + 1) * self.stride]
        if not self.fp8:
            return self._decode(entry[:self.pool[:, :, 0].numel() * 2].view(torch.bfloat16))
        rows = self.pool[:, :, 0, :, :, 0].numel()
        codes = entry[:rows * SHAPE[-1]].view(torch.float8_e4m3fn).float().view(rows, SHAPE[-1])
        scales = entry[self.scale_offset:self.scale_offset + rows * 4].view(torch.float32).view(rows, 1)
        return self._decode((codes * scales).to(torch.bfloat16))

    def close(self):
        torch.cuda.set_stream(self.caller_streams[0])
        self.engine.close()


@pytest.mark.parametrize("fmt", [ops.FORMAT_FP8, ops.FORMAT_RAW], ids=["fp8", "bf16"])
@pytest.mark.parametrize("split,staging,batched,noalloc,switch", [
    (True, 3, True, False, False), (True, 1, False, False, False), (False, 2, True, False, False),
    (True, 128, True, False, False), (True, 3, True, True, False), (False, 1, False, True, False),
    (True, 2, True, False, True), (False, 1, False, False, True)])
def test_random_caller_sequences_give_the_sequential_result(gpu, fmt, split, staging, batched, noalloc, switch):
    for seed in range(6):
        backend = GpuBackend(gpu, seed, fmt, split, staging, noalloc)
        try:
            caller = Caller(random.Random(seed), backend, BLOCKS, SLOTS, batched=batched, switch_streams=switch)
            caller.run(ROUNDS)
            bad = caller.check()
            assert not bad, f"seed {seed}: {bad[:5]}\n" + "\n".join(caller.log[-30:])
        finally:
            backend.close()
