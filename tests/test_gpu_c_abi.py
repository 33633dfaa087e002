"""libkvx from plain C: tests/c_abi/roundtrip.c links libkvx and libamdhip64 only (no Python, no torch) and
runs an FP8 save + restore, a BF16 round trip through the copy engine and two rejected calls; its output is
checked here against the oracle."""

import subprocess
from pathlib import Path

import numpy as np
import pytest

from kvx import _lib, ops
from oracle import kvx_oracle as oracle

pytestmark = pytest.mark.gpu

BINARY = Path(__file__).resolve().parent / "c_abi" / "roundtrip"
L, NB, BS, H, HD = 2, 6, 16, 2, 128


def test_a_plain_c_program_saves_and_restores_through_the_c_abi(gpu, tmp_path):
    assert BINARY.exists(), "build() compiles tests/c_abi/roundtrip.c"
    out = tmp_path / "roundtrip.bin"
    proc = subprocess.run([str(BINARY), str(out)], capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "0 check failures" in proc.stdout
    layout = _lib.BlockLayout(NB * BS * H * HD, BS * H * HD, 2 * L, BS * H, HD, NB, 2, _lib.SCALE_FP32)
    _, offset, stride = ops.entry_layout(layout, ops.FORMAT_FP8)
    data = np.fromfile(out, dtype=np.uint8)
    pool_bytes = 2 * L * NB * BS * H * HD * 2
    assert data.size == 3 * pool_bytes + 2 * stride
    shape = (2, L, NB, BS, H, HD)
    before = data[:pool_bytes].view(np.uint16).reshape(shape)
    staged = data[pool_bytes:pool_bytes + 2 * stride].reshape(2, stride)
    after_fp8 = data[pool_bytes + 2 * stride:2 * pool_bytes + 2 * stride].view(np.uint16).reshape(shape)
    after_raw = data[2 * pool_bytes + 2 * stride:].view(np.uint16).reshape(shape)
    for i, (src, dst) in enumerate([(4, 0), (1, 3)]):
        codes, scales = oracle.save_block_fp8(before, src, True)
        assert np.array_equal(staged[i, :codes.size], codes.ravel()), f"FP8 payload of block {src}"
        assert np.array_equal(staged[i, offset:offset + scales.nbytes], scales.view(np.uint8).ravel())
        assert np.array_equal(after_fp8[:, :, dst], oracle.dequantize(codes, scales, True)), f"restore into {dst}"
    for b in (1, 2, 4, 5):
        assert np.array_equal(after_fp8[:, :, b], before[:, :, b])
    # BF16 through pinned host slots: blocks 2 and 5 land in blocks 4 and 1; the rest is unchanged.
    assert np.array_equal(after_raw[:, :, 4], after_fp8[:, :, 2])
    assert np.array_equal(after_raw[:, :, 1], after_fp8[:, :, 5])
    for b in (0, 2, 3, 5):
        assert np.array_equal(after_raw[:, :, b], after_fp8[:, :, b])
