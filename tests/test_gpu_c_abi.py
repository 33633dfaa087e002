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


STRESS = Path(__file__).resolve().parent / "c_abi" / "engine_stress"


def run_stress(seed: int, split: int, debug: int = 0, iterations: int = 1500) -> tuple[int, str]:
    assert STRESS.exists(), "build() compiles tests/c_abi/engine_stress.c"
    proc = subprocess.run([str(STRESS), str(seed), str(iterations), str(split), str(debug)], capture_output=True,
                          text=True, timeout=120)
    assert proc.returncode in (0, 4), proc.stdout + proc.stderr  # 4: mismatches, every call succeeded
    line = proc.stdout.strip().splitlines()[-1]
    return int(line.split()[0]), proc.stdout


@pytest.mark.parametrize("seed,split", [(1, 1), (2, 1), (3, 0), (4, 0)])
def test_a_random_c_workload_keeps_every_block_and_slot_intact(gpu, seed, split):
    mismatches, out = run_stress(seed, split)
    assert mismatches == 0, out


@pytest.mark.parametrize("flag", [_lib.DEBUG_SKIP_SAVE_WAIT, _lib.DEBUG_SKIP_SLOT_READ_WAIT,
                                  _lib.DEBUG_SKIP_REUSE_WAIT, _lib.DEBUG_SKIP_VICTIM_WAIT])
def test_the_c_workload_catches_a_dropped_ordering_rule(gpu, flag):
    # Negative control for the test above (split streams): with one rule dropped, some seed's checkpoints fail.
    assert any(run_stress(seed, 1, flag)[0] > 0 for seed in (1, 2, 3))
