"""Pins the oracle (oracle/kvx_oracle.c) before it is trusted to judge the kernels.

Each check is independent of the oracle's own formulas: torch's CPU
conversion and codec routines (the library the reference runs), committed
fixtures written by them, hand-derived known answers, and the reference's own
acceptance bound (bench/test_cpu_cache_optimizations.py:71-73).
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import kvx_oracle as oracle
from oracle import torch_path

GOLDEN = np.load(Path(__file__).resolve().parent / "golden" / "fp8_codec.npz")
CHUNK = 1 << 24


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def bf16_tensor(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def fp32_patterns(first: int, count: int) -> torch.Tensor:
    return torch.arange(first, first + count, dtype=torch.int64).to(torch.int32).view(torch.float32)


def test_fast_division_is_ieee_for_every_significand_pair():
    # The kernels' reciprocal-FMA quotient, over all 2^30 (bf16, fp32) significand pairs.
    assert oracle.fastdiv_mismatches() == 0


def test_e4m3_encoder_matches_torch_on_every_relevant_fp32():
    # Every non-negative pattern up to 512 (past the 480 NaN boundary), exhaustively.
    end = 0x44000000
    for first in range(0, end, CHUNK):
        count = min(CHUNK, end - first)
        ours = oracle.e4m3_of_bits(first, count)
        ref = fp32_patterns(first, count).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        bad = np.flatnonzero(ours != ref)
        assert bad.size == 0, f"first mismatch at fp32 bits {first + int(bad[0]):#x}"


def test_e4m3_encoder_sign_nan_and_overflow_samples():
    # Negative values, large values, infinities and NaNs on a stride.
    for first in (0x80000000, 0x44000000, 0xC4000000):
        count = 0x3C000000
        idx = np.arange(0, count, 4099, dtype=np.int64) + first
        f = torch.from_numpy(idx.astype(np.uint32).view(np.int32)).view(torch.float32)
        ref = f.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        ours = np.array([oracle.lib().kvx_oracle_e4m3(float(v)) for v in f.numpy()[:20000]], dtype=np.uint8)
        assert np.array_equal(ours, ref[:20000])
    for special in (float("inf"), float("-inf"), float("nan"), 480.0, -480.0, 464.0, 464.00003):
        ref = torch.tensor([special]).to(torch.float8_e4m3fn).view(torch.uint8).item()
        assert oracle.lib().kvx_oracle_e4m3(special) == ref, special


def test_bf16_rounding_matches_torch_on_every_non_nan_fp32():
    for first in range(0, 1 << 32, CHUNK * 4):
        count = CHUNK * 4
        f = fp32_patterns(first, count)
        ref = bf16_bits(f.to(torch.bfloat16))
        ours = oracle.bf16_of_bits(first, count)
        finite = ~np.isnan(f.numpy())
        bad = np.flatnonzero((ours != ref) & finite)
        assert bad.size == 0, f"first mismatch at fp32 bits {first + int(bad[0]):#x}"
        assert np.all((ours[~finite] & 0x7FFF) > 0x7F80)  # NaN stays NaN


def test_e4m3_decoder_matches_torch_for_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    ours = oracle.e4m3_decode(codes)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan) and nan.sum() == 2
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


@pytest.mark.parametrize("hd", [128, 64, 256, 4])
@pytest.mark.parametrize("scale", ["fp32", "bf16"])
def test_codec_matches_golden_fixtures(hd, scale):
    x = GOLDEN[f"x_hd{hd}"]
    codes, scales = oracle.quantize(x, scale == "fp32")
    assert np.array_equal(codes, GOLDEN[f"codes_hd{hd}_{scale}"])
    assert np.array_equal(scales.view(np.uint8), GOLDEN[f"scale_hd{hd}_{scale}"].view(np.uint8))
    back = oracle.dequantize(GOLDEN[f"codes_hd{hd}_{scale}"], GOLDEN[f"scale_hd{hd}_{scale}"], scale == "fp32")
    assert np.array_equal(back, GOLDEN[f"back_hd{hd}_{scale}"])


def finite_bf16_rows(rows: int, hd: int, seed: int) -> np.ndarray:
    """Uniform over finite bf16 bit patterns: every exponent, both signs, subnormals."""
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 1 << 16, size=(rows, hd), dtype=np.uint32).astype(np.uint16)
    # Narrow some rows to a random exponent window so the row amax does not
    # always dominate every element (exercises mid-range quotients).
    narrow = rng.random(rows) < 0.5
    window = rng.integers(0x0080, 0x7E00, size=rows).astype(np.uint32)
    low = (bits.astype(np.uint32) & 0x807F) | ((window[:, None] + (bits.astype(np.uint32) & 0x0380)) & 0x7F80)
    bits[narrow] = low[narrow].astype(np.uint16)
    bits[(bits & 0x7F80) == 0x7F80] &= 0xBFFF  # fold inf/NaN patterns into finite ones
    return bits


@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.bfloat16])
def test_codec_matches_torch_on_random_finite_rows(scale_dtype):
    x = finite_bf16_rows(2048, 128, seed=7)
    t = bf16_tensor(x)
    payload = torch.empty(t.shape, dtype=torch.float8_e4m3fn)
    scale = torch.empty((t.shape[0], 1), dtype=scale_dtype)
    torch_path.fp8_quantize(t, payload, scale)
    codes, scales = oracle.quantize(x, scale_dtype == torch.float32)
    assert np.array_equal(codes, payload.view(torch.uint8).numpy())
    ref_scale = scale.numpy() if scale_dtype == torch.float32 else bf16_bits(scale)
    assert np.array_equal(scales.view(np.uint8), ref_scale.view(np.uint8))
    back = torch.empty_like(t)
    torch_path.fp8_dequantize(payload, scale, back)
    assert np.array_equal(oracle.dequantize(codes, scales, scale_dtype == torch.float32), bf16_bits(back))


@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.bfloat16])
def test_dequantize_matches_torch_for_all_codes_and_scales(scale_dtype):
    rng = np.random.default_rng(3)
    scales = np.concatenate([
        np.float32([1e-30, 1.0, 2.0 ** -126, 2.0 ** -149, 7.5e35, 1.0 / 448]),
        (rng.standard_normal(250) * 10.0 ** rng.integers(-30, 30, 250)).astype(np.float32).__abs__(),
    ]).astype(np.float32)
    codes = np.tile(np.arange(256, dtype=np.uint8), (scales.size, 1))
    t_scale = torch.from_numpy(scales[:, None]).to(scale_dtype)
    target = torch.empty(codes.shape, dtype=torch.bfloat16)
    torch_path.fp8_dequantize(torch.from_numpy(codes).view(torch.float8_e4m3fn), t_scale, target)
    s_in = scales[:, None] if scale_dtype == torch.float32 else bf16_bits(t_scale)
    ours = oracle.dequantize(codes, s_in, scale_dtype == torch.float32)
    ref = bf16_bits(target)
    nan = (codes & 0x7F) == 0x7F
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.all((ours[nan] & 0x7FFF) > 0x7F80)


def test_known_answers_from_the_e4m3_grid():
    # amax 448 makes the scale exactly 1, so codes are e4m3 of x itself.
    row = np.zeros(16, dtype=np.float32)
    row[:10] = [448.0, 1.0625, 1.1875, 2.0 ** -10, 3 * 2.0 ** -10, -(2.0 ** -10), 232.0, -0.0, -3.0, 0.015625]
    codes, scales = oracle.quantize(bf16_bits(torch.from_numpy(row).to(torch.bfloat16))[None], True)
    assert scales[0, 0] == 1.0
    # 1.0625 ties 1.0|1.125 -> 1.0 (0x38); 1.1875 ties 1.125|1.25 -> 1.25 (0x3A);
    # 2^-10 ties 0|2^-9 -> 0; 3*2^-10 ties 2^-9|2^-8 -> 2^-8 (0x02); 232 ties
    # 224|240 -> 224 (0x76); -0.0 keeps its sign (0x80); 2^-6 is the first normal (0x08).
    assert codes[0, :10].tolist() == [0x7E, 0x38, 0x3A, 0x00, 0x02, 0x80, 0x76, 0x80, 0xC4, 0x08]
    zero, _ = oracle.quantize(np.zeros((1, 8), dtype=np.uint16), True)
    _, zero_scale = oracle.quantize(np.zeros((1, 8), dtype=np.uint16), True)
    assert zero.sum() == 0 and zero_scale.view(np.uint32)[0, 0] == np.float32(1e-30).view(np.uint32)
    single = np.zeros((1, 8), dtype=np.uint16)
    single[0, 3] = bf16_bits(torch.tensor([-0.3], dtype=torch.bfloat16))[0]
    codes, _ = oracle.quantize(single, False)
    assert codes[0, 3] == 0xFE and codes[0, [0, 1, 2, 4]].tolist() == [0, 0, 0, 0]


def test_nan_and_inf_rows_follow_torch_by_class():
    x = bf16_bits(torch.tensor([[1.0, float("nan"), 2.0, 3.0], [1.0, float("inf"), -2.0, 0.0]],
                               dtype=torch.bfloat16))
    codes, scales = oracle.quantize(x, True)
    assert np.isnan(scales[0, 0]) and np.all((codes[0] & 0x7F) == 0x7F)
    assert np.isinf(scales[1, 0])
    assert codes[1].tolist()[2:] == [0x80, 0x00] and (codes[1, 1] & 0x7F) == 0x7F


def test_round_trip_stays_within_the_reference_bound():
    # bench/test_cpu_cache_optimizations.py:71-73: |restored - source| <= amax(|row|) / 16.
    g = torch.Generator().manual_seed(11)
    t = (torch.randn((4096, 128), generator=g) / torch.randn((4096, 128, 4), generator=g).square().mean(-1).sqrt())
    t[:, :4] *= 20
    x = bf16_bits(t.to(torch.bfloat16))
    for fp32 in (True, False):
        codes, scales = oracle.quantize(x, fp32)
        back = bf16_tensor(oracle.dequantize(codes, scales, fp32)).float()
        src = bf16_tensor(x).float()
        assert torch.all((back - src).abs() <= src.abs().amax(-1, keepdim=True) / 16)


def test_store_kvcache_closed_form_matches_a_loop():
    rng = np.random.default_rng(5)
    n, h, hd, slots = 9, 2, 4, 32
    key = rng.integers(0, 60000, size=(n, h, hd), dtype=np.uint16)
    value = rng.integers(0, 60000, size=(n, h, hd), dtype=np.uint16)
    mapping = np.array([5, -1, 0, 31, 7, -1, 40, 12, 3], dtype=np.int32)
    k = np.full((slots // 8, 8, h, hd), 0xBEEF, dtype=np.uint16)
    v = k.copy()
    k_loop, v_loop = k.copy(), v.copy()
    oracle.store_kvcache(key, value, k, v, mapping)
    for i, s in enumerate(mapping):
        if 0 <= s < slots:
            k_loop.reshape(slots, -1)[s] = key[i].ravel()
            v_loop.reshape(slots, -1)[s] = value[i].ravel()
    assert np.array_equal(k, k_loop) and np.array_equal(v, v_loop)


@pytest.mark.parametrize("count", [1, 4, 5, 11, 12])
def test_token_gather_matches_a_per_token_loop(count):
    """Token t of a handoff payload is row t % BS of block table[t // BS] (kv_handoff.py:51-55)."""
    rng = np.random.default_rng(count)
    pool = rng.integers(0, 1 << 16, size=(2, 3, 5, 4, 2, 3), dtype=np.uint16)
    table = [3, 0, 4]
    dense = oracle.gather_tokens(pool, table, count)
    assert dense.shape == (2, 3, count, 2, 3)
    for t in range(count):
        assert np.array_equal(dense[:, :, t], pool[:, :, table[t // 4], t % 4]), f"token {t}"


@pytest.mark.parametrize("count", [1, 4, 6, 12])
def test_token_scatter_writes_exactly_the_payload_rows(count):
    """Scatter puts token t at row t % BS of block table[t // BS] (kv_handoff.py:112-118) and touches nothing else."""
    rng = np.random.default_rng(100 + count)
    pool = rng.integers(0, 1 << 16, size=(2, 3, 5, 4, 2, 3), dtype=np.uint16)
    dense = rng.integers(0, 1 << 16, size=(2, 3, count, 2, 3), dtype=np.uint16)
    table = [2, 4, 1]
    want = pool.copy()
    for t in range(count):
        want[:, :, table[t // 4], t % 4] = dense[:, :, t]
    oracle.scatter_tokens(pool, table, dense)
    assert np.array_equal(pool, want)
    assert np.array_equal(oracle.gather_tokens(pool, table, count), dense)
