"""Parity of libkvx's HIP kernels (through the C ABI) with the oracle and the golden fixtures.

Bar: bit-exact codes, scales and dequantised bf16 for every finite row;
byte-exact block copies and paged writes (NaN bit patterns included).
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import bf16_bits, bf16_tensor, finite_bf16_rows, student_t_rows, u8
from kvx import ops
from oracle import kvx_oracle as oracle

pytestmark = pytest.mark.gpu

GOLDEN = np.load(Path(__file__).resolve().parent / "golden" / "fp8_codec.npz")


def quantize_on_device(x_bits: np.ndarray, scale_dtype, device):
    x = bf16_tensor(x_bits, device)
    payload = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=device)
    scale = torch.empty((*x.shape[:-1], 1), dtype=scale_dtype, device=device)
    ops.fp8_quantize(x, payload, scale)
    return payload, scale


def test_selftest_hardware_conversions_and_division(gpu):
    counters = ops.selftest(gpu)
    print(counters)
    assert counters["e4m3_encode_mismatch"] == 0
    assert counters["bf16_round_mismatch"] == 0
    assert counters["nan_not_preserved"] == 0
    assert counters["division_mismatch"] == 0
    assert counters["e4m3_decode_mismatch"] == 0
    assert counters["encode_inputs_2p20"] == 4096  # all 2^32 fp32 patterns swept
    assert counters["division_pairs_2p20"] == 1024  # all 2^30 significand pairs
    assert counters["decode_sweeps"] == 1


@pytest.mark.parametrize("hd", [128, 64, 256, 4])
@pytest.mark.parametrize("scale", ["fp32", "bf16"])
def test_codec_matches_golden_fixtures(gpu, hd, scale):
    dtype = torch.float32 if scale == "fp32" else torch.bfloat16
    payload, s = quantize_on_device(GOLDEN[f"x_hd{hd}"], dtype, gpu)
    torch.cuda.synchronize()
    assert np.array_equal(u8(payload), GOLDEN[f"codes_hd{hd}_{scale}"])
    assert np.array_equal(u8(s), GOLDEN[f"scale_hd{hd}_{scale}"].view(np.uint8))
    codes = torch.from_numpy(GOLDEN[f"codes_hd{hd}_{scale}"]).view(torch.float8_e4m3fn).to(gpu)
    golden_scale = GOLDEN[f"scale_hd{hd}_{scale}"]
    s_in = (torch.from_numpy(golden_scale) if scale == "fp32"
            else torch.from_numpy(golden_scale.view(np.int16)).view(torch.bfloat16)).to(gpu)
    back = torch.empty(codes.shape, dtype=torch.bfloat16, device=gpu)
    ops.fp8_dequantize(codes, s_in, back)
    assert np.array_equal(bf16_bits(back), GOLDEN[f"back_hd{hd}_{scale}"])


@pytest.mark.parametrize("hd", [128, 64, 256, 4, 96, 8])
@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.bfloat16])
def test_codec_matches_oracle_on_random_finite_rows(gpu, hd, scale_dtype):
    fp32 = scale_dtype == torch.float32
    # 8195 rows: not a multiple of any tile height, so the ragged last tile is exercised.
    x = np.concatenate([finite_bf16_rows(4096, hd, seed=hd), student_t_rows(4099, hd, seed=hd + 1)])
    payload, s = quantize_on_device(x, scale_dtype, gpu)
    codes, scales = oracle.quantize(x, fp32)
    got_codes, got_scales = u8(payload), u8(s)
    bad = np.argwhere(got_codes != codes)
    assert bad.size == 0, f"{len(bad)} code mismatches, first at row/col {bad[0]}"
    assert np.array_equal(got_scales, scales.view(np.uint8))
    back = torch.empty(payload.shape, dtype=torch.bfloat16, device=gpu)
    ops.fp8_dequantize(payload, s, back)
    assert np.array_equal(bf16_bits(back), oracle.dequantize(codes, scales, fp32))


def test_rows_with_nan_or_inf_keep_their_class(gpu):
    rows = torch.tensor([[1.0, float("nan"), 2.0, 3.0] * 32,
                         [1.0, float("inf"), -2.0, 0.0] * 32,
                         [-float("inf"), 1.0, 5.0, -0.0] * 32], dtype=torch.bfloat16)
    payload, s = quantize_on_device(bf16_bits(rows), torch.float32, gpu)
    codes, scales = u8(payload).reshape(3, 128), s.cpu().numpy().ravel()
    assert np.isnan(scales[0]) and np.all((codes[0] & 0x7F) == 0x7F)
    assert np.isinf(scales[1]) and np.isinf(scales[2])
    # Finite values over an infinite scale are signed zeros; inf/inf is NaN.
    assert codes[1, 2] == 0x80 and codes[1, 3] == 0x00 and (codes[1, 1] & 0x7F) == 0x7F
    assert codes[2, 1] == 0x00 and codes[2, 3] == 0x80 and (codes[2, 0] & 0x7F) == 0x7F


def test_codec_reads_strided_pool_views(gpu):
    g = torch.Generator(device=gpu).manual_seed(4)
    pool = torch.randn((2, 3, 5, 16, 2, 128), generator=g, device=gpu).to(torch.bfloat16)
    for block in (0, 2, 4):
        source = pool[:, :, block]
        payload = torch.empty(source.shape, dtype=torch.float8_e4m3fn, device=gpu)
        scale = torch.empty((*source.shape[:-1], 1), dtype=torch.float32, device=gpu)
        ops.fp8_quantize(source, payload, scale)
        codes, scales = oracle.quantize(bf16_bits(source), True)
        assert np.array_equal(u8(payload), codes) and np.array_equal(u8(scale), scales.view(np.uint8))
        target = torch.zeros_like(pool)
        ops.fp8_dequantize(payload, scale, target[:, :, block])
        assert np.array_equal(bf16_bits(target[:, :, block]), oracle.dequantize(codes, scales, True))
        others = [b for b in range(5) if b != block]
        assert torch.count_nonzero(target[:, :, others]) == 0
    # A view whose leading dims do not collapse (a transposed head axis) is split per plane.
    t = pool.permute(0, 1, 2, 4, 3, 5)[:, :, 1]
    payload = torch.empty(t.shape, dtype=torch.float8_e4m3fn, device=gpu)
    scale = torch.empty((*t.shape[:-1], 1), dtype=torch.bfloat16, device=gpu)
    ops.fp8_quantize(t, payload, scale)
    codes, scales = oracle.quantize(bf16_bits(t), False)
    assert np.array_equal(u8(payload), codes) and np.array_equal(u8(scale), scales.view(np.uint8))


def make_pool(device, layers=4, blocks=12, bs=256, heads=8, hd=128, seed=0):
    g = torch.Generator(device=device).manual_seed(seed)
    t = torch.randn((2, layers, blocks, bs, heads, hd), generator=g, device=device)
    chi = torch.randn((2, layers, blocks, bs, heads, hd), generator=g, device=device).square()
    return (t / chi.add_(1e-3).sqrt() * 0.5).to(torch.bfloat16)


# The vector kernels cover head_dim 64, 128 and 256 in tiles of 4-16 rows; the
# last three geometries leave a ragged last tile in every plane (15, 7 and 6 rows).
# heads=1, hd=128 is one tensor-parallel rank's share of Qwen3-8B at TP=8.
@pytest.mark.parametrize("geometry", [dict(), dict(layers=2, blocks=6, bs=256, heads=1, hd=4),
                                      dict(layers=3, blocks=6, bs=256, heads=1, hd=128),
                                      dict(layers=3, blocks=7, bs=32, heads=3, hd=96),
                                      dict(layers=2, blocks=6, bs=5, heads=3, hd=128),
                                      dict(layers=1, blocks=6, bs=7, heads=1, hd=64),
                                      dict(layers=2, blocks=6, bs=3, heads=2, hd=256)])
@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.bfloat16])
def test_fp8_block_save_and_restore_match_the_oracle(gpu, geometry, scale_dtype):
    pool = make_pool(gpu, **geometry)
    fp32 = scale_dtype == torch.float32
    layout = ops.pool_layout(pool, scale_dtype)
    logical, offset, stride = ops.entry_layout(layout, ops.FORMAT_FP8)
    nb = pool.shape[2]
    sources = list(dict.fromkeys([3, 0, nb - 1, 5]))  # distinct: one call may not name a destination twice
    dests = list(dict.fromkeys([1, 2, 4, nb - 2]))[:len(sources)]
    staging = torch.full((len(sources) * stride,), 0xAB, dtype=torch.uint8, device=gpu)
    entries = [staging.data_ptr() + i * stride for i in range(len(sources))]
    ops.save_blocks(pool, sources, entries, ops.FORMAT_FP8, scale_dtype)
    host_pool = bf16_bits(pool)
    staged = u8(staging).reshape(len(sources), stride)
    rows = layout.planes * layout.plane_rows
    sbytes = 4 if fp32 else 2
    for i, b in enumerate(sources):
        codes, scales = oracle.save_block_fp8(host_pool, b, fp32)
        assert np.array_equal(staged[i, :codes.size], codes.ravel()), f"payload of block {b}"
        assert np.array_equal(staged[i, offset:offset + rows * sbytes], scales.view(np.uint8).ravel())
    canary = pool.clone()
    ops.restore_blocks(pool, dests, entries, ops.FORMAT_FP8, scale_dtype)
    after = bf16_bits(pool)
    for i, (b, d) in enumerate(zip(sources, dests)):
        codes, scales = oracle.save_block_fp8(host_pool, b, fp32)
        expect = oracle.dequantize(codes, scales, fp32)
        assert np.array_equal(after[:, :, d], expect), f"restore of block {b} into {d}"
    untouched = [b for b in range(nb) if b not in dests]
    assert torch.equal(pool[:, :, untouched], canary[:, :, untouched])


def ulp_distance(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """|a - b| in units in the last place, for finite non-negative floats of one dtype (ordered as integers)."""
    itype = torch.int32 if a.dtype == torch.float32 else torch.int16
    return (a.view(itype).to(torch.int64) - b.view(itype).to(torch.int64)).abs()


@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.bfloat16])
def test_fp8_kernels_match_the_reference_torch_chain_on_the_gpu(gpu, scale_dtype):
    """Same seeded blocks through kvx and through the reference's own torch ops (cpu_prefix_cache.py:20-28)
    on this GPU: scales within 1 ulp, payload bit-exact given identical scales, restore bit-exact."""
    from oracle import torch_path

    pool = make_pool(gpu, layers=36, blocks=4)  # Qwen3-8B block shape, Student-t values
    g = torch.Generator(device=gpu).manual_seed(9)
    bits = torch.randint(-32768, 32768, pool[:, :, 3].shape, generator=g, device=gpu, dtype=torch.int32)
    bits = torch.where((bits & 0x7F80) == 0x7F80, bits & ~0x4000, bits)  # finite bf16 bit patterns only
    pool[:, :, 3] = bits.to(torch.int16).view(torch.bfloat16)
    for b in range(4):
        source = pool[:, :, b]
        ours_p = torch.empty(source.shape, dtype=torch.float8_e4m3fn, device=gpu)
        ours_s = torch.empty((*source.shape[:-1], 1), dtype=scale_dtype, device=gpu)
        ops.fp8_quantize(source, ours_p, ours_s)
        ref_p, ref_s = torch.empty_like(ours_p), torch.empty_like(ours_s)
        torch_path.fp8_quantize(source, ref_p, ref_s)
        assert int(ulp_distance(ours_s, ref_s).max()) <= 1, f"block {b}: scales more than 1 ulp apart"
        same = (ours_s == ref_s).squeeze(-1)
        assert torch.equal(ours_p.view(torch.uint8)[same], ref_p.view(torch.uint8)[same]), f"block {b}"
        # Where a scale differs, the reference's payload formula with our scale gives our codes.
        if not bool(same.all()):
            redo = torch.empty_like(ref_p)
            redo.copy_((source.float() / ours_s.float()).clamp_(-448.0, 448.0))
            assert torch.equal(ours_p.view(torch.uint8), redo.view(torch.uint8)), f"block {b}"
        ours_t, ref_t = torch.empty_like(source), torch.empty_like(source)
        ops.fp8_dequantize(ours_p, ours_s, ours_t)
        torch_path.fp8_dequantize(ours_p, ours_s, ref_t)
        assert torch.equal(ours_t.view(torch.int16), ref_t.view(torch.int16)), f"block {b} restore"


def byte_pattern_pool(device, shape=(2, 3, 9, 256, 2, 64)):
    """Pool bytes i % 256: every bf16 bit pattern class, NaNs included (test_cpu_prefix_cache.py:15-18)."""
    pool = torch.empty(shape, dtype=torch.bfloat16, device=device)
    raw = torch.arange(pool.numel() * 2, dtype=torch.int64, device=device).remainder(256).to(torch.uint8)
    pool.view(torch.uint8).copy_(raw.view(pool.view(torch.uint8).shape))
    return pool


@pytest.mark.parametrize("shape", [(2, 3, 9, 256, 2, 64), (2, 2, 5, 256, 1, 4), (2, 1, 4, 3, 1, 3),
                                   (2, 2, 5, 16, 1, 8), (2, 2, 6, 24, 3, 8)])
def test_bf16_block_gather_and_scatter_are_byte_exact(gpu, shape):
    # Planes of 64 KiB and 2 KiB fill whole 1 KiB copy tiles; 256 B and 1,152 B planes end in a partial tile; 18 B
    # planes take the 2-byte generic kernel.
    pool = byte_pattern_pool(gpu, shape)
    layout = ops.pool_layout(pool)
    _, _, stride = ops.entry_layout(layout, ops.FORMAT_RAW)
    nb = shape[2]
    dests = list(dict.fromkeys([1, 3, nb - 2]))  # distinct: one call may not name a destination twice
    sources = [nb - 1, 0, 2][:len(dests)]
    staging = torch.zeros(len(sources) * stride, dtype=torch.uint8, device=gpu)
    entries = [staging.data_ptr() + i * stride for i in range(len(sources))]
    before = u8(pool).reshape(pool.shape + (2,))
    ops.save_blocks(pool, sources, entries, ops.FORMAT_RAW)
    staged = u8(staging).reshape(len(sources), stride)
    block_bytes = before[:, :, 0].size
    for i, b in enumerate(sources):
        assert np.array_equal(staged[i, :block_bytes], np.ascontiguousarray(before[:, :, b]).ravel())
    ops.restore_blocks(pool, dests, entries, ops.FORMAT_RAW)
    after = u8(pool).reshape(pool.shape + (2,))
    expect = before.copy()
    for b, d in zip(sources, dests):
        expect[:, :, d] = before[:, :, b]
    assert np.array_equal(after, expect)


def test_block_copies_to_pinned_host_entries(gpu):
    # Entries may live in mapped pinned host memory: the kernels then move the
    # block across the host link themselves (no staging, no DMA engine).
    pool = make_pool(gpu, layers=2, blocks=4)
    layout = ops.pool_layout(pool, torch.float32)
    _, offset, stride = ops.entry_layout(layout, ops.FORMAT_FP8)
    host = torch.zeros(2 * stride, dtype=torch.uint8, pin_memory=True)
    entries = [host.data_ptr(), host.data_ptr() + stride]
    ops.save_blocks(pool, [2, 0], entries, ops.FORMAT_FP8, torch.float32)
    torch.cuda.synchronize()
    host_pool = bf16_bits(pool)
    for i, b in enumerate([2, 0]):
        codes, scales = oracle.save_block_fp8(host_pool, b, True)
        assert np.array_equal(host.numpy()[i * stride:i * stride + codes.size], codes.ravel())
    ops.restore_blocks(pool, [1, 3], entries, ops.FORMAT_FP8, torch.float32)
    after = bf16_bits(pool)
    for b, d in zip([2, 0], [1, 3]):
        codes, scales = oracle.save_block_fp8(host_pool, b, True)
        assert np.array_equal(after[:, :, d], oracle.dequantize(codes, scales, True))


def fused_qkv(n, q_heads, kv_heads, hd, device, seed):
    g = torch.Generator(device=device).manual_seed(seed)
    qkv = torch.randn((n, (q_heads + 2 * kv_heads) * hd), generator=g, device=device).to(torch.bfloat16)
    q, k, v = qkv.split([q_heads * hd, kv_heads * hd, kv_heads * hd], dim=-1)
    return k.contiguous().view(n, kv_heads, hd), v.view(n, kv_heads, hd)  # V stays a strided view


@pytest.mark.parametrize("heads,hd", [(8, 128), (1, 4), (3, 96), (2, 64)])
def test_store_kvcache_matches_the_closed_form(gpu, heads, hd):
    n, num_blocks, bs = 1000, 8, 256
    key, value = fused_qkv(n, 32, heads, hd, gpu, seed=heads)
    assert value.stride(0) == (32 + 2 * heads) * hd  # the fused QKV row stride
    pool = torch.empty((2, 1, num_blocks, bs, heads, hd), dtype=torch.bfloat16, device=gpu)
    pool[0].fill_(-7.0)  # distinct canaries for the K and V caches
    pool[1].fill_(-5.0)
    k_cache, v_cache = pool[0, 0], pool[1, 0]
    rng = np.random.default_rng(heads)
    slots = rng.permutation(num_blocks * bs)[:n].astype(np.int32)
    slots[rng.random(n) < 0.1] = -1  # graph padding
    slots[5] = num_blocks * bs + 3   # outside the cache: written nowhere
    mapping = torch.from_numpy(slots).to(gpu)
    k_ref, v_ref = bf16_bits(k_cache), bf16_bits(v_cache)  # the caches before the kernel
    oracle.store_kvcache(bf16_bits(key), bf16_bits(value), k_ref, v_ref, slots)
    ops.store_kvcache(key, value, k_cache, v_cache, mapping)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(k_cache), k_ref) and np.array_equal(bf16_bits(v_cache), v_ref)
    untouched = num_blocks * bs * heads * hd - int(((slots >= 0) & (slots < num_blocks * bs)).sum()) * heads * hd
    for cache, canary in ((k_cache, -7.0), (v_cache, -5.0)):
        assert (bf16_bits(cache) == bf16_bits(torch.tensor(canary, dtype=torch.bfloat16))).sum() == untouched


def test_store_kvcache_replays_inside_a_hip_graph(gpu):
    # Decode captures store_kvcache in a graph (model_runner.py:244-250); slots change between replays.
    n, heads, hd, slots_total = 64, 8, 128, 4 * 256
    key = torch.zeros((n, heads, hd), dtype=torch.bfloat16, device=gpu)
    value = torch.zeros_like(key)
    pool = torch.zeros((2, 1, 4, 256, heads, hd), dtype=torch.bfloat16, device=gpu)
    mapping = torch.full((n,), -1, dtype=torch.int32, device=gpu)
    stream = torch.cuda.Stream(gpu)
    stream.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(stream):
        ops.store_kvcache(key, value, pool[0, 0], pool[1, 0], mapping)  # warm-up outside capture
    torch.cuda.current_stream(gpu).wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.store_kvcache(key, value, pool[0, 0], pool[1, 0], mapping)
    rng = np.random.default_rng(9)
    expect_k = np.zeros((slots_total, heads * hd), dtype=np.uint16)
    expect_v = expect_k.copy()
    for step in range(4):
        key.copy_(torch.randn(key.shape, device=gpu))
        value.copy_(torch.randn(value.shape, device=gpu))
        slots = rng.permutation(slots_total)[:n].astype(np.int32)
        slots[:step] = -1
        mapping.copy_(torch.from_numpy(slots))
        graph.replay()
        torch.cuda.synchronize()
        oracle.store_kvcache(bf16_bits(key), bf16_bits(value), expect_k, expect_v, slots)
        assert np.array_equal(bf16_bits(pool[0, 0]).reshape(slots_total, -1), expect_k), step
        assert np.array_equal(bf16_bits(pool[1, 0]).reshape(slots_total, -1), expect_v), step


@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.bfloat16])
def test_fp8_block_save_and_restore_replay_inside_a_hip_graph(gpu, scale_dtype):
    # Block lists travel in the kernel arguments, so a captured save + restore
    # replays with no host work; each replay must match the eager result.
    pool = make_pool(gpu, layers=3, blocks=6)
    layout = ops.pool_layout(pool, scale_dtype)
    _, offset, stride = ops.entry_layout(layout, ops.FORMAT_FP8)
    sources, dests = [4, 1], [0, 5]
    staging = torch.zeros(len(sources) * stride, dtype=torch.uint8, device=gpu)
    entries = [staging.data_ptr() + i * stride for i in range(len(sources))]

    def step():
        ops.save_blocks(pool, sources, entries, ops.FORMAT_FP8, scale_dtype)
        ops.restore_blocks(pool, dests, entries, ops.FORMAT_FP8, scale_dtype)

    stream = torch.cuda.Stream(gpu)
    stream.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(stream):
        step()  # warm-up outside capture
    torch.cuda.current_stream(gpu).wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    g = torch.Generator(device=gpu).manual_seed(3)
    for replay in range(4):
        fresh = torch.randn(pool[:, :, sources].shape, generator=g, device=gpu) * (replay + 1)
        pool[:, :, sources] = fresh.to(torch.bfloat16)  # eager work between replays
        torch.cuda.synchronize()
        before = pool.clone()
        graph.replay()
        torch.cuda.synchronize()
        replayed, replayed_entries = pool.clone(), staging.clone()
        pool.copy_(before)
        step()
        torch.cuda.synchronize()
        assert torch.equal(replayed.view(torch.int16), pool.view(torch.int16)), replay
        assert torch.equal(replayed_entries, staging), replay
        host_pool = bf16_bits(before)
        for b, d in zip(sources, dests):
            codes, scales = oracle.save_block_fp8(host_pool, b, scale_dtype == torch.float32)
            expect = oracle.dequantize(codes, scales, scale_dtype == torch.float32)
            assert np.array_equal(bf16_bits(replayed[:, :, d]), expect), (replay, b)


def test_empty_and_all_padding_inputs_are_no_ops(gpu):
    pool = make_pool(gpu, layers=2, blocks=3)
    before = pool.clone()
    heads, hd = pool.shape[4], pool.shape[5]
    key = torch.randn((5, heads, hd), device=gpu).to(torch.bfloat16)
    # No tokens; only padding slots (-1, decode graph padding); only slots outside the cache.
    ops.store_kvcache(key[:0], key[:0], pool[0, 0], pool[1, 0], torch.empty(0, dtype=torch.int32, device=gpu))
    ops.store_kvcache(key, key, pool[0, 0], pool[1, 0], torch.full((5,), -1, dtype=torch.int32, device=gpu))
    outside = pool.shape[2] * pool.shape[3]
    ops.store_kvcache(key, key, pool[0, 0], pool[1, 0],
                      torch.arange(outside, outside + 5, dtype=torch.int32, device=gpu))
    # Empty block lists and zero-row codec tensors.
    ops.save_blocks(pool, [], [], ops.FORMAT_FP8, torch.float32)
    ops.restore_blocks(pool, [], [], ops.FORMAT_RAW)
    rows = pool[0, 0, 0, :0]
    ops.fp8_quantize(rows, torch.empty(rows.shape, dtype=torch.float8_e4m3fn, device=gpu),
                     torch.empty((*rows.shape[:-1], 1), dtype=torch.float32, device=gpu))
    # Zero-token handoff copies.
    dense = torch.empty((2, pool.shape[1], 0, heads, hd), dtype=pool.dtype, device=gpu)
    ops.gather_tokens(pool, [], 0, dense)
    ops.scatter_tokens(pool, [], 0, dense)
    torch.cuda.synchronize()
    assert torch.equal(pool.view(torch.int16), before.view(torch.int16))


def test_calls_longer_than_one_launch_cover_every_block(gpu):
    # A launch covers at most 128 blocks and longer calls are split: 150 blocks
    # (a ragged second launch of 22) through the FP8 codec and the token copies.
    pool = make_pool(gpu, layers=2, blocks=320, bs=4, heads=2, hd=128, seed=3)
    nb, bs = pool.shape[2], pool.shape[3]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(11)).tolist()
    sources, dests = perm[:150], perm[150:300]
    src_bits = bf16_bits(pool)
    untouched = [b for b in range(nb) if b not in set(dests)]
    for scale_dtype in (torch.float32, torch.bfloat16):
        fp32 = scale_dtype == torch.float32
        layout = ops.pool_layout(pool, scale_dtype)
        _, _, stride = ops.entry_layout(layout, ops.FORMAT_FP8)
        staging = torch.full((len(sources) * stride,), 0xAB, dtype=torch.uint8, device=gpu)
        entries = [staging.data_ptr() + i * stride for i in range(len(sources))]
        target = pool.clone()
        ops.save_blocks(pool, sources, entries, ops.FORMAT_FP8, scale_dtype)
        ops.restore_blocks(target, dests, entries, ops.FORMAT_FP8, scale_dtype)
        after = bf16_bits(target)
        for b, d in zip(sources, dests):
            codes, scales = oracle.save_block_fp8(src_bits, b, fp32)
            assert np.array_equal(after[:, :, d], oracle.dequantize(codes, scales, fp32)), (scale_dtype, b, d)
        assert np.array_equal(after[:, :, untouched], src_bits[:, :, untouched])
    # Token copies: 597 tokens span 150 blocks, the last holding one token.
    tokens = len(sources) * bs - 3
    dense = torch.empty((2, pool.shape[1], tokens, *pool.shape[-2:]), dtype=pool.dtype, device=gpu)
    ops.gather_tokens(pool, sources, tokens, dense)
    expect = src_bits[:, :, sources].reshape(2, pool.shape[1], len(sources) * bs, *pool.shape[-2:])[:, :, :tokens]
    assert np.array_equal(bf16_bits(dense), expect)
    target = pool.clone()
    ops.scatter_tokens(target, dests, tokens, dense)
    after = bf16_bits(target)
    written = after[:, :, dests].reshape(2, pool.shape[1], len(dests) * bs, *pool.shape[-2:])
    assert np.array_equal(written[:, :, :tokens], expect)
    assert np.array_equal(after[:, :, dests[-1], 1:], src_bits[:, :, dests[-1], 1:])
    assert np.array_equal(after[:, :, untouched], src_bits[:, :, untouched])
