"""KV handoff on a ROCm pool: the token-copy kernels (BF16 and FP8) and the engine's detach/resume.

The kernels are checked against the oracle's closed form of the reference's
copy (index_select over the block table, then a slice; kv_handoff.py:51-55)
and, for FP8, the oracle's codec (cpu_prefix_cache.py:20-28) applied to it.
The engine tests cover bench/test_engine_handoff.py's scenarios for both
payload formats.
"""

from dataclasses import replace

import numpy as np
import pytest
import torch

import kvx.engine.kv_handoff as kv_handoff
from engine_fixtures import cached_engine, params, step
from helpers import bf16_bits, finite_bf16_rows
from kvx import ops
from oracle import kvx_oracle as oracle

pytestmark = pytest.mark.gpu

SHAPES = [((2, 3, 300, 256, 2, 128), 300 * 256 - 77),  # > 128 blocks per call, ragged last block
          ((2, 2, 6, 256, 1, 4), 1),                   # the reference tests' geometry (generic kernels)
          ((2, 2, 6, 256, 1, 4), 513),
          ((2, 4, 9, 256, 8, 128), 2 * 256),           # exact blocks
          ((2, 2, 5, 256, 8, 128), 256 + 3)]


def random_pool(gpu, shape, seed, finite=False):
    pool = torch.empty(shape, dtype=torch.bfloat16, device=gpu)
    if finite:
        rows = finite_bf16_rows(pool.numel() // shape[-1], shape[-1], seed)
        pool.view(torch.int16).copy_(torch.from_numpy(rows.view(np.int16)).view(shape))
    else:
        pool.view(torch.int16).random_(-32768, 32768, generator=torch.Generator(device=gpu).manual_seed(seed))
    return pool


def table_for(shape, tokens, seed=1):
    need = -(-tokens // shape[3])
    return torch.randperm(shape[2], generator=torch.Generator().manual_seed(seed))[:need].tolist()


@pytest.mark.parametrize("shape,tokens", SHAPES)
def test_token_gather_and_scatter_match_the_index_select_formulation(gpu, shape, tokens):
    pool = random_pool(gpu, shape, tokens)
    table = table_for(shape, tokens)
    host = bf16_bits(pool)
    expect = oracle.gather_tokens(host, table, tokens)
    out = torch.empty((2, shape[1], tokens, *shape[-2:]), dtype=pool.dtype, device=gpu)
    ops.gather_tokens(pool, table, tokens, out)
    assert np.array_equal(bf16_bits(out), expect)
    pinned = torch.empty(out.shape, dtype=out.dtype, pin_memory=True)
    ops.gather_tokens(pool, table, tokens, pinned)  # straight into pinned host memory
    torch.cuda.synchronize()
    assert np.array_equal(pinned.view(torch.int16).numpy().view(np.uint16), expect)
    dest = torch.zeros_like(pool)
    ops.scatter_tokens(dest, table, tokens, out)
    want = np.zeros_like(host)
    oracle.scatter_tokens(want, table, expect)
    assert np.array_equal(bf16_bits(dest), want)  # exactly the tokens' rows change


@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape,tokens", SHAPES)
def test_fp8_token_gather_is_the_codec_of_the_gathered_tokens(gpu, shape, tokens, scale_dtype):
    pool = random_pool(gpu, shape, tokens + 7, finite=True)
    table = table_for(shape, tokens, seed=3)
    fp32 = scale_dtype == torch.float32
    codes, scales = oracle.quantize(oracle.gather_tokens(bf16_bits(pool), table, tokens), fp32)
    dense = (2, shape[1], tokens, *shape[-2:])
    for where in ("device", "pinned"):
        kw = {"device": gpu} if where == "device" else {"pin_memory": True}
        payload = torch.empty(dense, dtype=torch.float8_e4m3fn, **kw)
        scale = torch.empty((*dense[:-1], 1), dtype=scale_dtype, **kw)
        ops.gather_tokens_fp8(pool, table, tokens, payload, scale)
        torch.cuda.synchronize()
        assert np.array_equal(payload.cpu().view(torch.uint8).numpy(), codes), f"{where} payload"
        got_scales = scale.cpu().view(torch.int32 if fp32 else torch.int16).numpy()
        assert np.array_equal(got_scales, scales.view(np.int32 if fp32 else np.int16)), f"{where} scales"
    # Scatter (dequantise) into a fresh pool: exactly the tokens' rows change, to the oracle's dequantisation.
    dest = torch.zeros_like(pool)
    ops.scatter_tokens_fp8(dest, table, tokens, payload.to(gpu), scale.to(gpu))
    want = np.zeros(shape, dtype=np.uint16)
    oracle.scatter_tokens(want, table, oracle.dequantize(codes, scales, fp32))
    assert np.array_equal(bf16_bits(dest), want)


@pytest.mark.parametrize("first,end", [(0, 6), (1, 4), (5, 6)])
def test_token_copies_of_a_plane_range_are_that_slice_of_the_full_copy(gpu, first, end):
    shape, tokens = SHAPES[0]  # 6 (K/V, layer) planes, > 128 blocks, ragged last block
    pool = random_pool(gpu, shape, 11, finite=True)
    table = table_for(shape, tokens, seed=5)
    host = bf16_bits(pool)
    full = oracle.gather_tokens(host, table, tokens).reshape(-1, tokens, *shape[-2:])
    part = torch.empty((end - first, tokens, *shape[-2:]), dtype=pool.dtype, device=gpu)
    ops.gather_tokens(pool, table, tokens, part, planes=(first, end))
    assert np.array_equal(bf16_bits(part), full[first:end])
    payload = torch.empty(part.shape, dtype=torch.float8_e4m3fn, device=gpu)
    scale = torch.empty((*part.shape[:-1], 1), dtype=torch.float32, device=gpu)
    ops.gather_tokens_fp8(pool, table, tokens, payload, scale, planes=(first, end))
    codes, scales = oracle.quantize(full[first:end], True)
    assert np.array_equal(payload.cpu().view(torch.uint8).numpy(), codes)
    assert np.array_equal(scale.cpu().view(torch.int32).numpy(), scales.view(np.int32))
    # Scatters of the range write exactly those planes' token rows.
    want = np.zeros(shape, dtype=np.uint16)
    planes = want.reshape(-1, *shape[2:])
    for p in range(first, end):
        view = planes[p:p + 1].reshape(1, 1, *shape[2:])
        oracle.scatter_tokens(view, table, full[p:p + 1].reshape(1, 1, tokens, *shape[-2:]))
    dest = torch.zeros_like(pool)
    ops.scatter_tokens(dest, table, tokens, part, planes=(first, end))
    assert np.array_equal(bf16_bits(dest), want)
    dest.zero_()
    ops.scatter_tokens_fp8(dest, table, tokens, payload, scale, planes=(first, end))
    for p in range(first, end):
        view = planes[p:p + 1].reshape(1, 1, *shape[2:])
        back = oracle.dequantize(codes[p - first:p - first + 1], scales[p - first:p - first + 1], True)
        oracle.scatter_tokens(view, table, back.reshape(1, 1, tokens, *shape[-2:]))
    assert np.array_equal(bf16_bits(dest), want)


def test_token_copies_reject_short_tables_and_bad_buffers(gpu):
    pool = torch.zeros((2, 2, 4, 256, 1, 4), dtype=torch.bfloat16, device=gpu)
    out = torch.empty((2, 2, 300, 1, 4), dtype=pool.dtype, device=gpu)
    with pytest.raises(IndexError, match="need 2 blocks"):
        ops.gather_tokens(pool, [0], 300, out)
    with pytest.raises(IndexError, match="block id 9"):
        ops.gather_tokens(pool, [0, 9], 300, out)
    with pytest.raises(ValueError, match="contiguous"):
        ops.gather_tokens(pool, [0, 1], 299, out)
    with pytest.raises(ValueError, match="pinned"):
        ops.gather_tokens(pool, [0, 1], 300, torch.empty(out.shape, dtype=out.dtype))
    payload = torch.empty(out.shape, dtype=torch.float8_e4m3fn, device=gpu)
    scale = torch.empty((*out.shape[:-1], 1), dtype=torch.float32, device=gpu)
    with pytest.raises(IndexError, match="need 2 blocks"):
        ops.gather_tokens_fp8(pool, [3], 300, payload, scale)
    with pytest.raises(ValueError, match="twice"):
        ops.scatter_tokens_fp8(pool, [1, 1], 300, payload, scale)
    with pytest.raises(ValueError, match="scatter reads device memory"):
        ops.scatter_tokens_fp8(pool, [0, 1], 300, payload.cpu().pin_memory(), scale)


def running_request(gpu, length=5, max_tokens=3, batches=None, **engine):
    """An engine whose only request has been prefilled (one completion token, one pending)."""
    engine_ = cached_engine(gpu, batches or [[10]], **engine)
    request_id = engine_.add_request([1] * length, params(max_tokens=max_tokens))
    step(engine_)
    return engine_, request_id


FORMATS = [pytest.param({}, id="bf16"), pytest.param({"fp8": True}, id="fp8-fp32"),
           pytest.param({"fp8": True, "scale_dtype": torch.bfloat16}, id="fp8-bf16")]


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("length", [255, 256, 257])
def test_detach_then_resume_carries_the_kv_and_decode_continues(gpu, length, fmt):
    source, source_id = running_request(gpu, length=length)
    pool = source.model_runner.kv_cache
    table = source.scheduler.running[0].block_table.copy()
    snapshot = source.detach_request(source_id, **fmt)
    tokens = oracle.gather_tokens(bf16_bits(pool), table, length)
    if fmt:
        fp32 = fmt.get("scale_dtype", torch.float32) == torch.float32
        codes, scales = oracle.quantize(tokens, fp32)
        assert np.array_equal(snapshot.kv.view(torch.uint8).numpy(), codes)
        assert np.array_equal(snapshot.scale.view(torch.uint8).numpy(), scales.view(np.uint8))
        assert snapshot.payload_bytes == codes.nbytes + scales.nbytes  # about half of the BF16 payload
        tokens = oracle.dequantize(codes, scales, fp32)
    else:
        assert np.array_equal(snapshot.kv.view(torch.int16).numpy().view(np.uint16), tokens)
    assert snapshot.token_ids == [1] * length + [10] and snapshot.num_cached_tokens == length
    assert source.scheduler.block_manager.used_block_ids == set(table)  # the source keeps its blocks
    destination = cached_engine(gpu, [[11], [12]])
    destination.model_runner.kv_cache.fill_(-1)
    destination_id = destination.resume_request(snapshot)
    seq = destination.scheduler.running[0]
    assert destination_id == seq.seq_id != source_id
    assert not seq.is_prefill and seq.num_cached_tokens == length and seq.completion_token_ids == [10]
    assert len(seq.block_table) == -(-length // 256)
    assert np.array_equal(oracle.gather_tokens(bf16_bits(destination.model_runner.kv_cache), seq.block_table,
                                               length), tokens)
    assert kv_handoff.verify_imported_kv(destination.model_runner, seq, snapshot)
    manager = destination.scheduler.block_manager
    assert (manager.blocks[seq.block_table[0]].hash != -1) == (length >= 256)  # full blocks are published
    source.release_detached_request(source_id)
    assert step(destination).num_tokens == -1
    final = step(destination)
    assert final.outputs == [(destination_id, [10, 11, 12])]
    assert all(not prefill for prefill, _ in destination.model_runner.calls)
    assert not manager.used_block_ids


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("group", [1, 3])
def test_handoff_in_plane_groups_carries_the_kv(gpu, fmt, group, monkeypatch):
    """Export and import move the payload through staging a group of planes at a time.

    The staging is shrunk to `group` planes of this 700-token request, so the pool's 4 planes go in groups of
    1 or of 3 and 1."""
    source, source_id = running_request(gpu, length=700, budget=1024)
    pool = source.model_runner.kv_cache
    row = pool.shape[-1] * (2 if not fmt else 1) + (0 if not fmt else fmt.get("scale_dtype", torch.float32).itemsize)
    monkeypatch.setattr(kv_handoff, "_STAGING_BYTES", group * 700 * pool.shape[-2] * row)
    assert len(kv_handoff._plane_groups(pool, 700, torch.bfloat16 if not fmt else torch.float8_e4m3fn,
                                        fmt.get("scale_dtype", torch.float32) if fmt else None)) == -(-4 // group)
    table = source.scheduler.running[0].block_table.copy()
    tokens = oracle.gather_tokens(bf16_bits(pool), table, 700)
    snapshot = source.detach_request(source_id, **fmt)
    if fmt:
        fp32 = fmt.get("scale_dtype", torch.float32) == torch.float32
        codes, scales = oracle.quantize(tokens, fp32)
        assert np.array_equal(snapshot.kv.view(torch.uint8).numpy(), codes)
        assert np.array_equal(snapshot.scale.view(torch.uint8).numpy(), scales.view(np.uint8))
        tokens = oracle.dequantize(codes, scales, fp32)
    else:
        assert np.array_equal(snapshot.kv.view(torch.int16).numpy().view(np.uint16), tokens)
    destination = cached_engine(gpu, [[11]], budget=1024)
    destination.model_runner.kv_cache.fill_(-1)
    destination.resume_request(snapshot)
    seq = destination.scheduler.running[0]
    assert np.array_equal(oracle.gather_tokens(bf16_bits(destination.model_runner.kv_cache), seq.block_table, 700),
                          tokens)


@pytest.mark.parametrize("fmt", FORMATS)
def test_import_leaves_the_payload_free_for_reuse(gpu, fmt):
    """Once import_kv returns, the snapshot's pinned memory may be dropped and reused at once.

    import_kv is called directly, not through resume_request, so nothing
    but import_kv itself orders the payload's last read before the reuse.
    """
    source, source_id = running_request(gpu, length=700, budget=1024)
    snapshot = source.detach_request(source_id, **fmt)
    expected = kv_handoff.KVSnapshot(**{**snapshot.__dict__, "kv": snapshot.kv.clone(),
                                        "scale": None if snapshot.scale is None else snapshot.scale.clone()})
    destination = cached_engine(gpu, [[11]])
    seq = kv_handoff.import_kv(destination.model_runner, destination.scheduler.block_manager, snapshot)
    nbytes = snapshot.payload_bytes
    del snapshot
    for _ in range(4):  # the host allocator hands the freed pinned blocks out again
        junk = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
        junk.fill_(0x5A)
    assert kv_handoff.verify_imported_kv(destination.model_runner, seq, expected)


def test_reattach_continues_the_original_request(gpu):
    source, request_id = running_request(gpu, batches=[[10], [11], [12]])
    source.detach_request(request_id)
    assert source.is_finished()
    assert source.reattach_request(request_id) == request_id
    assert step(source).outputs == []
    assert step(source).outputs == [(request_id, [10, 11, 12])]
    assert not source.scheduler.block_manager.used_block_ids


def test_other_requests_progress_while_one_is_detached(gpu):
    source, request_id = running_request(gpu, batches=[[10], [20]])
    blocks = set(source.scheduler.running[0].block_table)
    source.detach_request(request_id)
    other = source.add_request([2], params(max_tokens=1))
    assert step(source).outputs == [(other, [20])]
    with pytest.raises(ValueError, match="already detached"):
        source.detach_request(request_id)
    assert source.scheduler.block_manager.used_block_ids == blocks
    source.release_detached_request(request_id)
    assert not source.scheduler.block_manager.used_block_ids
    with pytest.raises(KeyError):
        source.release_detached_request(request_id)
    with pytest.raises(KeyError):
        source.reattach_request(request_id)


def test_a_failed_export_keeps_the_request_running(gpu, monkeypatch):
    source, request_id = running_request(gpu)
    seq = source.scheduler.running[0]
    blocks = set(seq.block_table)

    def fail(*args, **kwargs):
        raise RuntimeError("export failed")

    monkeypatch.setattr(kv_handoff, "export_kv", fail)
    with pytest.raises(RuntimeError, match="export failed"):
        source.detach_request(request_id)
    assert list(source.scheduler.running) == [seq]
    assert source.scheduler.block_manager.used_block_ids == blocks


def test_only_running_requests_between_steps_can_be_detached(gpu):
    source = cached_engine(gpu, [[90], [91], [10]], budget=2)
    request_id = source.add_request([1] * 5, params(max_tokens=1))
    with pytest.raises(ValueError, match="handoff boundary"):
        source.detach_request(request_id)  # still waiting
    step(source)
    with pytest.raises(ValueError, match="handoff boundary"):
        source.detach_request(request_id)  # partially prefilled
    step(source)
    step(source)
    for rid in (request_id, -1):  # finished, unknown
        with pytest.raises(ValueError, match="handoff boundary"):
            source.detach_request(rid)
    assert not source.scheduler.block_manager.used_block_ids


@pytest.mark.parametrize("mismatch", ["dtype", "block_size", "shape", "finished", "fp8_without_scale"])
def test_resume_rejects_a_snapshot_that_does_not_fit_without_allocating(gpu, mismatch):
    source, request_id = running_request(gpu)
    snapshot = source.detach_request(request_id, fp8=mismatch == "fp8_without_scale")
    changed = {"dtype": {"kv": snapshot.kv.to(torch.float16)}, "block_size": {"block_size": 512},
               "shape": {"kv": snapshot.kv[:, :, :-1]}, "finished": {"max_tokens": 1},
               "fp8_without_scale": {"scale": None}}[mismatch]
    destination = cached_engine(gpu, [])
    with pytest.raises(ValueError):
        destination.resume_request(replace(snapshot, **changed))
    assert destination.is_finished() and not destination.scheduler.block_manager.used_block_ids


def test_resume_without_free_blocks_leaves_the_destination_as_it_was(gpu):
    source, source_id = running_request(gpu, length=257, batches=[[10], [11], [12]])
    snapshot = source.detach_request(source_id)
    destination = cached_engine(gpu, [[20]], num_blocks=1)
    existing_id = destination.add_request([2], params(max_tokens=2))
    step(destination)
    existing = destination.scheduler.running[0]
    with pytest.raises(MemoryError):
        destination.resume_request(snapshot)
    assert list(destination.scheduler.running) == [existing] and existing.seq_id == existing_id
    assert destination.scheduler.block_manager.used_block_ids == set(existing.block_table)
    assert source.reattach_request(source_id) == source_id


def test_a_failed_import_releases_the_blocks_it_took(gpu, monkeypatch):
    source, request_id = running_request(gpu, length=256)
    snapshot = source.detach_request(request_id)
    destination = cached_engine(gpu, [])
    manager = destination.scheduler.block_manager

    def fail(seq):
        raise RuntimeError("import failed")

    monkeypatch.setattr(manager, "hash_blocks", fail)
    with pytest.raises(RuntimeError, match="import failed"):
        destination.resume_request(snapshot)
    assert destination.is_finished() and not manager.used_block_ids and len(manager.free_block_ids) == 16


def test_exit_releases_detached_requests(gpu):
    source, request_id = running_request(gpu)
    source.detach_request(request_id)
    manager = source.scheduler.block_manager
    source.exit()
    assert not manager.used_block_ids
    assert source.model_runner.calls[-1] == "exit"
