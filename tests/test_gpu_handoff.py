"""KV handoff (detach/export, resume/import) over libkvx's token copies.

Restates bench/test_engine_handoff.py on a ROCm pool, and checks the token
gather/scatter kernels against the reference's own formulation of the same
copy (index_select over the block table, then a slice; kv_handoff.py:51-55)
evaluated in numpy.
"""

from dataclasses import replace
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import kvx.engine.kv_handoff as kv_handoff
from engine_fixtures import cached_engine, params
from kvx import ops
from kvx.engine.llm_engine import TokenEvent
from kvx.engine.sequence import Sequence

pytestmark = pytest.mark.gpu


def bytes_of(t):
    return t.contiguous().cpu().view(torch.uint8).numpy()


@pytest.mark.parametrize("shape,tokens", [((2, 3, 300, 256, 2, 128), 300 * 256 - 77),  # > 128 blocks, ragged
                                          ((2, 2, 6, 256, 1, 4), 1),
                                          ((2, 2, 6, 256, 1, 4), 513),
                                          ((2, 4, 9, 256, 8, 128), 2 * 256)])
def test_token_gather_and_scatter_match_the_index_select_formulation(gpu, shape, tokens):
    g = torch.Generator(device=gpu).manual_seed(tokens)
    pool = torch.empty(shape, dtype=torch.bfloat16, device=gpu)
    pool.view(torch.int16).random_(-32768, 32768, generator=g)
    nb, bs = shape[2], shape[3]
    need = -(-tokens // bs)
    table = torch.randperm(nb, generator=torch.Generator().manual_seed(1))[:need].tolist()
    out = torch.empty((2, shape[1], tokens, *shape[-2:]), dtype=pool.dtype, device=gpu)
    ops.gather_tokens(pool, table, tokens, out)
    host = pool.cpu().view(torch.int16).numpy()
    expect = host[:, :, table].reshape(2, shape[1], need * bs, *shape[-2:])[:, :, :tokens]
    assert np.array_equal(out.cpu().view(torch.int16).numpy(), expect)
    pinned = torch.empty(out.shape, dtype=out.dtype, pin_memory=True)
    ops.gather_tokens(pool, table, tokens, pinned)  # straight into mapped host memory
    torch.cuda.synchronize()
    assert np.array_equal(pinned.view(torch.int16).numpy(), expect)
    # Scatter into a fresh pool: exactly the tokens' rows change.
    dest = torch.zeros_like(pool)
    ops.scatter_tokens(dest, table, tokens, out)
    got = dest.cpu().view(torch.int16).numpy()
    want = np.zeros_like(host)
    flat = want[:, :, table].reshape(2, shape[1], need * bs, *shape[-2:])
    flat[:, :, :tokens] = expect
    want[:, :, table] = flat.reshape(2, shape[1], need, bs, *shape[-2:])
    assert np.array_equal(got, want)


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


def prefilled_engine(gpu, length=5, max_tokens=3, batches=None):
    engine = cached_engine(gpu, batches or [[10]])
    request_id = engine.add_request([1] * length, params(max_tokens=max_tokens))
    engine.step_with_events()
    return engine, request_id


def test_detach_preserves_source_blocks_and_other_requests_can_progress(gpu):
    source, request_id = prefilled_engine(gpu, batches=[[10], [20]])
    original = source.scheduler.running[0]
    blocks = original.block_table.copy()
    snapshot = source.detach_request(request_id)
    assert snapshot.token_ids == [1] * 5 + [10] and snapshot.num_cached_tokens == 5
    assert source._detached_requests[request_id] is original and original.block_table == blocks
    assert source.scheduler.block_manager.used_block_ids == set(blocks)
    assert source.is_finished()
    other = source.add_request([2], params(max_tokens=1))
    result = source.step_with_events()
    assert result.token_events == [TokenEvent(other, 0, 20, True)]
    with pytest.raises(ValueError, match="already detached"):
        source.detach_request(request_id)
    source.release_detached_request(request_id)
    assert not source._detached_requests and not source.scheduler.block_manager.used_block_ids
    with pytest.raises(KeyError):
        source.release_detached_request(request_id)
    with pytest.raises(KeyError):
        source.reattach_request(request_id)


def test_reattach_continues_original_id_and_output_position(gpu):
    source, request_id = prefilled_engine(gpu, batches=[[10], [11], [12]])
    source.detach_request(request_id)
    assert source.reattach_request(request_id) == request_id
    assert source.step_with_events().token_events == [TokenEvent(request_id, 1, 11, False)]
    final = source.step_with_events()
    assert final.token_events == [TokenEvent(request_id, 2, 12, True)]
    assert final.outputs == [(request_id, [10, 11, 12])]
    assert not source.scheduler.block_manager.used_block_ids


def test_failed_export_keeps_request_running_and_blocks_owned(gpu, monkeypatch):
    source, request_id = prefilled_engine(gpu)
    original = source.scheduler.running[0]
    blocks = set(original.block_table)

    def fail(*args):
        raise RuntimeError("export failed")

    monkeypatch.setattr(kv_handoff, "export_kv", fail)
    with pytest.raises(RuntimeError, match="export failed"):
        source.detach_request(request_id)
    assert list(source.scheduler.running) == [original] and not source._detached_requests
    assert source.scheduler.block_manager.used_block_ids == blocks


def test_detach_rejects_queued_partial_prefill_finished_and_unknown_requests(gpu):
    source = cached_engine(gpu, [[90], [91], [10]], budget=2)
    request_id = source.add_request([1] * 5, params(max_tokens=1))
    with pytest.raises(ValueError, match="handoff boundary"):
        source.detach_request(request_id)
    source.step_with_events()
    with pytest.raises(ValueError, match="handoff boundary"):
        source.detach_request(request_id)
    source.step_with_events()
    source.step_with_events()
    for rid in (request_id, -1):
        with pytest.raises(ValueError, match="handoff boundary"):
            source.detach_request(rid)
    assert not source._detached_requests and not source.scheduler.block_manager.used_block_ids


@pytest.mark.parametrize("length", [255, 256, 257])
def test_resume_imports_exact_kv_and_continues_decode_without_replaying_first_token(gpu, length):
    source, source_id = prefilled_engine(gpu, length=length)
    snapshot = source.detach_request(source_id)
    pool = source.model_runner.kv_cache
    table = source._detached_requests[source_id].block_table
    expect = pool.cpu()[:, :, table].flatten(2, 3)[:, :, :length]
    assert np.array_equal(bytes_of(snapshot.kv), bytes_of(expect))
    destination = cached_engine(gpu, [[11], [12]])
    destination.model_runner.kv_cache.fill_(-1)
    destination_id = destination.resume_request(snapshot)
    seq = destination.scheduler.running[0]
    manager = destination.scheduler.block_manager
    assert destination_id == seq.seq_id != source_id
    assert not seq.is_prefill and seq.num_cached_tokens == length and seq.completion_token_ids == [10]
    assert len(seq.block_table) == (length + 255) // 256
    assert kv_handoff.verify_imported_kv(destination.model_runner, seq, snapshot)
    if length >= 256:
        assert manager.blocks[seq.block_table[0]].hash != -1
    source.release_detached_request(source_id)
    first = destination.step_with_events()
    assert first.num_tokens == -1 and first.token_events == [TokenEvent(destination_id, 1, 11, False)]
    final = destination.step_with_events()
    assert final.outputs == [(destination_id, [10, 11, 12])]
    assert all(not prefill for prefill, _ in destination.model_runner.calls)
    assert not manager.used_block_ids


@pytest.mark.parametrize("mismatch", ["dtype", "block_size", "shape", "finished"])
def test_resume_rejects_invalid_snapshot_without_admitting_or_allocating(gpu, mismatch):
    source, request_id = prefilled_engine(gpu)
    snapshot = source.detach_request(request_id)
    if mismatch == "dtype":
        snapshot = replace(snapshot, kv=snapshot.kv.to(torch.float16))
    elif mismatch == "block_size":
        snapshot = replace(snapshot, block_size=512)
    elif mismatch == "shape":
        snapshot = replace(snapshot, kv=snapshot.kv[:, :, :-1])
    else:
        snapshot = replace(snapshot, max_tokens=1)
    destination = cached_engine(gpu, [])
    with pytest.raises(ValueError):
        destination.resume_request(snapshot)
    assert destination.is_finished() and not destination.scheduler.block_manager.used_block_ids
    assert request_id in source._detached_requests


def test_resume_out_of_blocks_preserves_existing_destination_and_source_can_reattach(gpu):
    source, source_id = prefilled_engine(gpu, length=257, batches=[[10], [11], [12]])
    snapshot = source.detach_request(source_id)
    destination = cached_engine(gpu, [[20]], num_blocks=1)
    existing_id = destination.add_request([2], params(max_tokens=2))
    destination.step_with_events()
    existing = destination.scheduler.running[0]
    blocks = set(existing.block_table)
    with pytest.raises(MemoryError):
        destination.resume_request(snapshot)
    assert list(destination.scheduler.running) == [existing] and existing.seq_id == existing_id
    assert destination.scheduler.block_manager.used_block_ids == blocks
    assert source.reattach_request(source_id) == source_id
    assert source.step_with_events().token_events == [TokenEvent(source_id, 1, 11, False)]


def test_failed_import_releases_allocated_destination_blocks(gpu, monkeypatch):
    source, request_id = prefilled_engine(gpu, length=256)
    snapshot = source.detach_request(request_id)
    destination = cached_engine(gpu, [])
    manager = destination.scheduler.block_manager

    def fail(seq):
        raise RuntimeError("import failed")

    monkeypatch.setattr(manager, "hash_blocks", fail)
    with pytest.raises(RuntimeError, match="import failed"):
        destination.resume_request(snapshot)
    assert destination.is_finished() and not manager.used_block_ids and len(manager.free_block_ids) == 16
    assert request_id in source._detached_requests


@pytest.mark.parametrize("sync_fails", [False, True])
def test_cuda_import_waits_for_readiness_before_admission_and_rolls_back_on_failure(gpu, monkeypatch, sync_fails):
    """bench/test_engine_handoff.py:198-233: the device sync precedes admission; its failure releases blocks."""
    source, request_id = prefilled_engine(gpu)
    snapshot = source.detach_request(request_id)
    destination = cached_engine(gpu, [])
    manager = destination.scheduler.block_manager
    destination.model_runner.kv_cache = SimpleNamespace(device=gpu)
    imported, synchronized = [], []

    def fake_import(runner, block_manager, snap):
        seq = Sequence(snap.token_ids[:snap.num_prompt_tokens], params(max_tokens=3))
        seq.append_token(10)
        block_manager.allocate_for_resume(seq, snap.num_cached_tokens)
        imported.append(seq)
        return seq

    def synchronize(device):
        assert device == gpu
        assert not destination.scheduler.running
        synchronized.append(device)
        if sync_fails:
            raise RuntimeError("copy failed")

    monkeypatch.setattr(kv_handoff, "import_kv", fake_import)
    monkeypatch.setattr(torch.cuda, "synchronize", synchronize)
    if sync_fails:
        with pytest.raises(RuntimeError, match="copy failed"):
            destination.resume_request(snapshot)
        assert not destination.scheduler.running and not manager.used_block_ids
    else:
        assert destination.resume_request(snapshot) == imported[0].seq_id
        assert list(destination.scheduler.running) == imported
    assert synchronized == [gpu]


def test_exit_releases_detached_source_blocks(gpu):
    source, request_id = prefilled_engine(gpu)
    source.detach_request(request_id)
    manager = source.scheduler.block_manager
    source.exit()
    assert not source._detached_requests and not manager.used_block_ids
    assert source.model_runner.calls[-1] == "exit"


def test_detach_and_resume_emit_phase_records(gpu, caplog):
    """bench/test_handoff_timing.py:118-151."""
    import json
    import logging

    import kvx.engine.handoff_timing as timing

    caplog.set_level(logging.DEBUG, logger="nanovllm.kv_handoff")
    timing.enable(True)
    try:
        source, source_id = prefilled_engine(gpu, length=5)
        snapshot = source.detach_request(source_id)
        records = [json.loads(r.message) for r in caplog.records]
        assert [r["op"] for r in records] == ["export_kv", "detach_request"]
        export, detach = records
        assert set(export["phases_ms"]) == {"gather_blocks", "pack", "copy_to_host"}
        assert set(detach["phases_ms"]) == {"export", "unschedule"}
        assert export["num_tokens"] == 5
        assert snapshot.payload_bytes == export["payload_bytes"] > 0

        caplog.records.clear()
        destination = cached_engine(gpu, [[11], [12]])
        destination.model_runner.kv_cache.fill_(-1)
        destination.resume_request(snapshot)
        records = [json.loads(r.message) for r in caplog.records]
        assert [r["op"] for r in records] == ["import_kv", "resume_request"]
        imported, resume = records
        assert set(imported["phases_ms"]) == {"validate", "rebuild_sequence", "allocate_blocks", "copy_to_device",
                                              "scatter_blocks", "publish_cache"}
        assert set(resume["phases_ms"]) == {"import", "cuda_sync", "admit"}
        assert resume["seq_id"] == destination.scheduler.running[0].seq_id
        assert imported["total_ms"] <= resume["phases_ms"]["import"] + 1e-3  # nested: import inside resume's phase
        assert kv_handoff.verify_imported_kv(destination.model_runner, destination.scheduler.running[0], snapshot)
    finally:
        timing.enable(False)
