"""Phase timing of the KV handoff operations (kvx.engine.handoff_timing).

Restates the unit tests of bench/test_handoff_timing.py:41-117 (the engine-level
test, :118-151, runs on a GPU pool in tests/test_gpu_handoff.py).
"""

import json
import logging
from types import SimpleNamespace

import pytest

import kvx.engine.handoff_timing as timing


@pytest.fixture
def timing_off():
    timing.enable(False)
    yield timing
    timing.enable(False)


@pytest.fixture
def timing_on(timing_off):
    timing.enable(True)


@pytest.fixture
def records(caplog):
    caplog.set_level(logging.DEBUG, logger="nanovllm.kv_handoff")
    return caplog


def parsed(record):
    return json.loads(record.message)


def test_disabled_timer_records_nothing(timing_off):
    timer = timing.PhaseTimer("export_kv", seq_id=1)
    with timer.phase("gather"):
        pass
    assert timer.finish(payload_bytes=10) is None
    assert timer.phases == {}


def test_enabled_timer_logs_structured_record(timing_on, records):
    timer = timing.PhaseTimer("export_kv", seq_id=7)
    with timer.phase("gather"):
        sum(range(1000))
    record = timer.finish(payload_bytes=4096)
    assert record["op"] == "export_kv" and record["seq_id"] == 7 and record["payload_bytes"] == 4096
    assert set(record["phases_ms"]) == {"gather"}
    assert record["total_ms"] >= record["phases_ms"]["gather"]
    assert record["unaccounted_ms"] >= 0.0 and record["timing_overhead_ms"] >= 0.0
    assert len(records.records) == 1 and parsed(records.records[0]) == record


def test_repeated_phase_names_accumulate(timing_on, records):
    timer = timing.PhaseTimer("op")
    for _ in range(3):
        with timer.phase("loop"):
            pass
    record = timer.finish()
    assert set(record["phases_ms"]) == {"loop"}
    assert record["total_ms"] >= record["phases_ms"]["loop"]
    # Three phase records: the measured cost of one empty record is charged three times.
    assert record["timing_overhead_ms"] == pytest.approx(3 * timing._phase_cost_s() * 1e3, rel=1e-3)


def test_phase_overhead_calibration_is_positive_and_cached(timing_off):
    first = timing._phase_cost_s()
    assert first > 0 and timing._phase_cost_s() == first


def test_abort_logs_error_and_returns_record(timing_on, records):
    record = timing.PhaseTimer("import_kv", num_cached_tokens=5).abort(ValueError("bad layout"))
    assert record["error"] == "ValueError: bad layout" and record["op"] == "import_kv"
    assert parsed(records.records[0]) == record


def test_lazy_extra_fields_resolve_only_when_enabled(timing_on, records):
    payload = SimpleNamespace(payload_bytes=1234)
    assert timing.PhaseTimer("import_kv").finish(payload_bytes=lambda: payload.payload_bytes)["payload_bytes"] == 1234
    timing.enable(False)
    calls = []
    assert timing.PhaseTimer("import_kv").finish(payload_bytes=lambda: calls.append(1)) is None
    assert calls == []


def test_timer_captures_enabled_state_at_construction(timing_on):
    timer = timing.PhaseTimer("export_kv")
    timing.enable(False)
    with timer.phase("gather"):
        pass
    assert set(timer.finish()["phases_ms"]) == {"gather"}


def test_enable_attaches_a_debug_handler_only_to_an_unconfigured_logger(timing_off):
    logger = logging.getLogger("nanovllm.kv_handoff")
    saved_handlers, saved_level = logger.handlers[:], logger.level
    try:
        logger.handlers.clear()
        logger.setLevel(logging.NOTSET)
        timing.enable(True)
        assert len(logger.handlers) == 1 and logger.level == logging.DEBUG
        timing.enable(True)
        assert len(logger.handlers) == 1  # not added twice
    finally:
        logger.handlers[:] = saved_handlers
        logger.setLevel(saved_level)
