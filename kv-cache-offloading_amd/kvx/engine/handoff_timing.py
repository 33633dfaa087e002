"""Optional phase timing of the KV handoff operations (nanovllm/engine/handoff_timing.py).

Off by default. NANOVLLM_HANDOFF_DEBUG=1 in the environment (read when this
module is imported) or enable() turns it on; then every export_kv, import_kv,
detach_request and resume_request emits one JSON line at DEBUG level on the
"nanovllm.kv_handoff" logger, the reference's logger and record format:

    {"op": ..., <context and extra fields>, "total_ms": ..., "phases_ms": {...},
     "unaccounted_ms": ..., "timing_overhead_ms": ...}

Phases with the same name accumulate. unaccounted_ms is the total minus the
phases (gaps and instrumentation); timing_overhead_ms is the number of phase
records times the cost of one empty record, measured once per process. Extra
fields may be zero-argument callables, evaluated only when timing is on. A
timer keeps the on/off state it was created with; while off, phase() is a
nullcontext and finish()/abort() return None without logging.
"""

import json
import logging
import os
import time
from contextlib import nullcontext

logger = logging.getLogger("nanovllm.kv_handoff")

_enabled = False
_record_cost_s = None  # seconds per empty phase record, measured on first use


def enable(enabled: bool = True):
    """Switch phase timing on or off for the process. Switching it on gives the
    logger a stderr handler at DEBUG level if it has no handler or level yet."""
    global _enabled
    _enabled = bool(enabled)
    if _enabled and not logger.handlers and logger.level == logging.NOTSET:
        handler = logging.StreamHandler()
        handler.setFormatter(logging.Formatter("%(message)s"))
        logger.addHandler(handler)
        logger.setLevel(logging.DEBUG)


def is_enabled() -> bool:
    return _enabled


enable(os.environ.get("NANOVLLM_HANDOFF_DEBUG", "") not in ("", "0"))


def _ms(seconds: float) -> float:
    # Microsecond-scale phases (and the timing cost itself) need more than three decimals.
    return round(seconds * 1000.0, 6)


class _Phase:
    __slots__ = ("timer", "name", "t0")

    def __init__(self, timer, name):
        self.timer, self.name = timer, name

    def __enter__(self):
        self.t0 = time.perf_counter()
        return self

    def __exit__(self, *exc):
        spent = time.perf_counter() - self.t0
        self.timer.phases[self.name] = self.timer.phases.get(self.name, 0.0) + spent
        self.timer.phase_records += 1
        return False


def _phase_cost_s() -> float:
    """Cost of one empty phase record, timed over 2000 records once per process."""
    global _record_cost_s
    if _record_cost_s is None:
        probe = PhaseTimer.__new__(PhaseTimer)
        probe.enabled, probe.phases, probe.phase_records = True, {}, 0
        n = 2000
        t0 = time.perf_counter()
        for _ in range(n):
            with _Phase(probe, "calibration"):
                pass
        _record_cost_s = max((time.perf_counter() - t0) / n, 1e-9)
    return _record_cost_s


class PhaseTimer:
    """Named phases of one handoff operation, logged as one JSON record by finish() or abort()."""

    def __init__(self, operation: str, **context):
        self.operation = operation
        self.context = context
        self.enabled = _enabled
        self.phases: dict[str, float] = {}
        self.phase_records = 0
        self._t0 = time.perf_counter() if self.enabled else None

    def phase(self, name: str):
        return _Phase(self, name) if self.enabled else nullcontext()

    def _emit(self, extra: dict) -> dict:
        fields = {key: value() if callable(value) else value for key, value in extra.items()}
        total = time.perf_counter() - self._t0
        record = {"op": self.operation, **self.context, **fields,
                  "total_ms": _ms(total),
                  "phases_ms": {name: _ms(spent) for name, spent in self.phases.items()},
                  "unaccounted_ms": _ms(total - sum(self.phases.values())),
                  "timing_overhead_ms": _ms(self.phase_records * _phase_cost_s())}
        logger.debug(json.dumps(record))
        return record

    def finish(self, **extra):
        return self._emit(extra) if self.enabled else None

    def abort(self, error: BaseException, **extra):
        if not self.enabled:
            return None
        return self._emit({"error": f"{type(error).__name__}: {error}", **extra})
