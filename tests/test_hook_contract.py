"""kvx's block manager and scheduler issue the reference's CPU-tier hooks, in the reference's order.

tests/golden/hook_traces.json holds the traces of tests/hook_scenarios.py
recorded on the reference's own BlockManager and Scheduler
(tests/golden/make_hook_traces.py): every _preserve_before_recycle,
_preserve_on_release, before_block_reuse, before_block_use and _copy_entry
call with its arguments, interleaved with pool snapshots (free order,
references, published hashes, block tables) and each step's outcome. kvx's
engine must reproduce them exactly, so a CPU tier that works under one works
under the other, and so kvx's CPUBlockCache, driven by kvx's engine in the
GPU tests, sees the reference BlockManager's call pattern.
"""

import json
from pathlib import Path
from types import SimpleNamespace

import pytest

import hook_scenarios
from kvx.engine.block_manager import BlockManager
from kvx.engine.scheduler import Scheduler
from kvx.engine.sequence import SamplingParams, Sequence

GOLDEN = Path(__file__).resolve().parent / "golden" / "hook_traces.json"
KVX = SimpleNamespace(BlockManager=BlockManager, Sequence=Sequence, SamplingParams=SamplingParams,
                      Scheduler=Scheduler)


def golden():
    return json.loads(GOLDEN.read_text())


def test_every_scenario_has_a_recorded_trace():
    assert set(golden()) == set(hook_scenarios.SCENARIOS)


@pytest.mark.parametrize("name", sorted(hook_scenarios.SCENARIOS))
def test_trace_matches_the_reference(name):
    expected = golden()[name]
    got = json.loads(json.dumps(hook_scenarios.SCENARIOS[name](KVX)))
    for i, (want, have) in enumerate(zip(expected, got)):
        assert have == want, f"{name}: event {i} differs\n reference: {want}\n kvx:       {have}"
    assert len(got) == len(expected), f"{name}: {len(got)} events, the reference recorded {len(expected)}"


def test_the_traces_exercise_every_hook():
    kinds = {event[0] for trace in golden().values() for event in trace}
    assert {"preserve_before_recycle", "preserve_on_release", "before_block_reuse", "before_block_use",
            "copy_entry", "budget_skip", "raised", "scheduled"} <= kinds
    waits = {event[3] for trace in golden().values() for event in trace if event[0] == "copy_entry"}
    assert waits == {True, False}
