"""Writes tests/golden/hook_traces.json: the reference BlockManager's and Scheduler's hook traces.

Runs the scenarios of tests/hook_scenarios.py on the reference's
nanovllm/engine/block_manager.py and nanovllm/engine/scheduler.py, loaded
file by file from /root/reference the way the reference's own tests load
engine modules (bench/test_engine_events.py:17-44), so nanovllm/__init__.py
(which imports flash-attn and the model) never runs. Only this script
touches the reference; the committed JSON is data (scenario outcomes, hook
calls and pool snapshots), read by tests/test_hook_contract.py.

Run: python tests/golden/make_hook_traces.py
"""

import importlib.util
import json
import sys
import types
from pathlib import Path

HERE = Path(__file__).resolve().parent
REFERENCE = Path("/root/reference/nanovllm_upstream/nanovllm")
OUT = HERE / "hook_traces.json"


def load_reference():
    for name, path in (("nanovllm", REFERENCE), ("nanovllm.engine", REFERENCE / "engine")):
        package = types.ModuleType(name)
        package.__path__ = [str(path)]
        sys.modules[name] = package
    modules = {}
    for name, path in (("nanovllm.sampling_params", REFERENCE / "sampling_params.py"),
                       ("nanovllm.config", REFERENCE / "config.py"),
                       ("nanovllm.engine.sequence", REFERENCE / "engine" / "sequence.py"),
                       ("nanovllm.engine.block_manager", REFERENCE / "engine" / "block_manager.py"),
                       ("nanovllm.engine.scheduler", REFERENCE / "engine" / "scheduler.py")):
        spec = importlib.util.spec_from_file_location(name, path)
        module = importlib.util.module_from_spec(spec)
        sys.modules[name] = module
        spec.loader.exec_module(module)
        modules[name.rsplit(".", 1)[-1]] = module
    return types.SimpleNamespace(BlockManager=modules["block_manager"].BlockManager,
                                 Sequence=modules["sequence"].Sequence,
                                 SamplingParams=modules["sampling_params"].SamplingParams,
                                 Scheduler=modules["scheduler"].Scheduler)


def main():
    sys.path.insert(0, str(HERE.parent))
    import hook_scenarios

    traces = hook_scenarios.run_all(load_reference())
    OUT.write_text(json.dumps(traces, indent=None, separators=(",", ":")) + "\n")
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(traces)} scenarios)")


if __name__ == "__main__":
    main()
