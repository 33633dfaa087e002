"""bench.py's command-line contract that needs no GPU."""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_exits_with_a_message():
    run = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=120)
    assert run.returncode == 2
    assert "one GPU" in run.stderr and not run.stdout.strip()
