"""bench.py's command-line contract that needs no GPU."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused_with_a_message():
    done = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          timeout=300, cwd=ROOT)
    assert done.returncode == 2
    assert "measures one GPU" in done.stderr


def test_help_names_the_profiling_switches():
    done = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--help"], capture_output=True, text=True,
                          timeout=300, cwd=ROOT)
    assert done.returncode == 0
    for flag in ("--steps", "--warmup", "--gpus", "--only-prefill", "--copy-calibration"):
        assert flag in done.stdout
