"""CPU checks of bench.py's command line: the refusals that happen before any GPU work."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _run(*args: str) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT, capture_output=True, text=True,
                          timeout=120)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one MI355X" in r.stderr and "--gpus 1" in r.stderr
    assert r.stdout == ""


def test_zero_operands_only_for_analysis_runs():
    r = _run("--operands", "zeros")
    assert r.returncode == 2
    assert "analysis mode" in r.stderr
