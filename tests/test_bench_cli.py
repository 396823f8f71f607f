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


def test_analysis_modes_are_not_part_of_the_bench():
    """The bench measures the BASELINE workloads only: the operand and library-comparison
    analysis switches are not accepted (argparse refuses unknown options with status 2)."""

    for flag in ("--operands", "--vs-library", "--mfma-ceiling"):
        r = _run(flag)
        assert r.returncode == 2 and "unrecognized arguments" in r.stderr, flag
