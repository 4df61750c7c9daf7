"""bench.py's command-line contract on the host: more than one GPU is refused with a message, and without a
visible GPU it stops with an error instead of timing anything on the CPU."""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=300, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = _run("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


def test_no_gpu_stops_before_timing():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible here")
    r = _run("--steps", "1", "--warmup", "0", "--no-cpu-baseline", "--no-extra", "--no-counters")
    assert r.returncode == 1
    assert "no ROCm GPU" in r.stderr
    assert r.stdout.strip() == ""
