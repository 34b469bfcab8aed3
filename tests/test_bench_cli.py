"""bench.py's contract pieces that run without a GPU: more than one GPU is
refused with a message, and the default run lengths are sized by time."""

from __future__ import annotations

import os
import subprocess
import sys
import time
import types

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_run_lengths_sized_by_time():
    calls = []

    def run_once():
        calls.append(1)
        time.sleep(0.002)

    args = types.SimpleNamespace(warmup=None, steps=None)
    warmup, steps = bench.resolve_counts(args, run_once, lambda: None)
    assert len(calls) == 2                       # one untimed, one timed launch
    # ~2 ms a step: ~0.3 s of warm-up, ~1 s timed (sleep overshoot lowers both)
    assert 5 <= warmup <= bench.WARMUP_SECONDS / 0.002
    assert 20 <= steps <= bench.TIMED_SECONDS / 0.002


def test_explicit_run_lengths_are_kept():
    args = types.SimpleNamespace(warmup=3, steps=7)
    assert bench.resolve_counts(args, lambda: None, lambda: None) == (3, 7)
