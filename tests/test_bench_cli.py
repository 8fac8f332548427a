"""bench.py's command line (CPU): more than one GPU is refused with a
message, and every workload is offered."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=120)


def test_more_than_one_gpu_is_refused():
    proc = run("--gpus", "2")
    assert proc.returncode == 2
    assert "one GPU only" in proc.stderr
    assert proc.stdout == ""


def test_every_workload_is_offered():
    proc = run("--help")
    assert proc.returncode == 0
    for name in ("decode", "prefill", "step-metadata", "qk-norm-rope", "greedy", "engine",
                 "append", "gather", "long-decode"):
        assert name in proc.stdout
