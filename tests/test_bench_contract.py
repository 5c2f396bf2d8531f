"""CPU: bench.py's command-line contract (one GPU only; no GPU, no run)."""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=300, cwd=ROOT)


def test_multi_gpu_request_exits_with_a_message():
    res = run_bench("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert res.returncode == 2
    assert "one GPU" in res.stderr and res.stdout == ""


def test_no_gpu_exits_without_a_result_line():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present: the bench would run")
    res = run_bench("--steps", "1", "--warmup", "0")
    assert res.returncode == 2
    assert "GPU" in res.stderr and res.stdout == ""
