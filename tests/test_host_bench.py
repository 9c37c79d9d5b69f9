"""bench.py's command-line contract on a host without a GPU: one GPU only,
and a clear refusal rather than a CPU fallback."""

import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _run(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True,
                          text=True, timeout=300, cwd=ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    result = _run("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert result.returncode == 2
    assert "one GPU" in result.stderr and "--gpus 2" in result.stderr
    assert result.stdout == ""


def test_without_a_device_bench_refuses_instead_of_falling_back():
    import torch

    if torch.cuda.device_count() > 0:
        pytest.skip("a HIP device is present; the GPU bench is not a host test")
    result = _run("--steps", "1", "--warmup", "0")
    assert result.returncode == 2
    assert "HIP device" in result.stderr
    assert result.stdout == ""
