"""bench.py's command-line contract, checked without a GPU: more than one GPU
is refused before anything is initialised, and on a host without a usable HIP
device the run stops with the reason instead of measuring a host fallback."""

import os
import subprocess
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(*args):
    return subprocess.run(
        [sys.executable, os.path.join(ROOT, "bench.py"), *args],
        cwd=ROOT,
        capture_output=True,
        text=True,
        timeout=300,
    )


@pytest.mark.parametrize("n", ["2", "8"])
def test_more_than_one_gpu_is_refused(n):
    res = run_bench("--gpus", n)
    assert res.returncode == 2
    assert "one GPU only" in res.stderr and f"--gpus {n}" in res.stderr
    assert res.stdout == ""


@pytest.mark.skipif(torch.cuda.is_available(), reason="needs a host without a GPU")
def test_no_device_stops_with_the_reason():
    res = run_bench("--steps", "1", "--warmup", "0", "--no-extra", "--no-cpu")
    assert res.returncode != 0
    assert "HIP path unavailable" in res.stderr
    assert not any(line.startswith("{") for line in res.stdout.splitlines())
