"""bench.py's command line on a machine without a GPU: the multi-GPU request
is refused before any device work, and a missing GPU is reported, both with
exit status 2 and no JSON line on stdout."""
import subprocess
import sys
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parents[1]


def run_bench(*args):
    return subprocess.run([sys.executable, str(REPO / "bench.py"), *args], capture_output=True,
                          text=True, timeout=300)


def test_more_than_one_gpu_is_refused():
    r = run_bench("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the message on a machine without a GPU")
def test_missing_gpu_is_reported():
    r = run_bench("--steps", "1", "--warmup", "0")
    assert r.returncode == 2
    assert "no GPU" in r.stderr and r.stdout == ""
