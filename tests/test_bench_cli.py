"""bench.py's command line without a GPU: more than one GPU is refused with
a message (the benchmark measures one), and so is a run on a host without a
ROCm device; neither touches a GPU."""
import os
import subprocess
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=300, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = _bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr


@pytest.mark.skipif(torch.cuda.is_available(), reason="a GPU is present")
def test_no_gpu_is_refused():
    r = _bench("--steps", "1", "--warmup", "0")
    assert r.returncode == 2
    assert "needs a ROCm GPU" in r.stderr
    assert r.stdout.strip() == ""
