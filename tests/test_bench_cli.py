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


@pytest.mark.parametrize("nbytes", [1 << 20, 6_256_120, 27_525_120, 47_185_920, 178_257_920,
                                    356_515_840, 600 << 20])
@pytest.mark.parametrize("iters", [1, 20, 100, 200])
def test_rotation_covers_the_caches(nbytes, iters):
    """copies_for's rotation: when the timed launches cycle through the
    copies, every copy is read again only after at least 512 MiB of the
    others; when they use fewer copies than that, the untimed flush reads at
    least 512 MiB of the rest just before them."""
    sys.path.insert(0, os.path.join(ROOT, "vram-compression_amd"))
    import rans_bench as B
    rot = 512 << 20
    n = B.copies_for(iters, nbytes, rot)
    assert n >= 2
    if iters >= n:
        assert (n - 1) * nbytes >= rot
    else:
        assert (n - iters) * nbytes >= rot


def test_traffic_only_for_the_measured_sources():
    """roofline.traffic comes from counters measured on one build: the line
    carries it only when the library sources hash to the recorded value,
    and says why otherwise."""
    sys.path.insert(0, ROOT)
    import bench
    h = bench.library_source_hash()
    assert len(h) == 12 and int(h, 16) >= 0
    key = next(iter(bench.PMC_TRAFFIC_KIB))
    rec = bench.PMC_TRAFFIC_KIB[key]
    t, note = bench.pmc_traffic(*key, rec["source_hash"])
    assert t == int((rec["fetch_kib"] * 2.0 + rec["write_kib"] * 1.0) * 1024) and "rocprofv3" in note
    t, note = bench.pmc_traffic(*key, "0" * 12)
    assert t is None and "measured on library sources" in note
    t, note = bench.pmc_traffic(1, 64, 1, "refill", h)
    assert t is None and "tiling" in note
