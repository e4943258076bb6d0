"""Shared test setup: puts the package directory and the oracle on sys.path
and registers the `gpu` marker (tests that need a gfx950 device)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "vram-compression_amd")
ORACLE = os.path.join(ROOT, "oracle")
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (PKG, ORACLE):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_collection_modifyitems(config, items):
    # Tests marked slow run only when RUN_SLOW=1 (none is marked at present:
    # all 18 published records run by default).
    if os.environ.get("RUN_SLOW") == "1":
        return
    skip = pytest.mark.skip(reason="slow CPU case; set RUN_SLOW=1")
    for item in items:
        if "slow" in item.keywords:
            item.add_marker(skip)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm gfx950 GPU")
    config.addinivalue_line("markers", "slow: long CPU test (the largest published records)")


@pytest.fixture(scope="session")
def oracle():
    if not os.path.exists(os.path.join(ORACLE, "liboracle.so")):
        subprocess.check_call(["make", "-s", "-C", ORACLE])
    import oracle as O
    O.load()
    return O


@pytest.fixture(scope="session")
def rans():
    import rans as R
    if not os.path.exists(R.LIB):
        raise RuntimeError("librans_hip.so is not built: run `python -c 'import __graft_entry__ as g; g.build()'`")
    R._LIB = R.load_lib(R.LIB)
    return R


@pytest.fixture(scope="session")
def lib(rans):
    return rans._LIB


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    return np.load(os.path.join(GOLDEN, "reference_vectors.npz"))
