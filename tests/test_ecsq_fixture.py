"""Codes with ECSQ-GPTQ + waterfilling statistics (tests/golden/ecsq_wf_kv.npz,
written by tests/golden/make_ecsq_golden.py, which imports the reference's
exp/quant.py and runs its ecsq with waterfilling, quant.py:122-156, on a
synthetic random-init layer): the fixture agrees
with its recorded statistics, those sit inside the reference's published
range (results/Qwen2.5-1.5B__ecsq_wf_3.25.json, copied into the statistics
file by the generator), and the codes, escapes included, survive the w64
encoder and both host decoders exactly."""
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def ecsq():
    z = np.load(os.path.join(GOLDEN, "ecsq_wf_kv.npz"))
    stats = json.load(open(os.path.join(GOLDEN, "ecsq_wf_stats.json")))
    return z["codes"].astype(np.int32), z["step"], stats


def test_fixture_matches_its_statistics(ecsq):
    codes, step, stats = ecsq
    fx = stats["fixture"]
    assert codes.shape == (fx["rows"], fx["cols"]) == (256, 1536)
    assert step.shape == (1536,) and step.dtype == np.float32 and np.all(step > 0)
    assert np.unique(codes).size == fx["levels"]
    assert np.count_nonzero(np.abs(codes) > 127) == fx["escapes"] > 0
    assert np.abs(codes).max() == fx["max_abs_code"]
    # waterfilling: per-column steps spread over orders of magnitude
    assert step.max() / step.min() > 10


def test_statistics_within_published_range(ecsq):
    """The group the fixture comes from (q/k/v) hits the target entropy as
    the reference's does (3.25 b/w minus 16 bits per column of side
    information) and has a level count inside the published range over the
    28 layers; its escapes are the codes the reference's 8-bit encoder would
    refuse (kernel/rans.py:66)."""
    _, _, stats = ecsq
    g = stats["groups"]["qkv"]
    assert g["bpw"] == pytest.approx(3.25, abs=0.002)
    assert g["code_entropy"] == pytest.approx(g["published_code_entropy_median"], abs=0.002)
    assert g["published_levels"]["min"] <= g["levels"] <= g["published_levels"]["max"]
    assert g["escapes"] > 0 and g["max_abs_code"] > 127
    for name, h in stats["groups"].items():
        assert h["bpw"] == pytest.approx(3.25, abs=0.002), name


@pytest.mark.parametrize("tiling", [None, (1, 1536), (8, 512), (16, 768, 2)])
def test_ecsq_codes_round_trip(rans, oracle, ecsq, tiling):
    codes, _, stats = ecsq
    if tiling is None:
        R, C = rans.pick_tiling(*codes.shape)
        enc = rans.encode(codes, R, C, 1)
    else:
        enc = rans.encode(codes, *tiling)
    assert len(enc["esc_pos"]) == stats["fixture"]["escapes"]
    np.testing.assert_array_equal(rans.decode_ref(enc), codes)
    np.testing.assert_array_equal(oracle.w64_decode(enc), codes)
