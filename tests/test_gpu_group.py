"""Grouped GEMV launches (rans_w64_gemv_group through rans.gemv_group):
several matrices that share x in one launch.  Each output must be bitwise
the output of the matrix's own rans_w64_gemv, and within the GEMV bar of
the float64 oracle."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

REL_L2 = 1e-3


def _rel_l2(y, ref):
    y = np.asarray(y, np.float64)
    return float(np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-300))


def _members(rans, oracle, rows_list, cols, seed, esc=0.002, R=None, C=None):
    rng = np.random.default_rng(seed)
    if R is None:
        R, C = rans.pick_group_tiling(rows_list, cols)
    out = []
    for i, rows in enumerate(rows_list):
        codes = oracle.synth_codes(rows, cols, 3.0 + 0.5 * i, seed=seed + i)
        codes[0, 0], codes[-1, -1] = 4, -4
        hit = rng.random(codes.shape) < esc
        codes[hit] = rng.integers(128, 700, size=int(hit.sum())) * rng.choice([-1, 1], int(hit.sum()))
        step = (rng.random(cols) + 0.25).astype(np.float32)
        m = rans.RansMatrix(rans.encode(codes, R, C, 1), torch.from_numpy(step), rans.build())
        out.append((m, codes, step))
    return out


@pytest.mark.parametrize("rows_list,cols", [((1536, 256, 256), 1536),   # q, k, v of a 1.5B layer
                                            ((896, 128, 128), 896),     # q, k, v of a 0.5B layer
                                            ((8960, 8960), 1536)])      # gate, up
@pytest.mark.parametrize("batch,f32", [(1, False), (3, False), (4, True), (5, False)])
def test_group_matches_single_launches(rans, oracle, rows_list, cols, batch, f32):
    print(f"case group {rows_list}x{cols} batch={batch} f32={f32}", flush=True)
    ms = _members(rans, oracle, rows_list, cols, seed=sum(rows_list) + batch)
    x = torch.from_numpy(np.random.default_rng(batch).standard_normal((batch, cols)).astype(np.float32)).cuda()
    if not f32:
        x = x.bfloat16()
    ys = rans.gemv_group([m for m, _, _ in ms], x)
    xf = x.float().cpu().numpy().astype(np.float64)
    for (m, codes, step), y in zip(ms, ys):
        assert torch.equal(y, m.gemv(x)), "grouped output differs from the single launch"
        ref = oracle.gemv_f64(codes, xf, step.astype(np.float64))
        for b in range(batch):
            assert _rel_l2(y[b].cpu().numpy(), ref[b]) <= REL_L2


def test_group_of_four_and_launch_is_one(rans, oracle):
    """Four members (the most one launch takes) go through the C ABI's
    grouped entry point itself; a fifth member makes gemv_group fall back
    to one launch per matrix, with the same results."""
    ms = _members(rans, oracle, (512, 256, 768, 256), 1024, seed=7, R=16, C=256)
    mats = [m for m, _, _ in ms]
    x = torch.randn(2, 1024, device="cuda").bfloat16()
    lib = mats[0].lib
    descs = (ctypes.c_void_p * 4)(*[ctypes.addressof(m._desc) for m in mats])
    ys = [torch.empty(2, m.rows, device="cuda") for m in mats]
    yps = (ctypes.c_void_p * 4)(*[y.data_ptr() for y in ys])
    rc = lib.rans_w64_gemv_group(descs, 4, x.data_ptr(), rans.X_BF16, 2, yps,
                                    torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    for m, y in zip(mats, ys):
        assert torch.equal(y, m.gemv(x))
    five = mats + [mats[0]]
    for m, y in zip(five, rans.gemv_group(five, x[0])):
        assert torch.equal(y, m.gemv(x[0]))


def test_group_falls_back_when_not_groupable(rans, oracle):
    """Members with different tile heights cannot share a launch: the C ABI
    refuses, gemv_group runs them one by one, results unchanged."""
    a = _members(rans, oracle, (512,), 1024, seed=3, R=16, C=256)[0][0]
    b = _members(rans, oracle, (512,), 1024, seed=4, R=8, C=256)[0][0]
    x = torch.randn(1024, device="cuda").bfloat16()
    descs = (ctypes.c_void_p * 2)(ctypes.addressof(a._desc), ctypes.addressof(b._desc))
    ys = [torch.empty(512, device="cuda") for _ in range(2)]
    yps = (ctypes.c_void_p * 2)(*[y.data_ptr() for y in ys])
    assert a.lib.rans_w64_gemv_group(descs, 2, x.data_ptr(), rans.X_BF16, 1, yps,
                                        torch.cuda.current_stream().cuda_stream) == -1
    ya, yb = rans.gemv_group([a, b], x)
    assert torch.equal(ya, a.gemv(x)) and torch.equal(yb, b.gemv(x))


def test_group_graph_replay_matches_eager(rans, oracle):
    """A grouped launch captured in a HIP graph: every replay (with eager
    work in between) equals the eager result."""
    ms = [m for m, _, _ in _members(rans, oracle, (1536, 256, 256), 1536, seed=11)]
    x = torch.randn(1, 1536, device="cuda").bfloat16()
    want = [y.clone() for y in rans.gemv_group(ms, x)]
    ys = [torch.zeros_like(y) for y in want]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        rans.gemv_group(ms, x, ys)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rans.gemv_group(ms, x, ys)
    for rep in range(4):
        for y in ys:
            y.zero_()
        ms[0].gemv(torch.randn(1, 1536, device="cuda").bfloat16())  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        for y, w in zip(ys, want):
            assert torch.equal(y, w), rep
