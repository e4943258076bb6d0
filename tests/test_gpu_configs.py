"""Parity of the HIP path on the benchmark configurations' own workloads and
on the reference's own tilings, through the C ABI, against the oracle.

Bars as in test_gpu_parity: decoded codes bit-exact, bf16 decode bit-exact
against bf16(code*step), GEMV relative L2 <= 1e-3 against the oracle's
float64 dequant+GEMV (and the reference's max-abs-relative < 1e-4 where its
test applies it, kernel/bench.py:55-56)."""
import ctypes
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

REL_L2 = 1e-3


@pytest.fixture(scope="module")
def dev(rans):
    if not torch.cuda.is_available():
        raise RuntimeError("GPU tests need a ROCm device")
    return torch.device("cuda")


def _rel_l2(y, ref):
    y = np.asarray(y, np.float64)
    return float(np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-300))


def _check(rans, oracle, lib, codes, R, C, step, x, x_bf16):
    """encode(codes, R, C) with the reference's tiling, then every device
    path against the oracle.  Returns the matrix."""
    enc = rans.encode(codes, R, C)
    m = rans.RansMatrix(enc, torch.from_numpy(step), lib)
    np.testing.assert_array_equal(m.decode_codes().cpu().numpy(), codes)
    want = (torch.from_numpy(codes.astype(np.float32)) * torch.from_numpy(step)).bfloat16()
    assert torch.equal(m.decode().cpu().view(torch.int16), want.view(torch.int16))
    xt = torch.from_numpy(x).cuda()
    if x_bf16:
        xt = xt.bfloat16()
    y = m.gemv(xt).cpu().numpy().astype(np.float64)
    ref = oracle.gemv_f64(codes, xt.float().cpu().numpy().astype(np.float64),
                          step.astype(np.float64))
    assert _rel_l2(y, ref) <= REL_L2, _rel_l2(y, ref)
    return m, y, ref


def test_config1_512x256(rans, oracle, lib, dev):
    """Configuration 1 on the HIP path: 512x256 Laplace codes at 3.25 bits
    (one per-tensor step), encoded with the reference's 32-lane tiling
    R=512, C=256 (mapped to 16x256 tiles), f32 x ~ N(0,1), checked against
    dense dequant.x as kernel/bench.py:38-56 does."""
    import rans_bench as B
    print("case config 1 512x256 R=512 C=256", flush=True)
    codes = B.synth_codes_full(512, 256, 3.25, seed=512 + 256)
    step = np.full(256, 0.0123, np.float32)
    x = np.random.default_rng(1).standard_normal(256).astype(np.float32)
    m, y, ref = _check(rans, oracle, lib, codes, 512, 256, step, x, x_bf16=False)
    assert (m.R, m.C, m.S) == (16, 256, 1)
    assert np.abs(y - ref).max() / np.abs(ref).max() < 1e-4


@pytest.mark.parametrize("case", [(1536, 8960, 8, 8960, 3.25), (32, 64, 1, 32, 1.0),
                                  (1536, 8960, 16, 8960, 3.25), (5120, 5120, 16, 512, 3.0)],
                         ids=lambda c: "x".join(map(str, c[:4])))
def test_reference_tilings(rans, oracle, lib, dev, case):
    """The reference's own tilings through encode and the GPU: R=8, C=8960
    (its published tiling of 1536x8960, results/kernel_bench.json:128-129),
    its test shape 32x64 with R=1, C=32 (kernel/bench.py:42), and two more of
    its sweep (kernel/bench.py:100-103), with log-normal steps and bf16 x."""
    import rans_bench as B
    rows, cols, R, C, bits = case
    print(f"case reference tiling {case}", flush=True)
    codes = B.synth_codes_full(rows, cols, bits, seed=rows + cols)
    step = B.lognormal_steps(cols, seed=rows)
    x = np.random.default_rng(2).standard_normal(cols).astype(np.float32)
    _check(rans, oracle, lib, codes, R, C, step, x, x_bf16=True)


@pytest.mark.parametrize("case", [(64, 96, 1, 32, True), (70, 96, 35, 96, True),
                                  (512, 2080, 16, 32, False), (2048, 1568, 8, 1568, True)],
                         ids=lambda c: "x".join(map(str, c[:4])))
def test_odd_multiple_of_32_columns(rans, oracle, lib, dev, case):
    """cols an odd multiple of 32 (the reference needs only C % 32 == 0,
    kernel/rans.py:57): stored with 32 appended columns, whose zero step and
    zero-padded x add nothing.  Decode paths bit-exact at the matrix's own
    shape; GEMV at batch 1 and 4 within the bar of the oracle; a grouped
    launch of two such matrices bitwise their single launches.  1% escapes."""
    import rans_bench as B
    rows, cols, R, C, xbf = case
    print(f"case odd-32 columns {case}", flush=True)
    codes = B.synth_codes_full(rows, cols, 3.25, seed=rows + cols, escape_frac=0.01)
    step = B.lognormal_steps(cols, seed=cols)
    x = np.random.default_rng(3).standard_normal(cols).astype(np.float32)
    m, _, _ = _check(rans, oracle, lib, codes, R, C, step, x, x_bf16=xbf)
    assert m.stream_cols == cols + 32
    xb = torch.randn(4, cols, device="cuda")
    xb = xb.bfloat16() if xbf else xb
    y4 = m.gemv(xb).cpu().numpy()
    ref4 = oracle.gemv_f64(codes, xb.float().cpu().numpy().astype(np.float64),
                           step.astype(np.float64))
    assert _rel_l2(y4, ref4) <= REL_L2
    codes2 = B.synth_codes_full(rows, cols, 3.25, seed=rows + cols + 1, escape_frac=0.01)
    m2 = rans.RansMatrix(rans.encode(codes2, R, C), torch.from_numpy(step), lib)
    ys = rans.gemv_group([m, m2], xb)
    assert torch.equal(ys[0], m.gemv(xb)) and torch.equal(ys[1], m2.gemv(xb))


def test_scalar_step_broadcasts(rans, lib, dev):
    """A one-value step (a per-tensor scale) acts as that value in every
    column, as the reference's x * step broadcast would: bitwise the same
    GEMV and decode as the explicit per-column vector."""
    import rans_bench as B
    print("case scalar step 256x512", flush=True)
    codes = B.synth_codes_full(256, 512, 3.25, seed=7)
    enc = rans.encode(codes, 8, 512)
    a = rans.RansMatrix(enc, torch.tensor(0.0123), lib)
    b = rans.RansMatrix(enc, torch.full((512,), 0.0123), lib)
    x = torch.randn(3, 512, device="cuda").bfloat16()
    assert torch.equal(a.gemv(x), b.gemv(x))
    assert torch.equal(a.decode(), b.decode())


CHAIN_LAYERS = int(os.environ.get("CHAIN_TEST_LAYERS", "28"))


def test_config4_chain(rans, oracle, lib, dev):
    """Configuration 4: the per-token chain of a Qwen2.5-1.5B-shaped weight
    set at 3.25 bits (full-size layers, q/k/v and gate/up as grouped
    launches), captured once in a HIP graph and replayed three times with
    other device work in between.  Every matrix's output on every replay is
    bitwise its own single launch and within the bar of the oracle."""
    import rans_bench as B
    L = CHAIN_LAYERS
    print(f"case chain {L} layers grouped", flush=True)
    ch = B.build_chain(bits=3.25, layers=L, seed=0, grouped=True, batch=1, tune=True,
                       keep_codes=True, bf16=False, lib=lib)
    mats = ch["mats"]
    assert len(mats) == 7 * L and len(ch["launches"]) == 4 * L
    assert any(len(launch) == 3 for launch in ch["launches"])  # q/k/v grouped
    single = [m.gemv(ch["xs"][m.cols][0]).clone() for m in mats]
    for i, m in enumerate(mats):
        x = ch["xs"][m.cols][0].float().cpu().numpy().astype(np.float64)
        ref = oracle.gemv_f64(ch["codes"][i], x, ch["steps"][i].astype(np.float64))
        assert _rel_l2(single[i].cpu().numpy(), ref) <= REL_L2, (i, ch["names"][i])
    ys = [torch.empty(1, m.rows, device="cuda") for m in mats]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        B.run_chain(ch, ys)  # first launches of each kernel outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        B.run_chain(ch, ys)
    for rep in range(3):
        for y in ys:
            y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for i, y in enumerate(ys):
            assert torch.equal(y[0], single[i]), (rep, i, ch["names"][i])
        # eager work between replays
        torch.randn(1 << 20, device="cuda").sum().item()


def test_paired_rows_need_lds_for_both(rans, lib, dev):
    """Two tile rows per workgroup hold both rows' staged blocks.  8192x10240
    in 16x2560 tiles at 3.25 bits (512 tile rows, 4 waves of ~16.8 KB each)
    fits one row per workgroup (~100 KB) but not two (~167 KB): the library
    keeps one row per workgroup, the launch succeeds and matches the launch
    forced onto the 4-byte table entries (never paired) bit for bit."""
    import rans_bench as B
    print("case paired rows LDS bound 8192x10240", flush=True)
    rows, cols = 8192, 10240
    codes = B.synth_codes_full(rows, cols, 3.25, seed=7)
    step = torch.from_numpy(B.lognormal_steps(cols, seed=7))
    enc = rans.encode(codes, 16, 2560, 1)
    assert enc["max_tile_words"] > 8000
    m = rans.RansMatrix(enc, step, lib, flags=rans.F_TABLE8)
    m4 = rans.RansMatrix(enc, step, lib, flags=rans.F_TABLE4)
    assert lib.rans_gemv_rows2(ctypes.byref(m._desc), rans.X_BF16, 1) == 0
    x = torch.randn(cols, device="cuda").bfloat16()
    assert torch.equal(m.gemv(x).cpu(), m4.gemv(x).cpu())


def test_paired_rows_query(rans, lib, dev):
    """rans_gemv_rows2 says which launches pair tile rows: 1536x8960 in
    3x2240 tiles (512 tile rows, two per CU) does at batch 1 and 4, and in
    3x1792 tiles at batch 1; with the 4-byte table entries forced, or at
    S = 2, it does not."""
    import rans_bench as B
    print("case paired rows query", flush=True)
    codes = B.synth_codes_full(1536, 8960, 3.25, seed=3)
    step = torch.from_numpy(B.lognormal_steps(8960, seed=3))
    m = rans.RansMatrix(rans.encode(codes, 3, 2240, 1), step, lib)
    for batch in (1, 4):
        assert lib.rans_gemv_rows2(ctypes.byref(m._desc), rans.X_BF16, batch) == 1
    # five column tiles per row: workgroups of 10 waves
    m5 = rans.RansMatrix(rans.encode(codes, 3, 1792, 1), step, lib)
    assert lib.rans_gemv_rows2(ctypes.byref(m5._desc), rans.X_BF16, 1) == 1
    m4 = rans.RansMatrix(rans.encode(codes, 3, 2240, 1), step, lib, flags=rans.F_TABLE4)
    assert lib.rans_gemv_rows2(ctypes.byref(m4._desc), rans.X_BF16, 1) == 0
    m2 = rans.RansMatrix(rans.encode(codes, 3, 1792, 2), step, lib)
    assert lib.rans_gemv_rows2(ctypes.byref(m2._desc), rans.X_BF16, 1) == 0


def test_ecsq_wf_fixture(rans, oracle, lib, dev):
    """Codes with ECSQ-GPTQ + waterfilling statistics (tests/golden/
    ecsq_wf_kv.npz: 246 levels, 24 escapes up to |196|) with their own
    per-column steps: every device path against the oracle, alone and tiled
    eight times into the q/k/v group's 2048x1536 shape (the configuration
    row of rans_bench.configs)."""
    import rans_bench as B
    print("case ecsq-wf fixture", flush=True)
    codes, step = B.ecsq_fixture()
    rng = np.random.default_rng(9)
    x = rng.standard_normal(codes.shape[1]).astype(np.float32)
    _check(rans, oracle, lib, codes, *rans.pick_tiling(*codes.shape), step, x, x_bf16=True)
    big, step = B.ecsq_fixture(rows=2048)
    m, _, _ = _check(rans, oracle, lib, big, *rans.pick_tiling(*big.shape), step, x, x_bf16=True)
    xb = torch.randn(4, big.shape[1], device="cuda").bfloat16()
    ref = oracle.gemv_f64(big, xb.float().cpu().numpy().astype(np.float64),
                          step.astype(np.float64))
    assert _rel_l2(m.gemv(xb).cpu().numpy(), ref) <= REL_L2


def test_random_reference_tilings_on_gpu(rans, oracle, lib, dev):
    """Seeded random shapes and (R, C) under the reference's preconditions
    only (any R, C % 32 == 0, cols possibly an odd multiple of 32), mapped by
    encode: decoded codes bit-exact, bf16 decode bit-exact, GEMV at a random
    batch within the bar of the oracle; ~0.5% escapes."""
    rng = np.random.default_rng(77)
    for case in range(16):
        R = int(rng.integers(1, 41))
        C = 32 * int(rng.integers(1, 40))
        rows = R * int(rng.integers(1, 5))
        cols = C * int(rng.integers(1, 4))
        batch = int(rng.integers(1, 6))
        print(f"case random reference tiling {case}: {rows}x{cols} R={R} C={C} batch={batch}",
              flush=True)
        codes = oracle.synth_codes(rows, cols, float(rng.uniform(1.5, 5.5)), seed=100 + case)
        codes[0, 0], codes[-1, -1] = 5, -5
        hit = rng.random(codes.shape) < 0.005
        codes[hit] = rng.integers(128, 3000, size=int(hit.sum())) * rng.choice([-1, 1], int(hit.sum()))
        step = (rng.random(cols) + 0.25).astype(np.float32)
        m = rans.RansMatrix(rans.encode(codes, R, C), torch.from_numpy(step), lib)
        np.testing.assert_array_equal(m.decode_codes().cpu().numpy(), codes)
        want = (torch.from_numpy(codes.astype(np.float32)) * torch.from_numpy(step)).bfloat16()
        assert torch.equal(m.decode().cpu().view(torch.int16), want.view(torch.int16))
        x = torch.from_numpy(rng.standard_normal((batch, cols)).astype(np.float32)).cuda().bfloat16()
        y = m.gemv(x).cpu().numpy()
        ref = oracle.gemv_f64(codes, x.float().cpu().numpy().astype(np.float64), step.astype(np.float64))
        for b in range(batch):
            assert _rel_l2(y[b], ref[b]) <= REL_L2, (case, b)
