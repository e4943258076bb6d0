"""Parity of the HIP kernels (through the C ABI) with the CPU oracle.

Bars: decoded codes bit-exact; bf16 decode bit-exact against
bf16(code*step) (round to nearest even); GEMV relative L2 <= 1e-3 against the
oracle's float64 dequant+GEMV (and, on the reference's own test shapes, its
max-abs-relative < 1e-4 criterion, kernel/bench.py:55-56)."""
import ctypes

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


def _check_matrix(rans, oracle, lib, codes, R, C, S, step, xs, bf16_x=True, exact_bf16=True):
    rows, cols = codes.shape
    enc = rans.encode(codes, R, C, S)
    m = rans.RansMatrix(enc, torch.from_numpy(step), lib)
    got = m.decode_codes().cpu().numpy()
    np.testing.assert_array_equal(got, codes)
    if exact_bf16:
        dec = m.decode().cpu()
        want = (torch.from_numpy(codes.astype(np.float32)) * torch.from_numpy(step)).bfloat16()
        assert torch.equal(dec.view(torch.int16), want.view(torch.int16))
    for x in xs:
        xt = torch.from_numpy(x).to("cuda")
        if bf16_x:
            xt = xt.bfloat16()
        xf = xt.float().cpu().numpy().astype(np.float64)
        y = m.gemv(xt).cpu().numpy()
        ref = oracle.gemv_f64(codes, xf, step.astype(np.float64))
        assert _rel_l2(y, ref) <= REL_L2, _rel_l2(y, ref)
    return m, enc


REF_TEST_SHAPES = [(64, 256, 4, 256, 1, 3.0), (128, 512, 8, 128, 1, 2.0),
                   (256, 1024, 16, 512, 2, 4.0), (32, 64, 1, 64, 1, 1.0),
                   (64, 512, 2, 256, 4, 3.0), (128, 1024, 8, 128, 1, 3.0)]


@pytest.mark.parametrize("shape", REF_TEST_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_reference_test_shapes(rans, oracle, lib, dev, shape):
    rows, cols, R, C, S, bits = shape
    print(f"case {shape}", flush=True)
    codes = oracle.synth_codes(rows, cols, bits, seed=rows)
    rng = np.random.default_rng(rows)
    step = (rng.random(cols) + 0.5).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    m, enc = _check_matrix(rans, oracle, lib, codes, R, C, S, step, [x], bf16_x=False)
    np.testing.assert_array_equal(oracle.w64_decode(enc), codes)
    y = m.gemv(torch.from_numpy(x).cuda()).cpu().numpy().astype(np.float64)
    ref = oracle.gemv_f64(codes, x.astype(np.float64), step.astype(np.float64))
    assert np.abs(y - ref).max() / np.abs(ref).max() < 1e-4


def test_q_proj_4p25_bits(rans, oracle, lib, dev):
    """1536x1536, N(0,1) codes at 4.25 bits, one per-tensor step, bf16 x."""
    import rans_bench as B
    print("case q_proj 1536x1536 @4.25", flush=True)
    codes = B.synth_codes_full(1536, 1536, 4.25, dist="gauss", seed=1536 + 1536)
    step = np.full(1536, 0.0123, np.float32)
    rng = np.random.default_rng(2)
    xs = [rng.standard_normal(1536).astype(np.float32) for _ in range(2)]
    for S in (1, 2):
        R, C = B.pick_tiling(1536, 1536, S=S)
        _check_matrix(rans, oracle, lib, codes, R, C, S, step, xs)


@pytest.mark.parametrize("rows,cols", [(8960, 1536), (1536, 8960)])
def test_mlp_waterfill_escapes(rans, oracle, lib, dev, rows, cols):
    """Laplace codes at 2.25 bits, log-normal per-column steps, 0.1% escapes."""
    import rans_bench as B
    print(f"case mlp {rows}x{cols} @2.25 escapes", flush=True)
    codes = B.synth_codes_full(rows, cols, 2.25, seed=rows + cols, escape_frac=0.001)
    step = B.lognormal_steps(cols, seed=rows)
    x = np.random.default_rng(3).standard_normal(cols).astype(np.float32)
    R, C = B.pick_tiling(rows, cols, S=1)
    m, enc = _check_matrix(rans, oracle, lib, codes, R, C, 1, step, [x], exact_bf16=False)
    assert len(enc["esc_pos"]) > 0
    # bf16 decode including escapes
    dec = m.decode().cpu()
    want = (torch.from_numpy(codes.astype(np.float32)) * torch.from_numpy(step)).bfloat16()
    assert torch.equal(dec.view(torch.int16), want.view(torch.int16))


def test_metric_shape(rans, oracle, lib, dev):
    """1536x8960 at 3.25 bits/weight (full-tensor entropy), log-normal steps."""
    import rans_bench as B
    print("case metric 1536x8960 @3.25", flush=True)
    codes = B.synth_codes_full(1536, 8960, 3.25, seed=1536 + 8960)
    step = B.lognormal_steps(8960, seed=1536 + 8960)
    rng = np.random.default_rng(4)
    xs = [rng.standard_normal(8960).astype(np.float32) for _ in range(2)]
    for S in (1, 2):
        R, C = B.pick_tiling(1536, 8960, S=S)
        _check_matrix(rans, oracle, lib, codes, R, C, S, step, xs, exact_bf16=(S == 1))


def test_split_k_deterministic(rans, oracle, lib, dev):
    """More column tiles than waves per workgroup: partials + last-workgroup
    reduction; repeated launches must agree bit for bit (counters reset)."""
    rows, cols = 256, 8192
    print("case split-k", flush=True)
    codes = oracle.synth_codes(rows, cols, 3.0, seed=11)
    step = (np.random.default_rng(5).random(cols) + 0.5).astype(np.float32)
    x = np.random.default_rng(6).standard_normal(cols).astype(np.float32)
    for R, C in [(8, 256), (4, 128), (16, 512)]:
        enc = rans.encode(codes, R, C, 1)
        m = rans.RansMatrix(enc, torch.from_numpy(step), lib)
        assert m.workspace is not None
        xt = torch.from_numpy(x).cuda()
        ys = [m.gemv(xt).cpu().numpy() for _ in range(4)]
        for y in ys[1:]:
            np.testing.assert_array_equal(y, ys[0])
        ref = oracle.gemv_f64(codes, x.astype(np.float64), step.astype(np.float64))
        assert _rel_l2(ys[0], ref) <= REL_L2


@pytest.mark.parametrize("batch", [1, 2, 3, 4, 5, 6, 7])
def test_batch(rans, oracle, lib, dev, batch):
    rows, cols = 512, 2048
    print(f"case batch {batch}", flush=True)
    codes = oracle.synth_codes(rows, cols, 3.0, seed=12)
    step = (np.random.default_rng(7).random(cols) * 0.01 + 0.005).astype(np.float32)
    xb = np.random.default_rng(8).standard_normal((batch, cols)).astype(np.float32)
    for R, C, S in [(8, 512, 1), (4, 2048, 2)]:
        enc = rans.encode(codes, R, C, S)
        m = rans.RansMatrix(enc, torch.from_numpy(step), lib)
        for dt in (torch.float32, torch.bfloat16):
            xt = torch.from_numpy(xb).cuda().to(dt)
            y = m.gemv(xt).cpu().numpy()
            assert y.shape == (batch, rows)
            xf = xt.float().cpu().numpy().astype(np.float64)
            ref = oracle.gemv_f64(codes, xf, step.astype(np.float64))
            for b in range(batch):
                assert _rel_l2(y[b], ref[b]) <= REL_L2
                # every batch row equals the batch-1 kernel's result
                y1 = m.gemv(xt[b]).cpu().numpy()
                np.testing.assert_allclose(y[b], y1, rtol=1e-5, atol=1e-5 * np.abs(y1).max())


def test_heavy_tail_escapes_batch4(rans, oracle, lib, dev):
    """Student-t(3) codes at 2.25 bits with 1% escapes, batch 1 and 4
    (the 27B-class configuration at reduced rows)."""
    import rans_bench as B
    rows, cols = 1280, 5120
    print("case student-t escapes", flush=True)
    codes = B.synth_codes_full(rows, cols, 2.25, dist="student3", seed=9, escape_frac=0.01)
    step = B.lognormal_steps(cols, seed=9)
    xb = np.random.default_rng(9).standard_normal((4, cols)).astype(np.float32)
    R, C = B.pick_tiling(rows, cols, S=1)
    enc = rans.encode(codes, R, C, 1)
    m = rans.RansMatrix(enc, torch.from_numpy(step), lib)
    np.testing.assert_array_equal(m.decode_codes().cpu().numpy(), codes)
    xt = torch.from_numpy(xb).cuda().bfloat16()
    y = m.gemv(xt).cpu().numpy()
    ref = oracle.gemv_f64(codes, xt.float().cpu().numpy().astype(np.float64), step.astype(np.float64))
    for b in range(4):
        assert _rel_l2(y[b], ref[b]) <= REL_L2


def test_graph_replay_matches_eager(rans, oracle, lib, dev):
    rows, cols = 512, 4096
    print("case graph replay", flush=True)
    codes = oracle.synth_codes(rows, cols, 3.0, seed=13)
    step = np.full(cols, 0.01, np.float32)
    for R, C in [(8, 512), (4, 256)]:  # one workgroup per tile row / split-K
        enc = rans.encode(codes, R, C, 1)
        m = rans.RansMatrix(enc, torch.from_numpy(step), lib)
        x = torch.randn(cols, device="cuda").bfloat16()
        y = torch.empty(rows, device="cuda")
        eager = m.gemv(x).clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            m.gemv(x, y)
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            m.gemv(x, y)
        for _ in range(3):
            y.fill_(float("nan"))
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, eager)
            m.gemv(x * 2)  # eager work between replays
            torch.cuda.synchronize()


# rows x cols: the int4 kernel's 4-row workgroups of 1 and 8 waves and its
# 8-row workgroups of 4 waves (both dimensions from 4096), row counts not
# multiples of them, blocks per row that leave a one-block tail (17, 33, 65)
# or run the two-block loop (1088; 257 = one pair and a tail)
@pytest.mark.parametrize("rows,cols", [(256, 1024), (4099, 1056), (8200, 2080), (16390, 544),
                                       (300, 34816), (4097, 8224)])
def test_int4_baseline(rans, lib, dev, rows, cols):
    print(f"case int4 {rows}x{cols}", flush=True)
    codes = np.random.default_rng(rows).integers(-8, 8, size=(rows, cols))
    step = torch.rand(cols) + 0.5
    m4 = rans.Int4Matrix(codes, step, lib)
    x = torch.randn(cols, device="cuda")
    y_ref = torch.from_numpy(codes).double().cuda() @ (x.double() * step.double().cuda())
    y = m4.gemv(x)
    assert torch.allclose(y.double(), y_ref, rtol=1e-4, atol=1e-3)


# rows x cols: odd row counts (the last two-row workgroup has one row),
# 16-byte chunk counts that take 1 to 8 waves, leave a one-chunk tail or run
# several passes of 8 waves; the 1536x8960 headline shape
@pytest.mark.parametrize("rows,cols", [(7, 136), (2049, 1544), (4100, 5120), (8197, 17408),
                                       (1536, 8960)])
def test_bf16_comparator(rans, lib, dev, rows, cols):
    """The dense bf16 GEMV against float64 of the same bf16 values (f32
    accumulation: relative L2 within 1e-5)."""
    print(f"case bf16 gemv {rows}x{cols}", flush=True)
    g = torch.Generator().manual_seed(rows)
    W = torch.randn(rows, cols, generator=g).bfloat16()
    x = torch.randn(cols, generator=g).bfloat16()
    mb = rans.Bf16Matrix(W, lib)
    y = mb.gemv(x.cuda())
    y_ref = W.double() @ x.double()
    err = (torch.linalg.vector_norm(y.cpu().double() - y_ref) / torch.linalg.vector_norm(y_ref)).item()
    assert err < 1e-5, err


@pytest.mark.parametrize("R,C,S", [(4, 256, 1), (8, 512, 2), (16, 128, 1), (2, 256, 4)])
def test_word_fetch_policies_agree(rans, oracle, lib, dev, R, C, S):
    """Both word-fetch policies of the GEMV (every lane re-reads each step,
    or only lanes that consumed their word) decode the same symbols in the
    same order: outputs are bitwise equal, and match the oracle."""
    rows, cols = 256, 1024
    print(f"case word fetch R={R} C={C} S={S}", flush=True)
    codes = oracle.synth_codes(rows, cols, 3.25, seed=R * 100 + S)
    codes[5, 7] = 300  # one escape
    rng = np.random.default_rng(R)
    step = (rng.random(cols) + 0.5).astype(np.float32)
    enc = rans.encode(codes, R, C, S)
    x = torch.from_numpy(rng.standard_normal((4, cols)).astype(np.float32)).cuda().bfloat16()
    ys = []
    for flags in (rans.F_WORDS_ALWAYS, rans.F_WORDS_REFILL, 0):
        m = rans.RansMatrix(enc, torch.from_numpy(step), lib, flags=flags)
        ys.append(m.gemv(x).cpu())
    assert torch.equal(ys[0], ys[1]) and torch.equal(ys[0], ys[2])
    m = rans.RansMatrix(enc, torch.from_numpy(step), lib)
    assert m.tune(batch=4) in (rans.F_WORDS_ALWAYS, rans.F_WORDS_REFILL)
    assert torch.equal(m.gemv(x).cpu(), ys[0])
    ref = oracle.gemv_f64(codes, x.float().cpu().numpy().astype(np.float64),
                          step.astype(np.float64))
    assert _rel_l2(ys[0].numpy(), ref) <= REL_L2


def test_matrix_from_container_file(rans, oracle, lib, dev, tmp_path):
    """A matrix saved with rans_io and memory-mapped back gives the same
    GEMV, bit for bit, as the in-memory encoding, with the stored flags."""
    import rans_io
    print("case container round trip 512x2048", flush=True)
    codes = oracle.synth_codes(512, 2048, 3.25, seed=11)
    codes[1, 2] = -500
    step = (np.random.default_rng(5).random(2048) + 0.5).astype(np.float32)
    enc = rans.encode(codes, 8, 512, 1)
    path = str(tmp_path / "m.w64")
    rans_io.save(path, [dict(name="m", enc=enc, step=step, flags=rans.F_WORDS_REFILL)])
    (e,) = rans_io.load(path)
    a = rans.RansMatrix(enc, torch.from_numpy(step), lib)
    b = rans.RansMatrix(e["enc"], torch.from_numpy(np.array(e["step"])), lib, flags=e["flags"])
    assert b.flags == rans.F_WORDS_REFILL
    x = torch.randn(2048, device="cuda").bfloat16()
    assert torch.equal(a.gemv(x), b.gemv(x))
    np.testing.assert_array_equal(b.decode_codes().cpu().numpy(), codes)


@pytest.mark.parametrize("rows,cols", [(25600, 5120), (5120, 25600)])
def test_full_size_27b_shapes(rans, oracle, lib, dev, rows, cols):
    """The 27B-class shapes at full size (131M weights), the configuration's
    own workload: Student-t(3) codes at 2.25 bits of full-tensor entropy
    with 1% escapes (~1.3M, |code| in [128, 600)): every code bit-exact,
    GEMV at batch 1 and 4 against the float64 oracle, both word-fetch
    policies bitwise equal."""
    import rans_bench as B
    print(f"case full size {rows}x{cols}", flush=True)
    codes = B.synth_codes_full(rows, cols, 2.25, dist="student3", seed=rows + cols,
                               escape_frac=0.01)
    R, C = rans.pick_tiling(rows, cols)
    enc = rans.encode(codes, R, C, 1)
    step = np.exp(0.5 * np.random.default_rng(cols).standard_normal(cols)).astype(np.float32)
    m = rans.RansMatrix(enc, torch.from_numpy(step), lib)
    got = m.decode_codes().cpu().numpy()
    assert np.array_equal(got, codes)
    del got
    x = torch.randn(4, cols, device="cuda").bfloat16()
    ref = oracle.gemv_f64(codes, x.float().cpu().numpy().astype(np.float64),
                          step.astype(np.float64))
    m._desc.flags = rans.F_WORDS_ALWAYS
    y4 = m.gemv(x).cpu()
    y1 = m.gemv(x[0]).cpu()
    m._desc.flags = rans.F_WORDS_REFILL
    assert torch.equal(m.gemv(x).cpu(), y4)
    assert _rel_l2(y4.numpy(), ref) <= REL_L2
    assert _rel_l2(y1.numpy(), ref[0]) <= REL_L2
    # more workgroups than the chip holds at once: batch 1 runs on the
    # 4-byte table entries, batch 4 on the 8-byte ones; forcing either
    # layout changes no bit
    assert m.table_lds4 is not None
    assert lib.rans_gemv_table4(ctypes.byref(m._desc), rans.X_BF16, 1) == 1
    assert lib.rans_gemv_table4(ctypes.byref(m._desc), rans.X_BF16, 4) == 0
    m._desc.flags = rans.F_WORDS_REFILL | rans.F_TABLE8
    assert torch.equal(m.gemv(x[0]).cpu(), y1)
    m._desc.flags = rans.F_WORDS_REFILL | rans.F_TABLE4
    assert torch.equal(m.gemv(x).cpu(), y4)


def test_no_escape_flag(rans, oracle, lib, dev):
    """A matrix without escapes gets RANS_F_NO_ESCAPES from the wrapper; the
    kernels then skip the side table.  Same outputs, bit for bit, as with
    the side table walked (flag cleared)."""
    print("case no-escape flag", flush=True)
    codes = oracle.synth_codes(384, 2048, 3.25, seed=21)
    step = (np.random.default_rng(3).random(2048) + 0.5).astype(np.float32)
    enc = rans.encode(codes, 8, 512, 1)
    m = rans.RansMatrix(enc, torch.from_numpy(step), lib)
    assert m.flags & rans.F_NO_ESCAPES
    x = torch.randn(4, 2048, device="cuda").bfloat16()
    y_skip, d_skip = m.gemv(x).cpu(), m.decode().cpu()
    m._desc.flags = m.flags & ~rans.F_NO_ESCAPES
    assert torch.equal(m.gemv(x).cpu(), y_skip)
    assert torch.equal(m.decode().cpu(), d_skip)
    np.testing.assert_array_equal(m.decode_codes().cpu().numpy(), codes)


@pytest.mark.parametrize("rows,cols,R,C", [(4096, 256, 2, 256), (2048, 512, 4, 256),
                                           (1536, 768, 1, 256), (1536, 8960, 3, 2240)])
def test_few_column_tiles(rans, oracle, lib, dev, rows, cols, R, C):
    """Many tile rows of few column tiles (1, 2, 3 and 4 per row: one
    workgroup of that many waves per tile row).  Escapes in several rows,
    batch 1, 3 and 4, both word-fetch policies bitwise equal, GEMV against
    the float64 oracle."""
    print(f"case few column tiles {rows}x{cols} R={R} C={C}", flush=True)
    codes = oracle.synth_codes(rows, cols, 3.0, seed=rows + C)
    rng = np.random.default_rng(R)
    hit = rng.random(codes.shape) < 0.002
    codes[hit] = rng.integers(128, 700, size=int(hit.sum())) * rng.choice([-1, 1], int(hit.sum()))
    step = (rng.random(cols) + 0.5).astype(np.float32)
    enc = rans.encode(codes, R, C, 1)
    x = torch.from_numpy(rng.standard_normal((4, cols)).astype(np.float32)).cuda().bfloat16()
    ref = oracle.gemv_f64(codes, x.float().cpu().numpy().astype(np.float64), step.astype(np.float64))
    ys = []
    for flags in (rans.F_WORDS_ALWAYS, rans.F_WORDS_REFILL):
        m = rans.RansMatrix(enc, torch.from_numpy(step), lib, flags=flags)
        np.testing.assert_array_equal(m.decode_codes().cpu().numpy(), codes)
        y4 = m.gemv(x).cpu()
        y3 = m.gemv(x[:3].contiguous()).cpu()
        y1 = m.gemv(x[1]).cpu()
        for b in range(4):
            assert _rel_l2(y4[b].numpy(), ref[b]) <= REL_L2
        assert _rel_l2(y3.numpy(), ref[:3]) <= REL_L2
        assert _rel_l2(y1.numpy(), ref[1]) <= REL_L2
        ys.append((y4, y3, y1))
    for a, b in zip(*ys):
        assert torch.equal(a, b)


def test_random_geometries(rans, oracle, lib, dev):
    """Seeded random tile geometries over every compiled R and S (columns
    per tile a random multiple of 64*S, several tile rows and columns),
    codes at a random rate with ~0.5% escapes: codes bit-exact, bf16
    decode bit-exact, GEMV against the float64 oracle at a random batch
    with bf16 or f32 x, both word-fetch policies bitwise equal."""
    rng = np.random.default_rng(2024)
    for case in range(24):
        R = int(rng.choice([1, 2, 3, 4, 8, 16]))
        S = int(rng.choice([1, 2, 4]))
        C = 64 * S * int(rng.integers(1, 5))
        rows = R * int(rng.integers(1, 9))
        cols = C * int(rng.integers(1, 11))
        bits = float(rng.uniform(1.5, 6.0))
        batch = int(rng.integers(1, 7))
        f32 = bool(rng.integers(0, 2))
        print(f"case random {case}: {rows}x{cols} R={R} C={C} S={S} bits={bits:.2f} "
              f"batch={batch} f32={f32}", flush=True)
        codes = oracle.synth_codes(rows, cols, bits, seed=case)
        codes[0, 0], codes[-1, -1] = 7, -7  # at least two symbols, even in a tiny matrix
        hit = rng.random(codes.shape) < 0.005
        codes[hit] = rng.integers(128, 3000, size=int(hit.sum())) * rng.choice([-1, 1], int(hit.sum()))
        step = (rng.random(cols) + 0.25).astype(np.float32)
        enc = rans.encode(codes, R, C, S)
        x = torch.from_numpy(rng.standard_normal((batch, cols)).astype(np.float32)).cuda()
        if not f32:
            x = x.bfloat16()
        ref = oracle.gemv_f64(codes, x.float().cpu().numpy().astype(np.float64),
                              step.astype(np.float64))
        ys = []
        for flags in (rans.F_WORDS_ALWAYS, rans.F_WORDS_REFILL):
            m = rans.RansMatrix(enc, torch.from_numpy(step), lib, flags=flags)
            np.testing.assert_array_equal(m.decode_codes().cpu().numpy(), codes)
            y = m.gemv(x).cpu()
            for b in range(batch):
                assert _rel_l2(y[b].numpy(), ref[b]) <= REL_L2, (case, b)
            ys.append(y)
        assert torch.equal(ys[0], ys[1])
        dec = m.decode().cpu()
        want = (torch.from_numpy(codes.astype(np.float32)) * torch.from_numpy(step)).bfloat16()
        assert torch.equal(dec.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("rows,cols,C,batch", [
    (35, 192, 192, 4),         # one tile, one wave: 140 (row, batch) sums for 64 threads
    (70, 384, 192, 4),         # two waves per workgroup
    (105, 1024, 64, 3),        # 16 column tiles: two column groups (split reduction)
    (140, 576, 64, 1),         # 9 column tiles: three waves, three groups
    (8960, 1536, 192, 1),      # Qwen2.5-1.5B gate/up: 2048 tiles of 35 x 192
])
def test_r35_tiles(rans, oracle, lib, dev, rows, cols, C, batch):
    """Tiles of 35 rows (one state per lane): codes bit-exact, bf16 decode
    bit-exact, GEMV against the float64 oracle with ~0.2% escapes, for both
    word-fetch policies (bitwise equal), at batch 1, 3 and 4; R=35 with two
    states per lane has no kernel and is refused."""
    print(f"case r35 {rows}x{cols} C={C} batch={batch}", flush=True)
    rng = np.random.default_rng(rows + cols)
    codes = oracle.synth_codes(rows, cols, 3.25, seed=rows)
    codes[0, 0], codes[-1, -1] = 5, -5
    hit = rng.random(codes.shape) < 0.002
    codes[hit] = rng.integers(128, 900, size=int(hit.sum())) * rng.choice([-1, 1], int(hit.sum()))
    step = (rng.random(cols) + 0.25).astype(np.float32)
    assert rans.pick_tiling(8960, 1536) == (35, 192)
    enc = rans.encode(codes, 35, C, 1)
    x = torch.from_numpy(rng.standard_normal((batch, cols)).astype(np.float32)).cuda().bfloat16()
    ref = oracle.gemv_f64(codes, x.float().cpu().numpy().astype(np.float64), step.astype(np.float64))
    ys = []
    for flags in (rans.F_WORDS_ALWAYS, rans.F_WORDS_REFILL):
        m = rans.RansMatrix(enc, torch.from_numpy(step), lib, flags=flags)
        np.testing.assert_array_equal(m.decode_codes().cpu().numpy(), codes)
        y = m.gemv(x).cpu()
        for b in range(batch):
            assert _rel_l2(y[b].numpy(), ref[b]) <= REL_L2, (flags, b)
        ys.append(y)
    assert torch.equal(ys[0], ys[1])
    dec = m.decode().cpu()
    want = (torch.from_numpy(codes.astype(np.float32)) * torch.from_numpy(step)).bfloat16()
    assert torch.equal(dec.view(torch.int16), want.view(torch.int16))
    if cols % 128 == 0 and C % 128 == 0:
        m2 = rans.RansMatrix(rans.encode(codes, 35, C, 2), torch.from_numpy(step), lib)
        with pytest.raises(AssertionError, match="HIP error -1"):
            m2.gemv(x)


@pytest.mark.parametrize("rows,cols,C,batch", [
    (20, 192, 192, 4),         # one tile, one wave: 80 (row, batch) sums
    (40, 1280, 640, 4),        # two tile rows of two column tiles
    (60, 1024, 64, 3),         # 16 column tiles: two column groups (split reduction)
    (2560, 5120, 640, 1),      # 128 tile rows of the 25600x5120 tiling
])
def test_r20_tiles(rans, oracle, lib, dev, rows, cols, C, batch):
    """Tiles of 20 rows (one state per lane, the large-matrix height):
    codes bit-exact, bf16 decode bit-exact, GEMV against the float64 oracle
    with ~0.2% escapes for both word-fetch policies (bitwise equal) at batch
    1, 3 and 4, and with both table-entry layouts forced (bitwise equal)."""
    print(f"case r20 {rows}x{cols} C={C} batch={batch}", flush=True)
    rng = np.random.default_rng(rows + cols)
    codes = oracle.synth_codes(rows, cols, 2.5, seed=rows)
    codes[0, 0], codes[-1, -1] = 5, -5
    hit = rng.random(codes.shape) < 0.002
    codes[hit] = rng.integers(128, 900, size=int(hit.sum())) * rng.choice([-1, 1], int(hit.sum()))
    step = (rng.random(cols) + 0.25).astype(np.float32)
    enc = rans.encode(codes, 20, C, 1)
    assert rans.tiling_of(enc) == (20, C, 1)
    x = torch.from_numpy(rng.standard_normal((batch, cols)).astype(np.float32)).cuda().bfloat16()
    ref = oracle.gemv_f64(codes, x.float().cpu().numpy().astype(np.float64), step.astype(np.float64))
    ys = []
    for flags in (rans.F_WORDS_ALWAYS, rans.F_WORDS_REFILL, rans.F_WORDS_REFILL | rans.F_TABLE4,
                  rans.F_WORDS_REFILL | rans.F_TABLE8):
        m = rans.RansMatrix(enc, torch.from_numpy(step), lib, flags=flags)
        np.testing.assert_array_equal(m.decode_codes().cpu().numpy(), codes)
        y = m.gemv(x).cpu()
        for b in range(batch):
            assert _rel_l2(y[b].numpy(), ref[b]) <= REL_L2, (flags, b)
        ys.append(y)
        y1 = m.gemv(x[0]).cpu()
        assert _rel_l2(y1.numpy(), ref[0]) <= REL_L2, flags
    assert all(torch.equal(ys[0], y) for y in ys[1:])
    dec = m.decode().cpu()
    want = (torch.from_numpy(codes.astype(np.float32)) * torch.from_numpy(step)).bfloat16()
    assert torch.equal(dec.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("R,C", [(1, 256), (2, 256), (3, 512), (4, 256), (8, 512), (16, 128),
                                 (20, 512), (35, 192)])
def test_table_entry_layouts_agree(rans, oracle, lib, dev, R, C):
    """The 8-byte and the 4-byte LDS table entries decode the same symbols:
    forced either way, GEMV outputs are bitwise equal at batch 1, 4 and 5
    (f32 and bf16 x), escapes included, and match the oracle."""
    rows, cols = {35: 35 * 24, 20: 20 * 24}.get(R, 384), 1536
    print(f"case table entries R={R} C={C}", flush=True)
    codes = oracle.synth_codes(rows, cols, 3.25, seed=R * 7 + 1)
    codes[3, 11] = 250  # escapes of both signs
    codes[rows - 1, cols - 2] = -400
    rng = np.random.default_rng(R)
    step = np.exp(0.5 * rng.standard_normal(cols)).astype(np.float32)
    enc = rans.encode(codes, R, C, 1)
    m8 = rans.RansMatrix(enc, torch.from_numpy(step), lib, flags=rans.F_TABLE8)
    m4 = rans.RansMatrix(enc, torch.from_numpy(step), lib, flags=rans.F_TABLE4)
    assert m8.table_lds4 is None and m4.table_lds4 is not None
    assert m4.nbytes == m8.nbytes + 16384
    for batch in (1, 4, 5):
        x = torch.from_numpy(rng.standard_normal((batch, cols)).astype(np.float32)).cuda()
        for xt in (x, x.bfloat16()):
            y8 = m8.gemv(xt).cpu()
            y4 = m4.gemv(xt).cpu()
            assert torch.equal(y8, y4), (batch, xt.dtype)
        ref = oracle.gemv_f64(codes, x.bfloat16().float().cpu().numpy().astype(np.float64),
                              step.astype(np.float64))
        assert _rel_l2(y4.numpy(), ref) <= REL_L2


def test_table_entries_choice(rans, lib, dev):
    """The library keeps the 8-byte entries for launches whose workgroups
    all fit on the chip at once (1536x8960 in 3x2240 tiles: 512
    workgroups), and the wrapper then uploads no 4-byte image."""
    import rans_bench as B
    print("case table entry choice 1536x8960", flush=True)
    codes = B.synth_codes_full(1536, 8960, 3.25, dist="laplace", seed=3)
    enc = rans.encode(codes, 3, 2240, 1)
    m = rans.RansMatrix(enc, torch.ones(8960), lib)
    assert m.table_lds4 is None
    for batch in (1, 4):
        assert lib.rans_gemv_table4(ctypes.byref(m._desc), rans.X_BF16, batch) == 0


def test_two_tile_rows_per_workgroup(rans, oracle, lib, dev):
    """1536x8960 in 3x2240 tiles (512 tile rows of 4 waves) runs two tile
    rows per workgroup, 256 workgroups that share one table copy each.
    Forcing the 4-byte table entries keeps one tile row per workgroup: the
    two launches agree bit for bit (each row's sum runs over the same waves
    in the same order), at batch 1, 4 and 5, escapes included."""
    import rans_bench as B
    print("case two tile rows per workgroup 1536x8960", flush=True)
    codes = B.synth_codes_full(1536, 8960, 2.25, dist="laplace", seed=5, escape_frac=0.001)
    step = torch.from_numpy(B.lognormal_steps(8960, seed=5))
    enc = rans.encode(codes, 3, 2240, 1)
    m2 = rans.RansMatrix(enc, step, lib)
    m1 = rans.RansMatrix(enc, step, lib, flags=rans.F_TABLE4)
    for batch in (1, 4, 5):
        x = torch.randn(batch, 8960, device="cuda").bfloat16()
        y2 = m2.gemv(x).cpu()
        assert torch.equal(y2, m1.gemv(x).cpu()), batch
        ref = oracle.gemv_f64(codes, x.float().cpu().numpy().astype(np.float64),
                              step.numpy().astype(np.float64))
        assert _rel_l2(y2.numpy(), ref) <= REL_L2


def test_table_choice_inside_graph_capture(rans, oracle, lib, dev):
    """32768x256 in 1x256 tiles is 32768 one-wave workgroups, more than the
    chip holds at once, so batch 1 runs on the 4-byte table entries.  The
    library's first occupancy query for the f32-x kernel happens while a HIP
    graph is being captured; every replay (with eager work between them)
    equals the eager launch and the 8-byte entries, bit for bit."""
    rows, cols = 32768, 256
    print("case table choice under graph capture 32768x256", flush=True)
    codes = oracle.synth_codes(rows, cols, 3.25, seed=21)
    codes[100, 5] = -200
    step = np.exp(0.5 * np.random.default_rng(4).standard_normal(cols)).astype(np.float32)
    enc = rans.encode(codes, 1, 256, 1)
    m = rans.RansMatrix(enc, torch.from_numpy(step), lib)
    assert m.table_lds4 is not None
    assert lib.rans_gemv_table4(ctypes.byref(m._desc), rans.X_BF16, 1) == 1
    assert lib.rans_gemv_table4(ctypes.byref(m._desc), rans.X_BF16, 4) == 0
    # 5 vectors are one batch-8 launch (8-byte entries); 9 add a batch-1 one
    assert lib.rans_gemv_table4(ctypes.byref(m._desc), rans.X_BF16, 5) == 0
    assert lib.rans_gemv_table4(ctypes.byref(m._desc), rans.X_BF16, 9) == 1
    x = torch.randn(cols, device="cuda")
    base = m._desc.flags & ~(rans.F_TABLE4 | rans.F_TABLE8)
    # load both kernels outside the capture; forced choices skip the query
    m._desc.flags = base | rans.F_TABLE8
    y8 = m.gemv(x).clone()
    m._desc.flags = base | rans.F_TABLE4
    y4 = m.gemv(x).clone()
    torch.cuda.synchronize()
    assert torch.equal(y8, y4)
    ref = oracle.gemv_f64(codes, x.cpu().numpy().astype(np.float64), step.astype(np.float64))
    assert _rel_l2(y4.cpu().numpy(), ref) <= REL_L2
    m._desc.flags = base
    y = torch.empty(rows, device="cuda")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        m.gemv(x, y)
    for _ in range(3):
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, y8)
        m.gemv(x * 2)  # eager work between replays
        torch.cuda.synchronize()
    assert torch.equal(m.gemv(x), y8)


@pytest.mark.parametrize("R,C", [(3, 256), (16, 128), (20, 640), (35, 192)])
def test_escape_value_extremes(rans, oracle, lib, dev, R, C):
    """The side table's 16-bit values at their extremes (-32768, 32767, and
    the smallest escapes -128 and 128) come back through the kernels'
    sign-extending loads: int32 and bf16 decodes bit-exact, GEMV within the
    bar, on the single-pass, split-K and LDS-escape (R = 35) paths."""
    rows, cols = R * 8, C * (16 if R == 16 else 6)  # 16 column tiles: two column groups
    print(f"case escape extremes R={R} C={C}", flush=True)
    codes = oracle.synth_codes(rows, cols, 3.0, seed=R)
    rng = np.random.default_rng(R)
    for v in (-32768, 32767, -128, 128, -129, 4095):
        for _ in range(3):
            codes[rng.integers(rows), rng.integers(cols)] = v
    step = np.exp(0.3 * rng.standard_normal(cols)).astype(np.float32)
    enc = rans.encode(codes, R, C, 1)
    assert enc["esc_val"].min() == -32768 and enc["esc_val"].max() == 32767
    m = rans.RansMatrix(enc, torch.from_numpy(step), lib)
    np.testing.assert_array_equal(m.decode_codes().cpu().numpy(), codes)
    want = (torch.from_numpy(codes.astype(np.float32)) * torch.from_numpy(step)).bfloat16()
    assert torch.equal(m.decode().cpu().view(torch.int16), want.view(torch.int16))
    for batch in (1, 4):
        x = torch.from_numpy(rng.standard_normal((batch, cols)).astype(np.float32)).cuda().bfloat16()
        ref = oracle.gemv_f64(codes, x.float().cpu().numpy().astype(np.float64),
                              step.astype(np.float64))
        assert _rel_l2(m.gemv(x).cpu().numpy(), ref) <= REL_L2


@pytest.mark.parametrize("tile_rows", [512, 513, 514])
@pytest.mark.parametrize("C", [2240, 1792])
def test_two_tile_rows_odd_and_even(rans, oracle, lib, dev, tile_rows, C):
    """A grid of at least twice the CUs pairs tile rows only when their
    count is even and pairing does not raise the most waves a CU holds.
    On 256 CUs: 512 tile rows of 3x2240 or 3x1792 tiles pair them (8 waves
    per workgroup for four column tiles per row, 10 for five); 513 keep one
    row per workgroup (odd); 514 do too (257 pairs would put two on one
    CU, 16 or 20 waves, where one-row workgroups put at most 12 or 15).
    All agree with the one-row launch (forced through the 4-byte table
    entries) bit for bit, and with the oracle."""
    import rans_bench as B
    rows, cols = 3 * tile_rows, 8960
    print(f"case tile rows {tile_rows} C={C}", flush=True)
    codes = B.synth_codes_full(rows, cols, 3.25, dist="laplace", seed=tile_rows)
    codes[rows - 1, cols - 1] = 900  # an escape in the last tile row
    step = torch.from_numpy(B.lognormal_steps(cols, seed=tile_rows))
    enc = rans.encode(codes, 3, C, 1)
    m = rans.RansMatrix(enc, step, lib)
    m1 = rans.RansMatrix(enc, step, lib, flags=rans.F_TABLE4)
    # the library's own answer, on MI355X's 256 CUs
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        want = 1 if tile_rows == 512 else 0
        assert lib.rans_gemv_rows2(ctypes.byref(m._desc), rans.X_BF16, 1) == want
    assert lib.rans_gemv_rows2(ctypes.byref(m1._desc), rans.X_BF16, 1) == 0
    for batch in (1, 4, 8):
        x = torch.randn(batch, cols, device="cuda").bfloat16()
        y = m.gemv(x).cpu()
        # batch 8: the batch-8 kernel (paired rows too) against one-vector
        # launches of the one-row kernel, which sum in the same order
        y1 = m1.gemv(x).cpu() if batch < 8 else \
            torch.cat([m1.gemv(x[i:i + 1]).cpu() for i in range(batch)])
        assert torch.equal(y, y1)
        ref = oracle.gemv_f64(codes, x.float().cpu().numpy().astype(np.float64),
                              step.numpy().astype(np.float64))
        assert _rel_l2(y.numpy(), ref) <= REL_L2


@pytest.mark.parametrize("R,C", [(1, 256), (3, 2240), (8, 384), (16, 256)])
def test_batch_kernels_agree(rans, oracle, lib, dev, R, C):
    """The batch-1, -4 and -8 kernels sum each vector's products in the same
    order: a batch of 1 to 9 vectors, however it is split into launches
    (5 to 8 vectors on the batch-8 kernel where tiles have at most 8 rows,
    chunks of 4 on the batch-4 kernel otherwise, a single vector on the
    batch-1 kernel), gives bitwise the outputs of one launch per vector, with
    escapes, and matches the float64 oracle."""
    rows, cols = {1: 64, 3: 384, 8: 256, 16: 256}[R], {256: 1024, 2240: 4480, 384: 1536}[C]
    print(f"case batch kernels R={R} C={C}", flush=True)
    codes = oracle.synth_codes(rows, cols, 3.25, seed=R)
    rng = np.random.default_rng(R)
    hit = rng.random(codes.shape) < 0.003
    codes[hit] = rng.integers(128, 700, size=int(hit.sum())) * rng.choice([-1, 1], int(hit.sum()))
    step = np.exp(0.4 * rng.standard_normal(cols)).astype(np.float32)
    m = rans.RansMatrix(rans.encode(codes, R, C, 1), torch.from_numpy(step), lib)
    x = torch.from_numpy(rng.standard_normal((9, cols)).astype(np.float32)).cuda().bfloat16()
    singles = torch.stack([m.gemv(x[b]) for b in range(9)]).cpu()
    ref = oracle.gemv_f64(codes, x.float().cpu().numpy().astype(np.float64), step.astype(np.float64))
    for batch in range(1, 10):
        y = m.gemv(x[:batch]).cpu()
        assert torch.equal(y, singles[:batch]), batch
    assert _rel_l2(singles.numpy(), ref) <= REL_L2
