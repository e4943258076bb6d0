"""The drop-in contract of encode(codes, R, C) on the CPU: every tiling the
reference's own test and benchmark pass (kernel/bench.py:41-42 and the
R/C sweep of kernel/bench.py:84-103) is accepted, mapped to a legal w64 tile
and decoded back exactly, and the returned dict carries the reference's keys
(kernel/rans.py:93-98) with the reference's meaning."""
import ctypes

import numpy as np
import pytest

# kernel/bench.py:41-42: (rows, cols, R, C, bits)
REF_TEST = [(64, 256, 4, 256, 3.0), (128, 512, 8, 128, 2.0), (256, 1024, 16, 512, 4.0),
            (32, 64, 1, 32, 1.0)]
# kernel/bench.py:84-87
REF_BENCH_SHAPES = {"1.5B qkv": (2048, 1536), "1.5B gate_up": (17920, 1536),
                    "1.5B down": (1536, 8960), "27B-like attn": (5120, 5120),
                    "27B-like gate_up": (34816, 5120), "27B-like down": (5120, 17408)}
REF_KEYS = ("words", "offs", "table", "R", "C", "shape", "bits_payload", "bits_state_offs",
            "bits_table", "entropy_model")


def bench_sweep(rows, cols):
    """(R, C) pairs of kernel/bench.py:100-103 for one shape."""
    out = []
    for R in (4, 8, 16):
        for C in sorted({cols, 512, 1024, 2048} & set(range(32, cols + 1, 32))):
            if cols % C or rows % R:
                continue
            out.append((R, C))
    return out


def _codes(rows, cols, seed, delta=0.45):
    """round(Laplace(0,1)/delta) clipped to [-127, 127] (about 3 bits per
    code), drawn by inverse CDF from 16-bit uniforms: fast at 178 M codes."""
    rng = np.random.default_rng(seed)
    u = (np.arange(65536) + 0.5) / 65536
    lap = np.where(u < 0.5, np.log(2 * u), -np.log(2 - 2 * u))
    lut = np.clip(np.round(lap / delta), -127, 127).astype(np.int32)
    return lut[rng.integers(0, 65536, size=(rows, cols), dtype=np.uint16)]


def _check_enc(rans, enc, codes, R, C):
    rows, cols = codes.shape
    for k in REF_KEYS:
        assert k in enc, k
    assert (enc["R"], enc["C"], tuple(enc["shape"])) == (R, C, (rows, cols))
    tR, tC, tS = rans.tiling_of(enc)
    # the stored width: cols, or cols + 32 when cols is an odd multiple of 32
    scols = rans.stream_cols(enc)
    assert scols == cols + (32 if cols % 64 else 0)
    # the mapped tile: a compiled height dividing R, a multiple of 64 within
    # one (or, for C % 64 == 32, two) of the reference's tiles
    assert R % tR == 0 and tR in rans.SUPPORTED_R
    assert tC % (64 * tS) == 0 and scols % tC == 0
    if scols == cols:
        assert (C if C % 64 == 0 else 2 * C) % tC == 0
    else:
        assert tC <= 2 * C
    assert tR * tC <= 65536 and tR * tC // (64 * tS) <= rans.MAX_STATE_SYMBOLS
    # offs: one word offset per state (the reference's per-lane offs), each
    # at its state's stream, in state order after the tile's initial states
    nstates = (rows // tR) * (scols // tC) * 64 * tS
    assert enc["offs"].dtype == np.uint32 and enc["offs"].size == nstates
    ends = enc["offs"].astype(np.int64) + rans.stream_lengths(enc)
    ntiles = (rows // tR) * (scols // tC)
    per_tile = ends.reshape(ntiles, -1)
    starts = enc["offs"].astype(np.int64).reshape(ntiles, -1)
    np.testing.assert_array_equal(starts[:, 1:], per_tile[:, :-1])
    np.testing.assert_array_equal(starts[:, 0],
                                  enc["tile_off"][:-1] + (enc["tile_meta"] >> 16))
    assert np.all(per_tile[:, -1] < enc["tile_off"][1:])  # the pad word follows
    assert np.array_equal(rans.decode_ref(enc), codes)


@pytest.mark.parametrize("case", REF_TEST, ids=lambda c: "x".join(map(str, c[:4])))
def test_reference_test_tilings(rans, oracle, case):
    rows, cols, R, C, bits = case
    codes = oracle.synth_codes(rows, cols, bits, seed=rows)
    enc = rans.encode(codes, R, C)
    _check_enc(rans, enc, codes, R, C)
    # the reference's bit accounting keys keep their meaning: payload words
    # over the weights, the 16 KB table over the weights
    assert enc["bits_table"] == pytest.approx(32 * 4096 / codes.size)
    assert enc["bits_payload"] >= 0


@pytest.mark.parametrize("name", list(REF_BENCH_SHAPES))
def test_reference_bench_sweep(rans, name):
    """Every (R, C) of the sweep on the first 1024 rows of the shape (the
    mapping depends on cols, R and C only; 1024 rows divide by every R of
    the sweep), then the shape at full size with the sweep's first tiling."""
    rows, cols = REF_BENCH_SHAPES[name]
    codes = _codes(rows, cols, seed=rows + cols)
    sweep = bench_sweep(rows, cols)
    assert sweep
    part = np.ascontiguousarray(codes[:1024])
    for R, C in sweep:
        _check_enc(rans, rans.encode(part, R, C), part, R, C)
    R, C = sweep[0]
    _check_enc(rans, rans.encode(codes, R, C), codes, R, C)


def test_published_tilings_map(rans):
    """The tilings of the published records (results/kernel_bench.json: e.g.
    R=8, C=8960 at 1536x8960) and configuration 1's 32-lane R=512, C=256."""
    cases = {(1536, 8960, 8, 8960): (8, 4480, 2), (5120, 5120, 16, 512): (16, 512, 1),
             (34816, 5120, 4, 512): (4, 512, 1), (5120, 17408, 4, 512): (4, 512, 1),
             (512, 256, 512, 256): (16, 256, 1), (32, 64, 1, 32): (1, 64, 1),
             (17920, 1536, 8, 1536): (8, 1536, 1), (2048, 1536, 4, 512): (4, 512, 1),
             (1536, 8960, 16, 8960): (16, 1792, 2)}
    for (rows, cols, R, C), want in cases.items():
        assert rans.w64_tiling(rows, cols, R, C) == want, (rows, cols, R, C)
    # a legal w64 tiling maps to itself, whatever the state count
    for rows, cols, R, C, S in ((1536, 8960, 3, 2240, 1), (8960, 1536, 35, 192, 1),
                                (25600, 5120, 16, 640, 1), (1536, 8960, 8, 1792, 2),
                                (1536, 8960, 16, 2240, 1)):
        assert rans.w64_tiling(rows, cols, R, C, S) == (R, C, S)


# cols an odd multiple of 32, which the reference accepts (kernel/rans.py:57
# asks only C % 32 == 0): (rows, cols, [C...])
ODD32 = [(64, 96, (32, 96)), (32, 160, (32, 160)), (48, 224, (32, 224)), (70, 96, (32, 96)),
         (6, 32, (32,)), (512, 2080, (32, 416, 2080))]


@pytest.mark.parametrize("case", ODD32, ids=lambda c: f"{c[0]}x{c[1]}")
def test_odd_multiple_of_32_columns(rans, oracle, case):
    """Every (R, C) the reference accepts on a matrix whose cols is an odd
    multiple of 32: stored with 32 appended columns of code 0 and decoded
    back to the matrix's own shape by the product's and the oracle's
    decoders; escapes included.  The bit accounting is per weight of the
    matrix, and the model entropy over its own codes."""
    rows, cols, Cs = case
    codes = _codes(rows, cols, seed=rows * cols)
    codes[::7, ::5] = 300  # escapes
    for R in [r for r in range(1, rows + 1) if rows % r == 0][:6]:
        for C in Cs:
            enc = rans.encode(codes, R, C)
            _check_enc(rans, enc, codes, R, C)
            np.testing.assert_array_equal(oracle.w64_decode(enc), codes)
    enc = rans.encode(codes, 1, Cs[0])
    assert enc["bits_table"] == pytest.approx(32 * 4096 / codes.size)
    # entropy_model: the matrix's own symbols under the stored table (fit to
    # them plus the appended zeros), a cross-entropy: at least their
    # empirical entropy (Gibbs), and close to the cross-entropy under the
    # unquantised mixture
    sym = np.where(np.abs(codes) <= 127, codes + 128, 0)
    n = np.bincount(sym.ravel(), minlength=256).astype(np.float64)
    p = n / codes.size
    q = n.copy()
    q[128] += rows * 32
    q /= q.sum()
    h = float(-(p[p > 0] * np.log2(p[p > 0])).sum())
    x = float(-(p[p > 0] * np.log2(q[p > 0])).sum())
    assert h - 1e-9 <= enc["entropy_model"], (h, enc["entropy_model"])
    assert abs(enc["entropy_model"] - x) < 0.02, (x, enc["entropy_model"])


def test_odd_multiple_of_32_container(rans, tmp_path):
    """A matrix stored with appended columns keeps its own shape and step
    through the container; the record's stored width is cols + 32."""
    import rans_io
    codes = _codes(96, 160, seed=3)
    step = np.linspace(0.5, 1.5, 160).astype(np.float32)
    enc = rans.encode(codes, 8, 32)
    path = str(tmp_path / "odd.w64")
    rans_io.save(path, [dict(name="m", enc=enc, step=step)])
    e = rans_io.load(path)[0]
    assert tuple(e["enc"]["shape"]) == (96, 160) and rans.stream_cols(e["enc"]) == 192
    np.testing.assert_array_equal(e["step"], step)
    np.testing.assert_array_equal(rans.decode_ref(e["enc"]), codes)


def test_reference_entry_points_check_arguments(rans):
    """The reference's launch_rans_gemv / launch_rans_decode argument lists
    (kernel/rans.py:25-29) reach entry points that check them before any
    device call: an R the reference has no kernel for returns its own -1
    (rans_gemv.cu:137-144), a null pointer RANS_EARG, a shape that does not
    divide RANS_EGEOMETRY.  (Decoding the reference's streams is tested on
    the GPU.)"""
    lib = ctypes.CDLL(rans.LIB)
    for name in ("launch_rans_gemv", "launch_rans_decode"):
        fn = getattr(lib, name)
        fn.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 5 + [ctypes.c_int] * 3 + [ctypes.c_void_p]
        fn.restype = ctypes.c_int
        for R in (3, 512, 0, -8):
            assert fn(R, 1, 2, 3, 4, 5, 1536, 8960, 8960, None) == -1
        assert fn(8, None, 2, 3, 4, 5, 1536, 8960, 8960, None) == -4
        assert fn(8, 1, 2, 3, 4, None, 1536, 8960, 8960, None) == -4
        assert fn(8, 1, 2, 3, 4, 5, 1536, 8960, 8976, None) == -2  # C does not divide cols
        assert fn(8, 1, 2, 3, 4, 5, 1536, 8960, 8944, None) == -2  # C % 32
        assert fn(16, 1, 2, 3, 4, 5, 1544, 8960, 8960, None) == -2  # R does not divide rows


def test_random_reference_tilings(rans, oracle):
    """Property test over the reference's preconditions: any R, any C with
    C % 32 == 0, rows = a*R and cols = b*C (odd multiples of 32 included),
    codes from narrow to wide (escapes up to the 16-bit limits).  encode
    accepts each, and both decoders give the codes back."""
    from hypothesis import given, settings, strategies as st

    @settings(max_examples=60, deadline=None, derandomize=True)
    @given(R=st.integers(1, 40), a=st.integers(1, 3), k=st.integers(1, 12),
           b=st.integers(1, 3), scale=st.floats(0.3, 40.0), esc=st.sampled_from([0.0, 0.01, 0.2]),
           seed=st.integers(0, 2**31 - 1))
    def prop(R, a, k, b, scale, esc, seed):
        C = 32 * k
        rows, cols = a * R, b * C
        rng = np.random.default_rng(seed)
        codes = np.clip(np.round(rng.laplace(size=(rows, cols)) * scale), -127, 127).astype(np.int64)
        mask = rng.random(codes.shape) < esc
        codes[mask] = rng.choice([-32768, -200, 128, 32767], size=int(mask.sum()))
        if np.unique(codes).size < 2:
            codes.flat[0] = codes.flat[0] + 1
        enc = rans.encode(codes, R, C)
        _check_enc(rans, enc, codes, R, C)
        np.testing.assert_array_equal(oracle.w64_decode(enc), codes)

    prop()


@pytest.mark.parametrize("i", range(4))
def test_reference_layout_encoder_matches_reference(rans, golden, i):
    """encode_reference_layout writes the reference's own encode output
    (kernel/rans.py:62-98) for its test shapes byte for byte: words (with
    the 8 trailing words), offs, table and the bit accounting."""
    rows, cols, R, C = (int(v) for v in golden[f"enc{i}_meta"])
    codes = golden[f"enc{i}_codes"].astype(np.int32)
    enc = rans.encode_reference_layout(codes, R, C)
    np.testing.assert_array_equal(enc["words"], golden[f"enc{i}_words"])
    np.testing.assert_array_equal(enc["offs"], golden[f"enc{i}_offs"])
    np.testing.assert_array_equal(enc["table"], golden[f"enc{i}_table"])
    bits = golden[f"enc{i}_bits"]
    assert enc["bits_payload"] == bits[1] and enc["bits_state_offs"] == bits[2]
    assert enc["bits_table"] == bits[3]
    assert abs(enc["entropy_model"] - bits[4]) < 1e-12
    assert (enc["R"], enc["C"], tuple(enc["shape"])) == (R, C, (rows, cols))


@pytest.mark.parametrize("case", [(1536, 8960, 8, 8960, 3.25), (96, 1536, 4, 512, 4.25),
                                  (48, 768, 16, 256, 2.25), (32, 64, 1, 32, 1.0)],
                         ids=lambda c: "x".join(map(str, c[:4])))
def test_reference_layout_encoder_matches_oracle(rans, oracle, case):
    """Larger shapes against the oracle's restatement of the reference's
    encoder, any thread count; codes at both ends of the 8-bit alphabet."""
    rows, cols, R, C, bits = case
    codes = oracle.synth_codes(rows, cols, bits, seed=rows + cols).astype(np.int32)
    codes[0, :2] = (-128, 127)
    want = oracle.encode_ref(codes, R, C)
    for threads in (1, 5):
        enc = rans.encode_reference_layout(codes, R, C, threads=threads)
        for k in ("words", "offs", "table"):
            np.testing.assert_array_equal(enc[k], want[k])
        assert enc["bits_payload"] == want["bits_payload"]
    with pytest.raises(AssertionError):
        rans.encode_reference_layout(np.where(codes == 127, 128, codes), R, C)


def test_pick_tiling_odd_multiple_of_32(rans, oracle):
    """pick_tiling tiles an odd multiple of 32 columns over its stored width,
    and encode takes that tile width (a multiple of 64 dividing the stored
    columns) as it is."""
    for rows, cols in ((64, 96), (1536, 1568), (256, 2080)):
        R, C = rans.pick_tiling(rows, cols)
        assert C % 64 == 0 and rans.w64_stream_cols(cols) % C == 0
        codes = _codes(rows, cols, seed=cols)
        enc = rans.encode(codes, R, C, 1)
        assert rans.tiling_of(enc) == (R, C, 1)
        np.testing.assert_array_equal(rans.decode_ref(enc), codes)
        np.testing.assert_array_equal(oracle.w64_decode(enc), codes)
    with pytest.raises(AssertionError):
        rans.encode(_codes(64, 128, 1), 16, 96)  # 96 divides neither 128 nor a padded width


def test_pick_tiling_large_matrix_rounds(rans):
    """Above 32M weights pick_tiling weighs the launch's last round of
    resident workgroups: 25600x5120 takes 20x640 tiles (1280 tile rows, the
    last of 768-workgroup rounds two thirds full) over 16x640 (1600 tile
    rows, the last round 8% full), 5120x17408 keeps 4x2176 over 8x2176 (last
    round a quarter full), and the other benchmark shapes keep their
    tilings.  Below 32M weights the 20-row height is not a candidate."""
    assert rans.pick_tiling(25600, 5120) == (20, 640)
    assert rans.pick_tiling(25600, 5120, bits=2.25) == (20, 640)
    assert rans.pick_tiling(5120, 17408) == (4, 2176)
    assert rans.pick_tiling(5120, 25600) == (4, 3200)
    assert rans.pick_tiling(34816, 5120) == (16, 640)
    assert rans.pick_tiling(1536, 8960) == (3, 2240)
    assert rans.pick_tiling(8960, 1536) == (35, 192)
    assert rans.pick_tiling(2560, 5120)[0] != 20  # 13M weights
    rounds, fill = rans.last_round_fill(25600, 5120, 16, 640, bits=2.25)
    assert rounds > 2 and fill < 0.1
    rounds, fill = rans.last_round_fill(25600, 5120, 20, 640, bits=2.25)
    assert 1 < rounds < 2 and fill > 0.6
    assert rans.last_round_fill(5120, 17408, 8, 2176)[1] < 0.5
    # two states per lane never take the 20-row (one state per lane) height
    assert rans.pick_tiling(25600, 5120, S=2)[0] != 20
    assert rans.w64_tiling(40, 1280, 20, 640, 2)[0] != 20


def test_r20_round_trip(rans, oracle):
    """The 20-row height through the host encoder and both host decoders,
    escapes included; encode keeps (20, C, 1) as given."""
    codes = _codes(60, 1280, seed=20)
    codes[5, 7], codes[59, 1279] = 300, -1000
    enc = rans.encode(codes, 20, 640, 1)
    assert rans.tiling_of(enc) == (20, 640, 1)
    np.testing.assert_array_equal(rans.decode_ref(enc), codes)
    np.testing.assert_array_equal(oracle.w64_decode(enc), codes)


def test_layout_tags_keep_the_two_formats_apart(rans, oracle):
    """encode() writes the w64 layout and says so; the reference-layout
    encoder says ref32; an untagged dict is w64 when it carries tile
    offsets (the reference's own encode writes none).  Each matrix class
    refuses the other layout before it needs a GPU, so a w64 dict cannot
    be decoded as 32-lane streams by the reference's entry points."""
    codes = oracle.synth_codes(64, 256, 3.0, seed=5)
    w64 = rans.encode(codes, 8, 256)
    ref = rans.encode_reference_layout(codes, 8, 256)
    assert w64["layout"] == rans.LAYOUT_W64 and ref["layout"] == rans.LAYOUT_REF32
    assert rans.layout_of({k: v for k, v in w64.items() if k != "layout"}) == rans.LAYOUT_W64
    untagged = {k: v for k, v in ref.items() if k != "layout"}
    assert rans.layout_of(untagged) == rans.LAYOUT_REF32
    step = np.ones(256, np.float32)
    with pytest.raises(AssertionError, match="32-lane"):
        rans.ReferenceLayoutMatrix(w64, step, None)
    with pytest.raises(AssertionError, match="w64"):
        rans.RansMatrix(ref, step, None)
    with pytest.raises(AssertionError, match="w64"):
        rans.RansMatrix(untagged, step, None)
    with pytest.raises(AssertionError, match="unknown"):
        rans.layout_of(dict(w64, layout="w32"))
