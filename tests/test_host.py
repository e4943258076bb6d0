"""Host side of the product (librans_hip.so's C++ encoder/decoder and the
Python wrapper) checked against the oracle on the CPU."""
import ctypes

import numpy as np
import pytest

SHAPES = [  # rows, cols, R, C, S, bits
    (64, 256, 4, 256, 1, 3.0),
    (128, 512, 8, 128, 1, 2.0),
    (256, 1024, 16, 512, 2, 4.0),
    (32, 64, 1, 64, 1, 1.0),
    (64, 512, 2, 256, 4, 3.0),
    (48, 768, 16, 384, 2, 5.0),
    (96, 1280, 8, 640, 1, 2.25),
]


def _ids(s):
    return "x".join(str(v) for v in s)


@pytest.mark.parametrize("shape", SHAPES, ids=_ids)
def test_round_trip_matches_oracle(rans, oracle, shape):
    rows, cols, R, C, S, bits = shape
    codes = oracle.synth_codes(rows, cols, bits, seed=rows + cols)
    enc = rans.encode(codes, R, C, S)
    np.testing.assert_array_equal(rans.decode_ref(enc), codes)
    np.testing.assert_array_equal(oracle.w64_decode(enc), codes)


@pytest.mark.parametrize("shape", SHAPES, ids=_ids)
def test_streams_equal_reference_encoder(rans, oracle, shape):
    """Each w64 state's stream is exactly what the reference encoder
    (kernel/rans.py:62-98, restated in the oracle) emits for that state's
    symbol sequence: same table, same initial state, same words."""
    rows, cols, R, C, S, bits = shape
    codes = oracle.synth_codes(rows, cols, bits, seed=rows + cols + 1)
    enc = rans.encode(codes, R, C, S)
    sym = (codes + 128).astype(np.uint8)
    freq, cum, table = oracle.build_table(sym)
    np.testing.assert_array_equal(enc["table"], table)
    seqs = np.ascontiguousarray(oracle.w64_order(sym, R, C, S))
    lanes, n = seqs.shape
    lib = oracle.load()
    cap = lanes * (n + 2) + 8
    words = np.zeros(cap, np.uint16)
    offs = np.zeros(lanes, np.uint32)
    counts = np.zeros(lanes, np.int64)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    assert lib.orc_encode_lanes(p(seqs), lanes, n, p(freq), p(cum), p(words), cap, p(offs)) == 0
    assert lib.orc_count_words(p(seqs), lanes, n, p(freq), p(cum), p(counts)) == 0
    nst = 64 * S
    # each state's stored length is its stream's word count, or its tile's
    # base where the tile's counts spread over more than 16 values (the
    # shorter streams padded up to it)
    ntiles = lanes // nst
    cnt = counts.reshape(ntiles, nst)
    base = np.maximum(cnt.min(axis=1), cnt.max(axis=1) - 15)
    np.testing.assert_array_equal(enc["tile_meta"] & 0xFF, base)
    np.testing.assert_array_equal(rans.stream_lengths(enc),
                                  np.maximum(cnt, base[:, None]).ravel())
    # the initial states read back from the tiles' bit-packed mantissas,
    # and the streams at the offsets the lengths give
    st0 = rans.initial_states(enc)
    starts = rans.stream_offsets(enc)
    for j in range(lanes):
        o = int(offs[j])
        assert int(st0[j]) == (int(words[o]) << 16) | int(words[o + 1])
        assert (int(enc["slen"][j]) >> 4) == int(st0[j]).bit_length() - 17
        ref_words = words[o + 2:o + 2 + counts[j]]
        start = int(starts[j])
        np.testing.assert_array_equal(enc["words"][start:start + counts[j]], ref_words)


def test_escapes_round_trip(rans, oracle):
    rng = np.random.default_rng(0)
    codes = oracle.synth_codes(128, 256, 2.0, seed=1)
    m = rng.random(codes.shape) < 0.01
    codes[m] = rng.integers(128, 600, m.sum()) * rng.choice([-1, 1], m.sum())
    codes[0, 0] = -128  # the reference alphabet's lowest code is an escape here
    codes[5, 7] = 32767  # the 16-bit side table's extremes
    codes[6, 8] = -32768
    R, C = 4, 128
    enc = rans.encode(codes, R, C, 1)
    esc = (codes < -127) | (codes > 127)
    assert len(enc["esc_pos"]) == int(esc.sum())
    np.testing.assert_array_equal(rans.decode_ref(enc), codes)
    np.testing.assert_array_equal(oracle.w64_decode(enc), codes)
    # side table per tile, in column order (rows ascending within a column),
    # rebuilt here by brute force from the codes
    ncb = codes.shape[1] // C
    tp = enc["esc_tileptr"]
    assert tp[0] == 0 and tp[-1] == len(enc["esc_pos"]) and len(tp) == codes.size // (R * C) + 1
    for t in range(len(tp) - 1):
        rb, cb = divmod(t, ncb)
        want_pos, want_val = [], []
        for c in range(C):
            for r in range(R):
                v = codes[rb * R + r, cb * C + c]
                if esc[rb * R + r, cb * C + c]:
                    want_pos.append(c * R + r)
                    want_val.append(v)
        np.testing.assert_array_equal(enc["esc_pos"][tp[t]:tp[t + 1]], want_pos)
        np.testing.assert_array_equal(enc["esc_val"][tp[t]:tp[t + 1]], want_val)


def test_escape_side_table_must_match_stream(rans, oracle):
    codes = oracle.synth_codes(64, 256, 3.0, seed=3)
    codes[3, 4] = 500
    enc = rans.encode(codes, 4, 256, 1)
    codes[2, 9] = -300
    enc = rans.encode(codes, 4, 256, 1)
    np.testing.assert_array_equal(enc["esc_pos"], [4 * 4 + 3, 9 * 4 + 2])  # c*R + r
    pos, val = enc["esc_pos"], enc["esc_val"]
    for bad_pos, bad_val in [(pos + 4, val),                   # one column to the right
                             (pos[::-1].copy(), val[::-1].copy()),  # not ascending
                             (pos + 4 * 256, val),             # past the tile's last column
                             (np.array([pos[0], pos[0]]), val)]:  # one entry twice
        bad = dict(enc, esc_pos=bad_pos.astype(np.uint16), esc_val=bad_val.astype(np.int16))
        with pytest.raises(AssertionError):
            rans.decode_ref(bad)
        with pytest.raises(AssertionError):
            oracle.w64_decode(bad)


def state_bit(enc, t, j):
    """Absolute bit offset (in enc["words"] read as a little-endian bit
    stream) of the initial-state mantissa of state j of tile t."""
    ntiles = enc["tile_off"].size - 1
    nb = 16 + (enc["slen"].astype(np.int64).reshape(ntiles, -1)[t] >> 4)
    return int(enc["tile_off"][t]) * 16 + int(nb[:j].sum())


def flip_bit(words, bit):
    words[bit >> 4] ^= np.uint16(1 << (bit & 15))


def test_corrupt_state_detected(rans, oracle):
    """A flipped bit in a state's stored initial value (a low mantissa bit of
    state 0) is caught by the final-state check of both decoders."""
    codes = oracle.synth_codes(64, 256, 3.0, seed=4)
    enc = rans.encode(codes, 4, 256, 1)
    bad = dict(enc, words=enc["words"].copy())
    flip_bit(bad["words"], state_bit(enc, 0, 0) + 3)
    with pytest.raises(AssertionError):
        rans.decode_ref(bad)
    with pytest.raises(AssertionError):
        oracle.w64_decode(bad)


def test_first_failing_tile_is_reported(rans, oracle):
    """With two corrupted tiles the host decoder (tiles decoded in parallel)
    reports the lower tile's state, as a tile-by-tile decode does."""
    import ctypes
    codes = oracle.synth_codes(256, 1024, 3.0, seed=17)
    enc = rans.encode(codes, 8, 256, 1)
    nst = 64
    bad = dict(enc, words=enc["words"].copy())
    flip_bit(bad["words"], state_bit(enc, 9, 5) + 2)    # tile 9, state 5
    flip_bit(bad["words"], state_bit(enc, 3, 40) + 7)   # tile 3, state 40: reported
    keep = []
    d = rans._host_desc(bad, keep)
    out = np.zeros(codes.shape, np.int32)
    rc = rans._host_lib().rans_w64_decode_host(ctypes.byref(d), rans._p(out))
    assert rc == 3 * nst + 40 + 1


def test_encode_rejects_bad_input(rans):
    ok = np.random.default_rng(0).integers(-3, 4, size=(16, 128)).astype(np.int32)
    with pytest.raises(AssertionError):
        rans.encode(np.full((16, 128), 5, np.int32), 4, 128)  # single symbol
    with pytest.raises(AssertionError):
        rans.encode(ok, 3, 128)  # rows % R
    with pytest.raises(AssertionError):
        rans.encode(ok, 4, 96)  # cols % C
    with pytest.raises(AssertionError):
        rans.encode(ok, 4, 80)  # C % 32 (the reference's own precondition)
    with pytest.raises(AssertionError):
        rans.encode(ok, 4, 128, S=4)  # no tile of the given S fits C % (64*S)
    with pytest.raises(AssertionError):
        rans.encode(np.zeros((0, 128), np.int32), 1, 128)
    # a code beyond the side table's 16-bit values
    for v in (32768, -32769, 2 ** 30):
        wide_code = ok.copy()
        wide_code[3, 5] = v
        with pytest.raises(AssertionError, match="32767"):
            rans.encode(wide_code, 4, 128)
    # streams beyond 255 words (1024 symbols of ~8 bits each: a tile's
    # length base does not fit its byte) when the caller fixes one state per
    # lane on a tile the format holds
    wide = np.random.default_rng(2).integers(-127, 128, size=(16, 4096)).astype(np.int32)
    with pytest.raises(AssertionError, match="255"):
        rans.encode(wide, 16, 4096, S=1)
    # the encoder entry point itself refuses a tile beyond 65536 codes (the
    # side table's 16-bit positions)
    h = ctypes.c_void_p()
    info = np.zeros(7, np.int64)
    big = np.zeros((16, 8192), np.int32)
    big[0, 0] = 1
    rc = rans._host_lib().rans_w64_encode(rans._p(big), 16, 8192, 16, 8192, 1, 1,
                                          ctypes.byref(h), rans._p(info))
    assert rc == -2


def test_encode_maps_oversized_requests(rans):
    """Tilings beyond the format's limits are mapped, not refused: a tile of
    more than 65536 codes becomes column sub-tiles, and states of more than
    338 symbols get more states per lane; the round trip is exact."""
    rng = np.random.default_rng(2)
    wide = rng.integers(-127, 128, size=(16, 4096)).astype(np.int32)
    enc = rans.encode(wide, 16, 4096)
    assert (enc["R"], enc["C"]) == (16, 4096)
    assert rans.tiling_of(enc) == (16, 4096, 4)
    np.testing.assert_array_equal(rans.decode_ref(enc), wide)
    big = rng.integers(-127, 128, size=(16, 65536)).astype(np.int32)
    enc = rans.encode(big, 16, 65536)
    assert rans.tiling_of(enc) == (16, 4096, 4)
    np.testing.assert_array_equal(rans.decode_ref(enc), big)


def test_stream_lengths_must_match(rans, oracle):
    """A stored length one word off (state 0's, so state 1 also starts one
    word off) is caught by both decoders."""
    codes = oracle.synth_codes(64, 256, 3.0, seed=5)
    enc = rans.encode(codes, 4, 256, 1)
    bad = dict(enc, slen=enc["slen"].copy())
    bad["slen"][0] ^= 1  # the low bit of the length delta
    with pytest.raises(AssertionError):
        rans.decode_ref(bad)
    with pytest.raises(AssertionError):
        oracle.w64_decode(bad)


def test_build_table_matches_oracle(rans, oracle, golden):
    for name in ["two_symbols", "tie_argmax", "rare_overflow", "half_even", "laplace"]:
        sym = golden[f"tab_{name}_sym"]
        for a, b in zip(rans.build_table(sym), oracle.build_table(sym)):
            np.testing.assert_array_equal(a, b)


def test_table_lds_image(rans, oracle, golden):
    """The LDS image the kernels copy verbatim: per slot of symbol y,
    {freq[y] | code<<24, slot - cum[y]} with code = y-128 (0 for the escape
    symbol), rebuilt here from freq/cum rather than from the packed table."""
    for name in ["two_symbols", "tie_argmax", "laplace"]:
        sym = golden[f"tab_{name}_sym"]
        freq, cum, table = oracle.build_table(sym)
        img = rans.table_lds(table)
        assert img.dtype == np.uint32 and img.size == 8192
        for y in np.nonzero(freq)[0]:
            code = 0 if y == 0 else int(y) - 128
            slots = np.arange(cum[y], cum[y] + freq[y])
            np.testing.assert_array_equal(img[2 * slots], np.uint32(freq[y] | ((code & 0xFF) << 24)))
            np.testing.assert_array_equal(img[2 * slots + 1], (slots - cum[y]).astype(np.uint32))
    esc = np.zeros(4096, np.uint32)  # every slot the escape symbol 0 with freq 4096-like fields
    esc[:] = 0 | (5 << 8) | (3 << 20)
    img = rans.table_lds(esc)
    assert np.all(img[0::2] == 5) and np.all(img[1::2] == 3)


def test_table_lds4_image(rans, oracle, golden):
    """The 4-byte LDS entries: per slot of symbol y, freq[y] | (slot -
    cum[y])<<12 | code<<24, rebuilt from freq/cum.  Decoding the fields as
    the kernel does (mask, 12-bit extract, arithmetic shift) gives the
    reference's next state freq*(x>>12) + (x & 4095) - cum for every slot."""
    x = np.random.default_rng(1).integers(1 << 16, 1 << 32, size=4096, dtype=np.uint64)
    for name in ["two_symbols", "tie_argmax", "laplace"]:
        sym = golden[f"tab_{name}_sym"]
        freq, cum, table = oracle.build_table(sym)
        img = rans.table_lds4(table)
        assert img.dtype == np.uint32 and img.size == 4096
        for y in np.nonzero(freq)[0]:
            code = 0 if y == 0 else int(y) - 128
            slots = np.arange(cum[y], cum[y] + freq[y])
            want = freq[y] | ((slots - cum[y]) << 12) | ((code & 0xFF) << 24)
            np.testing.assert_array_equal(img[slots], want.astype(np.uint32))
        xs = (x & ~np.uint64(0xFFF)) | np.arange(4096, dtype=np.uint64)  # state in every slot
        e = img[np.arange(4096)].astype(np.uint64)
        ns = (e & 0xFFF) * (xs >> 12) + ((e >> 12) & 0xFFF)
        ys = np.nonzero(freq)[0]  # symbol of each slot: cum ascends with the symbol
        s_of = ys[np.searchsorted(np.cumsum(freq[ys]), np.arange(4096), side="right")]
        ref = freq[s_of].astype(np.uint64) * (xs >> 12) + (xs & 0xFFF) - cum[s_of].astype(np.uint64)
        np.testing.assert_array_equal(ns, ref)
        codes = img.view(np.int32) >> 24
        np.testing.assert_array_equal(codes, np.where(s_of == 0, 0, s_of - 128))


def test_lane_order_matches_oracle(rans, oracle):
    a = np.arange(32 * 1024).reshape(32, 1024)
    for R, C, S in [(1, 64, 1), (4, 256, 2), (8, 1024, 4), (32, 512, 1)]:
        np.testing.assert_array_equal(rans.lane_order(a, R, C, S), oracle.w64_order(a, R, C, S))


def test_bit_accounting(rans, oracle):
    rows, cols, R, C, S = 256, 1024, 8, 512, 1
    codes = oracle.synth_codes(rows, cols, 3.0, seed=9)
    enc = rans.encode(codes, R, C, S)
    N = rows * cols
    sym = (codes + 128).astype(np.uint8)
    seqs = oracle.w64_order(sym, R, C, S)
    freq, cum, _ = oracle.build_table(sym)
    lib = oracle.load()
    counts = np.zeros(seqs.shape[0], np.int64)
    s = np.ascontiguousarray(seqs)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    assert lib.orc_count_words(p(s), s.shape[0], s.shape[1], p(freq), p(cum), p(counts)) == 0
    assert enc["bits_payload"] == 16 * counts.sum() / N
    nstates = seqs.shape[0]
    ntiles = (rows // R) * (cols // C)
    pad = len(enc["words"]) - counts.sum()
    assert enc["bits_state_offs"] == (8 * nstates + 32 * (2 * ntiles + 1) + 16 * pad) / N
    assert enc["bits_table"] == 32 * 4096 / N
    # the words beyond the payload: each tile's bit-packed initial states
    # (16 + e bits per state, rounded up to words), the streams padded up to
    # their tile's length base, and 1 to 8 words closing each block
    e = enc["slen"].astype(np.int64).reshape(ntiles, -1) >> 4
    blob = (np.sum(16 + e, axis=1) + 15) // 16
    np.testing.assert_array_equal(enc["tile_meta"] >> 16, blob)
    lpad = rans.stream_lengths(enc).sum() - counts.sum()
    assert ntiles <= pad - blob.sum() - lpad <= 8 * ntiles
    assert np.all(np.diff(enc["tile_off"].astype(np.int64)) % 8 == 0)
    # model entropy (from the encoder's symbol counts) against the direct mean
    direct = -np.log2(freq[sym.ravel()] / 4096).mean()
    assert abs(enc["entropy_model"] - direct) < 1e-9


def test_encoder_threads_identical(rans, oracle):
    """The threaded encoder (parallel symbol mapping, histogram and tiles)
    gives the same stream for any thread count, escapes included."""
    codes = oracle.synth_codes(1536, 1024, 3.25, seed=21)
    rng = np.random.default_rng(21)
    hit = rng.random(codes.shape) < 0.003
    codes[hit] = rng.integers(128, 900, size=int(hit.sum()))
    a = rans.encode(codes, 8, 512, 1, threads=1)
    for th in (3, 8):
        b = rans.encode(codes, 8, 512, 1, threads=th)
        for k in ("words", "tile_off", "slen", "tile_meta", "table", "esc_tileptr", "esc_pos",
                  "esc_val"):
            np.testing.assert_array_equal(a[k], b[k])
        assert a["entropy_model"] == b["entropy_model"]


def test_bench_generators(rans, oracle, golden):
    import rans_bench as B
    for i in range(4):
        rows, cols, R, C = (int(v) for v in golden[f"enc{i}_meta"])
        bits = float(golden[f"enc{i}_bits"][0])
        np.testing.assert_array_equal(B.synth_codes(rows, cols, bits, seed=rows),
                                      golden[f"enc{i}_codes"])
    c = B.synth_codes_full(512, 1024, 3.25, seed=5)
    assert abs(B.entropy(c) - 3.25) <= 0.005
    assert B.entropy_fast(c) == pytest.approx(B.entropy(c), abs=1e-12)
    c = B.synth_codes_full(256, 1024, 2.25, dist="student3", seed=6, escape_frac=0.01)
    assert abs(int(((c < -127) | (c > 127)).sum()) - 0.01 * c.size) <= 0.002 * c.size
    st = B.lognormal_steps(1024, seed=1)
    assert st.shape == (1024,) and np.all(st > 0)
    for rows, cols in [(1536, 8960), (8960, 1536), (256, 1536), (25600, 5120)]:
        for S in (1, 2):
            R, C = B.pick_tiling(rows, cols, S=S)
            assert rows % R == 0 and cols % C == 0 and C % (64 * S) == 0


def test_w64_format_golden(rans):
    """The encoder's exact output on the committed fixture (escapes, two
    states per lane, 35-row tiles): a change to the stream bytes is a
    format change.  tests/golden/make_w64_golden.py wrote the fixture."""
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "w64_format_vectors.npz")
    g = np.load(path)
    for name in ("esc", "s2", "r35"):
        rows, cols, R, C, S, mtw, msw = (int(v) for v in g[f"{name}_meta"])
        codes = g[f"{name}_codes"].astype(np.int32)
        assert codes.shape == (rows, cols)
        enc = rans.encode(codes, R, C, S)
        for k in ("words", "tile_off", "tile_meta", "slen", "esc_tileptr", "esc_pos", "esc_val"):
            np.testing.assert_array_equal(enc[k], g[f"{name}_{k}"], err_msg=f"{name}.{k}")
        assert (enc["max_tile_words"], enc["max_state_words"]) == (mtw, msw)
        np.testing.assert_array_equal(rans.decode_ref(enc), codes)
