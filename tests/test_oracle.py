"""Pins the CPU oracle (oracle/) before anything is checked against it:
the reference's own vectors (tests/golden/reference_vectors.npz, written by
tests/golden/make_golden.py from kernel/rans.py and kernel/bench.py), the 18
published benchmark records (results/kernel_bench.json: exact entropies and
emitted word counts), closed forms and brute force."""
import itertools
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TABLE_CASES = ["two_symbols", "tie_argmax", "rare_overflow", "half_even", "laplace", "uniform256"]


@pytest.mark.parametrize("name", TABLE_CASES)
def test_build_table_matches_reference(oracle, golden, name):
    sym = golden[f"tab_{name}_sym"]
    for fn in (oracle.build_table, oracle.build_table_np):
        freq, cum, table = fn(sym)
        np.testing.assert_array_equal(freq, golden[f"tab_{name}_freq"])
        np.testing.assert_array_equal(cum, golden[f"tab_{name}_cum"])
        np.testing.assert_array_equal(table, golden[f"tab_{name}_table"])


@pytest.mark.parametrize("name", TABLE_CASES)
def test_table_is_textbook_rans_slot_map(oracle, golden, name):
    """Every slot decodes to the symbol whose [cum, cum+freq) interval holds
    it, with bias = slot - cum (Duda's static rANS decode table)."""
    sym = golden[f"tab_{name}_sym"]
    freq, cum, table = oracle.build_table(sym)
    counts = np.bincount(sym, minlength=256)
    assert freq.sum() == oracle.M
    assert np.all((freq >= 1) == (counts > 0))
    assert freq.max() < oracle.M
    slots = np.arange(oracle.M)
    s = table & 0xFF
    f = (table >> 8) & 0xFFF
    b = table >> 20
    np.testing.assert_array_equal(f, freq[s])
    np.testing.assert_array_equal(b, slots - cum[s])
    assert np.all((cum[s] <= slots) & (slots < cum[s] + freq[s]))


def test_build_table_rejects_degenerate(oracle):
    with pytest.raises(ValueError):
        oracle.build_table(np.full(100, 7, np.uint8))
    with pytest.raises(ValueError):
        oracle.build_table_np(np.full(100, 7, np.uint8))


@pytest.mark.parametrize("i", range(4))
def test_encode_matches_reference_words(oracle, golden, i):
    rows, cols, R, C = (int(v) for v in golden[f"enc{i}_meta"])
    codes = golden[f"enc{i}_codes"].astype(np.int32)
    enc = oracle.encode_ref(codes, R, C)
    np.testing.assert_array_equal(enc["words"], golden[f"enc{i}_words"])
    np.testing.assert_array_equal(enc["offs"], golden[f"enc{i}_offs"])
    np.testing.assert_array_equal(enc["table"], golden[f"enc{i}_table"])
    bits = golden[f"enc{i}_bits"]
    assert enc["bits_payload"] == bits[1]
    assert enc["bits_state_offs"] == bits[2]
    assert enc["bits_table"] == bits[3]
    assert abs(enc["entropy_model"] - bits[4]) < 1e-12


@pytest.mark.parametrize("i", range(4))
def test_decode_reference_stream(oracle, golden, i):
    rows, cols, R, C = (int(v) for v in golden[f"enc{i}_meta"])
    codes = golden[f"enc{i}_codes"].astype(np.int64)
    enc = dict(words=golden[f"enc{i}_words"], offs=golden[f"enc{i}_offs"],
               table=golden[f"enc{i}_table"], R=R, C=C, shape=(rows, cols))
    np.testing.assert_array_equal(oracle.decode_ref(enc), codes)
    if rows * cols <= 64 * 256:
        np.testing.assert_array_equal(oracle.decode_ref_py(enc), codes)


@pytest.mark.parametrize("i", range(4))
def test_synth_codes_matches_reference(oracle, golden, i):
    rows, cols, R, C = (int(v) for v in golden[f"enc{i}_meta"])
    bits = float(golden[f"enc{i}_bits"][0])
    codes = oracle.synth_codes(rows, cols, bits, seed=rows)
    np.testing.assert_array_equal(codes, golden[f"enc{i}_codes"])
    assert oracle.entropy(codes) == golden[f"enc{i}_bits"][5]


def test_synth_codes_gauss_matches_reference(oracle, golden):
    np.testing.assert_array_equal(oracle.synth_codes(48, 96, 2.5, dist="gauss", seed=7),
                                  golden["synth_gauss_48x96_2.5_seed7"])


def _records():
    with open(os.path.join(GOLDEN, "kernel_bench_records.json")) as f:
        return json.load(f)


def _entropy_bincount(codes):
    cnt = np.bincount((codes.ravel() + 127).astype(np.int64))
    cnt = cnt[cnt > 0]
    p = cnt / cnt.sum()
    return float(-(p * np.log2(p)).sum())


def _record_params():
    # all 18 records at full size (about 90 s on 8 cores, the 178M-weight
    # shape 13-18 s each)
    return [pytest.param(r, id=f"{r['rows']}x{r['cols']}@{r['target_bits']}")
            for r in _records()]


@pytest.mark.parametrize("rec", _record_params())
def test_published_record_word_count(oracle, rec):
    """Entropy to 1e-12 and the exact emitted word count of every published
    record: pins synth_codes, build_table, lane_order and the encoder's
    renormalisation rule at full size (e.g. 2,583,223 words at 1536x8960)."""
    codes = oracle.synth_codes(rec["rows"], rec["cols"], rec["target_bits"], seed=rec["seed"])
    assert abs(_entropy_bincount(codes) - rec["entropy"]) < 1e-12
    assert oracle.count_words_ref(codes, rec["R"], rec["C"]) == rec["payload_words"]
    N = rec["rows"] * rec["cols"]
    lanes = (rec["rows"] // rec["R"]) * (rec["cols"] // rec["C"]) * 32
    assert abs((64 * lanes + 32 * 4096) / N - rec["bits_overhead"]) < 1e-12


def _encode_streams(oracle, S, freq, cum):
    """Reference-layout encode of an arbitrary lane-major symbol matrix."""
    import ctypes
    lib = oracle.load()
    S = np.ascontiguousarray(S, np.uint8)
    lanes, n = S.shape
    cap = lanes * (n + 2) + 8
    words = np.zeros(cap, np.uint16)
    offs = np.zeros(lanes, np.uint32)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    rc = lib.orc_encode_lanes(p(S), lanes, n, p(freq), p(cum), p(words), cap, p(offs))
    assert rc == 0
    return words, offs


def _decode_streams(oracle, words, offs, lanes, n, table):
    import ctypes
    lib = oracle.load()
    out = np.zeros((lanes, n), np.uint8)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    rc = lib.orc_decode_lanes(p(words), words.size, p(offs), lanes, n, p(table), p(out))
    return rc, out


@pytest.mark.parametrize("freqs", [(3000, 1000, 96), (4094, 1, 1), (1365, 1365, 1366)])
def test_bruteforce_round_trip(oracle, freqs):
    """Every sequence of length 1..7 over a 3-symbol alphabet (including one
    at probability 1/4096, 12 bits per symbol) round-trips and ends in 2^16."""
    sym_ids = np.array([5, 128, 250])
    counts = np.zeros(256, np.int64)
    counts[sym_ids] = freqs
    sym = np.repeat(np.arange(256, dtype=np.uint8), counts)
    freq, cum, table = oracle.build_table(sym)
    np.testing.assert_array_equal(freq[sym_ids], freqs)
    for n in range(1, 8):
        seqs = np.array(list(itertools.product(range(3), repeat=n)), np.int64)
        S = sym_ids[seqs].astype(np.uint8)
        words, offs = _encode_streams(oracle, S, freq, cum)
        rc, out = _decode_streams(oracle, words, offs, S.shape[0], n, table)
        assert rc == 0
        np.testing.assert_array_equal(out, S)
        # renormalisation emits at most one word per symbol
        lens = np.diff(offs.astype(np.int64)) - 2
        assert np.all((lens >= 0) & (lens <= n))


def test_word_count_tracks_information(oracle):
    """Emitted bits approach the model information content: sum(-log2 p)
    minus the final-state slack (16 + log2 of the final state - 16 bits)."""
    rng = np.random.default_rng(3)
    codes = np.clip(np.round(rng.laplace(size=(256, 512)) * 2), -127, 127).astype(np.int32)
    enc = oracle.encode_ref(codes, 8, 512)
    sym = (codes.ravel() + 128).astype(np.uint8)
    freq = oracle.build_table(sym)[0]
    info = float(-np.log2(freq[sym] / oracle.M).sum())
    emitted = 16 * int(enc["counts"].sum())
    lanes = len(enc["offs"])
    # each lane's final state carries between 0 and 16 bits of the message;
    # integer division costs a small fraction of a bit per symbol
    assert info - 16 * lanes - 0.01 * codes.size <= emitted <= info + 0.01 * codes.size


def test_decode_detects_truncation(oracle, golden):
    rows, cols, R, C = (int(v) for v in golden["enc0_meta"])
    words = golden["enc0_words"].copy()
    offs = golden["enc0_offs"].copy()
    # drop the first lane's initial state: every lane reads a shifted stream
    enc = dict(words=words[1:], offs=np.maximum(offs.astype(np.int64) - 1, 0).astype(np.uint32),
               table=golden["enc0_table"], R=R, C=C, shape=(rows, cols))
    with pytest.raises(AssertionError):
        oracle.decode_ref(enc)


def test_gemv_f64_closed_forms(oracle):
    rng = np.random.default_rng(0)
    cols = 96
    x = rng.standard_normal(cols)
    step = rng.random(cols) + 0.5
    eye = np.eye(cols, dtype=np.int32) * 3
    np.testing.assert_array_equal(oracle.gemv_f64(eye, x, step), 3.0 * (x * step))
    codes = rng.integers(-300, 300, size=(40, cols)).astype(np.int32)
    want = codes.astype(np.float64) @ (x * step)
    np.testing.assert_allclose(oracle.gemv_f64(codes, x, step), want, rtol=1e-12, atol=1e-9)
    xb = rng.standard_normal((4, cols))
    yb = oracle.gemv_f64(codes, xb, step)
    np.testing.assert_allclose(yb, (codes.astype(np.float64) @ (xb * step).T).T, rtol=1e-12, atol=1e-9)


@pytest.mark.parametrize("R,C,S", [(1, 64, 1), (4, 128, 1), (2, 256, 2), (8, 512, 4)])
def test_w64_order_is_a_permutation(oracle, R, C, S):
    rows, cols = 16, 1024
    a = np.arange(rows * cols).reshape(rows, cols)
    o = oracle.w64_order(a, R, C, S)
    assert o.shape == ((rows // R) * (cols // C) * 64 * S, (C // (64 * S)) * R)
    np.testing.assert_array_equal(oracle.w64_unorder(o, rows, cols, R, C, S), a)
    # state 0 of tile 0: column 0 then the next column of that state, rows inner
    assert list(o[0, :R]) == [r * cols for r in range(R)]
    if C // (64 * S) > 1:
        assert o[0, R] == 64 * S
    # lane l of state slot s starts at column 64*s + l
    assert o[64 * (S - 1) + 5, 0] == 64 * (S - 1) + 5
