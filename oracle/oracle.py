"""ORACLE -- test infrastructure only.

CPU checker for the entropy-coded GEMV.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this module; the shipped library never does, and the product path fails
loudly without its HIP extension instead of falling back here.

It restates, from scratch, the reference coder of snuri00/vram-compression
(``kernel/rans.py``, ``kernel/bench.py``) in numpy plus the plain-C helpers in
``rans_oracle.c`` (loaded through ctypes):

=====================  =========================================  ==================
function               reference                                  pinned by
=====================  =========================================  ==================
build_table            kernel/rans.py:34-51                       tests/golden fixtures
                                                                  (reference output),
                                                                  C twin, invariants
lane_order/unorder     kernel/rans.py:55-59, 122-123              inverse round trip,
                                                                  golden fixtures
encode_ref             kernel/rans.py:62-98                       golden words/offs,
                                                                  kernel_bench.json
                                                                  word counts
decode_ref_py /        kernel/rans.py:101-123                     round trip, golden
decode_ref                                                        fixtures, brute force
entropy, synth_codes   kernel/bench.py:20-35                      kernel_bench.json
                                                                  entropies
gemv_f64               kernel/rans_gemv.cu:4-6 (y = code@(x*s))   closed form on
                                                                  one-hot codes
w64_* (layout of the   the same per-stream arithmetic on the      round trip and
wavefront format)      64-lane layout this library ships          per-stream equality
                                                                  with encode_ref
=====================  =========================================  ==================
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

SCALE_BITS = 12
M = 1 << SCALE_BITS
RANS_L = 1 << 16
OFFSET = 128
ESC = 0  # symbol 0 (code -128 in the reference alphabet) is the escape symbol

_lib = None


def load():
    """ctypes handle on the C restatement (built by oracle/Makefile)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
    lib = ctypes.CDLL(LIB_PATH)
    P = ctypes.c_void_p
    I64 = ctypes.c_int64
    lib.orc_build_table.argtypes = [P, I64, P, P, P]
    lib.orc_count_words.argtypes = [P, I64, I64, P, P, P]
    lib.orc_encode_lanes.argtypes = [P, I64, I64, P, P, P, I64, P]
    lib.orc_decode_streams.argtypes = [P, I64, P, P, I64, I64, P, P]
    lib.orc_decode_lanes.argtypes = [P, I64, P, I64, I64, P, P]
    lib.orc_gemv_f64.argtypes = [P, I64, I64, P, I64, P, P]
    for f in (lib.orc_build_table, lib.orc_count_words, lib.orc_encode_lanes,
              lib.orc_decode_streams, lib.orc_decode_lanes, lib.orc_gemv_f64):
        f.restype = ctypes.c_int
    _lib = lib
    return lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


# ----------------------------------------------------------------- bench.py
def entropy(codes):
    """Empirical entropy in bits/symbol (kernel/bench.py:20-23)."""
    _, c = np.unique(codes, return_counts=True)
    p = c / c.sum()
    return float(-(p * np.log2(p)).sum())


def synth_codes(rows, cols, target_bits, dist="laplace", seed=0):
    """kernel/bench.py:26-35: w ~ Laplace (or N(0,1)) from default_rng(seed);
    40-step bisection of log(step) in [-12, 6] on the entropy of the first
    min(rows, 256) rows; codes = clip(round(w/step), -127, 127)."""
    rng = np.random.default_rng(seed)
    w = rng.laplace(size=(rows, cols)) if dist == "laplace" else rng.standard_normal((rows, cols))
    lo, hi = -12.0, 6.0
    for _ in range(40):
        mid = (lo + hi) / 2
        h = entropy(np.round(w[: min(rows, 256)] / np.exp(mid)))
        lo, hi = (mid, hi) if h > target_bits else (lo, mid)
    return np.clip(np.round(w / np.exp((lo + hi) / 2)), -127, 127).astype(np.int32)


# ------------------------------------------------------------------- table
def build_table_np(sym):
    """numpy restatement of kernel/rans.py:34-51 (kept separate from the C
    twin so each checks the other)."""
    counts = np.bincount(np.asarray(sym, np.uint8).ravel(), minlength=256).astype(np.float64)
    if counts.sum() == 0:
        raise ValueError("empty symbol array")
    present = counts > 0
    freq = np.zeros(256, np.int64)
    freq[present] = np.maximum(1, np.round(counts[present] * M / counts.sum())).astype(np.int64)
    while freq.sum() != M:
        diff = M - freq.sum()
        i = int(np.argmax(freq))
        freq[i] += max(diff, 1 - freq[i]) if diff < 0 else diff
    if freq.max() >= M:
        raise ValueError("degenerate distribution (single symbol)")
    cum = np.concatenate([[0], np.cumsum(freq)[:-1]]).astype(np.int64)
    table = np.zeros(M, np.uint32)
    for s in np.nonzero(freq)[0]:
        k = np.arange(freq[s], dtype=np.uint32)
        table[cum[s] + k] = np.uint32(s) | (np.uint32(freq[s]) << 8) | (k << 20)
    return freq, cum, table


def build_table(sym):
    """C restatement of kernel/rans.py:34-51 (same contract as build_table_np)."""
    lib = load()
    s = np.ascontiguousarray(np.asarray(sym, np.uint8).ravel())
    freq = np.zeros(256, np.int64)
    cum = np.zeros(256, np.int64)
    table = np.zeros(M, np.uint32)
    rc = lib.orc_build_table(_p(s), s.size, _p(freq), _p(cum), _p(table))
    if rc == -1:
        raise ValueError("empty symbol array")
    if rc == -2:
        raise ValueError("degenerate distribution (single symbol)")
    return freq, cum, table


# -------------------------------------------------------- reference layout
def lane_order(sym, R, C):
    """kernel/rans.py:55-59: (rb r cb k l) -> (rb cb l k r), 32 lanes."""
    rows, cols = sym.shape
    if rows % R or cols % C or C % 32:
        raise ValueError("shape not divisible by R, C or C % 32 != 0")
    a = sym.reshape(rows // R, R, cols // C, C // 32, 32)
    return a.transpose(0, 2, 4, 3, 1).reshape(-1, (C // 32) * R)


def lane_unorder(S, rows, cols, R, C):
    """Inverse of lane_order (kernel/rans.py:122-123)."""
    a = S.reshape(rows // R, cols // C, 32, C // 32, R).transpose(0, 4, 1, 3, 2)
    return a.reshape(rows, cols)


def encode_ref(codes, R, C):
    """kernel/rans.py:62-98 (reference 32-lane layout), via the C twin."""
    lib = load()
    sym = codes.astype(np.int64) + OFFSET
    if sym.min() < 0 or sym.max() > 255:
        raise ValueError("code out of 8-bit alphabet")
    sym = sym.astype(np.uint8)
    freq, cum, table = build_table(sym)
    S = np.ascontiguousarray(lane_order(sym, R, C))
    lanes, n = S.shape
    counts = np.zeros(lanes, np.int64)
    rc = lib.orc_count_words(_p(S), lanes, n, _p(freq), _p(cum), _p(counts))
    assert rc == 0, rc
    cap = int(counts.sum()) + 2 * lanes + 8
    words = np.zeros(cap, np.uint16)
    offs = np.zeros(lanes, np.uint32)
    rc = lib.orc_encode_lanes(_p(S), lanes, n, _p(freq), _p(cum), _p(words), cap, _p(offs))
    assert rc == 0, rc
    N = codes.size
    p = freq[sym.ravel()] / M
    return dict(words=words, offs=offs, table=table, R=R, C=C, shape=codes.shape,
                bits_payload=16 * int(counts.sum()) / N, bits_state_offs=64 * lanes / N,
                bits_table=32 * M / N, entropy_model=float(-np.log2(p).mean()),
                counts=counts)


def count_words_ref(codes, R, C):
    """Total emitted words of encode_ref without building the stream."""
    lib = load()
    sym = (codes.astype(np.int64) + OFFSET).astype(np.uint8)
    freq, cum, _ = build_table(sym)
    S = np.ascontiguousarray(lane_order(sym, R, C))
    counts = np.zeros(S.shape[0], np.int64)
    rc = lib.orc_count_words(_p(S), S.shape[0], S.shape[1], _p(freq), _p(cum), _p(counts))
    assert rc == 0, rc
    return int(counts.sum())


def decode_ref(enc):
    """kernel/rans.py:101-123 via the C twin (raises on a bad final state)."""
    lib = load()
    rows, cols = enc["shape"]
    R, C = enc["R"], enc["C"]
    lanes = len(enc["offs"])
    n = (C // 32) * R
    out = np.zeros((lanes, n), np.uint8)
    w = np.ascontiguousarray(enc["words"], np.uint16)
    rc = lib.orc_decode_lanes(_p(w), w.size, _p(np.ascontiguousarray(enc["offs"], np.uint32)),
                              lanes, n, _p(np.ascontiguousarray(enc["table"], np.uint32)), _p(out))
    if rc != 0:
        raise AssertionError(f"stream did not return to initial state (lane {-rc - 1})")
    return lane_unorder(out.astype(np.int64) - OFFSET, rows, cols, R, C)


def decode_ref_py(enc, max_lanes=None):
    """Pure-Python scalar loop, one lane at a time (kernel/rans.py:101-123).
    For small inputs only; also the scalar CPU baseline.  With max_lanes, only
    the first max_lanes lanes are decoded and their lane-major symbol rows
    returned (a bounded timing sample)."""
    rows, cols = enc["shape"]
    R, C = enc["R"], enc["C"]
    tab = enc["table"].astype(np.int64).tolist()
    lanes = len(enc["offs"]) if max_lanes is None else min(max_lanes, len(enc["offs"]))
    # lanes' streams are consecutive: a sample converts only the words it reads
    end = len(enc["words"]) if lanes == len(enc["offs"]) else int(enc["offs"][lanes])
    w = enc["words"][:end].astype(np.int64).tolist()
    n = (C // 32) * R
    S = np.zeros((lanes, n), np.int64)
    for li in range(lanes):
        p = int(enc["offs"][li])
        st = (w[p] << 16) | w[p + 1]
        p += 2
        row = S[li]
        for i in range(n):
            e = tab[st & (M - 1)]
            st = ((e >> 8) & 0xFFF) * (st >> SCALE_BITS) + (e >> 20)
            if st < RANS_L:
                st = (st << 16) | w[p]
                p += 1
            row[i] = (e & 0xFF) - OFFSET
        if st != RANS_L:
            raise AssertionError("stream did not return to initial state")
    if max_lanes is not None:
        return S
    return lane_unorder(S, rows, cols, R, C)


# ------------------------------------------- wavefront (64-lane) layout
def w64_order(sym, R, C, S):
    """Symbol sequence of every state of the 64-lane layout, lane-major.

    Tile (rb, cb) holds rows rb*R.. and columns cb*C..; state j = s*64 + l
    decodes, for k in range(C // (64*S)) and r in range(R) (k-major, r-minor),
    the symbol at row rb*R + r, column cb*C + 64*(S*k + s) + l."""
    rows, cols = sym.shape
    a = sym.reshape(rows // R, R, cols // C, C // (64 * S), S, 64)  # rb r cb k s l
    return a.transpose(0, 2, 4, 5, 3, 1).reshape(-1, (C // (64 * S)) * R)


def w64_unorder(Sm, rows, cols, R, C, S):
    a = Sm.reshape(rows // R, cols // C, S, 64, C // (64 * S), R)  # rb cb s l k r
    return a.transpose(0, 5, 1, 4, 2, 3).reshape(rows, cols)


def w64_decode(enc):
    """Decode an encoded matrix of the 64-lane layout to int64 codes on the
    CPU: the reference per-stream step (kernel/rans.py:110-121) on every
    state, then the inverse layout permutation, then the escape side table.
    Raises AssertionError on a stream that does not end in state 2^16."""
    lib = load()
    rows, ocols = enc["shape"]
    # the stream's columns: the matrix's own plus any appended to reach a
    # multiple of 64 (dropped from the result)
    cols = int(enc.get("stream_cols", ocols))
    # the w64 tiling (tile_R, tile_C); R and C of the dict are the tiling the
    # encoder was asked for, which it may have mapped to another tile
    R, C, S = enc.get("tile_R", enc["R"]), enc.get("tile_C", enc["C"]), enc["S"]
    tile_off = enc["tile_off"].astype(np.int64)
    ntiles = (rows // R) * (cols // C)
    nst = 64 * S
    n = (C // nst) * R
    w = np.ascontiguousarray(enc["words"], np.uint16)
    # a tile block opens with its states' initial values, each as 16 + e
    # bits below an implicit leading one (e in the high half of the state's
    # slen byte), bit-packed in state order (bit i of the block is bit i%16
    # of its word i/16); blob_words (tile_meta >> 16) words of them, then the
    # streams in state order, each base (tile_meta & 255) + (slen & 15) words
    meta = enc["tile_meta"].astype(np.int64)[:ntiles]
    sl = enc["slen"].astype(np.int64).reshape(ntiles, nst)
    nb = 16 + (sl >> 4)
    bit0 = tile_off[:ntiles, None] * 16 + np.cumsum(nb, axis=1) - nb
    if np.any(np.cumsum(nb, axis=1)[:, -1] > 16 * (meta >> 16)):
        raise AssertionError("initial states overrun their tile's blob")
    mant = np.zeros((ntiles, nst), np.int64)
    for i in range(31):
        b = bit0 + i
        bitv = (w[np.minimum(b >> 4, w.size - 1)].astype(np.int64) >> (b & 15)) & 1
        mant |= np.where(i < nb, bitv << i, 0)
    st0 = (mant | (np.int64(1) << nb)).ravel().astype(np.uint32)
    slen = (meta & 0xFF)[:, None] + (sl & 15)
    starts_in_tile = (meta >> 16)[:, None] + np.cumsum(slen, axis=1) - slen
    start = (tile_off[:ntiles, None] + starts_in_tile).ravel()
    out = np.zeros((ntiles * nst, n), np.uint8)
    start = np.ascontiguousarray(start, np.int64)
    rc = lib.orc_decode_streams(_p(w), w.size, _p(st0), _p(start), ntiles * nst, n,
                                _p(np.ascontiguousarray(enc["table"], np.uint32)), _p(out))
    if rc != 0:
        raise AssertionError(f"stream did not return to initial state (state {-rc - 1})")
    sym = w64_unorder(out, rows, cols, R, C, S)
    codes = sym.astype(np.int64) - OFFSET
    esc_mask = sym == ESC
    # side table per tile: tile t owns entries tp[t]..tp[t+1], each at tile
    # row pos % R, tile column pos // R, strictly ascending within the tile
    tp = enc["esc_tileptr"].astype(np.int64)
    pos = enc["esc_pos"].astype(np.int64)
    eval_ = enc["esc_val"].astype(np.int64)
    if tp.size != ntiles + 1 or tp[0] != 0 or np.any(np.diff(tp) < 0) or tp[-1] != pos.size:
        raise AssertionError("escape tile pointers malformed")
    t = np.repeat(np.arange(ntiles), np.diff(tp))
    r, c = pos % R, pos // R
    if np.any(pos < 0) or np.any(c >= C):
        raise AssertionError("escape position outside its tile")
    same = t[1:] == t[:-1]
    if np.any(pos[1:][same] <= pos[:-1][same]):
        raise AssertionError("escape positions not strictly ascending within a tile")
    ncb = cols // C
    er, ec = (t // ncb) * R + r, (t % ncb) * C + c
    flagged = np.zeros_like(esc_mask)
    flagged[er, ec] = True
    if not np.array_equal(flagged, esc_mask):
        raise AssertionError("escape side table disagrees with escape symbols in the stream")
    codes[er, ec] = eval_
    return codes[:, :ocols]


# ---------------------------------------------------------------- gemv
def gemv_f64(codes, x, step):
    """y = codes @ (x * step) in float64 (kernel/rans_gemv.cu:4-6).
    x is (cols,) or (B, cols); returns (rows,) or (B, rows)."""
    lib = load()
    c = np.ascontiguousarray(codes, np.int32)
    rows, cols = c.shape
    xb = np.atleast_2d(np.asarray(x, np.float64))
    xb = np.ascontiguousarray(xb)
    st = np.ascontiguousarray(np.asarray(step, np.float64).reshape(cols))
    y = np.zeros((xb.shape[0], rows), np.float64)
    rc = lib.orc_gemv_f64(_p(c), rows, cols, _p(xb), xb.shape[0], _p(st), _p(y))
    assert rc == 0
    return y[0] if np.ndim(x) == 1 else y
