"""Host side of the wavefront-interleaved rANS GEMV for MI355X: table
building, the w64 encoder and host decoder (C++ in librans_hip.so), and
ctypes wrappers around the HIP kernels.

Mirrors the interface of kernel/rans.py of snuri00/vram-compression:
``build``, ``build_table``, ``lane_order``, ``encode``, ``decode_ref``,
``RansMatrix`` (``.gemv``, ``.decode``, ``.nbytes``) and ``Int4Matrix``, with
the same argument meaning and the same assert-on-error behaviour.  What
changes is the stream layout (64-lane tiles, S states per lane, escapes), so
``encode`` takes an extra ``S`` and accepts codes outside [-128, 127].

PyTorch is used only for device buffers and streams; every GPU operation is
a hand-written HIP kernel in librans_hip.so.  There is no CPU fallback:
``RansMatrix`` raises when the library or a GPU is missing.
"""
import copy
import ctypes
import os
import subprocess

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
LIB = os.path.join(HERE, "librans_hip.so")
SOURCES = [os.path.join(CSRC, "rans_gemv.hip"), os.path.join(CSRC, "ref32_gemv.hip"),
           os.path.join(CSRC, "w64_host.cpp")]
HEADERS = [os.path.join(INCLUDE, "vramc_rans.h")]

SCALE_BITS = 12
M = 1 << SCALE_BITS
RANS_L = 1 << 16
OFFSET = 128
ESC = 0  # escape symbol: codes outside [-127, 127]
LANES = 64

X_F32, X_BF16 = 0, 1
# stream layouts, recorded as enc["layout"]: the wavefront-interleaved w64
# format of `encode`, and the reference's own 32-lane format
# (encode_reference_layout, or the reference's encode itself)
LAYOUT_W64, LAYOUT_REF32 = "w64", "ref32"
# rans_w64_matrix.flags: word fetch of the GEMV (0 = library default), and
# the empty-side-table promise (set by RansMatrix itself)
F_WORDS_ALWAYS, F_WORDS_REFILL, F_WORDS_MASK, F_NO_ESCAPES = 1, 2, 3, 4
F_TABLE8, F_TABLE4 = 8, 16
# tile heights with compiled kernels.  SUPPORTED_R are the candidates of
# every tiling choice (35 only with one state per lane); LARGE_R (one state
# per lane) are compiled for large matrices, where pick_tiling considers
# them too, and taken wherever a caller asks for them.
SUPPORTED_R = (35, 16, 8, 4, 3, 2, 1)
LARGE_R = (20,)
ONE_STATE_R = (35,) + LARGE_R

HIPCC_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared",
               # packed fp32 VALU ops stay disabled on this platform
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


class RansMatrixDesc(ctypes.Structure):
    """ctypes mirror of rans_w64_matrix (include/vramc_rans.h)."""
    _fields_ = [("rows", ctypes.c_int32), ("cols", ctypes.c_int32),
                ("R", ctypes.c_int32), ("C", ctypes.c_int32), ("S", ctypes.c_int32),
                ("max_tile_words", ctypes.c_int32), ("max_state_words", ctypes.c_int32),
                ("flags", ctypes.c_int32),
                ("words", ctypes.c_void_p), ("tile_off", ctypes.c_void_p),
                ("slen", ctypes.c_void_p), ("tile_meta", ctypes.c_void_p),
                ("table", ctypes.c_void_p), ("table_lds", ctypes.c_void_p),
                ("esc_tileptr", ctypes.c_void_p),
                ("esc_pos", ctypes.c_void_p), ("esc_val", ctypes.c_void_p),
                ("step", ctypes.c_void_p), ("workspace", ctypes.c_void_p),
                ("workspace_bytes", ctypes.c_int64), ("table_lds4", ctypes.c_void_p)]


EXPORTS = ("rans_w64_gemv", "rans_w64_gemv_noalloc", "rans_gemv_workspace_bytes", "rans_gemv_table4",
           "rans_gemv_rows2", "rans_w64_gemv_group", "launch_rans_gemv", "launch_rans_decode",
           "rans_w64_decode",
           "rans_w64_decode_codes", "launch_int4_gemv", "bf16_gemv", "rans_build_table",
           "rans_table_lds",
           "rans_table_lds4",
           "rans_w64_encode", "rans_w64_encode_fetch", "rans_w64_encode_counts",
           "rans_w64_encode_free",
           "rans_w64_decode_host", "rans_ref32_encode")


def compile_lib(arch="gfx950", out=LIB):
    """Compile librans_hip.so with hipcc for ``arch`` (always recompiles)."""
    tmp = out + ".tmp"
    cmd = ["hipcc", f"--offload-arch={arch}", *HIPCC_FLAGS, "-o", tmp, *SOURCES]
    subprocess.check_call(cmd, stderr=subprocess.DEVNULL if os.environ.get("RANS_QUIET") else None)
    os.replace(tmp, out)
    return out


def _stale(lib):
    if not os.path.exists(lib):
        return True
    t = os.path.getmtime(lib)
    return any(os.path.getmtime(s) > t for s in SOURCES + HEADERS)


def load_lib(path=LIB):
    """ctypes handle with argtypes set for every exported symbol; raises
    AttributeError if one is missing (as rans.py:25-29 does)."""
    lib = ctypes.CDLL(path)
    P, I32, I64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    D = ctypes.POINTER(RansMatrixDesc)
    sig = {
        "rans_w64_gemv": ([D, P, ctypes.c_int, ctypes.c_int, P, P], ctypes.c_int),
        "rans_w64_gemv_noalloc": ([D, P, ctypes.c_int, ctypes.c_int, P, P], ctypes.c_int),
        "rans_gemv_workspace_bytes": ([D, ctypes.c_int], I64),
        "rans_gemv_table4": ([D, ctypes.c_int, ctypes.c_int], ctypes.c_int),
        "rans_gemv_rows2": ([D, ctypes.c_int, ctypes.c_int], ctypes.c_int),
        "rans_w64_gemv_group": ([P, ctypes.c_int, P, ctypes.c_int, ctypes.c_int, P, P],
                                ctypes.c_int),
        # the reference's own argument lists and stream format
        # (kernel/rans.py:25-29)
        "launch_rans_gemv": ([ctypes.c_int] + [P] * 5 + [ctypes.c_int] * 3 + [P], ctypes.c_int),
        "launch_rans_decode": ([ctypes.c_int] + [P] * 5 + [ctypes.c_int] * 3 + [P], ctypes.c_int),
        "rans_w64_decode": ([D, P, P], ctypes.c_int),
        "rans_w64_decode_codes": ([D, P, P], ctypes.c_int),
        "launch_int4_gemv": ([P, P, P, ctypes.c_int, ctypes.c_int, P], ctypes.c_int),
        "bf16_gemv": ([P, P, P, ctypes.c_int, ctypes.c_int, P], ctypes.c_int),
        "rans_build_table": ([P, I64, P, P, P], ctypes.c_int),
        "rans_table_lds": ([P, P], ctypes.c_int),
        "rans_table_lds4": ([P, P], ctypes.c_int),
        "rans_w64_encode": ([P, I32, I32, I32, I32, I32, I32, ctypes.POINTER(P), P], ctypes.c_int),
        "rans_w64_encode_fetch": ([P] * 10, ctypes.c_int),
        "rans_w64_encode_counts": ([P, P], ctypes.c_int),
        "rans_w64_encode_free": ([P], None),
        "rans_w64_decode_host": ([D, P], ctypes.c_int),
        "rans_ref32_encode": ([P, I32, I32, I32, I32, I32, P, I64, P, P, P], ctypes.c_int),
    }
    for name, (args, res) in sig.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = res
    return lib


_LIB = None


def build(arch="gfx950"):
    """Compile librans_hip.so when a source is newer than it (rans.py:19-30)
    and return the ctypes handle."""
    global _LIB
    if _stale(LIB):
        compile_lib(arch)
        _LIB = None
    if _LIB is None:
        _LIB = load_lib(LIB)
    return _LIB


def _host_lib():
    """The library for host-only calls (encoder, table, host decoder)."""
    return _LIB if _LIB is not None else build()


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


# --------------------------------------------------------------------- table
def build_table(sym):
    """sym: uint8 symbols.  Returns (freq[256], cum[256], table[4096]) with
    12-bit probabilities, the quantisation of rans.py:34-51."""
    s = np.ascontiguousarray(np.asarray(sym, np.uint8).ravel())
    freq = np.zeros(256, np.int64)
    cum = np.zeros(256, np.int64)
    table = np.zeros(M, np.uint32)
    rc = _host_lib().rans_build_table(_p(s), s.size, _p(freq), _p(cum), _p(table))
    assert rc == 0, "degenerate distribution (single symbol)"
    return freq, cum, table


def table_lds(table, lib=None):
    """The 32 KB LDS image of a packed table (uint32[8192]): per slot
    {freq | code<<24, slot - cum}, code 0 for the escape symbol."""
    t = np.ascontiguousarray(np.asarray(table, np.uint32).ravel())
    assert t.size == M, "table must have 4096 slots"
    out = np.zeros(2 * M, np.uint32)
    rc = (lib or _host_lib()).rans_table_lds(_p(t), _p(out))
    assert rc == 0, f"rans_table_lds failed ({rc})"
    return out


def table_lds4(table, lib=None):
    """The 16 KB image of 4-byte LDS entries (uint32[4096]): per slot
    freq | (slot - cum)<<12 | code<<24, code 0 for the escape symbol."""
    t = np.ascontiguousarray(np.asarray(table, np.uint32).ravel())
    assert t.size == M, "table must have 4096 slots"
    out = np.zeros(M, np.uint32)
    rc = (lib or _host_lib()).rans_table_lds4(_p(t), _p(out))
    assert rc == 0, f"rans_table_lds4 failed ({rc})"
    return out


# ------------------------------------------------------------------ encoding
def lane_order(sym, R, C, S=1):
    """Symbols in decode order, one row per rANS state (rans.py:55-59 for the
    64-lane layout): tile (rb, cb), state j = s*64 + l, symbol i = k*R + r is
    sym[rb*R + r, cb*C + 64*(S*k + s) + l]."""
    rows, cols = sym.shape
    assert rows % R == 0 and cols % C == 0 and C % (LANES * S) == 0
    a = sym.reshape(rows // R, R, cols // C, C // (LANES * S), S, LANES)  # rb r cb k s l
    return a.transpose(0, 2, 4, 5, 3, 1).reshape(-1, (C // (LANES * S)) * R)


# Longest state sequence whose stream length fits the byte-wide slen: a
# symbol adds at most 12 bits, so n symbols emit at most 0.75n + 1 words.
MAX_STATE_SYMBOLS = 338
MAX_TILE_CODES = 65536  # 16-bit tile-local escape positions


def w64_stream_cols(cols):
    """Columns of the stored stream for a matrix of `cols` columns: cols
    itself when it is a multiple of 64 (one column per wavefront lane), else
    cols + 32 (the reference accepts any multiple of 32, kernel/rans.py:57;
    encode appends 32 columns of code 0, which the GEMV multiplies by a zero
    step and a zero x, and which decoding drops)."""
    assert cols % 32 == 0, "cols must be a multiple of 32"
    return cols + (-cols) % LANES


def stream_cols(enc):
    """Stored columns of an encoded matrix (its logical cols, or cols + 32)."""
    return int(enc.get("stream_cols", enc["shape"][1]))


def w64_tiling(rows, cols, R, C, S=None):
    """The w64 tiling (tile_R, tile_C, S) that encode uses for a requested
    (R, C): the reference's tiling parameters (kernel/rans.py:55-59, any
    R dividing rows and C dividing cols with C % 32 == 0) mapped to a legal
    tile of this format, over w64_stream_cols(cols) columns.  The decoded
    codes and GEMV results do not depend on the tiling; only speed and bits
    do.

    - tile_R: the largest compiled tile height dividing R (R = 512 gives 16,
      R = 6 gives 3);
    - tile_C: the widest multiple of 64 dividing C (or 2C when C % 64 == 32:
      two of the reference's 32-lane tiles side by side; when cols % 64 ==
      32 too, the widest multiple of 64 up to 2C that divides the padded
      columns) whose tile holds at most 65536 codes;
    - S: the given S if that tile is legal with it, else the fewest states
      per lane (1, 2, 4) that keep every state at most MAX_STATE_SYMBOLS
      symbols.
    A given S with a tile this format holds as it is ((R, C) compiled and
    within 65536 codes) is kept unchanged; the encoder then rejects a state
    whose stream outgrows its length byte.  A matrix with appended columns
    also takes, beyond the reference's C, a multiple of 64 dividing its
    stored columns (the tiles pick_tiling gives it)."""
    scols = w64_stream_cols(cols)
    # the reference's preconditions; a padded matrix also takes a tile width
    # of its stored columns (what pick_tiling gives it)
    assert rows % R == 0 and C % 32 == 0 and \
        (cols % C == 0 or (scols != cols and scols % C == 0 and C % LANES == 0)), \
        "shape not divisible into R x C tiles with C % 32 == 0"
    if S and R in SUPPORTED_R + LARGE_R and C % (LANES * S) == 0 and R * C <= MAX_TILE_CODES \
            and not (R in ONE_STATE_R and S != 1):
        return R, C, S
    tR = max(r for r in SUPPORTED_R if R % r == 0)
    if C % LANES == 0:
        base = C
    elif scols % (2 * C) == 0:
        base = 2 * C
    else:  # padded columns: the widest multiple of 64 below 2C dividing them
        base = next(c for c in range(2 * C - 2 * C % LANES, 0, -LANES) if scols % c == 0)
    assert scols % base == 0
    Ss = (S,) if S else (1, 2, 4)
    for tC in range(base, 0, -LANES):
        if base % tC or tR * tC > MAX_TILE_CODES:
            continue
        for s in Ss:
            if tC % (LANES * s) or (tR in ONE_STATE_R and s != 1):
                continue
            if tR * tC // (LANES * s) <= MAX_STATE_SYMBOLS:
                return tR, tC, s
    raise AssertionError(f"no legal w64 tiling for R={R}, C={C}, S={S}")


def stream_lengths(enc):
    """Stored words of every state's stream (int64, one per state in state
    order): its tile's base (tile_meta bits 0-7) plus the 4-bit delta in the
    low half of its slen byte."""
    ntiles = enc["tile_off"].size - 1
    base = (enc["tile_meta"].astype(np.int64) & 0xFF)[:ntiles, None]
    return (base + (enc["slen"].astype(np.int64).reshape(ntiles, -1) & 15)).reshape(-1)


def stream_offsets(enc):
    """Start of every state's stream in enc["words"] (uint32 word offsets,
    one per state in state order): the counterpart of the reference's
    per-lane ``offs`` (kernel/rans.py:86), derived from the tile offsets, the
    tile's initial-state words and the per-state stream lengths the format
    stores instead."""
    ntiles = enc["tile_off"].size - 1
    if ntiles == 0:
        return np.zeros(0, np.uint32)
    per = stream_lengths(enc).reshape(ntiles, -1)
    first = enc["tile_off"][:-1].astype(np.int64) + (enc["tile_meta"].astype(np.int64) >> 16)
    start = first[:, None] + np.cumsum(per, axis=1) - per
    return start.reshape(-1).astype(np.uint32)


def initial_states(enc):
    """Every state's initial decoder value (uint32, state order), read back
    from the format: exponent e in the high half of its slen byte, and its
    16 + e bits below the leading one bit-packed at the start of its tile's
    block, state after state (little-endian bit stream of the words)."""
    ntiles = enc["tile_off"].size - 1
    if ntiles == 0:
        return np.zeros(0, np.uint32)
    nst = enc["slen"].size // ntiles
    e = (enc["slen"].astype(np.int64) >> 4).reshape(ntiles, nst)
    nb = 16 + e
    bit = np.cumsum(nb, axis=1) - nb  # within the tile's blob
    words = np.asarray(enc["words"], np.uint16)
    start = enc["tile_off"][:-1].astype(np.int64)[:, None] * 16 + bit  # absolute bit
    x = np.zeros(start.shape, np.int64)
    for i in range(31):  # at most 31 mantissa bits
        b = start + i
        v = (words[np.minimum(b >> 4, words.size - 1)].astype(np.int64) >> (b & 15)) & 1
        x |= np.where(i < nb, v << i, 0)
    return (x | (np.int64(1) << nb)).reshape(-1).astype(np.uint32)


def encode(codes, R, C, S=None, threads=None):
    """codes: integer array (rows x cols) within [-32768, 32767]; values
    outside [-127, 127] go through the escape side table.  (R, C) are the
    reference's tiling parameters (rows % R == cols % C == C % 32 == 0,
    kernel/rans.py:57); the stream is laid out in the w64 tiling
    w64_tiling(rows, cols, R, C, S) gives, recorded as tile_R, tile_C and S.

    Returns a dict with the reference's keys (words, offs, table, R, C,
    shape, bits_payload, bits_state_offs, bits_table, entropy_model,
    rans.py:93-98) and the w64 stream: tile_off, tile_meta, slen (the
    initial states sit bit-packed in the words; initial_states reads them
    back), the escape side table (esc_tileptr, esc_pos, esc_val), tile_R,
    tile_C, S,
    stream_cols, max_tile_words, max_state_words, bits_escape, and
    layout = "w64".  offs keeps the reference's meaning (each stream's first
    word) but there is one stream per 64-lane state, not per 32-lane lane:
    the dict cannot go to launch_rans_gemv / launch_rans_decode or to
    ReferenceLayoutMatrix, which refuses it.  shape is
    the matrix's own; the stream holds stream_cols = w64_stream_cols(cols)
    columns (32 columns of code 0 appended when cols % 64 == 32).  Bit
    accounting, per weight of the matrix: bits_payload (renormalisation
    words), bits_state_offs (initial states, per-state length and exponent
    bytes, tile offsets and metadata, length and tile padding), bits_table
    (16 KB table), bits_escape (side table);
    appended columns are paid for in these.  entropy_model is over the
    matrix's own codes."""
    codes = np.ascontiguousarray(codes, dtype=np.int32)
    assert codes.ndim == 2 and codes.size > 0, "codes must be a non-empty matrix"
    rows, cols = codes.shape
    tR, tC, tS = w64_tiling(rows, cols, R, C, S)
    scols = w64_stream_cols(cols)
    if scols != cols:
        codes = np.ascontiguousarray(np.pad(codes, ((0, 0), (0, scols - cols))))
    lib = _host_lib()
    h = ctypes.c_void_p()
    info = np.zeros(7, np.int64)
    nthreads = threads or min(16, os.cpu_count() or 1)
    rc = lib.rans_w64_encode(_p(codes), rows, scols, tR, tC, tS, nthreads, ctypes.byref(h),
                             _p(info))
    assert rc != -5, "degenerate distribution (single symbol), or a code outside [-32768, 32767]"
    assert rc != -6, "a tile needs more than 65535 words, or a state more than 255: " \
                     "use smaller R or C"
    assert rc != -2, "tile geometry outside the format (R*C <= 65536)"
    assert rc == 0, f"encode failed ({rc})"
    nwords, ntiles, nstates, nesc, max_tile_words, payload_words, max_state_words = \
        (int(v) for v in info)
    words = np.zeros(nwords, np.uint16)
    tile_off = np.zeros(ntiles + 1, np.uint32)
    tile_meta = np.zeros(ntiles, np.uint32)
    slen = np.zeros(nstates, np.uint8)
    table = np.zeros(M, np.uint32)
    freq = np.zeros(256, np.int64)
    esc_tileptr = np.zeros(ntiles + 1, np.int32)
    esc_pos = np.zeros(nesc, np.uint16)
    esc_val = np.zeros(nesc, np.int16)
    counts = np.zeros(256, np.int64)
    try:
        rc = lib.rans_w64_encode_fetch(h, _p(words), _p(tile_off), _p(tile_meta), _p(slen),
                                       _p(table), _p(freq), _p(esc_tileptr), _p(esc_pos),
                                       _p(esc_val))
        assert rc == 0
        assert lib.rans_w64_encode_counts(h, _p(counts)) == 0
    finally:
        lib.rans_w64_encode_free(h)
    N = rows * cols
    counts[OFFSET] -= rows * (scols - cols)  # the appended zeros (symbol of code 0)
    # model entropy: -mean log2 p over the symbols, from the counts
    present = counts > 0
    entropy_model = float(-(counts[present] * np.log2(freq[present] / M)).sum() / N)
    pad_words = nwords - payload_words
    enc = dict(words=words, tile_off=tile_off, tile_meta=tile_meta, slen=slen, table=table,
               esc_tileptr=esc_tileptr, esc_pos=esc_pos, esc_val=esc_val,
               R=R, C=C, tile_R=tR, tile_C=tC, S=tS, shape=(rows, cols), stream_cols=scols,
               max_tile_words=max_tile_words, max_state_words=max_state_words,
               bits_payload=16 * payload_words / N,
               bits_state_offs=(8 * nstates + 32 * (2 * ntiles + 1) + 16 * pad_words) / N,
               bits_table=32 * M / N,
               bits_escape=(32 * (ntiles + 1) + 32 * nesc) / N,
               entropy_model=entropy_model, layout=LAYOUT_W64)
    enc["offs"] = stream_offsets(enc)
    return enc


def layout_of(enc):
    """The stream layout of an encoded dict: its "layout" tag, or for an
    untagged dict (the reference's own encode writes none) "w64" when it
    carries the w64 tile offsets and "ref32" otherwise."""
    tag = enc.get("layout")
    if tag is None:
        return LAYOUT_W64 if "tile_off" in enc else LAYOUT_REF32
    assert tag in (LAYOUT_W64, LAYOUT_REF32), f"unknown stream layout {tag!r}"
    return tag


def tiling_of(enc):
    """(tile_R, tile_C, S) of an encoded matrix."""
    return enc["tile_R"], enc["tile_C"], enc["S"]


# MI355X figures the large-matrix rule of pick_tiling estimates residency
# with: compute units, LDS bytes per CU, and what one workgroup of the
# batch-1 GEMV holds besides its staged tiles (the 16 KB table of 4-byte
# entries, which large launches use, and the reduction scratch)
MI355X_CUS = 256
LDS_PER_CU = 160 * 1024
GEMV_WG_FIXED_LDS = 16384 + 2048


def last_round_fill(rows, cols, R, C, bits=3.0, S=1):
    """(rounds, fill) of the batch-1 GEMV launch of a rows x cols matrix in
    R x C tiles at about `bits` bits per weight: workgroups (one tile row of
    min(ncb, 8) waves each) over those MI355X holds at once, as the LDS
    allows (the fixed part plus each wave's staged tile of R*C*bits/8
    bytes, at most 32 waves per CU), and the occupied fraction of the last
    round (1.0 when the rounds come out whole)."""
    ncb = w64_stream_cols(cols) // C
    waves = min(ncb, 8)
    nwg = (rows // R) * (ncb // waves)
    tile = R * C * bits / 8 + 16
    per_cu = min(32 // waves, int(LDS_PER_CU // (GEMV_WG_FIXED_LDS + waves * tile)))
    resident = max(per_cu, 1) * MI355X_CUS
    rounds = nwg / resident
    frac = rounds - int(rounds)
    return rounds, (frac if frac > 1e-9 else 1.0)


def pick_tiling(rows, cols, R=None, S=1, target_states=None, max_ncb=None, bits=3.0):
    """A legal (R, C) for the w64 format: C a multiple of 64*S dividing the
    stored columns (w64_stream_cols(cols)),
    R in {1, 2, 3, 4, 8, 16}, or 35 at S=1 (rows of 8960 = 256 x 35: 8960 x
    1536 becomes 2048 tiles of 35 x 192, two waves on every SIMD), or for
    matrices above 32M weights also 20 at S=1.  Chosen by measurement on
    MI355X:

    - states: about 105 symbols per state for mid-size matrices (at
      1536x8960 that is 2048 waves, two per SIMD: two waves on a SIMD slow
      each other by only ~15%, so a one-wave SIMD is mostly idle capacity);
      small ones get more states: up to 98304 at 64 or more symbols each,
      and at least 49152 (768 waves) down to 35 symbols each, below which
      the launch is latency-bound far above its byte count (1536x1536 at
      3.25 bits: 5.5 us with 49152 states, 8.1 us with 36864, +0.21
      bits/weight); matrices above 32M weights use about 160 symbols per
      state.  Fewer states cost less per-state overhead (a byte of length
      and exponent plus a 16 to 31-bit mantissa, ~26 bits beyond the
      entropy each), more states give more parallelism.
    - column tiles per tile row (ncb): 8 is best (8 waves of a workgroup
      share one LDS table, so more waves fit per CU), then 4-7 and 16 (the
      latter needs the split-K reduction); fewer than 4 repeat the table
      staging more often per tile.
    - above 32M weights the launch takes more than one round of resident
      workgroups (last_round_fill, at `bits` bits per weight), and a last
      round less than half full leaves most of the chip idle while its
      tiles decode: tilings with one are penalised, so 25600x5120 takes
      20x640 (1280 tile rows, last round 2/3 full: 51.9 us at batch 1,
      61.8 at batch 4, 2.880 bits/weight) over 16x640 (1600 tile rows, 8%:
      54.8 us, 64.7-68.5 us, 2.923 bits/weight), while 5120x17408 keeps
      4x2176 (35.4 us) over 8x2176 (44.0 us, last round 1/4 full).

    R: one tile height, or a list of candidates (default: every compiled
    one dividing rows); max_ncb: at most this many column tiles.  Columns
    that are an odd multiple of 32 are tiled over their stored width
    (w64_stream_cols)."""
    nst = 64 * S
    n = rows * cols
    cols = w64_stream_cols(cols)
    cands = [c for c in range(nst, cols + 1, nst)
             if cols % c == 0 and (max_ncb is None or cols // c <= max_ncb)]
    assert cands, f"cols={cols} has no divisor that is a multiple of {nst}"
    large = n >= (32 << 20)
    if R is None:
        heights = SUPPORTED_R + (LARGE_R if large else ())
        Rs = [r for r in heights if rows % r == 0 and (S == 1 or r not in ONE_STATE_R)]
    else:
        Rs = [R] if isinstance(R, int) else list(R)
    if target_states:
        target = target_states
    elif large:
        target = n // 160
    else:
        target = int(min(max(n // 105, min(98304, n // 64), min(49152, n // 35)), 262144))
    best = None
    for r in Rs:
        for c in cands:
            states = (rows // r) * (cols // c) * nst
            ncb = cols // c
            if ncb == 8:
                penalty = 0.0
            elif 4 <= ncb <= 7:
                penalty = 0.3 if n >= (32 << 20) else 0.0
            elif ncb == 16:
                penalty = 0.2
            else:
                penalty = 0.35 if ncb < 4 else 0.5
            if large:
                rounds, fill = last_round_fill(rows, cols, r, c, bits, S)
                if rounds > 1 and fill < 0.5:
                    penalty += 0.3
            key = (abs(np.log(states / target)) + penalty, -c)
            if best is None or key < best[0]:
                best = (key, r, c)
    return best[1], best[2]


def _host_desc(enc, keep):
    """rans_w64_matrix over host numpy arrays (for rans_w64_decode_host)."""
    arrs = {k: np.ascontiguousarray(enc[k]) for k in
            ("words", "tile_off", "tile_meta", "slen", "table", "esc_tileptr", "esc_pos",
             "esc_val")}
    keep.append(arrs)
    rows = enc["shape"][0]
    tR, tC, tS = tiling_of(enc)
    d = RansMatrixDesc(rows=rows, cols=stream_cols(enc), R=tR, C=tC, S=tS,
                       max_tile_words=enc["max_tile_words"],
                       max_state_words=enc["max_state_words"])
    for k, a in arrs.items():
        setattr(d, k, a.ctypes.data if a.size else None)
    return d


def decode_ref(enc):
    """Host decoder of the w64 stream (rans.py:101-123 semantics): returns
    int64 codes (rows x cols), escapes applied; asserts that every state
    returns to 2^16 and that the escape side table matches the stream."""
    rows, cols = enc["shape"]
    keep = []
    d = _host_desc(enc, keep)
    out = np.zeros((rows, stream_cols(enc)), np.int32)
    rc = _host_lib().rans_w64_decode_host(ctypes.byref(d), _p(out))
    assert rc <= 0, f"stream did not return to initial state (state {rc - 1})"
    assert rc == 0, f"corrupt stream or escape side table ({rc})"
    return out[:, :cols].astype(np.int64)


def fused_rows_limit(desc, lib, grouped=False):
    """Rows of x up to which the fused GEMV beats decoding to bf16 and a
    dense GEMM on MI355X: 16 where a batch of 5 to 8 rows runs as one launch
    of the batch-8 kernel (1536x8960 at 16 rows 29.9 against 38.6 us,
    1536x1536 14.1 against 14.6), else 8 (batch-4 launches: 8960x1536 at 12
    rows 32.7 against 25.6 us, 25600x5120 158.6 against 150.4).  The
    library's planner takes the batch-8 kernel only for a single matrix with
    one state per lane, tiles of at most 8 rows and one workgroup per tile
    row (no split-K: rans_gemv_workspace_bytes is 0); grouped launches
    (grouped=True) have no batch-8 kernel.  desc: a RansMatrixDesc; lib:
    the loaded library (the query is host code, no GPU needed)."""
    batch8 = (not grouped and desc.S == 1 and desc.R <= 8 and
              lib.rans_gemv_workspace_bytes(ctypes.byref(desc), 8) == 0)
    return 16 if batch8 else 8


# ------------------------------------------------------------------- device
def _require_gpu():
    if not torch.cuda.is_available():
        raise RuntimeError("RansMatrix needs a ROCm GPU (gfx950); no CPU fallback exists")


class RansMatrix:
    """Entropy-coded matrix resident on the GPU (rans.py:127-162)."""

    def __init__(self, enc, step, lib, flags=0):
        """flags: F_WORDS_ALWAYS / F_WORDS_REFILL picks the GEMV's word
        fetch and F_TABLE8 / F_TABLE4 its table entries (same results,
        different speed); 0 lets the library choose.  F_NO_ESCAPES is added
        here when the matrix has no escapes.  The 4-byte table image is
        uploaded only where the library would use it (rans_gemv_table4 at
        batch 1, bf16 x) or F_TABLE4 asks for it."""
        assert layout_of(enc) == LAYOUT_W64, \
            "RansMatrix takes the w64 layout of encode(); the reference's 32-lane layout " \
            "runs on ReferenceLayoutMatrix"
        _require_gpu()
        if lib is None:
            raise RuntimeError("librans_hip.so not loaded")
        self.lib = lib
        self.R, self.C, self.S = tiling_of(enc)
        self.rows, self.cols = enc["shape"]
        # stored columns: cols, or cols + 32 when cols % 64 == 32 (the
        # appended columns get a zero step here and a zero x in gemv)
        self.stream_cols = stream_cols(enc)
        dev = torch.device("cuda")

        def up(a, dt):
            a = np.ascontiguousarray(a)
            if not a.flags.writeable:  # e.g. a memory-mapped file (rans_io.load)
                a = a.copy()
            return torch.from_numpy(a.view(dt)).to(dev)

        self.words = up(enc["words"], np.int16)
        self.tile_off = up(enc["tile_off"], np.int32)
        self.slen = up(enc["slen"], np.uint8)
        self.tile_meta = up(enc["tile_meta"], np.int32)
        # the kernels read the table's LDS image; the packed table is only
        # for the host decoder and stays on the host
        self.table_lds = up(table_lds(enc["table"], lib), np.int32)
        self.esc_tileptr = up(enc["esc_tileptr"], np.int32)
        # never hand a zero-length buffer's (possibly null) pointer to the ABI
        self.esc_pos = up(enc["esc_pos"] if len(enc["esc_pos"]) else np.zeros(1, np.uint16), np.int16)
        self.esc_val = up(enc["esc_val"] if len(enc["esc_val"]) else np.zeros(1, np.int16), np.int16)
        # one value per column, or one for the whole matrix (broadcast, as
        # the reference's x * step would)
        step = torch.as_tensor(step).float().reshape(-1)
        assert step.numel() in (1, self.cols), "step must have one value per column (or one)"
        self.step = torch.zeros(self.stream_cols, dtype=torch.float32, device=dev)
        self.step[:self.cols] = step.to(dev).expand(self.cols)
        self.max_tile_words = int(enc["max_tile_words"])
        self.max_state_words = int(enc["max_state_words"])
        self._desc = RansMatrixDesc(
            rows=self.rows, cols=self.stream_cols, R=self.R, C=self.C, S=self.S,
            max_tile_words=self.max_tile_words, max_state_words=self.max_state_words,
            flags=(int(flags) & (F_WORDS_MASK | F_TABLE8 | F_TABLE4)) |
            (0 if len(enc["esc_pos"]) else F_NO_ESCAPES),
            words=self.words.data_ptr(), tile_off=self.tile_off.data_ptr(),
            slen=self.slen.data_ptr(), tile_meta=self.tile_meta.data_ptr(),
            table=None, table_lds=self.table_lds.data_ptr(),
            esc_tileptr=self.esc_tileptr.data_ptr(),
            esc_pos=self.esc_pos.data_ptr(), esc_val=self.esc_val.data_ptr(),
            step=self.step.data_ptr(), workspace=None, workspace_bytes=0)
        self.workspace = None
        self._ensure_workspace(4)
        self.table_lds4 = None
        if flags & F_TABLE4 or (not flags & F_TABLE8 and
                                lib.rans_gemv_table4(ctypes.byref(self._desc), X_BF16, 1) == 1):
            self.table_lds4 = up(table_lds4(enc["table"], lib), np.int32)
            self._desc.table_lds4 = self.table_lds4.data_ptr()
        # device bytes (the 32 KB table image in place of the 16 KB table,
        # plus the 16 KB image of 4-byte entries where it is used)
        imgs = (self.table_lds,) if self.table_lds4 is None else (self.table_lds, self.table_lds4)
        self.nbytes = sum(t.numel() * t.element_size() for t in
                          (self.words, self.tile_off, self.slen, self.tile_meta, *imgs,
                           self.esc_tileptr)) + 4 * int(len(enc["esc_pos"]))

    @property
    def fused_rows_limit(self):
        """Rows of x up to which this matrix's own GEMV launch beats
        decoding to bf16 and a dense GEMM (module-level fused_rows_limit)."""
        return fused_rows_limit(self._desc, self.lib)

    def tune(self, batch=1, x_dtype=torch.bfloat16, iters=20):
        """Time the two word-fetch policies of the GEMV on this matrix and
        keep the faster one.  Both give bitwise identical results; which is
        faster depends on the tile geometry and the matrix size.  Each
        policy's launches are captured in a HIP graph and replayed, so the
        events time back-to-back kernels rather than host launch overhead.
        Returns the chosen flag."""
        x = torch.randn(batch, self.cols, device="cuda").to(x_dtype)
        y = torch.empty(batch, self.rows, device="cuda")
        best = None
        keep = self._desc.flags & ~F_WORDS_MASK
        for f in (F_WORDS_ALWAYS, F_WORDS_REFILL):
            self._desc.flags = f | keep
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                self.gemv(x, y)  # first launch of this kernel outside the capture
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(iters):
                    self.gemv(x, y)
            g.replay()
            t0 = torch.cuda.Event(enable_timing=True)
            t1 = torch.cuda.Event(enable_timing=True)
            t0.record()
            g.replay()
            g.replay()
            t1.record()
            t1.synchronize()
            t = t0.elapsed_time(t1)
            del g
            if best is None or t < best[0]:
                best = (t, f)
        self._desc.flags = best[1] | keep
        return best[1]

    @property
    def flags(self):
        return int(self._desc.flags)

    def _ensure_workspace(self, batch):
        need = int(self.lib.rans_gemv_workspace_bytes(ctypes.byref(self._desc), batch))
        assert need >= 0, f"tile geometry not launchable ({need})"
        if need and (self.workspace is None or self.workspace.numel() < need):
            # zero once: the kernel keeps its counters at zero between launches
            self.workspace = torch.zeros(need, dtype=torch.uint8, device="cuda")
            self._desc.workspace = self.workspace.data_ptr()
            self._desc.workspace_bytes = need

    def gemv(self, x, y=None):
        """y = codes @ (x * step) for x of shape (cols,) or (B, cols), f32 or
        bf16; returns f32 (rows,) or (B, rows).  The step fold runs inside
        the kernel.  A matrix stored with 32 appended columns takes x
        through a zero-padded copy (the kernel reads stream_cols values per
        x row)."""
        assert x.is_cuda, "x must be a device tensor"
        squeeze = x.dim() == 1
        xb = x.reshape(1, -1) if squeeze else x
        assert xb.shape[-1] == self.cols
        xb, xd = _x_operand(xb, self.stream_cols)
        B = xb.shape[0]
        if y is None:
            y = torch.empty((B, self.rows) if not squeeze else (self.rows,),
                            device="cuda", dtype=torch.float32)
        assert y.dtype == torch.float32 and y.is_contiguous() and y.numel() == B * self.rows
        rc = self.lib.rans_w64_gemv(ctypes.byref(self._desc), xb.data_ptr(), xd, B,
                                       y.data_ptr(), torch.cuda.current_stream().cuda_stream)
        assert rc == 0, f"HIP error {rc}"
        return y

    def _decode_into(self, fn, out, dtype):
        if out is None:
            out = torch.empty(self.rows, self.cols, device="cuda", dtype=dtype)
        assert out.dtype == dtype and out.is_contiguous() and out.numel() == self.rows * self.cols
        # appended columns: decode the stored width, keep the matrix's own
        full = out if self.stream_cols == self.cols else \
            torch.empty(self.rows, self.stream_cols, device="cuda", dtype=dtype)
        rc = fn(ctypes.byref(self._desc), full.data_ptr(), torch.cuda.current_stream().cuda_stream)
        assert rc == 0, f"HIP error {rc}"
        if full is not out:
            out.view(self.rows, self.cols).copy_(full[:, :self.cols])
        return out

    def decode(self, out=None):
        """Dense bf16 rows x cols matrix code*step (rans.py:154-162)."""
        return self._decode_into(self.lib.rans_w64_decode, out, torch.bfloat16)

    def decode_codes(self, out=None):
        """Dense int32 codes on the GPU, escapes included (bit-exact path)."""
        return self._decode_into(self.lib.rans_w64_decode_codes, out, torch.int32)


GROUP_MAX = 4
_EUNSUPPORTED, _EGEOMETRY, _ECODES = -1, -2, -5


def pick_group_tiling(rows_list, cols, S=1):
    """One (R, C) for matrices that share x (a layer's q, k, v or gate, up),
    so that gemv_group can run them in one launch: the tiling pick_tiling
    gives the stacked matrix, among tile heights that divide every member's
    rows, with at most 8 column tiles (one workgroup per tile row)."""
    Rs = [r for r in (SUPPORTED_R if S == 1 else SUPPORTED_R[1:])
          if all(n % r == 0 for n in rows_list)]
    assert Rs, f"no compiled tile height divides all of {list(rows_list)}"
    return pick_tiling(sum(rows_list), cols, R=Rs, S=S, max_ncb=8)


def _x_operand(xb, scols):
    """x rows as the kernels read them: contiguous bf16 or f32, each row
    zero-padded to scols values (a matrix stored with appended columns)."""
    if xb.dtype == torch.bfloat16:
        xd = X_BF16
    else:
        xb, xd = xb.float(), X_F32
    if xb.shape[-1] != scols:
        xb = torch.nn.functional.pad(xb, (0, scols - xb.shape[-1]))
    return xb.contiguous(), xd


def gemv_group(matrices, x, ys=None):
    """[m.gemv(x) for m in matrices] for up to 4 RansMatrix objects sharing
    x, in one launch (rans_w64_gemv_group) when they can share one: same
    cols and R, one state per lane, one workgroup per tile row (encode them
    with pick_group_tiling).  Otherwise one launch per matrix.  Results are
    bitwise those of separate gemv calls.  Returns the list of y."""
    ms = list(matrices)
    assert 0 < len(ms), "no matrices"
    assert x.is_cuda, "x must be a device tensor"
    squeeze = x.dim() == 1
    xb0 = x.reshape(1, -1) if squeeze else x
    B = xb0.shape[0]
    if ys is None:
        ys = [torch.empty((B, m.rows) if not squeeze else (m.rows,), device="cuda",
                          dtype=torch.float32) for m in ms]
    assert len(ys) == len(ms)
    for m, y in zip(ms, ys):
        assert xb0.shape[-1] == m.cols
        assert y.dtype == torch.float32 and y.is_contiguous() and y.numel() == B * m.rows
    xb, xd = _x_operand(xb0, ms[0].stream_cols)
    if 1 < len(ms) <= GROUP_MAX:
        descs = (ctypes.c_void_p * len(ms))(*[ctypes.addressof(m._desc) for m in ms])
        yps = (ctypes.c_void_p * len(ms))(*[y.data_ptr() for y in ys])
        rc = ms[0].lib.rans_w64_gemv_group(descs, len(ms), xb.data_ptr(), xd, B, yps,
                                              torch.cuda.current_stream().cuda_stream)
        if rc == 0:
            return ys
        assert rc in (_EUNSUPPORTED, _EGEOMETRY), f"HIP error {rc}"
    for m, y in zip(ms, ys):
        m.gemv(xb0 if not squeeze else xb0[0], y)
    return ys


# ------------------------------------------------ the reference's own layout
def encode_reference_layout(codes, R, C, threads=None):
    """The reference's encode (kernel/rans.py:62-98) on its own 32-lane
    layout: words, offs and table as it writes them, in its dict (words,
    offs, table, R, C, shape, bits_payload, bits_state_offs, bits_table,
    entropy_model) plus layout = "ref32".  The input of
    ReferenceLayoutMatrix and of the reference-format entry points; `encode` gives the w64 layout, which
    decodes far faster.  codes must lie in [-128, 127]."""
    codes = np.ascontiguousarray(codes, dtype=np.int32)
    assert codes.ndim == 2 and codes.size > 0, "codes must be a non-empty matrix"
    rows, cols = codes.shape
    assert rows % R == 0 and cols % C == 0 and C % 32 == 0
    lanes = (rows // R) * (cols // C) * 32
    cap = 2 * lanes + codes.size + 8
    buf = np.zeros(cap, np.uint16)
    offs = np.zeros(lanes, np.uint32)
    table = np.zeros(M, np.uint32)
    info = np.zeros(2, np.int64)
    rc = _host_lib().rans_ref32_encode(_p(codes), rows, cols, R, C,
                                       threads or min(16, os.cpu_count() or 1), _p(buf), cap,
                                       _p(offs), _p(table), _p(info))
    assert rc != _ECODES, "code out of 8-bit alphabet, or a single-symbol distribution"
    assert rc == 0, f"encode failed ({rc})"
    n = codes.size
    # per-symbol frequencies from the table's slots, for the model entropy
    fr = np.zeros(256, np.int64)
    fr[table & 0xFF] = (table >> 8) & 0xFFF
    cnt = np.bincount((codes.ravel() + OFFSET), minlength=256)
    used = cnt > 0
    return dict(words=buf[:int(info[0])].copy(), offs=offs, table=table, R=R, C=C,
                shape=codes.shape, bits_payload=16 * int(info[1]) / n,
                bits_state_offs=64 * lanes / n, bits_table=32 * M / n,
                entropy_model=float(-(cnt[used] * np.log2(fr[used] / M)).sum() / n),
                layout=LAYOUT_REF32)


class ReferenceLayoutMatrix:
    """A matrix in the reference's own layout on the GPU, with the
    reference's RansMatrix contract (kernel/rans.py:127-162): gemv(x) folds
    x*step on the host side and runs launch_rans_gemv (y zeroed first when a
    row spans several column tiles, as the kernel adds into it); decode()
    runs launch_rans_decode.  For data encoded in that layout; RansMatrix on
    the w64 layout is the fast path."""

    def __init__(self, enc, step, lib):
        assert layout_of(enc) == LAYOUT_REF32, \
            "ReferenceLayoutMatrix takes the reference's 32-lane layout " \
            "(encode_reference_layout, or the reference's encode); the w64 dict of encode() " \
            "has one offs entry per 64-lane state and runs on RansMatrix"
        _require_gpu()
        self.lib = lib
        self.R, self.C = int(enc["R"]), int(enc["C"])
        self.rows, self.cols = (int(v) for v in enc["shape"])
        dev = torch.device("cuda")
        as_i = {"words": np.int16, "offs": np.int32, "table": np.int32}
        for key, dt in as_i.items():
            setattr(self, key, torch.from_numpy(np.ascontiguousarray(enc[key]).view(dt)).to(dev))
        step = torch.as_tensor(step).float().reshape(-1)
        assert step.numel() in (1, self.cols), "step must have one value per column (or one)"
        self.step = step.to(dev).expand(self.cols).contiguous()
        self.nbytes = sum(t.numel() * t.element_size() for t in (self.words, self.offs, self.table))

    def _call(self, fn, src, dst):
        rc = fn(self.R, self.words.data_ptr(), self.offs.data_ptr(), self.table.data_ptr(),
                src.data_ptr(), dst.data_ptr(), self.rows, self.cols, self.C,
                torch.cuda.current_stream().cuda_stream)
        assert rc == 0, f"HIP error {rc}"
        return dst

    def gemv(self, x, y=None):
        """y = codes @ (x * step) for x of shape (cols,); f32 (rows,)."""
        assert x.is_cuda and x.numel() == self.cols, "x must be a (cols,) device tensor"
        xs = (x.reshape(-1).float() * self.step).contiguous()
        split = self.cols != self.C
        if y is None:
            y = torch.zeros(self.rows, device="cuda") if split else torch.empty(self.rows, device="cuda")
        elif split:
            y.zero_()
        return self._call(self.lib.launch_rans_gemv, xs, y)

    def decode(self, out=None):
        """Dense bf16 rows x cols matrix code*step."""
        if out is None:
            out = torch.empty(self.rows, self.cols, device="cuda", dtype=torch.bfloat16)
        return self._call(self.lib.launch_rans_decode, self.step, out)


class Int4Matrix:
    """Fixed-rate 4-bit baseline (codes in [-8, 7]), rans.py:165-185."""

    def __init__(self, codes, step, lib):
        _require_gpu()
        self.lib = lib
        self.rows, self.cols = codes.shape
        assert self.cols % 32 == 0, "cols must be a multiple of 32"
        # eight biased nibbles per u32, column 8j+b at bits 4b..4b+3 of word j
        nib = (np.clip(codes, -8, 7) + 8).astype(np.uint32).reshape(self.rows, -1, 8)
        shifts = np.arange(0, 32, 4, dtype=np.uint32)
        words = np.bitwise_or.reduce(nib << shifts, axis=2).astype(np.uint32)
        self.w = torch.from_numpy(words.view(np.int32)).cuda()
        self.step = torch.as_tensor(step).float().cuda()
        self.nbytes = self.w.numel() * 4

    def clone(self):
        """The same matrix in its own device copy of the packed words (for
        timing over copies that displace each other from the caches)."""
        c = copy.copy(self)
        c.w = self.w.clone()
        return c

    def gemv(self, x, y=None):
        xs = (x.float() * self.step).contiguous()
        y = torch.empty(self.rows, device="cuda") if y is None else y
        rc = self.lib.launch_int4_gemv(self.w.data_ptr(), xs.data_ptr(), y.data_ptr(),
                                       self.rows, self.cols, torch.cuda.current_stream().cuda_stream)
        assert rc == 0, f"HIP error {rc}"
        return y


class Bf16Matrix:
    """Dense bf16 comparator: y = W x through the library's own bf16 GEMV
    (f32 accumulation and output), the product F.linear computes with the
    BLAS library (bench.py:96).  W: a (rows, cols) tensor or array, cols a
    multiple of 8; it is held as a contiguous bf16 copy on the GPU."""

    def __init__(self, W, lib):
        _require_gpu()
        self.lib = lib
        self.w = torch.as_tensor(W).to(device="cuda", dtype=torch.bfloat16).contiguous()
        self.rows, self.cols = self.w.shape
        assert self.cols % 8 == 0, "cols must be a multiple of 8"
        self.nbytes = self.w.numel() * 2

    def gemv(self, x, y=None):
        xb = x.to(device="cuda", dtype=torch.bfloat16).contiguous()
        assert xb.numel() == self.cols
        y = torch.empty(self.rows, device="cuda") if y is None else y
        rc = self.lib.bf16_gemv(self.w.data_ptr(), xb.data_ptr(), y.data_ptr(),
                                self.rows, self.cols, torch.cuda.current_stream().cuda_stream)
        assert rc == 0, f"HIP error {rc}"
        return y
