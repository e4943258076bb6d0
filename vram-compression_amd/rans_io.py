"""On-disk container for w64-encoded matrices (one or many per file).

The reference keeps encoded matrices only in memory (kernel/rans.py:62-98
returns a dict, kernel/bench.py re-encodes on every run).  A 1.31 G-weight
set takes minutes to encode, so it is stored once and memory-mapped on load:
every array is a zero-copy view of the file, ready to upload.

Layout (all integers little endian, every section 64-byte aligned):

    header, 64 bytes
        magic      8 bytes  b"VRAMCW64"
        version    u32      6 (1 to 5 held earlier stream layouts and are
                            not read: 4 and 5 a u32 initial state and a
                            byte length per state, 1 to 3 a row-CSR side
                            table, 16-bit stream offsets or a 32-bit side
                            table; re-encode such a matrix)
        nmat       u32      number of matrices
        index_off  u64      byte offset of the index
        file_bytes u64      total file size (truncation check)
        reserved   32 bytes zero
    index, nmat records of 256 bytes
        name       64 bytes UTF-8, NUL padded
        rows, cols, R, C, S, max_tile_words, max_state_words, flags   i32 x 8
                   (cols: the stored columns, stream_cols of the enc dict;
                   R, C, S: the w64 tiling, tile_R/tile_C/S of the enc dict)
        nwords, ntiles, nstates, nesc, payload_words                  u64 x 5
        entropy_model                                                 f64
        offsets of words, tile_off, slen, tile_meta, table,
                   esc_tileptr, esc_pos, esc_val, step                u64 x 9
        crc32 of the nine sections, in that order                     u32
        appended columns (0, or 32 when the matrix's cols % 64 == 32)  i32
        zero padding to 256 bytes
    sections
        words u16[nwords] (each tile's bit-packed initial states, then its
        streams), tile_off u32[ntiles+1], slen u8[nstates] (length delta |
        state exponent << 4), tile_meta u32[ntiles] (length base | blob
        words << 16), table u32[4096] (reference packing),
        esc_tileptr i32[ntiles+1], esc_pos u16[nesc], esc_val i16[nesc],
        step f32[cols - appended columns]

`flags` holds the launch options chosen for the matrix (the RANS_F_* word
fetch and table-entry bits; 0 = library defaults), so a tuned set reloads
with its tuning.
"""
import os
import struct
import zlib

import numpy as np

import rans

MAGIC = b"VRAMCW64"
VERSION = 6
READ_VERSIONS = (6,)
_HEADER = struct.Struct("<8sIIQQ32x")
_RECORD = struct.Struct("<64s8i5Qd9QIi")
RECORD_BYTES = 256
ALIGN = 64
_SECTIONS = (("words", np.uint16), ("tile_off", np.uint32), ("slen", np.uint8),
             ("tile_meta", np.uint32), ("table", np.uint32), ("esc_tileptr", np.int32),
             ("esc_pos", np.uint16), ("esc_val", np.int16), ("step", np.float32))
assert _HEADER.size == 64 and _RECORD.size <= RECORD_BYTES


def _align(n):
    return (n + ALIGN - 1) // ALIGN * ALIGN


def _section_lengths(cols, nwords, ntiles, nstates, nesc):
    """Entries of each section; cols: the matrix's own columns (step)."""
    return dict(words=nwords, tile_off=ntiles + 1, slen=nstates, tile_meta=ntiles,
                table=rans.M, esc_tileptr=ntiles + 1, esc_pos=nesc, esc_val=nesc, step=cols)


def save(path, entries):
    """Write `entries` (a list of dicts with keys name, enc, step and
    optionally flags) to `path`.  enc is the dict rans.encode returns; step
    is the per-column f32 step vector.  Writes to a temporary name and
    renames, so a reader never sees a partial file."""
    recs, blobs = [], []
    pos = _align(_HEADER.size + RECORD_BYTES * len(entries))
    for e in entries:
        enc = e["enc"]
        rows, cols = (int(v) for v in enc["shape"])
        scols = rans.stream_cols(enc)
        arrays = {}
        for key, dt in _SECTIONS:
            a = e["step"] if key == "step" else enc[key]
            arrays[key] = np.ascontiguousarray(np.asarray(a).reshape(-1), dtype=dt)
        n = _section_lengths(cols, arrays["words"].size, arrays["tile_off"].size - 1,
                             arrays["slen"].size, arrays["esc_pos"].size)
        for key, _ in _SECTIONS:
            assert arrays[key].size == n[key], f"{e['name']}: {key} has {arrays[key].size} " \
                                               f"entries, expected {n[key]}"
        payload_words = int(round(enc["bits_payload"] * rows * cols / 16))
        offs, crc = [], 0
        for key, _ in _SECTIONS:
            offs.append(pos)
            b = arrays[key].tobytes()
            crc = zlib.crc32(b, crc)
            blobs.append((pos, b))
            pos = _align(pos + len(b))
        name = e["name"].encode("utf-8")
        assert len(name) <= 64, "matrix names are at most 64 bytes of UTF-8"
        recs.append(_RECORD.pack(name, rows, scols, *rans.tiling_of(enc),
                                 enc["max_tile_words"], enc["max_state_words"],
                                 int(e.get("flags", 0)), arrays["words"].size,
                                 arrays["tile_off"].size - 1, arrays["slen"].size,
                                 arrays["esc_pos"].size, payload_words,
                                 float(enc.get("entropy_model", 0.0)), *offs, crc,
                                 scols - cols))
    total = pos
    tmp = f"{path}.tmp{os.getpid()}"
    with open(tmp, "wb") as f:
        f.write(_HEADER.pack(MAGIC, VERSION, len(entries), _HEADER.size, total))
        for r in recs:
            f.write(r.ljust(RECORD_BYTES, b"\0"))
        for off, b in blobs:
            f.seek(off)
            f.write(b)
        f.truncate(total)
    os.replace(tmp, path)
    return total


def load(path, verify=True, mmap=True):
    """Read a container written by `save`.  Returns a list of dicts with
    keys name, enc (the dict rans.encode returns, arrays as read-only views
    of the file when mmap; its R and C are the stored w64 tiling, since the
    tiling the encoder was asked for is not kept), step and flags.  Raises ValueError on a wrong
    magic or version, a truncated file, a section outside the file, or (with
    verify) a CRC mismatch."""
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        head = f.read(_HEADER.size)
        if len(head) < _HEADER.size:
            raise ValueError("not a w64 container: file shorter than its header")
        magic, version, nmat, index_off, file_bytes = _HEADER.unpack(head)
        if magic != MAGIC:
            raise ValueError("not a w64 container: bad magic")
        if version not in READ_VERSIONS:
            raise ValueError(f"unsupported w64 container version {version}")
        if file_bytes != size:
            raise ValueError(f"truncated or padded file: header says {file_bytes} bytes, "
                             f"file has {size}")
        if index_off + RECORD_BYTES * nmat > size:
            raise ValueError("index runs past the end of the file")
        f.seek(index_off)
        raw = f.read(RECORD_BYTES * nmat)
    buf = np.memmap(path, dtype=np.uint8, mode="r") if mmap else np.fromfile(path, np.uint8)
    out = []
    for i in range(nmat):
        v = _RECORD.unpack(raw[i * RECORD_BYTES:i * RECORD_BYTES + _RECORD.size])
        name = v[0].rstrip(b"\0").decode("utf-8")
        rows, cols, R, C, S, mtw, msw, flags = v[1:9]
        nwords, ntiles, nstates, nesc, payload_words = v[9:14]
        entropy_model = v[14]
        offs = v[15:24]
        crc_want = v[24]
        appended = v[25]
        if rows <= 0 or cols <= 0 or R <= 0 or C <= 0 or S <= 0 or rows % R or cols % C \
                or C % (64 * S) or ntiles != (rows // R) * (cols // C) \
                or nstates != ntiles * 64 * S or appended not in (0, 32):
            raise ValueError(f"{name}: inconsistent geometry in the index")
        scols, cols = cols, cols - appended
        n = _section_lengths(cols, nwords, ntiles, nstates, nesc)
        arrays, crc = {}, 0
        for (key, dt), off in zip(_SECTIONS, offs):
            nbytes = n[key] * np.dtype(dt).itemsize
            if off % ALIGN or off + nbytes > size:
                raise ValueError(f"{name}: section {key} lies outside the file")
            a = buf[off:off + nbytes]
            if verify:
                crc = zlib.crc32(a, crc)
            arrays[key] = a.view(dt)
        if verify and crc != crc_want:
            raise ValueError(f"{name}: CRC mismatch (file corrupted)")
        N = rows * cols
        pad = nwords - payload_words
        enc = dict(words=arrays["words"], tile_off=arrays["tile_off"], slen=arrays["slen"],
                   tile_meta=arrays["tile_meta"], table=arrays["table"],
                   esc_tileptr=arrays["esc_tileptr"], esc_pos=arrays["esc_pos"],
                   esc_val=arrays["esc_val"], R=R, C=C, tile_R=R, tile_C=C, S=S,
                   shape=(rows, cols), stream_cols=scols,
                   max_tile_words=mtw, max_state_words=msw,
                   bits_payload=16 * payload_words / N,
                   bits_state_offs=(8 * nstates + 32 * (2 * ntiles + 1) + 16 * pad) / N,
                   bits_table=32 * rans.M / N,
                   bits_escape=(32 * (ntiles + 1) + 32 * nesc) / N,
                   entropy_model=entropy_model, layout=rans.LAYOUT_W64)
        enc["offs"] = rans.stream_offsets(enc)
        out.append(dict(name=name, enc=enc, step=arrays["step"], flags=flags))
    return out
