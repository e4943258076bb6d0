"""On-disk container (rans_io): round trips, zero-copy loads and the
integrity checks a reader relies on."""
import os

import numpy as np
import pytest


@pytest.fixture()
def entries(rans, oracle):
    a = oracle.synth_codes(256, 1024, 3.0, seed=3)
    b = oracle.synth_codes(128, 512, 2.0, seed=4)
    b[3, 5], b[100, 7], b[100, 300] = 700, -129, 1000  # escapes
    out = []
    for name, codes, (R, C, S), flags in (("layer0.q", a, (4, 256, 1), 0),
                                          ("layer0.down", b, (8, 128, 2), 2)):
        enc = rans.encode(codes, R, C, S)
        step = np.random.default_rng(len(name)).random(codes.shape[1]).astype(np.float32) + 0.5
        out.append(dict(name=name, enc=enc, step=step, flags=flags, codes=codes))
    return out


KEYS = ("words", "tile_off", "slen", "tile_meta", "table", "esc_tileptr", "esc_pos", "esc_val")
SCALARS = ("R", "C", "S", "shape", "max_tile_words", "max_state_words", "bits_payload",
           "bits_state_offs", "bits_table", "bits_escape")


@pytest.mark.parametrize("mmap", [True, False])
def test_round_trip(rans, tmp_path, entries, mmap):
    import rans_io
    path = str(tmp_path / "set.w64")
    size = rans_io.save(path, entries)
    assert size == os.path.getsize(path) and size % rans_io.ALIGN == 0
    got = rans_io.load(path, mmap=mmap)
    assert [g["name"] for g in got] == [e["name"] for e in entries]
    for e, g in zip(entries, got):
        for k in KEYS:
            np.testing.assert_array_equal(g["enc"][k], e["enc"][k])
            assert g["enc"][k].dtype == e["enc"][k].dtype
        for k in SCALARS:
            assert tuple(np.atleast_1d(g["enc"][k])) == tuple(np.atleast_1d(e["enc"][k])), k
        np.testing.assert_array_equal(g["step"], e["step"])
        assert g["flags"] == e["flags"]
        np.testing.assert_array_equal(rans.decode_ref(g["enc"]), e["codes"])


def test_sections_are_aligned_views(tmp_path, entries):
    import rans_io
    path = str(tmp_path / "set.w64")
    rans_io.save(path, entries)
    got = rans_io.load(path)
    base = np.memmap(path, dtype=np.uint8, mode="r")
    for g in got:
        for k in KEYS:
            a = g["enc"][k]
            if a.size:
                assert isinstance(a.base, np.memmap) or isinstance(a, np.memmap)
                assert not a.flags.writeable


def test_corruption_is_detected(tmp_path, entries):
    import rans_io
    path = str(tmp_path / "set.w64")
    rans_io.save(path, entries)
    raw = bytearray(open(path, "rb").read())
    # a flipped bit in the last section of the file (the second matrix's step)
    bad = bytearray(raw)
    bad[-5] ^= 0x10
    p2 = str(tmp_path / "flip.w64")
    open(p2, "wb").write(bad)
    with pytest.raises(ValueError, match="CRC"):
        rans_io.load(p2)
    assert len(rans_io.load(p2, verify=False)) == 2  # integrity check can be skipped
    p3 = str(tmp_path / "short.w64")
    open(p3, "wb").write(raw[:-64])
    with pytest.raises(ValueError, match="truncated"):
        rans_io.load(p3)
    p4 = str(tmp_path / "magic.w64")
    open(p4, "wb").write(b"NOTAW64!" + raw[8:])
    with pytest.raises(ValueError, match="magic"):
        rans_io.load(p4)
    p5 = str(tmp_path / "tiny.w64")
    open(p5, "wb").write(raw[:20])
    with pytest.raises(ValueError):
        rans_io.load(p5)


def test_save_rejects_inconsistent_entries(rans, tmp_path, entries):
    import rans_io
    e = dict(entries[0])
    e["step"] = e["step"][:-1]  # one column short
    with pytest.raises(AssertionError):
        rans_io.save(str(tmp_path / "x.w64"), [e])


def test_version_6_written_and_earlier_refused(rans, tmp_path, entries):
    """The writer stamps version 6; files of the earlier stream layouts
    (versions 1 to 5) and unknown versions are refused with a ValueError
    naming the version."""
    import rans_io
    path = str(tmp_path / "set.w64")
    rans_io.save(path, entries)
    raw = bytearray(open(path, "rb").read())
    assert int.from_bytes(raw[8:12], "little") == rans_io.VERSION == 6
    got = rans_io.load(path)
    for e, g in zip(entries, got):
        np.testing.assert_array_equal(rans.decode_ref(g["enc"]), e["codes"])
    for version in (4, 5, 7):
        p = str(tmp_path / f"v{version}.w64")
        raw[8:12] = version.to_bytes(4, "little")
        open(p, "wb").write(raw)
        with pytest.raises(ValueError, match="version"):
            rans_io.load(p)


def test_appended_columns_round_trip(rans, oracle, tmp_path):
    """A matrix whose cols is an odd multiple of 32 (stored with 32 appended
    columns) keeps its own shape, step and codes through a container file,
    next to one without appended columns."""
    import rans_io
    odd = oracle.synth_codes(64, 224, 3.0, seed=11)
    even = oracle.synth_codes(64, 256, 3.0, seed=12)
    ents = []
    for name, codes in (("odd", odd), ("even", even)):
        enc = rans.encode(codes, 8, 32 if codes.shape[1] % 64 else 64)
        step = np.linspace(0.5, 1.5, codes.shape[1]).astype(np.float32)
        ents.append(dict(name=name, enc=enc, step=step, codes=codes))
    path = str(tmp_path / "odd.w64")
    rans_io.save(path, ents)
    got = rans_io.load(path)
    assert rans.stream_cols(got[0]["enc"]) == 256 and rans.stream_cols(got[1]["enc"]) == 256
    for e, g in zip(ents, got):
        assert tuple(g["enc"]["shape"]) == e["codes"].shape
        assert g["enc"]["layout"] == rans.LAYOUT_W64
        np.testing.assert_array_equal(g["step"], e["step"])
        np.testing.assert_array_equal(rans.decode_ref(g["enc"]), e["codes"])
