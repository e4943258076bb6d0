"""Writes w64_format_vectors.npz: the w64 encoder's exact output for three
small seeded matrices (one with escapes, one with two states per lane, one
35-row tiling).  The fixture pins the stream format and the container's
section contents, so that a change to the encoder that alters the bytes is
seen as a format change.  Run from the repository root after building:

    python tests/golden/make_w64_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "vram-compression_amd"))
import rans  # noqa: E402

# the table itself is pinned by the reference vectors (build_table)
KEYS = ("words", "tile_off", "tile_meta", "slen", "esc_tileptr", "esc_pos", "esc_val")
CASES = [  # name, rows, cols, R, C, S, escape fraction, seed
    ("esc", 24, 256, 3, 128, 1, 0.02, 1),
    ("s2", 16, 256, 8, 128, 2, 0.0, 2),
    ("r35", 70, 192, 35, 192, 1, 0.01, 3),
]


def case_codes(rows, cols, esc, seed):
    rng = np.random.default_rng(seed)
    codes = np.round(rng.laplace(size=(rows, cols)) * 3.0).astype(np.int32)
    hit = rng.random(codes.shape) < esc
    codes[hit] = rng.integers(128, 2000, size=int(hit.sum())) * rng.choice([-1, 1], int(hit.sum()))
    return codes


def main():
    out = {}
    for name, rows, cols, R, C, S, esc, seed in CASES:
        codes = case_codes(rows, cols, esc, seed)
        enc = rans.encode(codes, R, C, S, threads=1)
        assert np.abs(codes).max() < 2 ** 15
        out[f"{name}_codes"] = codes.astype(np.int16)  # stored small; every value fits
        for k in KEYS:
            out[f"{name}_{k}"] = np.asarray(enc[k])
        out[f"{name}_meta"] = np.array([rows, cols, R, C, S, enc["max_tile_words"],
                                        enc["max_state_words"]], np.int64)
    np.savez_compressed(os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                     "w64_format_vectors.npz"), **out)


if __name__ == "__main__":
    main()
