"""Runs the host encoders and decoder of a sanitizer build of w64_host.cpp
(path in argv[1]; started by tests/test_host_sanitizers.py in a process
with the AddressSanitizer runtime preloaded): w64 encode/decode at several
tilings with escapes and padded columns, the reference-layout encoder,
rejected inputs, and corrupted streams, which must be rejected without any
out-of-bounds access.  Prints "ok <cases>"."""
import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "vram-compression_amd"))
import rans  # noqa: E402

lib = ctypes.CDLL(sys.argv[1])
P, I32, I64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
lib.rans_w64_encode.argtypes = [P, I32, I32, I32, I32, I32, I32, ctypes.POINTER(P), P]
lib.rans_w64_encode_fetch.argtypes = [P] * 10
lib.rans_w64_encode_counts.argtypes = [P, P]
lib.rans_w64_encode_free.argtypes = [P]
lib.rans_w64_encode_free.restype = None
lib.rans_w64_decode_host.argtypes = [ctypes.POINTER(rans.RansMatrixDesc), P]
lib.rans_ref32_encode.argtypes = [P, I32, I32, I32, I32, I32, P, I64, P, P, P]
rans._LIB = lib  # the host calls of rans go to the sanitizer build

rng = np.random.default_rng(0)
cases = 0
for rows, cols, R, C, S, esc in [(64, 256, 4, 256, 1, 0.01), (35 * 4, 192, 35, 192, 1, 0.05),
                                 (48, 512, 16, 512, 2, 0.0), (32, 1024, 8, 1024, 4, 0.02),
                                 (6, 96, 3, 32, None, 0.1), (512, 2080, 16, 32, None, 0.01)]:
    for scale in (0.5, 3.0, 60.0):
        codes = np.clip(np.round(rng.laplace(size=(rows, cols)) * scale), -127, 127).astype(np.int32)
        m = rng.random(codes.shape) < esc
        codes[m] = rng.choice([-32768, -300, 200, 32767], size=int(m.sum()))
        enc = rans.encode(codes, R, C, S, threads=4)
        assert np.array_equal(rans.decode_ref(enc), codes)
        cases += 1
for rows, cols, R, C in [(64, 256, 4, 256), (128, 512, 8, 128), (32, 64, 1, 32), (96, 1536, 16, 512)]:
    codes = np.clip(np.round(rng.laplace(size=(rows, cols)) * 3), -128, 127).astype(np.int32)
    rans.encode_reference_layout(codes, R, C, threads=3)
    cases += 1
for fn in (lambda: rans.encode(np.full((64, 64), 5, np.int32), 4, 64),
           lambda: rans.encode_reference_layout(np.full((32, 64), 300, np.int32), 1, 32)):
    try:
        fn()
    except AssertionError:
        cases += 1
codes = np.clip(np.round(rng.laplace(size=(64, 256)) * 3), -127, 127).astype(np.int32)
enc = rans.encode(codes, 4, 256)
for k in range(30):
    bad = dict(enc, words=enc["words"].copy(), slen=enc["slen"].copy(),
               tile_meta=enc["tile_meta"].copy(), esc_pos=enc["esc_pos"].copy())
    if k % 3 == 0:
        bad["words"][rng.integers(0, bad["words"].size)] ^= 0xFFFF
    elif k % 3 == 1:
        bad["slen"][rng.integers(0, bad["slen"].size)] = rng.integers(0, 256)
    else:
        bad["tile_meta"][rng.integers(0, bad["tile_meta"].size)] ^= 0xFFFFFFFF
    try:
        rans.decode_ref(bad)
    except AssertionError:
        pass
    cases += 1
print("ok", cases)
