"""The C-ABI library loads on a machine without a GPU, exports every entry
point include/vramc_rans.h declares, and rejects bad arguments before any
HIP call (no compute happens in these tests)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vramc_rans.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^(?:int|int64_t|void)\s+(\w+)\s*\(", text, flags=re.M)


def test_header_declares_entry_points():
    names = _declared()
    assert "rans_w64_gemv" in names and "launch_int4_gemv" in names
    assert len(names) == len(set(names))


def test_every_declared_symbol_is_exported(rans, lib):
    for name in _declared():
        assert hasattr(lib, name), name
    assert set(_declared()) == set(rans.EXPORTS)


def _desc(rans, rows=256, cols=4096, R=8, C=256, S=1, mtw=1024):
    fake = 0x1000  # never dereferenced: every call below returns before launching
    return rans.RansMatrixDesc(rows=rows, cols=cols, R=R, C=C, S=S, max_tile_words=mtw,
                               max_state_words=64,
                               words=fake, tile_off=fake, slen=fake, tile_meta=fake, table=fake,
                               table_lds=fake,
                               esc_tileptr=fake, esc_pos=fake, esc_val=fake, step=fake,
                               workspace=None, workspace_bytes=0)


def test_argument_validation_without_gpu(rans, lib):
    d = _desc(rans)
    x = y = ctypes.c_void_p(0x2000)
    assert lib.rans_w64_gemv(None, x, 0, 1, y, None) == -2
    bad = _desc(rans, cols=4000)
    assert lib.rans_w64_gemv(ctypes.byref(bad), x, 0, 1, y, None) == -2
    r5 = _desc(rans, rows=255, R=5)  # no kernel compiled for R=5
    assert lib.rans_w64_gemv(ctypes.byref(r5), x, 0, 1, y, None) == -1
    assert lib.rans_w64_gemv(ctypes.byref(d), x, 7, 1, y, None) == -4
    assert lib.rans_w64_gemv(ctypes.byref(d), None, 0, 1, y, None) == -4
    assert lib.rans_w64_gemv(ctypes.byref(d), x, 0, 0, y, None) == -4
    # 16 column tiles: 8 waves per workgroup, 2 column groups -> split-K workspace
    assert lib.rans_w64_gemv(ctypes.byref(d), x, 0, 1, y, None) == -3
    need = lib.rans_gemv_workspace_bytes(ctypes.byref(d), 1)
    assert need == 256 + 2 * 1 * 256 * 4
    assert lib.rans_gemv_workspace_bytes(ctypes.byref(d), 4) == 256 + 2 * 4 * 256 * 4
    one = _desc(rans, cols=2048)  # 8 column tiles: one workgroup per tile row
    assert lib.rans_gemv_workspace_bytes(ctypes.byref(one), 1) == 0
    huge = _desc(rans, mtw=70000)
    assert lib.rans_gemv_workspace_bytes(ctypes.byref(huge), 1) == -2
    for flags in (3, 24, 32, -1):  # both word-fetch bits, both table bits, an unknown bit
        bad_flags = _desc(rans, cols=2048)
        bad_flags.flags = flags
        assert lib.rans_w64_gemv(ctypes.byref(bad_flags), x, 0, 1, y, None) == -2
        assert lib.rans_gemv_table4(ctypes.byref(bad_flags), 0, 1) == -2
    # the 4-byte table entries, forced: they need their image and one state per lane
    t4 = _desc(rans, cols=2048)
    t4.flags = rans.F_TABLE4
    assert lib.rans_w64_gemv(ctypes.byref(t4), x, 0, 1, y, None) == -4
    t4s2 = _desc(rans, cols=2048, S=2)
    t4s2.flags = rans.F_TABLE4
    t4s2.table_lds4 = 0x1000
    assert lib.rans_w64_gemv(ctypes.byref(t4s2), x, 0, 1, y, None) == -1
    assert lib.rans_gemv_table4(ctypes.byref(t4s2), 0, 1) == -1
    # forced choices are answered without the occupancy query
    t4.table_lds4 = 0x1000
    assert lib.rans_gemv_table4(ctypes.byref(t4), 1, 1) == 1
    t8 = _desc(rans, cols=2048)
    t8.flags = rans.F_TABLE8
    assert lib.rans_gemv_table4(ctypes.byref(t8), 1, 1) == 0
    assert lib.rans_gemv_table4(ctypes.byref(t8), 7, 1) == -4
    assert lib.rans_gemv_table4(ctypes.byref(t8), 1, 0) == -2
    assert lib.rans_table_lds4(None, y) == -4
    no_img = _desc(rans)
    no_img.table_lds = None  # the kernels need the table's LDS image
    assert lib.rans_w64_gemv(ctypes.byref(no_img), x, 0, 1, y, None) == -4
    assert lib.rans_w64_decode_codes(ctypes.byref(no_img), y, None) == -4
    assert lib.rans_table_lds(None, y) == -4
    assert lib.rans_w64_decode(None, y, None) == -2
    assert lib.rans_w64_decode_codes(ctypes.byref(d), None, None) == -4
    assert lib.launch_int4_gemv(None, x, y, 4, 64, None) == -4
    assert lib.launch_int4_gemv(x, x, y, 4, 48, None) == -2
    assert lib.launch_int4_gemv(x, ctypes.c_void_p(0x2004), y, 4, 64, None) == -2  # x not 16-byte aligned
    assert lib.bf16_gemv(None, x, y, 4, 64, None) == -4
    assert lib.bf16_gemv(x, x, y, 0, 64, None) == -4
    assert lib.bf16_gemv(x, x, y, 4, 60, None) == -2  # cols not a multiple of 8
    assert lib.bf16_gemv(ctypes.c_void_p(0x2008), x, y, 4, 64, None) == -2  # w not 16-byte aligned


def test_group_validation_without_gpu(rans, lib):
    """rans_w64_gemv_group refuses, before any launch, what one launch
    cannot run: no matrices, more than 4, different cols or R, two states
    per lane, or split-K tilings."""
    x = ctypes.c_void_p(0x2000)

    def call(descs, n=None, ys=None):
        arr = (ctypes.c_void_p * max(1, len(descs)))(*[ctypes.addressof(d) for d in descs])
        yarr = (ctypes.c_void_p * max(1, len(descs)))(*([0x3000] * len(descs) if ys is None else ys))
        return lib.rans_w64_gemv_group(arr, len(descs) if n is None else n, x, 0, 1, yarr, None)

    a = _desc(rans, cols=2048)  # 8 column tiles: one workgroup per tile row
    b = _desc(rans, rows=512, cols=2048)
    assert lib.rans_w64_gemv_group(None, 2, x, 0, 1, None, None) == -4
    assert call([a, b], n=0) == -4
    assert call([a] * 5) == -1
    assert call([a, _desc(rans, cols=4096, C=512)]) == -1  # different cols
    assert call([a, _desc(rans, rows=256, cols=2048, R=16)]) == -1  # different R
    assert call([_desc(rans, cols=2048, C=256, S=2)] * 2) == -1  # two states per lane
    assert call([_desc(rans)] * 2) == -1  # 16 column tiles: split-K
    assert call([a, b], ys=[0x3000, 0]) == -4  # a null y
    bad = _desc(rans, rows=512, cols=2048)
    bad.table_lds = None
    assert call([a, bad]) == -4


def test_product_fails_loudly_without_gpu(rans):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    import numpy as np
    codes = np.random.default_rng(0).integers(-3, 4, size=(8, 64)).astype(np.int32)
    enc = rans.encode(codes, 1, 64)
    with pytest.raises(RuntimeError):
        rans.RansMatrix(enc, np.ones(64, np.float32), rans._LIB)


def test_oracle_is_not_imported_by_the_product():
    pkg = os.path.join(ROOT, "vram-compression_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "import oracle" not in text and "liboracle" not in text, f


def test_header_compiles_as_c(tmp_path):
    """include/vramc_rans.h is plain C for non-Python bindings (cgo, JNI,
    a C caller): it compiles as C99 and as C++17."""
    import os
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None or not os.path.isdir("/opt/rocm/include"):
        pytest.skip("needs gcc and the ROCm headers")
    inc = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")
    src = tmp_path / "use.c"
    src.write_text('#include "vramc_rans.h"\n'
                   "int main(void) { rans_w64_matrix m = {0}; (void)m;\n"
                   "  return rans_w64_gemv_group ? 0 : 1; }\n")
    for std, lang in (("c99", "c"), ("c++17", "c++")):
        subprocess.check_call([gcc, f"-std={std}", "-x", lang, "-fsyntax-only", f"-I{inc}",
                               "-I/opt/rocm/include", "-D__HIP_PLATFORM_AMD__", str(src)])


def test_fused_rows_limit_follows_the_planner(rans, lib):
    """The crossover to decode + dense GEMM is 16 rows only where the
    library runs 5-8 rows as one batch-8 launch: a single matrix with one
    state per lane, tiles of at most 8 rows and no split over column
    groups.  Split-K tilings, taller tiles, more states per lane and
    grouped launches run batch-4 launches and cross over at 8."""
    single = _desc(rans, cols=2048)            # 8 column tiles: one workgroup per tile row
    assert lib.rans_gemv_workspace_bytes(ctypes.byref(single), 8) == 0
    assert rans.fused_rows_limit(single, lib) == 16
    assert rans.fused_rows_limit(single, lib, grouped=True) == 8
    split = _desc(rans)                         # 16 column tiles: two column groups
    assert lib.rans_gemv_workspace_bytes(ctypes.byref(split), 8) > 0
    assert rans.fused_rows_limit(split, lib) == 8
    tall = _desc(rans, rows=256, cols=2048, R=16)
    assert rans.fused_rows_limit(tall, lib) == 8
    two = _desc(rans, cols=2048, C=256, S=2)
    assert rans.fused_rows_limit(two, lib) == 8
    bad = _desc(rans, mtw=70000)                # outside the format: no launch at all
    assert rans.fused_rows_limit(bad, lib) == 8
