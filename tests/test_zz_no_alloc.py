"""rans_w64_gemv_noalloc: the GEMV entry point that allocates nothing (its
split-K partials and counters live in the library's per-GPU scratch array)
gives the results of rans_w64_gemv with a workspace, bit for bit, call after
call on the same GPU, and refuses launches beyond the array before touching
the device."""
import ctypes

import numpy as np
import pytest
import torch

REL_L2 = 1e-3


def _fake_desc(rans, rows, cols, R, C):
    fake = 0x1000  # never dereferenced: the calls below return before launching
    return rans.RansMatrixDesc(rows=rows, cols=cols, R=R, C=C, S=1, max_tile_words=1024,
                               max_state_words=64, words=fake, tile_off=fake, slen=fake,
                               tile_meta=fake, table=fake, table_lds=fake, esc_tileptr=fake,
                               esc_pos=fake, esc_val=fake, step=fake, workspace=None,
                               workspace_bytes=0)


def test_noalloc_refuses_beyond_scratch(rans, lib):
    """Sizes beyond the scratch array come back as RANS_ESCRATCH (-7) before
    any HIP call, so this runs without a GPU."""
    x = y = ctypes.c_void_p(0x2000)
    # 32768 tile rows of split-K counters: twice the 64 KiB counter region
    d = _fake_desc(rans, rows=32768, cols=4096, R=1, C=256)
    assert lib.rans_gemv_workspace_bytes(ctypes.byref(d), 1) > 0
    assert lib.rans_w64_gemv_noalloc(ctypes.byref(d), x, 1, 1, y, None) == -7
    # 32 column groups x 4 batch rows x 8192 rows of partials: 4 MiB
    d = _fake_desc(rans, rows=8192, cols=65536, R=8, C=256)
    assert lib.rans_w64_gemv_noalloc(ctypes.byref(d), x, 1, 4, y, None) == -7
    # the argument checks of rans_w64_gemv come first
    assert lib.rans_w64_gemv_noalloc(None, x, 1, 1, y, None) == -2
    assert lib.rans_w64_gemv_noalloc(ctypes.byref(d), None, 1, 1, y, None) == -4


@pytest.mark.gpu
def test_noalloc_matches_workspace_launch(rans, oracle, lib):
    """Two split-K matrices, the second smaller, each launched through both
    entry points at batch 1 and 4: bitwise equal outputs, within the bar of
    the oracle, and equal again on repeated calls (the counters return to
    zero).  A matrix without split-K takes the plain path."""
    if not torch.cuda.is_available():
        raise RuntimeError("GPU tests need a ROCm device")
    import rans_bench as B
    stream = torch.cuda.current_stream().cuda_stream
    # 16 column tiles per tile row, 8 waves per workgroup: two column groups
    for rows, cols, R, C, seed in ((768, 8192, 8, 512, 1), (256, 4096, 4, 256, 2),
                                   (512, 2048, 8, 256, 3)):
        print(f"case noalloc {rows}x{cols} R={R} C={C}", flush=True)
        codes = B.synth_codes_full(rows, cols, 3.25, seed=seed, escape_frac=0.002)
        step = B.lognormal_steps(cols, seed=seed)
        enc = rans.encode(codes, R, C, 1)
        m = rans.RansMatrix(enc, torch.from_numpy(step), lib)
        split = lib.rans_gemv_workspace_bytes(ctypes.byref(m._desc), 1) > 0
        assert split == (cols // C > 8)
        for batch in (1, 4, 1):
            x = torch.randn(batch, cols, device="cuda").bfloat16()
            want = m.gemv(x)
            for _ in range(2):
                y = torch.full((batch, rows), float("nan"), device="cuda")
                rc = lib.rans_w64_gemv_noalloc(ctypes.byref(m._desc), x.data_ptr(), rans.X_BF16,
                                               batch, y.data_ptr(), stream)
                assert rc == 0, rc
                torch.cuda.synchronize()
                assert torch.equal(y, want)
            ref = oracle.gemv_f64(codes, x.float().cpu().numpy().astype(np.float64),
                                  step.astype(np.float64))
            err = float(np.linalg.norm(y.cpu().numpy() - ref) / np.linalg.norm(ref))
            assert err <= REL_L2, err


@pytest.mark.gpu
def test_noalloc_under_graph_capture(rans, lib):
    """The entry point that allocates nothing is meant for callers under
    HIP graph capture.  Split-K launches at batch 1 and 4 are captured in
    one graph and replayed four times, with eager launches of the same
    entry point and synchronisations between replays: every replay equals
    the eager workspace launch bit for bit, so the scratch counters return
    to zero under replay as well as eagerly."""
    if not torch.cuda.is_available():
        raise RuntimeError("GPU tests need a ROCm device")
    import rans_bench as B
    rows, cols, R, C = 768, 8192, 8, 512  # 16 column tiles: two column groups
    print(f"case noalloc graph {rows}x{cols} R={R} C={C}", flush=True)
    codes = B.synth_codes_full(rows, cols, 3.25, seed=7, escape_frac=0.002)
    step = B.lognormal_steps(cols, seed=7)
    m = rans.RansMatrix(rans.encode(codes, R, C, 1), torch.from_numpy(step), lib)
    assert lib.rans_gemv_workspace_bytes(ctypes.byref(m._desc), 1) > 0
    xs = {b: torch.randn(b, cols, device="cuda").bfloat16() for b in (1, 4)}
    want = {b: m.gemv(x) for b, x in xs.items()}
    ys = {b: torch.empty(b, rows, device="cuda") for b in xs}
    torch.cuda.synchronize()

    def call(b, y, stream):
        return lib.rans_w64_gemv_noalloc(ctypes.byref(m._desc), xs[b].data_ptr(), rans.X_BF16,
                                         b, y.data_ptr(), stream)

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        s = torch.cuda.current_stream().cuda_stream
        rcs = [call(b, ys[b], s) for b in (1, 4)]
    assert rcs == [0, 0], rcs
    other = torch.empty(4, rows, device="cuda")
    for rep in range(4):
        for y in ys.values():
            y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for b in xs:
            assert torch.equal(ys[b], want[b]), (rep, b)
        # eager work on the same scratch between replays
        assert call(4, other, torch.cuda.current_stream().cuda_stream) == 0
        torch.cuda.synchronize()
        assert torch.equal(other, want[4]), rep
