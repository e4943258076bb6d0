"""The reference's own stream format on the GPU, through the reference's own
entry points and argument lists (launch_rans_gemv / launch_rans_decode,
rans_gemv.cu:146-162, as kernel/rans.py:25-29 binds them): the words, offs
and table of the reference's encode (its exact output for its test shapes,
the golden fixture, and the oracle's restatement of it for larger ones),
decoded bit-exact against bf16(code*step) and multiplied within the bar of
the oracle's float64 GEMV, also by the reference test's max-relative < 1e-4
(kernel/bench.py:53-56)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

REL_L2 = 1e-3


@pytest.fixture(scope="module")
def dev(rans):
    if not torch.cuda.is_available():
        raise RuntimeError("GPU tests need a ROCm device")
    return torch.device("cuda")


def _upload(enc):
    return (torch.from_numpy(np.ascontiguousarray(enc["words"]).view(np.int16)).cuda(),
            torch.from_numpy(np.ascontiguousarray(enc["offs"]).view(np.int32)).cuda(),
            torch.from_numpy(np.ascontiguousarray(enc["table"]).view(np.int32)).cuda())


def _run(lib, enc, codes, R, C, seed=0):
    """decode and GEMV through the reference's entry points; checks both."""
    rows, cols = codes.shape
    words, offs, table = _upload(enc)
    rng = np.random.default_rng(seed)
    step = torch.from_numpy((rng.random(cols) * 0.01 + 0.005).astype(np.float32)).cuda()
    st = torch.cuda.current_stream().cuda_stream
    out = torch.full((rows, cols), float("nan"), device="cuda", dtype=torch.bfloat16)
    rc = lib.launch_rans_decode(R, words.data_ptr(), offs.data_ptr(), table.data_ptr(),
                                step.data_ptr(), out.data_ptr(), rows, cols, C, st)
    assert rc == 0, rc
    want = (torch.from_numpy(codes.astype(np.float32)).cuda() * step).bfloat16()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    x = torch.from_numpy(rng.standard_normal(cols).astype(np.float32)).cuda()
    xs = (x * step).contiguous()
    # the reference's contract: y written when cols == C, else added into a zeroed y
    y = torch.full((rows,), float("nan"), device="cuda") if cols == C else torch.zeros(rows, device="cuda")
    rc = lib.launch_rans_gemv(R, words.data_ptr(), offs.data_ptr(), table.data_ptr(),
                              xs.data_ptr(), y.data_ptr(), rows, cols, C, st)
    assert rc == 0, rc
    torch.cuda.synchronize()
    yv = y.cpu().numpy().astype(np.float64)
    import oracle as O
    ref = O.gemv_f64(codes, xs.cpu().numpy().astype(np.float64), np.ones(cols))
    rel = float(np.linalg.norm(yv - ref) / max(np.linalg.norm(ref), 1e-300))
    assert rel <= REL_L2, rel
    assert np.abs(yv - ref).max() / max(np.abs(ref).max(), 1e-30) < 1e-4
    return words, offs, table, xs, y


@pytest.mark.parametrize("i", range(4))
def test_reference_encoded_golden(rans, lib, golden, dev, i):
    """The reference's own encode output for its test shapes
    (kernel/bench.py:41-42), byte for byte as it wrote them."""
    rows, cols, R, C = (int(v) for v in golden[f"enc{i}_meta"])
    print(f"case ref32 golden enc{i} {rows}x{cols} R={R} C={C}", flush=True)
    enc = dict(words=golden[f"enc{i}_words"], offs=golden[f"enc{i}_offs"],
               table=golden[f"enc{i}_table"])
    _run(lib, enc, golden[f"enc{i}_codes"].astype(np.int64), R, C, seed=i)


@pytest.mark.parametrize("case", [
    (1536, 8960, 8, 8960, 3.25),   # the published tiling of the headline shape
    (48, 768, 16, 256, 3.0),       # 9 tiles (an odd count, a half-empty last wave), 3 column tiles
    (64, 2048, 1, 512, 4.25),
    (128, 1024, 2, 1024, 2.25),
    (96, 1536, 4, 512, 3.25),
    (2048, 1536, 4, 512, 4.25),    # the reference's sweep tiling of the 1.5B qkv shape
], ids=lambda c: "x".join(map(str, c[:4])))
def test_reference_format_shapes(rans, oracle, lib, dev, case):
    """Larger shapes through the oracle's restatement of the reference's
    encoder (pinned to its words by the golden fixture), every R the
    reference compiles, one and several column tiles."""
    rows, cols, R, C, bits = case
    print(f"case ref32 {case}", flush=True)
    codes = oracle.synth_codes(rows, cols, bits, seed=rows + cols)
    _run(lib, oracle.encode_ref(codes, R, C), codes.astype(np.int64), R, C)


@pytest.mark.parametrize("rows", [16, 64])
def test_reference_format_spans_beyond_lds(rans, oracle, lib, dev, rows):
    """Near-uniform 8-bit codes in 16x8960 tiles (4480 symbols per stream):
    a wave's streams exceed its LDS slot, so the waves read their words from
    global memory; same results."""
    print(f"case ref32 global path {rows}x8960", flush=True)
    rng = np.random.default_rng(rows)
    codes = rng.integers(-128, 128, size=(rows, 8960)).astype(np.int64)
    enc = oracle.encode_ref(codes, 16, 8960)
    per_lane = np.diff(enc["offs"].astype(np.int64)).mean()
    assert 31 * per_lane + 4480 > 65536  # past the largest slot
    _run(lib, enc, codes, 16, 8960)


def test_reference_format_in_graph(rans, oracle, lib, dev):
    """Captured in a HIP graph (the caller's y zeroing as a fill kernel in
    the graph) and replayed three times with other work in between: every
    replay equals the eager launches."""
    print("case ref32 graph", flush=True)
    codes = oracle.synth_codes(64, 1024, 3.25, seed=5)
    R, C = 8, 512
    words, offs, table, xs, y0 = _run(lib, oracle.encode_ref(codes, R, C), codes.astype(np.int64), R, C)
    y = torch.zeros(64, device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y.zero_()
        rc = lib.launch_rans_gemv(R, words.data_ptr(), offs.data_ptr(), table.data_ptr(),
                                  xs.data_ptr(), y.data_ptr(), 64, 1024, C,
                                  torch.cuda.current_stream().cuda_stream)
        assert rc == 0, rc
    for _ in range(3):
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_allclose(y.cpu().numpy(), y0.cpu().numpy(), rtol=1e-5, atol=1e-6)
        torch.randn(1 << 20, device="cuda").sum().item()


def test_reference_format_unsupported_r(rans, oracle, lib, dev):
    """Configuration 1's R=512 has no kernel in the reference (its GPU path
    takes R in {1, 2, 4, 8, 16}): -1, as the reference returns."""
    codes = oracle.synth_codes(512, 256, 3.25, seed=1)
    words, offs, table = _upload(oracle.encode_ref(codes, 512, 256))
    y = torch.zeros(512, device="cuda")
    x = torch.zeros(256, device="cuda")
    assert lib.launch_rans_gemv(512, words.data_ptr(), offs.data_ptr(), table.data_ptr(),
                                x.data_ptr(), y.data_ptr(), 512, 256, 256,
                                torch.cuda.current_stream().cuda_stream) == -1


def test_reference_layout_matrix(rans, oracle, lib, dev):
    """encode_reference_layout + ReferenceLayoutMatrix, the reference's
    encode and RansMatrix contract (kernel/rans.py:62-162) on its own
    layout: the published tiling of the headline shape, decode bit-exact,
    gemv within the bar of the oracle (twice into the same y, which it
    zeroes itself when a row spans several column tiles), a one-value step."""
    import rans_bench as B
    print("case reference layout matrix 1536x8960 R=8 C=8960 and R=8 C=2240", flush=True)
    codes = B.synth_codes_full(1536, 8960, 3.25, seed=1536 + 8960)
    step = B.lognormal_steps(8960, seed=3)
    x = torch.randn(8960, device="cuda").bfloat16()
    for C in (8960, 2240):
        m = rans.ReferenceLayoutMatrix(rans.encode_reference_layout(codes, 8, C),
                                       torch.from_numpy(step), lib)
        want = (torch.from_numpy(codes.astype(np.float32)) * torch.from_numpy(step)).bfloat16()
        assert torch.equal(m.decode().cpu().view(torch.int16), want.view(torch.int16))
        ref = oracle.gemv_f64(codes, x.float().cpu().numpy().astype(np.float64),
                              step.astype(np.float64))
        y = torch.empty(1536, device="cuda")
        for _ in range(2):
            yv = m.gemv(x, y).cpu().numpy().astype(np.float64)
            assert np.linalg.norm(yv - ref) / np.linalg.norm(ref) <= REL_L2
    m1 = rans.ReferenceLayoutMatrix(rans.encode_reference_layout(codes[:64, :512], 8, 512),
                                    torch.tensor(0.02), lib)
    want = (torch.from_numpy(codes[:64, :512].astype(np.float32)) * 0.02).bfloat16()
    assert torch.equal(m1.decode().cpu().view(torch.int16), want.view(torch.int16))


def test_reference_format_exact_size_allocation(rans, lib, golden, dev):
    """`words` in an allocation of exactly its own size (hipMalloc of 3849
    words, not a whole number of 16-byte chunks): the last wave's span is cut
    at the allocation's end and its last words are staged one by one; the
    decode is still exact."""
    import ctypes
    rows, cols, R, C = (int(v) for v in golden["enc0_meta"])
    words = np.ascontiguousarray(golden["enc0_words"])
    assert words.nbytes % 16
    hip = ctypes.CDLL("libamdhip64.so")
    ptr = ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(ptr), ctypes.c_size_t(words.nbytes)) == 0
    try:
        assert hip.hipMemcpy(ptr, words.ctypes.data_as(ctypes.c_void_p),
                             ctypes.c_size_t(words.nbytes), 1) == 0  # host to device
        offs = torch.from_numpy(golden["enc0_offs"].view(np.int32)).cuda()
        table = torch.from_numpy(golden["enc0_table"].view(np.int32)).cuda()
        step = torch.full((cols,), 0.5, device="cuda")
        out = torch.full((rows, cols), float("nan"), device="cuda", dtype=torch.bfloat16)
        rc = lib.launch_rans_decode(R, ptr.value, offs.data_ptr(), table.data_ptr(),
                                    step.data_ptr(), out.data_ptr(), rows, cols, C,
                                    torch.cuda.current_stream().cuda_stream)
        assert rc == 0, rc
        torch.cuda.synchronize()
        want = (torch.from_numpy(golden["enc0_codes"].astype(np.float32)) * 0.5).bfloat16()
        assert torch.equal(out.cpu().view(torch.int16), want.view(torch.int16))
    finally:
        torch.cuda.synchronize()
        hip.hipFree(ptr)


def test_reference_format_unaligned_words(rans, lib, golden, dev):
    """`words` starting 2 bytes into an allocation (not 16-byte aligned): the
    spans are staged through registers instead of direct copies; same
    decode and GEMV."""
    rows, cols, R, C = (int(v) for v in golden["enc1_meta"])
    print(f"case ref32 unaligned words {rows}x{cols}", flush=True)
    w = golden["enc1_words"]
    buf = torch.zeros(w.size + 1, dtype=torch.int16, device="cuda")
    buf[1:] = torch.from_numpy(np.ascontiguousarray(w).view(np.int16)).cuda()
    words = buf[1:]
    assert words.data_ptr() % 16 != 0
    offs = torch.from_numpy(golden["enc1_offs"].view(np.int32)).cuda()
    table = torch.from_numpy(golden["enc1_table"].view(np.int32)).cuda()
    codes = golden["enc1_codes"].astype(np.int64)
    step = torch.full((cols,), 0.25, device="cuda")
    out = torch.empty(rows, cols, device="cuda", dtype=torch.bfloat16)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.launch_rans_decode(R, words.data_ptr(), offs.data_ptr(), table.data_ptr(),
                                  step.data_ptr(), out.data_ptr(), rows, cols, C, st) == 0
    want = (torch.from_numpy(codes.astype(np.float32)) * 0.25).bfloat16()
    assert torch.equal(out.cpu().view(torch.int16), want.view(torch.int16))
    x = torch.randn(cols, device="cuda")
    y = torch.zeros(rows, device="cuda")
    assert lib.launch_rans_gemv(R, words.data_ptr(), offs.data_ptr(), table.data_ptr(),
                                x.data_ptr(), y.data_ptr(), rows, cols, C, st) == 0
    import oracle as O
    ref = O.gemv_f64(codes, x.cpu().numpy().astype(np.float64), np.ones(cols))
    yv = y.cpu().numpy().astype(np.float64)
    assert np.linalg.norm(yv - ref) / np.linalg.norm(ref) <= REL_L2
