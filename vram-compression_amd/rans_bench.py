"""Usage:
  python vram-compression_amd/rans_bench.py test    # correctness on small shapes
  python vram-compression_amd/rans_bench.py bench   # timing sweep, JSON report
  python vram-compression_amd/rans_bench.py configs # the benchmark configurations
  python vram-compression_amd/rans_bench.py chain [grouped|separate|both] [LAYERS] [BATCH]
  python vram-compression_amd/rans_bench.py profile [ROWS COLS BITS DIST ESC R C N FETCH]

Mirror of kernel/bench.py of snuri00/vram-compression (same function names
and record keys, bench.py:20-126) for the w64 GEMV, plus the synthetic
workloads of the MI355X benchmark configurations: full-tensor entropy
targeting, Gaussian / Laplace / Student-t codes, forced escapes and
log-normal per-column (waterfilling) steps.

Timing is done on the device: a launch sequence is captured once in a HIP
graph and replayed between HIP events, so host dispatch cost (about 10-20 us
per Python-level call) does not hide a kernel of a few microseconds.
"""
import ctypes
import hashlib
import json
import os
import sys

import numpy as np
import torch

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import rans  # noqa: E402
from rans import encode, gemv_group, pick_group_tiling, pick_tiling  # noqa: E402,F401

RES = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "results")


# ----------------------------------------------------------- synthetic codes
def entropy(codes):
    """Empirical entropy, bits/symbol (bench.py:20-23)."""
    _, c = np.unique(codes, return_counts=True)
    p = c / c.sum()
    return float(-(p * np.log2(p)).sum())


def entropy_fast(codes):
    """Same value as entropy() for integer codes, via bincount (linear time)."""
    c = np.asarray(codes).ravel()
    lo = int(c.min())
    cnt = np.bincount((c - lo).astype(np.int64))
    cnt = cnt[cnt > 0]
    p = cnt / cnt.sum()
    return float(-(p * np.log2(p)).sum())


def synth_codes(rows, cols, target_bits, dist="laplace", seed=0):
    """bench.py:26-35 exactly: Laplace or N(0,1) weights from
    default_rng(seed), 40-step bisection of log(step) on the entropy of the
    first min(rows, 256) rows, codes clipped to [-127, 127]."""
    rng = np.random.default_rng(seed)
    w = rng.laplace(size=(rows, cols)) if dist == "laplace" else rng.standard_normal((rows, cols))
    lo, hi = -12.0, 6.0
    for _ in range(40):
        mid = (lo + hi) / 2
        h = entropy(np.round(w[: min(rows, 256)] / np.exp(mid)))
        lo, hi = (mid, hi) if h > target_bits else (lo, mid)
    return np.clip(np.round(w / np.exp((lo + hi) / 2)), -127, 127).astype(np.int32)


def _weights(rng, shape, dist):
    if dist == "laplace":
        return rng.laplace(size=shape)
    if dist == "gauss":
        return rng.standard_normal(shape)
    if dist == "student3":
        return rng.standard_t(3, size=shape)
    raise ValueError(dist)


def synth_codes_full(rows, cols, target_bits, dist="laplace", seed=0, escape_frac=0.0,
                     tol=0.005):
    """ECSQ-like codes round(w/step) with one step per tensor chosen so the
    FULL tensor's empirical entropy is target_bits +- tol (no clipping: the
    levels are unbounded).  The bisection runs on a 2^22-element sample and is
    refined on the full tensor.  escape_frac of the positions (chosen at
    random, each independently) are then forced to |code| in [128, 600),
    beyond the table range."""
    rng = np.random.default_rng(seed)
    w = _weights(rng, (rows, cols), dist)
    flat = w.ravel()
    sample = flat if flat.size <= 1 << 22 else flat[rng.choice(flat.size, 1 << 22, replace=False)]
    lo, hi = -12.0, 6.0
    for _ in range(40):
        mid = (lo + hi) / 2
        h = entropy_fast(np.round(sample / np.exp(mid)).astype(np.int64))
        lo, hi = (mid, hi) if h > target_bits else (lo, mid)
    logd = (lo + hi) / 2
    codes = np.round(w / np.exp(logd)).astype(np.int64)
    # refine on the full tensor (entropy decreases as the step grows)
    flo, fhi = logd - 0.05, logd + 0.05
    for _ in range(30):
        h = entropy_fast(codes)
        if abs(h - target_bits) <= tol:
            break
        flo, fhi = (logd, fhi) if h > target_bits else (flo, logd)
        logd = (flo + fhi) / 2
        codes = np.round(w / np.exp(logd)).astype(np.int64)
    codes = codes.astype(np.int32)
    if escape_frac > 0:
        pos = np.flatnonzero(rng.random(codes.size) < escape_frac)
        n = pos.size
        mag = rng.integers(128, 600, n)
        sign = np.where(rng.random(n) < 0.5, -1, 1)
        codes.ravel()[pos] = (sign * mag).astype(np.int32)
    return codes


ECSQ_FIXTURE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                            "tests", "golden", "ecsq_wf_kv.npz")


def ecsq_fixture(rows=None):
    """Codes with ECSQ-GPTQ + waterfilling statistics and their per-column
    steps: the k projection (256 x 1536) of a synthetic random-init
    Qwen2.5-1.5B layer quantised at 3.25 b/w by the reference's own ecsq
    with waterfilling (exp/quant.py:122-156, imported by
    tests/golden/make_ecsq_golden.py, which wrote the fixture).  rows: a multiple of 256, the 256 rows
    repeated to that height.  Returns (int32 codes, float32 steps)."""
    z = np.load(ECSQ_FIXTURE)
    codes = z["codes"].astype(np.int32)
    if rows is not None:
        assert rows % codes.shape[0] == 0, "rows must be a multiple of 256"
        codes = np.tile(codes, (rows // codes.shape[0], 1))
    return np.ascontiguousarray(codes), z["step"].astype(np.float32)


def lognormal_steps(cols, sigma=0.5, seed=0, scale=0.01):
    """Per-column waterfilling steps scale*exp(sigma*N(0,1))."""
    rng = np.random.default_rng(seed + 1)
    return (scale * np.exp(sigma * rng.standard_normal(cols))).astype(np.float32)


# ------------------------------------------------------------------- timing
def timeit(fn, iters=200):
    """Event timing of eager calls, as bench.py:69-79 (10 warm-ups); us/call.
    Includes host dispatch cost."""
    for _ in range(10):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(iters):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / iters * 1000


def copies_for(iters, nbytes, rotate_bytes=512 << 20):
    """Distinct copies of an nbytes operand for a rotated run of `iters`
    launches: n = ceil(rotate_bytes / nbytes) + 1 copies when iters >= n
    (the timed launches cycle through them, so every copy is read again only
    after the other n - 1, at least rotate_bytes), else iters + n (the timed
    launches use the first iters copies; an untimed flush replay reads the
    other n just before them)."""
    n = max(2, -(-rotate_bytes // nbytes) + 1)
    return n if iters >= n else iters + n


# hipEventDisableSystemFence (hip_runtime_api.h): the event records without a
# system-scope cache writeback and invalidate, which is a cost of the timing
# event and not of the work it brackets.  On MI355X the default events add
# ~10 us to a timed region (0.5 us per launch over 20 headline GEMVs, 11.1
# against 10.6 us; equal at 200).
HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000
_HIP = None


def _hip():
    global _HIP
    if _HIP is None:
        h = ctypes.CDLL("libamdhip64.so")
        h.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        h.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                          ctypes.c_void_p]
        h.hipEventDestroy.argtypes = [ctypes.c_void_p]
        _HIP = h
    return _HIP


def device_elapsed_us(run):
    """Device microseconds of the work run() queues on the current stream,
    between two HIP events recorded on that stream (created with
    hipEventDisableSystemFence); the host waits for the second."""
    h = _hip()
    stream = torch.cuda.current_stream().cuda_stream
    evs = []
    try:
        for _ in range(2):
            e = ctypes.c_void_p()
            rc = h.hipEventCreateWithFlags(ctypes.byref(e), HIP_EVENT_DISABLE_SYSTEM_FENCE)
            if rc != 0:
                raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")
            evs.append(e)
        if h.hipEventRecord(evs[0], stream) != 0:
            raise RuntimeError("hipEventRecord failed")
        run()
        if h.hipEventRecord(evs[1], stream) != 0 or h.hipEventSynchronize(evs[1]) != 0:
            raise RuntimeError("hipEventRecord / hipEventSynchronize failed")
        ms = ctypes.c_float()
        if h.hipEventElapsedTime(ctypes.byref(ms), evs[0], evs[1]) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value * 1000.0
    finally:
        for e in evs:
            h.hipEventDestroy(e)


# Untimed device work queued right before a timed region.  The GPU's clocks
# ramp up over a few milliseconds of load after an idle spell (the host-side
# encoding and uploads before each measurement): on MI355X, 20 headline GEMVs
# timed right after one untimed pass over the rotated copies read 11.2 us,
# after ~15 ms of untimed passes 10.6 us (25600x5120: 54.3 and 51.5 us).
WARM_US = 10000.0


def warm_then_time(timed, lead=None):
    """Device microseconds of timed.replay() (a captured graph), after
    replays of `lead` (default: timed itself), all queued back to back,
    totalling at least WARM_US of device time (at most 1000 replays, so a
    tiny graph does not turn into a host-bound loop); the last lead replay
    runs just before the timed one, so the start event does not wait for
    the host to submit it."""
    lead = lead or timed
    t_lead = device_elapsed_us(lead.replay)
    for _ in range(min(1000, max(1, -(-int(WARM_US) // max(1, int(t_lead)))))):
        lead.replay()
    t = device_elapsed_us(timed.replay)
    torch.cuda.synchronize()
    return t


def timeit_graph(fns, iters=200, warmup=10, rotate=False):
    """Device time per call: fns (one callable, or a list cycled through, one
    per rotating copy, sized by copies_for) are captured `iters` times in a
    HIP graph; the graph is replayed once untimed and then, after at least
    WARM_US of untimed replays (warm_then_time), timed between HIP events.
    With several copies, an untimed graph runs just before the
    timed replay: the copies the timed graph does not use (iters below
    len(fns)), else every copy once in order, so every timed call reads a
    copy that the other copies have displaced from the caches.  rotate is
    accepted for older callers and has no further effect.
    Returns microseconds per call."""
    if callable(fns):
        fns = [fns]
    for i in range(warmup):
        fns[i % len(fns)]()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for f in fns[:2]:
            f()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(iters):
            fns[i % len(fns)]()
    # untimed lead-in replayed just before the timed graph: with several
    # copies, the ones the timed calls do not use (iters < len(fns)) or every
    # copy once in order, so each timed call reads a copy all the others
    # followed; with one callable, the timed graph once more
    lead = g
    if len(fns) > 1:
        lead = torch.cuda.CUDAGraph()
        with torch.cuda.graph(lead):
            for f in (fns[iters:] if iters < len(fns) else fns):
                f()
    g.replay()
    lead.replay()
    torch.cuda.synchronize()
    return warm_then_time(g, lead) / iters


def test():
    """The reference's test (bench.py:38-66) on the w64 layout."""
    lib = rans.build()
    torch.manual_seed(0)
    for (rows, cols, R, C, S, bits) in [(64, 256, 4, 256, 1, 3.0), (128, 512, 8, 128, 1, 2.0),
                                        (256, 1024, 16, 512, 2, 4.0), (32, 64, 1, 64, 1, 1.0)]:
        codes = synth_codes(rows, cols, bits, seed=rows)
        enc = rans.encode(codes, R, C, S)
        ref = rans.decode_ref(enc)
        assert np.array_equal(ref, codes), "host decode mismatch"
        step = torch.rand(cols) + 0.5
        m = rans.RansMatrix(enc, step, lib)
        assert np.array_equal(m.decode_codes().cpu().numpy(), codes), "GPU code decode mismatch"
        dec = m.decode().float().cpu()
        want = torch.from_numpy(codes).float() * step
        assert torch.equal(dec, want.bfloat16().float()), "GPU decode mismatch"
        x = torch.randn(cols, device="cuda")
        y = m.gemv(x)
        y_ref = torch.from_numpy(codes).double().cuda() @ (x.double() * step.double().cuda())
        err = ((y.double() - y_ref).norm() / y_ref.norm()).item()
        assert err < 1e-3, f"GEMV mismatch {err}"
        print(f"ok  {rows}x{cols} R={R} C={C} S={S}  H={entropy(codes):.2f}  "
              f"payload={enc['bits_payload']:.3f}  overhead={enc['bits_state_offs']:.3f} bit/w  "
              f"gemv_rel_l2={err:.1e}")
    codes = np.random.default_rng(1).integers(-8, 8, size=(256, 1024))
    step = torch.rand(1024) + 0.5
    m4 = rans.Int4Matrix(codes, step, lib)
    x = torch.randn(1024, device="cuda")
    y_ref = torch.from_numpy(codes).float().cuda() @ (x * step.cuda())
    assert torch.allclose(m4.gemv(x), y_ref, rtol=1e-4, atol=1e-3)
    print("ok  int4 baseline")


def library_source_hash():
    """First 12 hex digits of the SHA-256 of the library's sources and
    header (rans.SOURCES, rans.HEADERS, in that order): names the build a
    measurement belongs to."""
    h = hashlib.sha256()
    for path in rans.SOURCES + rans.HEADERS:
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:12]


BENCH_FILE = "kernel_bench_mi355x.json"


def bench(rotate_bytes=512 << 20, iters=200, out_name=BENCH_FILE):
    """bench.py:82-126 on the w64 GEMV: the same 18 shapes and rates, codes
    from the same generator and seeds, the same record keys.  Every time is
    the device time of graph-replayed launches over rotated copies
    (copies_for: each timed launch reads a copy that at least rotate_bytes
    of other copies have displaced from the 256 MB Infinity Cache and the
    L2), for the rANS GEMV, F.linear (t_bf16_us), the library's bf16_gemv
    (t_bf16_hip_us), the int4 GEMV with its host fold (t_int4_us) and
    decode-to-bf16 + F.linear (t_decode_then_cublas_us).  The tiling is the
    library's pick_tiling with one and with two states per lane, the faster
    kept.  Writes results/<out_name>: {"meta": ..., "records": [...]}."""
    lib = rans.build()
    shapes = {"1.5B qkv": (2048, 1536), "1.5B gate_up": (17920, 1536), "1.5B down": (1536, 8960),
              "27B-like attn": (5120, 5120), "27B-like gate_up": (34816, 5120),
              "27B-like down": (5120, 17408)}
    out = []
    for name, (rows, cols) in shapes.items():
        for bits in (2.0, 3.0, 4.0):
            codes = synth_codes(rows, cols, bits, seed=rows + cols)
            step = torch.rand(cols) * 0.01 + 0.005
            x = torch.randn(cols, device="cuda")
            xb = x.bfloat16()
            nW = copies_for(iters, rows * cols * 2, rotate_bytes)
            W = (torch.from_numpy(codes).float() * step).bfloat16().cuda()
            Ws = [W] + [W.clone() for _ in range(nW - 1)]
            t_bf16 = timeit_graph([lambda W=W: torch.nn.functional.linear(xb, W) for W in Ws], iters)
            mbs = [rans.Bf16Matrix(W, lib) for W in Ws]
            yh = torch.empty(rows, device="cuda")
            t_bf16_hip = timeit_graph([lambda mb=mb: mb.gemv(xb, yh) for mb in mbs], iters)
            del Ws, mbs, W
            n4 = copies_for(iters, rows * cols // 2, rotate_bytes)
            m4 = rans.Int4Matrix(np.clip(codes, -8, 7), step, lib)
            m4s = [m4] + [m4.clone() for _ in range(n4 - 1)]
            y4 = torch.empty(rows, device="cuda")
            t_int4 = timeit_graph([lambda m4=m4: m4.gemv(x, y4) for m4 in m4s], iters)
            del m4s, m4
            best = None
            for S in (1, 2):
                R, C = pick_tiling(rows, cols, S=S)
                enc = rans.encode(codes, R, C, S)
                m = rans.RansMatrix(enc, step, lib)
                ncopy = copies_for(iters, m.nbytes, rotate_bytes)
                ms = [m] + [rans.RansMatrix(enc, step, lib) for _ in range(ncopy - 1)]
                yb = torch.empty(rows, device="cuda")
                t = timeit_graph([lambda mm=mm: mm.gemv(xb, yb) for mm in ms], iters)
                if best is None or t < best["t_rans_us"]:
                    best = dict(R=R, C=C, S=S, t_rans_us=t, bits_total=8 * m.nbytes / codes.size,
                                bits_payload=enc["bits_payload"],
                                bits_overhead=enc["bits_state_offs"] + enc["bits_table"] +
                                enc["bits_escape"], copies=ncopy, _ms=ms)
                else:
                    del ms
                del m
            ms = best.pop("_ms")
            buf = torch.empty(rows, cols, device="cuda", dtype=torch.bfloat16)
            best["t_decode_then_cublas_us"] = timeit_graph(
                [lambda mm=mm: torch.nn.functional.linear(xb, mm.decode(buf)) for mm in ms], iters)
            del ms, buf
            r = dict(shape=name, rows=rows, cols=cols, entropy=entropy_fast(codes),
                     t_bf16_us=t_bf16, t_bf16_hip_us=t_bf16_hip, t_int4_us=t_int4, **best,
                     bf16_copies=nW, int4_copies=n4)
            r["speedup_vs_bf16"] = t_bf16 / r["t_rans_us"]
            r["speedup_vs_bf16_hip"] = t_bf16_hip / r["t_rans_us"]
            r["speedup_vs_int4"] = t_int4 / r["t_rans_us"]
            print(json.dumps({k: (round(v, 3) if isinstance(v, float) else v) for k, v in r.items()}),
                  flush=True)
            out.append(r)
            torch.cuda.empty_cache()
    meta = dict(device=torch.cuda.get_device_name(0),
                arch=getattr(torch.cuda.get_device_properties(0), "gcnArchName", "gfx950"),
                torch=torch.__version__, hip=torch.version.hip,
                library_source_hash=library_source_hash(), iters=iters,
                rotate_bytes=rotate_bytes,
                timing="device time per launch of `iters` launches captured in one HIP graph, "
                       "replayed between HIP events, rotating over distinct copies",
                workload="kernel/bench.py:26-35 generator (synth_codes, seed rows+cols), one step "
                         "U[0.005, 0.015) per column, f32 x (bf16 for the bf16 and rANS GEMVs)")
    os.makedirs(RES, exist_ok=True)
    with open(os.path.join(RES, out_name), "w") as f:
        json.dump({"meta": meta, "records": out}, f, indent=1)


def bench_reference_layout(rotate_bytes=512 << 20, iters=200, out_name="kernel_bench_reflayout.json"):
    """bench.py:82-126 on the reference's own 32-lane layout
    (encode_reference_layout + ReferenceLayoutMatrix, launch_rans_gemv with
    the host fold): the same shapes, rates, record keys and (R, C) sweep,
    the best tiling picked on hot timings as the reference's bench does,
    then timed again over rotated copies (t_rans_us; the hot figure is
    t_rans_hot_us).  The comparators are left out: bench() measures them on
    the same inputs."""
    lib = rans.build()
    shapes = {"1.5B qkv": (2048, 1536), "1.5B gate_up": (17920, 1536), "1.5B down": (1536, 8960),
              "27B-like attn": (5120, 5120), "27B-like gate_up": (34816, 5120),
              "27B-like down": (5120, 17408)}
    out = []
    for name, (rows, cols) in shapes.items():
        for bits in (2.0, 3.0, 4.0):
            codes = synth_codes(rows, cols, bits, seed=rows + cols)
            step = torch.rand(cols) * 0.01 + 0.005
            x = torch.randn(cols, device="cuda")
            yb = torch.empty(rows, device="cuda")
            best = None
            for R in (4, 8, 16):
                for C in sorted({cols, 512, 1024, 2048} & set(range(32, cols + 1, 32))):
                    if cols % C or rows % R:
                        continue
                    enc = rans.encode_reference_layout(codes, R, C)
                    m = rans.ReferenceLayoutMatrix(enc, step, lib)
                    t = timeit_graph(lambda: m.gemv(x, yb), iters)
                    if best is None or t < best[0]:
                        best = (t, R, C, enc)
                    del m
            t_hot, R, C, enc = best
            m0 = rans.ReferenceLayoutMatrix(enc, step, lib)
            ncopy = copies_for(iters, m0.nbytes, rotate_bytes)
            ms = [m0] + [rans.ReferenceLayoutMatrix(enc, step, lib) for _ in range(ncopy - 1)]
            t = timeit_graph([lambda mm=mm: mm.gemv(x, yb) for mm in ms], iters, rotate=True)
            del ms
            r = dict(shape=name, rows=rows, cols=cols, entropy=entropy_fast(codes), R=R, C=C,
                     t_rans_us=t, t_rans_hot_us=t_hot, bits_total=8 * m0.nbytes / codes.size,
                     bits_payload=enc["bits_payload"],
                     bits_overhead=enc["bits_state_offs"] + enc["bits_table"], copies=ncopy)
            del m0
            print(json.dumps({k: (round(v, 3) if isinstance(v, float) else v) for k, v in r.items()}),
                  flush=True)
            out.append(r)
            torch.cuda.empty_cache()
    os.makedirs(RES, exist_ok=True)
    with open(os.path.join(RES, out_name), "w") as f:
        json.dump(out, f, indent=1)


# ------------------------------------------------ benchmark configurations
def qwen15b_layer_shapes():
    """(name, rows, cols) of one Qwen2.5-1.5B decoder layer's linear maps."""
    return [("q", 1536, 1536), ("k", 256, 1536), ("v", 256, 1536), ("o", 1536, 1536),
            ("gate", 8960, 1536), ("up", 8960, 1536), ("down", 1536, 8960)]


# Tilings of the per-token chain that spend its bits on more states where a
# launch is short, measured on MI355X (rotated copies, 3.25 bits, µs per
# launch, with compact state metadata):
# - o, 1536x1536: 3x512 5.16 at 4.46 bits/weight, against pick_tiling's 8x384
#   6.35 at 3.91 (3x384: 4.95 at 4.83);
# - down, 1536x8960: 3x1792 as the headline (3.4% faster than 3x2240);
# - the q/k/v group (2048 rows): 8x256, 1536 waves, against 16x256's 768.
# The whole chain then takes 993 us per token at 3.646 bits/weight against
# 1082 us at 3.573 with pick_tiling's tilings (one box, two runs each); the
# next denser choice (o 3x384) passes 3.66 bits.
CHAIN_TILING = {(1536, 1536): (3, 512), (1536, 8960): (3, 1792)}
CHAIN_GROUP_TILING = {"qkv": (8, 256)}


def chain_tiling(rows, cols):
    """Tiling for one matrix of the per-token chain: CHAIN_TILING's for the
    shapes it measured, else the library's default (pick_tiling)."""
    return CHAIN_TILING.get((rows, cols)) or pick_tiling(rows, cols, S=1)


HBM_PEAK_GBS = 8000.0  # MI355X HBM3E peak


def config_matrix(rows, cols, bits, dist, escape_frac, batch, seed, lib, R=None, C=None, S=1,
                  iters=100, rotate_bytes=512 << 20, codes=None, step=None):
    """Times one encoded matrix (rotated over >= rotate_bytes of copies),
    the bf16 F.linear and the library's bf16_gemv on the same shape and
    rotation; checks the GEMV.
    codes/step: a given matrix and its steps instead of synthetic ones.
    batch: rows of x, or a tuple of them (one record per entry, in order,
    all on the same encoded matrix and copies)."""
    batches = tuple(batch) if isinstance(batch, (tuple, list)) else (batch,)
    if codes is None:
        codes = synth_codes_full(rows, cols, bits, dist=dist, seed=seed, escape_frac=escape_frac)
        step = torch.from_numpy(lognormal_steps(cols, seed=seed))
    else:
        step = torch.from_numpy(np.asarray(step, np.float32))
    if R is None or C is None:
        R, C = pick_tiling(rows, cols, S=S, bits=bits)
    enc = encode(codes, R, C, S)
    m = rans.RansMatrix(enc, step, lib)
    ncopy = copies_for(iters, m.nbytes, rotate_bytes)
    nW = copies_for(iters, rows * cols * 2, rotate_bytes)
    W = (torch.from_numpy(codes.astype(np.float32)) * step).bfloat16().cuda()
    Ws = [W] + [W.clone() for _ in range(nW - 1)]
    mbs = [rans.Bf16Matrix(Wd, lib) for Wd in Ws]
    yh = torch.empty(rows, device="cuda")
    Wd64 = torch.from_numpy(codes).cuda().double().t()
    h = entropy_fast(codes)
    out = []
    for b in batches:
        flags = m.tune(batch=b)
        ms = [rans.RansMatrix(enc, step, lib, flags=flags) for _ in range(ncopy)]
        x = torch.randn(b, cols, device="cuda").bfloat16()
        y = torch.empty(b, rows, device="cuda")
        t_rans = timeit_graph([lambda mm=mm: mm.gemv(x, y) for mm in ms], iters, rotate=True)
        t_bf16 = timeit_graph([lambda Wd=Wd: torch.nn.functional.linear(x, Wd) for Wd in Ws],
                              iters, rotate=True)

        # the library's dense bf16_gemv on the same copies (one vector per
        # launch, so batch b takes b launches)
        def dense(mb, x=x, b=b):
            for i in range(b):
                mb.gemv(x[i], yh)

        t_bf16_hip = timeit_graph([lambda mb=mb: dense(mb) for mb in mbs], iters, rotate=True)
        # against the exact product codes @ (x * step) in float64 (the bf16
        # comparator's weights are themselves rounded)
        ref = (x.double() * step.double().cuda()) @ Wd64
        got = ms[0].gemv(x).double()
        err = float((got - ref).norm() / ref.norm())
        # bytes one launch must move: the matrix as the device holds it, x
        # (bf16), the step vector and y (f32)
        alg = m.nbytes + 2 * cols * b + 4 * cols + 4 * rows * b
        out.append(dict(rows=rows, cols=cols, bits_target=bits, dist=dist,
                        escape_frac=escape_frac, batch=b, R=R, C=C, S=S,
                        word_fetch={1: "always", 2: "refill"}[flags & 3],
                        entropy=h, bits_total=8 * m.nbytes / codes.size,
                        n_escapes=int(len(enc["esc_pos"])), t_rans_us=t_rans,
                        t_bf16_us=t_bf16, t_bf16_hip_us=t_bf16_hip,
                        effective_GBps=rows * cols * 2 / t_rans / 1e3,
                        compressed_GBps=m.nbytes / t_rans / 1e3,
                        compressed_bytes=int(m.nbytes), algorithmic_bytes=int(alg),
                        roofline_frac=alg / t_rans / 1e3 / HBM_PEAK_GBS,
                        speedup_vs_bf16=t_bf16 / t_rans, speedup_vs_bf16_hip=t_bf16_hip / t_rans,
                        rel_l2_vs_f64=err, copies=ncopy, bf16_copies=nW))
        del ms
    del mbs, Ws, m
    torch.cuda.empty_cache()
    return out if isinstance(batch, (tuple, list)) else out[0]


# projections of a layer that read the same activations
CHAIN_GROUPS = {"q": "qkv", "k": "qkv", "v": "qkv", "gate": "mlp", "up": "mlp"}


def build_chain(bits=3.25, layers=28, seed=0, grouped=False, batch=1, tune=False,
                keep_codes=False, bf16=True, lib=None):
    """The per-token chain's weight set: 7*layers matrices over a
    random-init Qwen2.5-1.5B-shaped model (one table per matrix, ECSQ-like
    Laplace codes at `bits` bits/weight, log-normal steps), encoded and
    uploaded, and its launch sequence.

    grouped: q, k, v and gate, up of a layer are tiled for one grouped
    launch each (CHAIN_GROUP_TILING, else pick_group_tiling).  tune: the
    word-fetch policy is timed once per shape, on the first layer
    (RansMatrix.tune, hot launches of one copy); off by default, since the
    library's policy was chosen on cold copies and the chain reads its
    weights cold (on o in 8x384 tiles tune picked "always", 7.2 us cold
    against "refill"'s 6.35).  keep_codes: keep each matrix's
    codes and step on the host (for a parity check).  bf16: also build the
    bf16 weights of the comparator chain.

    Returns a dict: mats (RansMatrix, chain order), names, launches (lists
    of matrix indices, one per launch), xs (one bf16 activation per cols, of
    `batch` rows), codes/steps (with keep_codes), Ws (bf16 weights), nbytes,
    nweights."""
    lib = lib or rans.build()
    rng = np.random.default_rng(seed)
    mats, names, launches, codes_l, steps_l, Ws, xs = [], [], [], [], [], [], {}
    nbytes = nweights = 0
    deltas, fetch = {}, {}
    shapes = qwen15b_layer_shapes()
    tiling = {name: chain_tiling(rows, cols) for name, rows, cols in shapes}
    if grouped:
        for g in set(CHAIN_GROUPS.values()):
            members = [(n, r, c) for n, r, c in shapes if CHAIN_GROUPS.get(n) == g]
            t = CHAIN_GROUP_TILING.get(g) or \
                pick_group_tiling([r for _, r, _ in members], members[0][2])
            for n, _, _ in members:
                tiling[n] = t
    # one step per shape, chosen on a sample, so every layer has ~`bits` bits
    for name, rows, cols in shapes:
        sample = rng.laplace(size=1 << 20)
        lo, hi = -12.0, 6.0
        for _ in range(40):
            mid = (lo + hi) / 2
            h = entropy_fast(np.round(sample / np.exp(mid)).astype(np.int64))
            lo, hi = (mid, hi) if h > bits else (lo, mid)
        deltas[name] = np.exp((lo + hi) / 2)
    for layer in range(layers):
        for name, rows, cols in shapes:
            codes = np.round(rng.laplace(size=(rows, cols)) / deltas[name]).astype(np.int32)
            stepv = lognormal_steps(cols, seed=seed + layer)
            R, C = tiling[name]
            enc = encode(codes, R, C, 1)
            # word-fetch policy tuned once per shape, on the first layer
            m = rans.RansMatrix(enc, torch.from_numpy(stepv), lib, flags=fetch.get(name, 0))
            if name not in fetch:
                fetch[name] = m.tune() if tune else m.flags & rans.F_WORDS_MASK
            i = len(mats)
            mats.append(m)
            names.append(name)
            g = CHAIN_GROUPS.get(name) if grouped else None
            if g and launches and CHAIN_GROUPS.get(names[launches[-1][0]]) == g \
                    and len(launches[-1]) < rans.GROUP_MAX:
                launches[-1].append(i)
            else:
                launches.append([i])
            nbytes += m.nbytes
            nweights += codes.size
            if keep_codes:
                codes_l.append(codes)
                steps_l.append(stepv)
            if bf16:
                Ws.append((torch.from_numpy(codes.astype(np.float32)) *
                           torch.from_numpy(stepv)).bfloat16().cuda())
            if cols not in xs:
                xs[cols] = torch.randn(batch, cols, device="cuda").bfloat16()
            print(f"chain: layer {layer} {name} encoded", file=sys.stderr, flush=True) \
                if name == "down" and layer % 7 == 0 else None
    return dict(mats=mats, names=names, launches=launches, xs=xs, codes=codes_l,
                steps=steps_l, Ws=Ws, nbytes=nbytes, nweights=nweights, batch=batch)


def run_chain(ch, ys):
    """Issues the chain's launches on the current stream: ys[i] receives
    matrix i's product (several matrices may share one buffer)."""
    mats = ch["mats"]
    for launch in ch["launches"]:
        if len(launch) > 1:
            gemv_group([mats[i] for i in launch], ch["xs"][mats[launch[0]].cols],
                       [ys[i] for i in launch])
        else:
            m = mats[launch[0]]
            m.gemv(ch["xs"][m.cols], ys[launch[0]])


def chain(bits=3.25, layers=28, seed=0, iters=3, grouped=False, batch=1):
    """Per-token chain of 7*layers batch-1 GEMVs over a random-init
    Qwen2.5-1.5B-shaped weight set (build_chain), graph-captured and
    replayed; the same chain with bf16 F.linear and, at batch 1, with the
    library's dense bf16_gemv.  Returns the total weight-pass latency of
    each.

    grouped: q, k, v and gate, up of a layer each run as one grouped launch
    (gemv_group, tiled with pick_group_tiling); the bf16 chain then runs q, k,
    v as one F.linear over the concatenated weights (faster than three),
    gate and up separately (the concatenated shape is slower in rocBLAS).
    batch: rows of x per GEMV (the same weights serve every row)."""
    ch = build_chain(bits, layers, seed, grouped, batch)
    mats, names = ch["mats"], ch["names"]
    # one output buffer per projection name, reused by every layer
    ybuf = {}
    for m, n in zip(mats, names):
        ybuf.setdefault(n, torch.empty(batch, m.rows, device="cuda"))
    ys = [ybuf[n] for n in names]
    Ws = ch["Ws"]
    if grouped:  # q, k, v weights of a layer concatenated for the bf16 chain
        Wl = []
        for launch in ch["launches"]:
            ws = [Ws[i] for i in launch]
            if CHAIN_GROUPS.get(names[launch[0]]) == "qkv":
                Wl.append(torch.cat(ws, 0).contiguous())
            else:
                Wl.extend(ws)
        Ws = Wl
    xs = ch["xs"]

    def run_bf16():
        for W in Ws:
            torch.nn.functional.linear(xs[W.shape[1]], W)

    t_rans = timeit_graph(lambda: run_chain(ch, ys), iters, warmup=2)
    t_bf16 = timeit_graph(run_bf16, iters, warmup=2)
    # the same bf16 weights through the library's dense bf16_gemv (batch 1)
    t_bf16_hip = None
    if batch == 1:
        mbs = [rans.Bf16Matrix(W, mats[0].lib) for W in Ws]
        yh = {}
        for mb in mbs:
            yh.setdefault(mb.rows, torch.empty(mb.rows, device="cuda"))

        def run_bf16_hip():
            for mb in mbs:
                mb.gemv(xs[mb.cols][0], yh[mb.rows])

        t_bf16_hip = timeit_graph(run_bf16_hip, iters, warmup=2)
        del mbs
    nweights, nbytes = ch["nweights"], ch["nbytes"]
    return dict(config=f"Qwen2.5-1.5B-shaped weight set, {layers} layers x 7 matrices, "
                f"batch {batch}" + (", q/k/v and gate/up grouped" if grouped else ""),
                gemvs=len(mats), launches=len(ch["launches"]), weights=nweights,
                bits_target=bits, bits_total=8 * nbytes / nweights, compressed_MB=nbytes / 1e6,
                bf16_MB=nweights * 2 / 1e6, t_rans_us=t_rans, t_bf16_us=t_bf16,
                t_bf16_hip_us=t_bf16_hip,
                effective_GBps=nweights * 2 / t_rans / 1e3, speedup_vs_bf16=t_bf16 / t_rans)


def configs():
    """The benchmark configurations beyond the headline shape: MLP shapes at
    2.25 bits with 0.1% escapes, q_proj at 4.25 bits, the headline shape at
    batch 8 (one launch of the batch-8 kernel), the 27B-class shapes
    with Student-t codes and 1% escapes at batch 1 and 4, and the per-token
    196-GEMV chain with separate and with grouped launches.  Prints one JSON
    line per result."""
    lib = rans.build()
    cases = [
        ("q_proj 4.25b gauss", 1536, 1536, 4.25, "gauss", 0.0, 1),
        ("1536x8960 3.25b laplace B8 (one batch-8 launch)", 1536, 8960, 3.25, "laplace", 0.0, 8),
        ("gate/up 2.25b esc0.1%", 8960, 1536, 2.25, "laplace", 0.001, 1),
        ("down 2.25b esc0.1%", 1536, 8960, 2.25, "laplace", 0.001, 1),
        ("27B 25600x5120 t3 2.25b esc1%", 25600, 5120, 2.25, "student3", 0.01, (1, 4)),
        ("27B 5120x25600 t3 2.25b esc1%", 5120, 25600, 2.25, "student3", 0.01, (1, 4)),
    ]
    for name, rows, cols, bits, dist, esc, batch in cases:
        rs = config_matrix(rows, cols, bits, dist, esc, batch, seed=rows + cols, lib=lib)
        for r in (rs if isinstance(rs, list) else [rs]):
            r["case"] = name if not isinstance(rs, list) else f"{name} B{r['batch']}"
            print(json.dumps({k: (round(v, 4) if isinstance(v, float) else v)
                              for k, v in r.items()}), flush=True)
    # ECSQ-GPTQ + waterfilling code statistics (the k projection's codes of a
    # synthetic layer, tiled to the q/k/v group's shape) with their own steps
    codes, step = ecsq_fixture(rows=2048)
    r = config_matrix(2048, 1536, 3.25, "ecsq_wf", 0.0, 1, seed=0, lib=lib, codes=codes,
                      step=step)
    r["case"] = "q/k/v 2048x1536 ECSQ-GPTQ+WF codes 3.25b (k slice x8)"
    print(json.dumps({k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}),
          flush=True)
    for grouped in (False, True):
        r = chain(grouped=grouped)
        print(json.dumps({k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}),
              flush=True)


def comparators(rows=1536, cols=8960, iters=100, rotate_bytes=512 << 20):
    """The uncompressed and fixed-rate comparators alone on one shape,
    rotated over >= rotate_bytes of copies: the library's dense bf16_gemv
    (random bf16 weights) and the int4 GEMV (random nibbles; its time
    includes the host fold x*step, as Int4Matrix.gemv does).  Prints one
    JSON line: rans_bench.py comparators [ROWS COLS]."""
    lib = rans.build()
    g = torch.Generator(device="cuda").manual_seed(rows + cols)
    W = torch.randn(rows, cols, device="cuda", generator=g).bfloat16()
    nW = copies_for(iters, rows * cols * 2, rotate_bytes)
    mbs = [rans.Bf16Matrix(W, lib)] + [rans.Bf16Matrix(W.clone(), lib) for _ in range(nW - 1)]
    xb = torch.randn(cols, device="cuda", generator=g).bfloat16()
    yb = torch.empty(rows, device="cuda")
    t_bf16 = timeit_graph([lambda mb=mb: mb.gemv(xb, yb) for mb in mbs], iters)
    del mbs, W
    codes = np.random.default_rng(rows + cols).integers(-8, 8, size=(rows, cols), dtype=np.int32)
    step = torch.rand(cols) + 0.5
    m4 = rans.Int4Matrix(codes, step, lib)
    n4 = copies_for(iters, rows * cols // 2, rotate_bytes)
    m4s = [m4] + [m4.clone() for _ in range(n4 - 1)]
    x = torch.randn(cols, device="cuda")
    y4 = torch.empty(rows, device="cuda")
    t_int4 = timeit_graph([lambda mm=mm: mm.gemv(x, y4) for mm in m4s], iters)
    del m4s, m4
    torch.cuda.empty_cache()
    r = dict(rows=rows, cols=cols, t_bf16_hip_us=t_bf16, bf16_GBps=rows * cols * 2 / t_bf16 / 1e3,
             bf16_copies=nW, t_int4_us=t_int4, int4_GBps=rows * cols / 2 / t_int4 / 1e3,
             int4_copies=n4)
    print(json.dumps({k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}),
          flush=True)
    return r


def profile(rows=25600, cols=5120, bits=2.25, dist="student3", escape_frac=0.01, R=0, C=0,
            launches=20, fetch="refill"):
    """One encoded matrix launched `launches` times at batch 1, then at
    batch 4 (bf16 x), for a profiler run: rans_bench.py profile [ROWS COLS
    BITS DIST ESC R C LAUNCHES FETCH].  The defaults are the 27B-class
    25600x5120 matrix of the configurations; R = C = 0 takes the library's
    tiling (pick_tiling at these bits)."""
    lib = rans.build()
    if not R or not C:
        R, C = pick_tiling(rows, cols, bits=bits)
    codes = synth_codes_full(rows, cols, bits, dist=dist, seed=rows + cols, escape_frac=escape_frac)
    step = torch.from_numpy(lognormal_steps(cols, seed=rows + cols))
    flags = {"always": rans.F_WORDS_ALWAYS, "refill": rans.F_WORDS_REFILL}[fetch]
    m = rans.RansMatrix(encode(codes, R, C, 1), step, lib, flags=flags)
    for batch in (1, 4):
        x = torch.randn(batch, cols, device="cuda").bfloat16()
        y = torch.empty(batch, rows, device="cuda")
        for _ in range(launches):
            m.gemv(x, y)
        torch.cuda.synchronize()
        print(f"profile {rows}x{cols} R={R} C={C} batch {batch}: {launches} launches", flush=True)


if __name__ == "__main__":
    if sys.argv[1] == "comparators":
        comparators(*(int(v) for v in sys.argv[2:4]))
    elif sys.argv[1] == "profile":
        types = (int, int, float, str, float, int, int, int, str)
        profile(*(t(v) for t, v in zip(types, sys.argv[2:])))
    elif sys.argv[1] == "chain":  # chain [grouped|separate|both] [layers] [batch]
        mode = sys.argv[2] if len(sys.argv) > 2 else "both"
        layers = int(sys.argv[3]) if len(sys.argv) > 3 else 28
        batch = int(sys.argv[4]) if len(sys.argv) > 4 else 1
        for grouped in {"grouped": (True,), "separate": (False,)}.get(mode, (False, True)):
            r = chain(layers=layers, grouped=grouped, batch=batch)
            print(json.dumps({k: (round(v, 4) if isinstance(v, float) else v)
                              for k, v in r.items()}), flush=True)
    elif sys.argv[1] == "bench" and sys.argv[2:] == ["reference"]:
        bench_reference_layout()
    else:
        {"test": test, "bench": bench, "configs": configs}[sys.argv[1]]()
