"""Benchmark of the fused rANS-decode + batch-1 GEMV on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1]

Workload: one down_proj-shaped (1536 x 8960) matrix of ECSQ-like integer
codes, round(w/step) with w ~ Laplace(0,1) from default_rng(1536+8960) and
one step chosen so the full tensor's empirical entropy is 3.25 bits, stored
in the w64 rANS format; log-normal (sigma 0.5) per-column waterfilling steps;
x ~ N(0,1) in bf16; batch 1.  A step is one GEMV y = codes @ (x*step).

Timing: W warm-up launches, at least 10 ms of untimed replays (the clocks
ramp up after the host-side encoding), then K launches captured in one HIP graph (so
Python dispatch cost is not measured) and replayed between two HIP events on
the launch stream, created with hipEventDisableSystemFence (the default
events' system-scope cache writeback and invalidate would add ~10 us to the
timed region).  Launches rotate over distinct encoded copies so that every
timed launch reads a copy that >= 512 MiB of other copies have passed through
the caches since its last read: the 256 MB Infinity Cache and the L2 cannot
serve the compressed stream, whatever K is (with K below the copies 512 MiB
take, an untimed replay over the other copies runs just before the timed
one).  A hot-cache figure (one copy) is reported separately, as is torch's
bf16 F.linear (rocBLAS/hipBLASLt) on the same shape and rotation.

Prints one JSON line.  `value` is the bf16-equivalent effective weight
throughput rows*cols*2 bytes / time per GEMV.
"""
import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "vram-compression_amd"))
import rans  # noqa: E402
import rans_bench as B  # noqa: E402

METRIC = "effective weight GB/s (bf16-equiv) + µs/GEMV at 1536x8960, 3.25 b/w"
ROWS, COLS, BITS = 1536, 8960, 3.25
HBM_PEAK_GBS = 8000.0
ROTATE_BYTES = 512 << 20

# Tiling of the headline configuration (tile rows, tile columns, states per
# lane): the fastest of the --sweep tilings that store at most 3.60 bits per
# weight (163,840 states: 3.589 bits, 10.00 us against 10.35 us for 3x2240 at
# 3.527 on one box); see pick_tiling for the trade-off between parallelism
# and per-state overhead.
DEFAULT_TILING = (3, 1792, 1)

# HBM traffic per launch of the headline kernel, from two rocprofv3 --pmc
# passes (FETCH_SIZE, then WRITE_SIZE) over 50 rotated launches.  Each counter
# is scaled by what it reads for an elementwise kernel that reads and writes
# 256 MiB: reads x2.0, writes x1.0.  Commands and counts:
# profiles/rans_w64_gemv_1536x8960_3.25b.md.  Keyed by (R, C, S, word fetch)
# and by the hash of the library sources they were measured on
# (library_source_hash): with other sources the line reports traffic null.
PMC_TRAFFIC_KIB = {(3, 1792, 1, "refill"): dict(source_hash="921d6e673b83", commit="e180c16",
                                                fetch_kib=3443.6, write_kib=12.0)}
PMC_FETCH_FACTOR, PMC_WRITE_FACTOR = 2.0, 1.0


library_source_hash = B.library_source_hash


def pmc_traffic(R, C, S, word_fetch, src_hash):
    """(HBM bytes per launch, note) of the headline kernel for this tiling
    and word fetch from the rocprofv3 counters, or (None, why) when no
    counter figure exists or it was measured on other library sources."""
    pmc = PMC_TRAFFIC_KIB.get((R, C, S, word_fetch))
    if pmc is None:
        return None, "no counter figure for this tiling"
    if pmc["source_hash"] != src_hash:
        return None, (f"the counter figure was measured on library sources {pmc['source_hash']}, "
                      f"these are {src_hash}")
    t = int((pmc["fetch_kib"] * PMC_FETCH_FACTOR + pmc["write_kib"] * PMC_WRITE_FACTOR) * 1024)
    return t, ("rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE per dispatch, scaled x2.0 / x1.0, "
               f"measured on library sources {src_hash} at commit {pmc['commit']} "
               "(profiles/rans_w64_gemv_1536x8960_3.25b.md)")


def algorithmic_bytes(enc, rows, cols, batch=1):
    """Bytes one GEMV must move: the whole compressed matrix as the device
    holds it (payload and padding words with each tile's bit-packed initial
    states, tile offsets and metadata, per-state length and exponent bytes,
    the 32 KB LDS image of the table, the escape side table), x (bf16), the
    step vector (f32) and y (f32)."""
    comp = (enc["words"].nbytes + enc["tile_off"].nbytes + enc["slen"].nbytes +
            enc["tile_meta"].nbytes + 2 * enc["table"].nbytes + enc["esc_tileptr"].nbytes +
            enc["esc_pos"].nbytes + enc["esc_val"].nbytes)
    return comp, comp + cols * 2 * batch + cols * 4 + rows * 4 * batch


def copies_for(steps, nbytes):
    """Copies of an nbytes operand for `steps` rotated launches
    (rans_bench.copies_for with the 512 MiB rotation)."""
    return B.copies_for(steps, nbytes, ROTATE_BYTES)


def graph_time_us(fns, steps, warmup, rotate=None):
    """Device microseconds per call of exactly `steps` calls captured in one
    HIP graph and replayed between two HIP events on the launch stream
    (rans_bench.device_elapsed_us: events without the system-scope fence).

    rotate (the number of copies the calls in fns rotate over, len(fns)):
    when steps is smaller than that, the timed graph runs calls 0..steps-1
    and a second, untimed graph runs all the others just before the timed
    replay; otherwise the timed calls cycle through all copies, after an
    untimed pass over every copy in order.  Either way every timed call
    reads a copy that at least 512 MiB of other copies have displaced from
    the 256 MB Infinity Cache and the L2 since its last read."""
    n = len(fns)
    for i in range(warmup):
        fns[i % n]()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fns[0]()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            fns[i % n]()
    # Untimed lead-in replayed just before the timed graph: when rotating,
    # the copies the timed launches do not use (steps < n) or every copy
    # once in order (steps >= n), so each timed launch reads a copy that at
    # least 512 MiB of other copies followed; else the timed graph itself.
    lead = None
    if rotate:
        lead = torch.cuda.CUDAGraph()
        with torch.cuda.graph(lead):
            for f in (fns[steps:] if steps < n else fns):
                f()
    g.replay()  # untimed: first replay uploads the graph
    if lead is not None:
        lead.replay()
    torch.cuda.synchronize()
    # At least 10 ms of untimed replays of the lead-in (or of the timed graph)
    # queued back to back bring the clocks to their loaded state, and the
    # timed replay is queued while the device still runs the last of them, so
    # the start event fires when that work ends and not while the host is
    # still submitting the timed graph: the events time the device's `steps`
    # launches (rans_bench.warm_then_time).  With the device idle at the start
    # event, 20 launches of the 1536x8960 GEMV read 0.5-0.9 us per launch
    # above their kernel time.
    return B.warm_then_time(g, lead) / steps


def rotation_record(steps, ncopy, nbytes):
    """What a rotated measurement read: copies, bytes, and the least data
    read between two reads of one copy."""
    cycle = ncopy if steps >= ncopy else ncopy - steps
    return {"copies": ncopy, "bytes": ncopy * nbytes, "timed_launches": steps,
            "copies_read_in_timed_region": min(steps, ncopy),
            "bytes_between_reads_of_a_copy": cycle * nbytes}


def cpu_baseline(codes, step, x, budget_s=12.0):
    """The oracle's scalar restatement of the reference decoder
    (kernel/rans.py:101-123, one core: a pure-Python loop) on a bounded
    sample of lanes of the reference 32-lane encoding (R=8, C=8960, the
    published tiling for this shape), extrapolated to the whole matrix, plus
    the numpy dense GEMV timed on the full matrix."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    from threadpoolctl import threadpool_info
    enc = oracle.encode_ref(np.clip(codes, -128, 127), 8, COLS)
    n = (COLS // 32) * 8
    t0 = time.perf_counter()
    oracle.decode_ref_py(enc, max_lanes=16)
    per_lane = (time.perf_counter() - t0) / 16
    lanes = int(max(16, min(len(enc["offs"]), budget_s / max(per_lane, 1e-9))))
    t0 = time.perf_counter()
    oracle.decode_ref_py(enc, max_lanes=lanes)
    t_dec = time.perf_counter() - t0
    per_sym = t_dec / (lanes * n)
    t_decode_full = per_sym * codes.size
    W = codes.astype(np.float32)
    xs = x.astype(np.float32) * step
    t0 = time.perf_counter()
    for _ in range(5):
        W @ xs
    t_gemv = (time.perf_counter() - t0) / 5
    t = t_decode_full + t_gemv
    blas = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    return {"value": ROWS * COLS * 2 / t / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": (f"scalar decode of {lanes} of {len(enc['offs'])} lanes ({lanes * n} symbols, "
                       f"{t_dec:.1f} s, {per_sym * 1e9:.0f} ns/symbol) extrapolated to "
                       f"{codes.size} symbols = {t_decode_full:.1f} s, plus numpy dense GEMV "
                       f"{t_gemv * 1e3:.1f} ms on {blas} BLAS threads"),
            "us_per_gemv": t * 1e6, "host_cpus": len(os.sched_getaffinity(0)),
            "numpy": np.__version__,
            "per_config": cpu_per_config(oracle, per_sym, t_gemv / codes.size)}


def _gemv_seconds(rows, cols, reps=3):
    W = np.ones((rows, cols), np.float32)
    xs = np.ones(cols, np.float32)
    t0 = time.perf_counter()
    for _ in range(reps):
        W @ xs
    return (time.perf_counter() - t0) / reps


def cpu_per_config(oracle, metric_s_per_symbol, metric_gemv_s_per_weight, budget_s=2.0):
    """The same CPU path on the other workloads: configurations 1-3 timed
    on a bounded sample of lanes of their reference 32-lane encoding (one
    tile row; codes outside [-128, 127] clipped to the reference alphabet)
    plus the full numpy GEMV; configurations 4-5 extrapolated from measured
    per-symbol and per-weight rates, and labelled so."""
    out = []

    def timed(name, codes, R, C, rows, cols):
        enc = oracle.encode_ref(np.clip(codes, -128, 127), R, C)
        n = (C // 32) * R
        t0 = time.perf_counter()
        oracle.decode_ref_py(enc, max_lanes=2)
        per_lane = (time.perf_counter() - t0) / 2
        lanes = int(max(2, min(len(enc["offs"]), budget_s / max(per_lane, 1e-9))))
        t0 = time.perf_counter()
        oracle.decode_ref_py(enc, max_lanes=lanes)
        per_sym = (time.perf_counter() - t0) / (lanes * n)
        t_gemv = _gemv_seconds(rows, cols)
        t = per_sym * rows * cols + t_gemv
        out.append({"config": name, "kind": "measured sample", "us_per_gemv": t * 1e6,
                    "ns_per_symbol": per_sym * 1e9,
                    "sample": f"{lanes * n} symbols of R={R} C={C} lanes, full numpy GEMV"})
        return per_sym

    c1 = B.synth_codes_full(512, 256, 3.25, seed=512 + 256)
    timed("1: 512x256 Laplace 3.25 b (reference CPU test path, R=512 C=256, 32 lanes)",
          c1, 512, 256, 512, 256)
    c2 = B.synth_codes_full(1536, 1536, 4.25, dist="gauss", seed=3072)
    timed("2: q_proj 1536x1536 N(0,1) 4.25 b", c2[:8], 8, 1536, 1536, 1536)
    c3 = B.synth_codes_full(8960, 1536, 2.25, seed=8960 + 1536, escape_frac=0.001)
    r3 = timed("3: gate/up 8960x1536 Laplace 2.25 b", c3[:8], 8, 1536, 8960, 1536)
    c3d = B.synth_codes_full(1536, 8960, 2.25, seed=8960 + 1536 + 1, escape_frac=0.001)
    timed("3: down 1536x8960 Laplace 2.25 b", c3d[:8], 8, 8960, 1536, 8960)
    n4 = 28 * (2 * 1536 * 1536 + 2 * 256 * 1536 + 3 * 8960 * 1536)
    out.append({"config": "4: 196-GEMV Qwen2.5-1.5B-shaped chain, 3.25 b",
                "kind": "extrapolated", "us_per_gemv": None,
                "us_per_chain": n4 * (metric_s_per_symbol + metric_gemv_s_per_weight) * 1e6,
                "sample": f"{n4} symbols at the metric shape's measured rate"})
    for shape in ((25600, 5120), (5120, 25600)):
        n5 = shape[0] * shape[1]
        out.append({"config": f"5: {shape[0]}x{shape[1]} Student-t 2.25 b, B=1",
                    "kind": "extrapolated",
                    "us_per_gemv": n5 * (r3 + metric_gemv_s_per_weight) * 1e6,
                    "sample": f"{n5} symbols at configuration 3's measured rate"})
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--tiling", type=str, default=None, help="R,C,S")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--word-fetch", choices=("tune", "always", "refill"), default="refill",
                    help="GEMV word-fetch policy: refill (the library's default for tiles of "
                         "3 or more rows), always, or tune (time both on the matrix; a 2x20-launch "
                         "timing that can pick either within noise)")
    ap.add_argument("--no-rocblas", action="store_true")
    ap.add_argument("--no-chain", action="store_true",
                    help="skip the per-token chain (196 GEMVs, grouped launches)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other benchmark configurations (q_proj at 4.25 bits, the MLP "
                         "shapes at 2.25 bits with escapes, the 27B-class shapes at batch 1 and 4)")
    ap.add_argument("--no-ecsq", action="store_true",
                    help="skip the row with ECSQ-GPTQ + waterfilling code statistics")
    ap.add_argument("--no-reflayout", action="store_true",
                    help="skip the reference's own 32-lane layout at its published tiling")
    ap.add_argument("--sweep", action="store_true", help="print a tiling sweep to stderr")
    ap.add_argument("--profile", action="store_true",
                    help="for rocprofv3: W eager warm-up launches, then K eager launches of the "
                         "headline GEMV, each on a copy no earlier launch read (the rotation of a "
                         "timed run with the same --steps), then one 256 MiB elementwise kernel "
                         "as the FETCH/WRITE calibration")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the library has no multi-GPU path "
              "(a matrix would shard by ranges of tile rows, one range per GPU)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)

    lib = rans.build()
    codes = B.synth_codes_full(ROWS, COLS, BITS, seed=ROWS + COLS)
    step = B.lognormal_steps(COLS, seed=ROWS + COLS)
    x = np.random.default_rng(0).standard_normal(COLS).astype(np.float32)
    xb = torch.from_numpy(x).cuda().bfloat16()
    step_t = torch.from_numpy(step)
    print(f"workload ready: entropy {B.entropy_fast(codes):.4f} bits", file=sys.stderr, flush=True)

    def pick_fetch(m):
        if args.word_fetch == "tune":
            return m.tune()
        return rans.F_WORDS_ALWAYS if args.word_fetch == "always" else rans.F_WORDS_REFILL

    def measure(R, C, S, steps):
        enc = rans.encode(codes, R, C, S)
        comp, alg = algorithmic_bytes(enc, ROWS, COLS)
        ncopy = copies_for(steps, comp)
        m0 = rans.RansMatrix(enc, step_t, lib)
        flags = pick_fetch(m0)
        ms = [m0] + [rans.RansMatrix(enc, step_t, lib, flags=flags) for _ in range(ncopy - 1)]
        y = torch.empty(ROWS, device="cuda")
        fns = [lambda m=m: m.gemv(xb, y) for m in ms]
        t_rot = graph_time_us(fns, steps, args.warmup, rotate=ncopy)
        t_hot = graph_time_us(fns[:1], steps, args.warmup)
        del ms, m0
        torch.cuda.empty_cache()
        measure.flags = flags
        return enc, comp, alg, ncopy, t_rot, t_hot

    if args.profile:
        R, C, S = (int(v) for v in args.tiling.split(",")) if args.tiling else DEFAULT_TILING
        enc = rans.encode(codes, R, C, S)
        comp, alg = algorithmic_bytes(enc, ROWS, COLS)
        # the rotation a timed run of the same --steps uses (copies_for):
        # every launch below reads a copy no earlier launch read
        ncopy = copies_for(args.steps, comp)
        m0 = rans.RansMatrix(enc, step_t, lib)
        flags = pick_fetch(m0)
        ms = [m0] + [rans.RansMatrix(enc, step_t, lib, flags=flags) for _ in range(ncopy - 1)]
        y = torch.empty(ROWS, device="cuda")
        # warm-up launches on the copies the profiled ones do not read, then
        # `steps` launches on copies 0..steps-1
        for i in range(args.warmup):
            ms[ncopy - 1 - i % (ncopy - args.steps)].gemv(xb, y)
        for i in range(args.steps):
            ms[i].gemv(xb, y)
        torch.cuda.synchronize()
        # calibration: an elementwise kernel that reads and writes 256 MiB
        src = torch.ones(64 << 20, dtype=torch.int32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        print(json.dumps({"profile": True, "R": R, "C": C, "S": S, "flags": flags,
                          "launches": args.warmup + args.steps, "profiled_launches": args.steps,
                          "library_source_hash": library_source_hash(),
                          "copies": ncopy, "algorithmic_bytes_per_launch": alg,
                          "compressed_bytes": comp, "calibration_copy_bytes": 256 << 20}), flush=True)
        return

    if args.sweep:
        # tilings of the headline shape, plus the reference's published one
        # (R=8, C=8960, mapped by encode to 8x4480 tiles with two states per lane)
        for S in (1, 2):
            for R in (1, 2, 3, 4, 8):
                for C in (640, 1280, 1792, 2240, 4480):
                    if C % (64 * S) or COLS % C or (R * C) // (64 * S) > rans.MAX_STATE_SYMBOLS:
                        continue
                    try:
                        enc, comp, alg, ncopy, t_rot, t_hot = measure(R, C, S, 100)
                    except AssertionError as e:
                        print(f"sweep R={R} C={C} S={S}: {e}", file=sys.stderr)
                        continue
                    bt = 8 * comp / codes.size
                    print(f"sweep R={R:2d} C={C:5d} S={S} states={enc['slen'].size:7d} "
                          f"bits_total={bt:.3f} rot={t_rot:7.2f}us hot={t_hot:7.2f}us "
                          f"eff={ROWS * COLS * 2 / t_rot / 1e3:7.1f}GB/s", file=sys.stderr, flush=True)

    R, C, S = (int(v) for v in args.tiling.split(",")) if args.tiling else DEFAULT_TILING
    enc, comp, alg, ncopy, t_rot, t_hot = measure(R, C, S, args.steps)
    bits_total = 8 * comp / codes.size
    print(f"rans gemv: {t_rot:.2f} us rotated, {t_hot:.2f} us hot", file=sys.stderr, flush=True)

    rocblas = None
    if not args.no_rocblas:
        W = (torch.from_numpy(codes.astype(np.float32)) * step_t).bfloat16()
        nW = copies_for(args.steps, ROWS * COLS * 2)
        Ws = [W.cuda() for _ in range(nW)]
        fns = [lambda Wd=Wd: torch.nn.functional.linear(xb, Wd) for Wd in Ws]
        tb_rot = graph_time_us(fns, args.steps, args.warmup, rotate=nW)
        tb_hot = graph_time_us(fns[:1], args.steps, args.warmup)
        rocblas = {"us_per_gemv": tb_rot, "effective_GBps": ROWS * COLS * 2 / tb_rot / 1e3,
                   "hot_us_per_gemv": tb_hot, "copies": nW,
                   "rotation": rotation_record(args.steps, nW, ROWS * COLS * 2),
                   "speedup_rans_vs_bf16": tb_rot / t_rot}
        # the library's own bf16 GEMV on the same copies: what an uncompressed
        # GEMV reaches near the HBM bound
        mbs = [rans.Bf16Matrix(Wd, lib) for Wd in Ws]
        yb16 = torch.empty(ROWS, device="cuda")
        th_rot = graph_time_us([lambda mb=mb: mb.gemv(xb, yb16) for mb in mbs], args.steps,
                               args.warmup, rotate=nW)
        rocblas["bf16_hip_us_per_gemv"] = th_rot
        rocblas["bf16_hip_GBps"] = ROWS * COLS * 2 / th_rot / 1e3
        rocblas["speedup_rans_vs_bf16_hip"] = th_rot / t_rot
        del Ws, fns, mbs
        # the reference's other comparators (kernel/bench.py:97-111): the
        # fixed-rate int4 GEMV (host fold + int4 kernel) and decode-to-bf16
        # followed by the bf16 GEMV
        n4 = copies_for(args.steps, ROWS * COLS // 2)
        m4 = rans.Int4Matrix(np.clip(codes, -8, 7), step_t, lib)
        m4s = [m4] + [m4.clone() for _ in range(n4 - 1)]
        xf = xb.float()
        y4 = torch.empty(ROWS, device="cuda")
        rocblas["int4_us_per_gemv"] = graph_time_us([lambda m4=m4: m4.gemv(xf, y4) for m4 in m4s],
                                                    args.steps, args.warmup, rotate=n4)
        del m4s, m4
        # decode to bf16, then F.linear (the reference's t_decode_then_cublas),
        # over the rotated compressed copies like every other comparator; the
        # bf16 buffer is the decode's output, rewritten by every call
        ndc = copies_for(args.steps, comp)
        mds = [rans.RansMatrix(enc, step_t, lib) for _ in range(ndc)]
        buf = torch.empty(ROWS, COLS, device="cuda", dtype=torch.bfloat16)
        rocblas["decode_then_bf16_us_per_gemv"] = graph_time_us(
            [lambda md=md: torch.nn.functional.linear(xb, md.decode(buf)) for md in mds],
            args.steps, args.warmup, rotate=ndc)
        rocblas["decode_then_bf16_copies"] = ndc
        del mds, buf
        torch.cuda.empty_cache()
        print(f"bf16 F.linear: {tb_rot:.2f} us rotated, {tb_hot:.2f} us hot; "
              f"bf16 HIP GEMV: {th_rot:.2f} us rotated", file=sys.stderr, flush=True)

    # The same matrix in the reference's own 32-lane layout at its published
    # tiling of this shape (R=8, C=8960: 6144 streams of 2240 symbols,
    # results/kernel_bench.json:128-129), through the reference's entry point
    # launch_rans_gemv with the host fold, rotated the same way.
    reflayout = None
    if not args.no_reflayout:
        renc = rans.encode_reference_layout(codes, 8, COLS)
        rm0 = rans.ReferenceLayoutMatrix(renc, step_t, lib)
        nr = copies_for(args.steps, rm0.nbytes)
        rms = [rm0] + [rans.ReferenceLayoutMatrix(renc, step_t, lib) for _ in range(nr - 1)]
        yr = torch.empty(ROWS, device="cuda")
        rfns = [lambda rm=rm: rm.gemv(xb, yr) for rm in rms]
        tr_rot = graph_time_us(rfns, args.steps, args.warmup, rotate=nr)
        tr_hot = graph_time_us(rfns[:1], args.steps, args.warmup)
        reflayout = {"R": 8, "C": COLS, "streams": int(renc["offs"].size),
                     "bits_total": 8 * rm0.nbytes / codes.size,
                     "us_per_gemv": tr_rot, "hot_us_per_gemv": tr_hot, "copies": nr,
                     "w64_speedup": tr_rot / t_rot,
                     "note": "host fold x*step plus launch_rans_gemv, as the reference's "
                             "RansMatrix.gemv does"}
        del rms, rm0, rfns
        torch.cuda.empty_cache()
        print(f"reference layout R=8 C={COLS}: {tr_rot:.2f} us rotated, {tr_hot:.2f} us hot",
              file=sys.stderr, flush=True)

    cpu = None if args.no_cpu else cpu_baseline(codes, step, torch.from_numpy(x).bfloat16().float().numpy())

    # The per-token chain of a Qwen2.5-1.5B-shaped weight set (28 layers x 7
    # matrices at 3.25 bits, batch 1), each layer's q/k/v and gate/up as one
    # grouped launch, against the bf16 chain with q/k/v concatenated.
    chain = None
    if not args.no_chain:
        r = B.chain(grouped=True)
        chain = {"us_per_token": r["t_rans_us"], "bf16_us_per_token": r["t_bf16_us"],
                 "bf16_hip_us_per_token": r["t_bf16_hip_us"],
                 "speedup_vs_bf16": r["speedup_vs_bf16"], "launches": r["launches"],
                 "gemvs": r["gemvs"], "bits_total": r["bits_total"],
                 "workload": r["config"]}
        torch.cuda.empty_cache()

    # codes with ECSQ-GPTQ + waterfilling statistics (the k projection of a
    # synthetic layer quantised by the reference's method, tiled to the q/k/v
    # group's 2048x1536) with their own per-column steps, batch 1
    ecsq = None
    if not args.no_ecsq:
        codes_e, step_e = B.ecsq_fixture(rows=2048)
        r = B.config_matrix(2048, 1536, 3.25, "ecsq_wf", 0.0, 1, 0, lib, codes=codes_e,
                            step=step_e, iters=args.steps)
        ecsq = {k: r[k] for k in ("rows", "cols", "R", "C", "entropy", "bits_total", "n_escapes",
                                  "t_rans_us", "t_bf16_us", "t_bf16_hip_us", "effective_GBps",
                                  "speedup_vs_bf16", "speedup_vs_bf16_hip", "algorithmic_bytes",
                                  "roofline_frac", "rel_l2_vs_f64", "copies")}
        ecsq["workload"] = ("q/k/v-shaped 2048x1536 ECSQ-GPTQ + waterfilling codes at 3.25 b/w "
                            "(246 levels, escapes up to |196|), own per-column steps, bf16 x, "
                            "batch 1")
        torch.cuda.empty_cache()

    # The other configurations of the benchmark, each timed like the
    # headline (rotated copies, HIP graph), beside F.linear and the library's
    # bf16_gemv on the same shape and rotation: q_proj 1536x1536 at 4.25 bits,
    # the MLP shapes at 2.25 bits with 0.1% escapes, and the 27B-class
    # shapes (Student-t(3) codes at 2.25 bits, 1% escapes, log-normal steps)
    # at batch 1 and 4.  Both 27B shapes use seed 30720, so the 5120x25600
    # codes are the 25600x5120 array reshaped (the generator's flat draw does
    # not depend on the shape): generated once.
    configs = None
    if not args.no_configs:
        configs = []
        keys = ("rows", "cols", "batch", "R", "C", "S", "word_fetch", "entropy", "bits_total",
                "n_escapes", "t_rans_us", "t_bf16_us", "t_bf16_hip_us", "effective_GBps",
                "compressed_GBps", "algorithmic_bytes", "roofline_frac", "speedup_vs_bf16",
                "speedup_vs_bf16_hip", "rel_l2_vs_f64", "copies", "bf16_copies")

        def add(name, records):
            for r in (records if isinstance(records, list) else [records]):
                rec = {"config": name, **{k: r[k] for k in keys}}
                if r["batch"] > 1:
                    rec["note"] = ("bf16_gemv takes one vector per launch: t_bf16_hip_us is "
                                   f"{r['batch']} launches")
                configs.append(rec)
                print(f"config {name} B={r['batch']}: {r['t_rans_us']:.2f} us "
                      f"(F.linear {r['t_bf16_us']:.2f}, bf16_gemv {r['t_bf16_hip_us']:.2f})",
                      file=sys.stderr, flush=True)

        add("2: q_proj 1536x1536 N(0,1) 4.25 b",
            B.config_matrix(1536, 1536, 4.25, "gauss", 0.0, 1, 3072, lib, iters=args.steps))
        add("3: gate/up 8960x1536 Laplace 2.25 b, 0.1% escapes",
            B.config_matrix(8960, 1536, 2.25, "laplace", 0.001, 1, 10496, lib, iters=args.steps))
        add("3: down 1536x8960 Laplace 2.25 b, 0.1% escapes",
            B.config_matrix(1536, 8960, 2.25, "laplace", 0.001, 1, 10496, lib, iters=args.steps))
        big = B.synth_codes_full(25600, 5120, 2.25, dist="student3", seed=30720,
                                 escape_frac=0.01)
        for rows, cols in ((25600, 5120), (5120, 25600)):
            add(f"5: {rows}x{cols} Student-t(3) 2.25 b, 1% escapes",
                B.config_matrix(rows, cols, 2.25, "student3", 0.01, (1, 4), 30720, lib,
                                iters=args.steps, codes=big.reshape(rows, cols),
                                step=B.lognormal_steps(cols, seed=30720)))
        del big
        torch.cuda.empty_cache()

    achieved = alg / (t_rot * 1e-6) / 1e9
    fetch_name = {rans.F_WORDS_ALWAYS: "always", rans.F_WORDS_REFILL: "refill"}.get(measure.flags & 3)
    src_hash = library_source_hash()
    traffic, traffic_note = pmc_traffic(R, C, S, fetch_name, src_hash)
    out = {
        "metric": METRIC,
        "value": ROWS * COLS * 2 / t_rot / 1e3,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": t_rot / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32 decode / f32 accumulate",
        "data": "synthetic",
        "config": {"workload": f"{ROWS}x{COLS} Laplace ECSQ codes at {BITS} bits/weight entropy, "
                               "log-normal per-column steps, bf16 x, batch 1",
                   "rows": ROWS, "cols": COLS, "batch": 1, "R": R, "C": C, "S": S,
                   "states": int(enc["slen"].size), "bits_total": bits_total,
                   "bits_payload": enc["bits_payload"], "rotating_copies": ncopy,
                   "rotation": rotation_record(args.steps, ncopy, comp),
                   "word_fetch": {1: "always", 2: "refill"}.get(measure.flags & 3, "default"),
                   "parallelism": "single GPU"},
        "us_per_gemv": t_rot,
        "hot_us_per_gemv": t_hot,
        "hot_effective_GBps": ROWS * COLS * 2 / t_hot / 1e3,
        "compressed_GBps": comp / t_rot / 1e3,
        "rocblas_bf16": rocblas,
        "reference_layout": reflayout,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "traffic_source": traffic_note,
                     "library_source_hash": src_hash,
                     "kernel": "rans_w64_gemv_kernel", "bytes_per_launch": alg},
        "cpu_baseline": cpu,
        "chain": chain,
        "ecsq_wf": ecsq,
        "configs": configs,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
