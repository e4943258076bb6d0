"""Writes tests/golden/reference_vectors.npz: input/output vectors of the
reference's own encoder, table builder and code generator
(kernel/rans.py:34-98, kernel/bench.py:20-35 of snuri00/vram-compression).

Why an import is needed: the published kernel_bench.json records pin the
number of words the encoder emits and the entropy of synth_codes, but not the
exact word values, the exact table of the rounding fix-up in tie and
negative-residue cases, or the code arrays themselves.  This script imports
the reference's numpy functions (its CUDA parts are never built or run) and
records those outputs as data.  It runs only where the reference checkout is
mounted (REFERENCE env var, default /root/reference); the committed .npz is
what the tests read.

    python tests/golden/make_golden.py

It also copies the fields of the reference's published benchmark records
(results/kernel_bench.json) that the tests check into
tests/golden/kernel_bench_records.json, with the derived payload word count
bits_payload*rows*cols/16 (an exact integer).
"""
import importlib.util
import json
import os
import sys

import numpy as np

REF = os.environ.get("REFERENCE", "/root/reference")
HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "reference_vectors.npz")
RECORDS = os.path.join(HERE, "kernel_bench_records.json")


def _load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def write_records():
    with open(os.path.join(REF, "results", "kernel_bench.json")) as f:
        recs = json.load(f)
    out = []
    for i, r in enumerate(recs):
        n = r["rows"] * r["cols"]
        out.append(dict(source=f"results/kernel_bench.json record {i}", shape=r["shape"],
                        rows=r["rows"], cols=r["cols"], R=r["R"], C=r["C"],
                        target_bits=float(round(r["entropy"])), seed=r["rows"] + r["cols"],
                        entropy=r["entropy"], payload_words=int(round(r["bits_payload"] * n / 16)),
                        bits_payload=r["bits_payload"], bits_overhead=r["bits_overhead"],
                        bits_total=r["bits_total"], t_bf16_us=r["t_bf16_us"],
                        t_rans_us=r["t_rans_us"], t_int4_us=r["t_int4_us"],
                        t_decode_then_cublas_us=r["t_decode_then_cublas_us"]))
    with open(RECORDS, "w") as f:
        json.dump(out, f, indent=1)
    print(f"wrote {RECORDS} ({len(out)} records)")


def main():
    write_records()
    ref_rans = _load("rans", os.path.join(REF, "kernel", "rans.py"))
    ref_bench = _load("ref_bench", os.path.join(REF, "kernel", "bench.py"))
    out = {}

    # encode/decode on the shapes of the reference's own test (bench.py:41-43)
    cases = [(64, 256, 4, 256, 3.0), (128, 512, 8, 128, 2.0), (256, 1024, 16, 512, 4.0),
             (32, 64, 1, 32, 1.0)]
    for i, (rows, cols, R, C, bits) in enumerate(cases):
        codes = ref_bench.synth_codes(rows, cols, bits, seed=rows)
        enc = ref_rans.encode(codes, R, C)
        out[f"enc{i}_meta"] = np.array([rows, cols, R, C], np.int64)
        out[f"enc{i}_bits"] = np.array([bits, enc["bits_payload"], enc["bits_state_offs"],
                                        enc["bits_table"], enc["entropy_model"],
                                        ref_bench.entropy(codes)], np.float64)
        out[f"enc{i}_codes"] = codes.astype(np.int8)
        out[f"enc{i}_words"] = enc["words"]
        out[f"enc{i}_offs"] = enc["offs"]
        out[f"enc{i}_table"] = enc["table"]

    # synth_codes: Gaussian branch and a non-square shape
    g = ref_bench.synth_codes(48, 96, 2.5, dist="gauss", seed=7)
    out["synth_gauss_48x96_2.5_seed7"] = g.astype(np.int8)

    # build_table edge cases (rans.py:36-50)
    rng = np.random.default_rng(123)
    tables = {
        "two_symbols": np.array([3] * 5 + [200] * 7, np.uint8),
        "tie_argmax": np.array([10] * 50 + [20] * 50 + [30] * 3, np.uint8),
        # many rare symbols: max(1, round(.)) pushes the sum above M
        "rare_overflow": np.concatenate([np.full(100000, 128, np.uint8),
                                         np.arange(256, dtype=np.uint8).repeat(3)]),
        # exact halves exercise round-half-even
        "half_even": np.concatenate([np.full(8191, 1, np.uint8), np.full(1, 2, np.uint8),
                                     np.full(8192, 3, np.uint8)]),
        "laplace": (np.clip(np.round(rng.laplace(size=20000) * 3), -127, 127) + 128).astype(np.uint8),
        "uniform256": rng.integers(0, 256, 5000).astype(np.uint8),
    }
    for name, sym in tables.items():
        freq, cum, table = ref_rans.build_table(sym)
        out[f"tab_{name}_sym"] = sym
        out[f"tab_{name}_freq"] = freq.astype(np.int64)
        out[f"tab_{name}_cum"] = np.asarray(cum, np.int64)
        out[f"tab_{name}_table"] = table

    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
