"""Writes ECSQ-GPTQ codes with waterfilling (the reference's ecsq_wf method)
for one random-init Qwen2.5-1.5B-shaped decoder layer, and their statistics
beside the reference's published ones.

    python tests/golden/make_ecsq_golden.py          # writes ecsq_wf_kv.npz, ecsq_wf_stats.json

Run in the build container only (CPU, torch; about a minute).  The
quantiser is the reference's own: exp/quant.py is imported from the
reference checkout ($REFERENCE, default /root/reference) and its
ecsq(W, H, 3.25, waterfill=True) (quant.py:122-156) quantises each group;
the codes and per-column steps of its final GPTQ pass are recorded from its
_ecsq_run (quant.py:117-119).  The layers are synthetic, since the
reference's model and calibration text need network access:

- weights: N(0, 0.02^2) scaled per input column by a log-normal factor, so
  the per-row excess kurtosis matches the published layer 0 of each group
  (results/Qwen2.5-1.5B__stats.json:6-16 and the three records after it,
  "kurtosis": qkv 1.10, o 0.97, gate_up 0.18, down 0.32);
- Hessian: H = X^T X / m over m = 4096 synthetic activation rows, X = a
  Gaussian with log-normal per-channel scales, a rank-32 correlated part and
  four massive channels, sized so diag(H) max/median is layer 0's published
  value per group ("diag_max_over_median": qkv 1609, o 178, gate_up 294,
  down 1758).

Outputs (both committed):
- ecsq_wf_kv.npz: the k projection's rows (1536..1791) of the quantised
  q/k/v group, int16 codes 256 x 1536, and the group's per-column steps
  (float32) = the fixture the tests encode and decode;
- ecsq_wf_stats.json: per group bpw, code entropy, levels, escapes (codes
  outside [-127, 127]) and the largest |code|, beside the published layer 0
  levels and the published range over the 28 layers
  (results/Qwen2.5-1.5B__ecsq_wf_3.25.json)."""
import importlib.util
import json
import math
import os
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF = os.environ.get("REFERENCE", "/root/reference")
REF_RESULTS = os.path.join(REF, "results", "Qwen2.5-1.5B__ecsq_wf_3.25.json")
BITS = 3.25

# group: rows, cols, kurtosis target, diag(H) max/median target
GROUPS = {"qkv": (2048, 1536, 1.10, 1609.0), "o": (1536, 1536, 0.97, 177.5),
          "gate_up": (17920, 1536, 0.18, 294.0), "down": (1536, 8960, 0.32, 1758.4)}


def load_quant():
    """The reference's quantiser module, exp/quant.py, imported from the
    reference checkout (it needs only math and torch)."""
    spec = importlib.util.spec_from_file_location("quant", os.path.join(REF, "exp", "quant.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["quant"] = mod
    spec.loader.exec_module(mod)
    return mod


def ecsq_wf(quant, W, H, target_bits):
    """Runs the reference's quant.ecsq(W, H, target_bits, waterfill=True)
    (exp/quant.py:122-156) and returns its integer codes and per-column
    steps with its info dict.  ecsq returns only the dequantised weights, so
    its module-level GPTQ pass _ecsq_run (exp/quant.py:117-119), which it
    calls last with the final steps, is wrapped to record those steps and
    the codes of that call."""
    seen = {}
    run = quant._ecsq_run

    def record(W_, Hinv, steps):
        Q, C = run(W_, Hinv, steps)
        seen["steps"], seen["codes"] = steps.clone(), C.clone()
        return Q, C

    quant._ecsq_run = record
    try:
        Q, info = quant.ecsq(W, H, target_bits, True)
    finally:
        quant._ecsq_run = run
    C, steps = seen["codes"], seen["steps"]
    # the recorded pass is the one whose output ecsq returned
    assert torch.equal(C.float() * steps, Q)
    return C, steps, info


def synth_layer(rows, cols, kurt, diag_ratio, gen, m=4096, rank=32):
    """Weights and input Hessian of one linear group (see the module
    docstring)."""
    # per-row excess kurtosis of a Gaussian scale mixture over columns with
    # log-normal scales exp(tau*z): 3*(exp(4 tau^2) - 1)
    tau = math.sqrt(math.log(1 + kurt / 3) / 4)
    colscale = torch.exp(tau * torch.randn(cols, generator=gen))
    W = 0.02 * torch.randn(rows, cols, generator=gen) * colscale
    # activations: log-normal channel scales, a correlated low-rank part and
    # four massive channels that set diag(H) max/median
    chs = torch.exp(0.5 * torch.randn(cols, generator=gen))
    X = torch.randn(m, cols, generator=gen) * chs
    X += torch.randn(m, rank, generator=gen) @ (0.3 * torch.randn(rank, cols, generator=gen))
    med = float(torch.median((X * X).mean(0)))
    big = torch.randperm(cols, generator=gen)[:4]
    X[:, big] *= math.sqrt(diag_ratio * med / float((X[:, big] ** 2).mean()))
    H = (X.t() @ X) / m
    return W, H


def main():
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    gen = torch.Generator().manual_seed(1536)
    quant = load_quant()
    ref = json.load(open(REF_RESULTS))["infos"]
    out = {"bits": BITS, "method": "ecsq_wf (exp/quant.py ecsq, imported), synthetic random-init layer", "groups": {}}
    fixture = None
    for g, (rows, cols, kurt, ratio) in GROUPS.items():
        t0 = time.time()
        W, H = synth_layer(rows, cols, kurt, ratio, gen)
        dh = torch.diag(H)
        C, steps, info = ecsq_wf(quant, W, H, BITS)
        c = C.numpy()
        pub = [x for x in ref if x["group"] == g]
        pub0 = [x for x in pub if x["layer"] == 0][0]
        out["groups"][g] = dict(
            rows=rows, cols=cols, **info,
            published_layer0=dict(levels=pub0["levels"], code_entropy=pub0["code_entropy"]),
            escapes=int(np.count_nonzero((c < -127) | (c > 127))),
            max_abs_code=int(np.abs(c).max()),
            diag_h_max_over_median=float(dh.max() / dh.median()),
            published_levels=dict(min=min(x["levels"] for x in pub),
                                  median=float(np.median([x["levels"] for x in pub])),
                                  max=max(x["levels"] for x in pub)),
            published_code_entropy_median=float(np.median([x["code_entropy"] for x in pub])))
        print(g, json.dumps(out["groups"][g]), f"{time.time() - t0:.0f}s", file=sys.stderr,
              flush=True)
        if g == "qkv":  # the k projection's rows of the group
            fixture = dict(codes=c[1536:1792].astype(np.int16), step=steps.numpy().astype(np.float32))
    np.savez_compressed(os.path.join(HERE, "ecsq_wf_kv.npz"), **fixture)
    k = fixture["codes"]
    out["fixture"] = dict(file="ecsq_wf_kv.npz", rows=int(k.shape[0]), cols=int(k.shape[1]),
                          source="rows 1536..1791 (the k projection) of the qkv group",
                          levels=int(np.unique(k).size),
                          escapes=int(np.count_nonzero((k < -127) | (k > 127))),
                          max_abs_code=int(np.abs(k).max()))
    with open(os.path.join(HERE, "ecsq_wf_stats.json"), "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out["fixture"]), file=sys.stderr)


if __name__ == "__main__":
    main()
