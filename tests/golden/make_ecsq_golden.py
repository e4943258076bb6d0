"""Writes ECSQ-GPTQ codes with waterfilling (the reference's ecsq_wf method)
for one random-init Qwen2.5-1.5B-shaped decoder layer, and their statistics
beside the reference's published ones.

    python tests/golden/make_ecsq_golden.py          # writes ecsq_wf_kv.npz, ecsq_wf_stats.json

Run in the build container only (CPU, torch; about a minute).  The
quantiser is restated from the documented steps of exp/quant.py (it is not
imported): hinv_chol (quant.py:28-45), gptq (quant.py:48-72) and ecsq with
waterfilling (quant.py:116-156).  Its inputs are synthetic, since the
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
import json
import math
import os
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF_RESULTS = "/root/reference/results/Qwen2.5-1.5B__ecsq_wf_3.25.json"
GROUP = 128
BITS = 3.25

# group: rows, cols, kurtosis target, diag(H) max/median target
GROUPS = {"qkv": (2048, 1536, 1.10, 1609.0), "o": (1536, 1536, 0.97, 177.5),
          "gate_up": (17920, 1536, 0.18, 294.0), "down": (1536, 8960, 0.32, 1758.4)}


def entropy_bits(codes):
    """Zero-order entropy of the integer codes (quant.py:22-25), by counts."""
    c = codes.reshape(-1).long()
    counts = torch.bincount(c - c.min())
    p = counts[counts > 0].double() / c.numel()
    return float(-(p * p.log2()).sum())


def hinv_chol(H, percdamp=0.01):
    """Upper Cholesky factor of (H + damp*I)^-1 in float64 (quant.py:28-45):
    dead channels get a unit diagonal, damp = percdamp * mean diag, raised
    again while the factorisation fails."""
    H = H.double().clone()
    dead = torch.diag(H) == 0
    H[dead, dead] = 1
    damp = percdamp * torch.diag(H).mean()
    H.diagonal().add_(damp)
    while True:
        L, info = torch.linalg.cholesky_ex(H)
        if info == 0:
            break
        H.diagonal().add_(damp)
    Hinv = torch.cholesky_inverse(L)
    U = torch.linalg.cholesky(Hinv, upper=True)
    return U.float(), dead


def gptq(W, Hinv, steps, blocksize=GROUP):
    """GPTQ / LDLQ with error feedback (quant.py:48-72) for the ECSQ column
    quantiser of quant.py:117-119: code = round(w / step_i), value = code *
    step_i.  Within a block each column's error, scaled by the inverse
    factor's diagonal, is pushed onto the block's later columns; at the end
    of a block its errors are pushed onto all later columns."""
    W = W.clone()
    n = W.shape[1]
    C = torch.zeros(W.shape, dtype=torch.int32)
    for i1 in range(0, n, blocksize):
        i2 = min(i1 + blocksize, n)
        W1 = W[:, i1:i2].clone()
        E1 = torch.zeros_like(W1)
        Hi = Hinv[i1:i2, i1:i2]
        for i in range(i2 - i1):
            w = W1[:, i]
            c = torch.round(w / steps[i1 + i])
            q = c * steps[i1 + i]
            C[:, i1 + i] = c.int()
            err = (w - q) / Hi[i, i]
            W1[:, i:] -= err.unsqueeze(1) @ Hi[i, i:].unsqueeze(0)
            E1[:, i] = err
        W[:, i2:] -= E1 @ Hinv[i1:i2, i2:]
    return C


def ecsq_wf(W, H, target_bits):
    """ECSQ with waterfilling (quant.py:122-156): per-column steps c * d_i with
    d = diag of the upper Cholesky factor of H^-1 over its mean; 16 bits of
    side information per column; c from 40 bisection steps on the
    round-to-nearest entropy, then two secant corrections on the GPTQ codes
    (dH/dlog2 c ~ -1), then the final GPTQ pass.  Returns codes, steps, info."""
    Hinv, dead = hinv_chol(H)
    W = W.clone()
    W[:, dead] = 0
    d = torch.diag(Hinv)
    base = d / d.mean()
    side = 16 * W.shape[1] / W.numel()
    target = target_bits - side

    def rtn_H(logc):
        return entropy_bits(torch.round(W / (math.exp(logc) * base)))

    lo, hi = math.log(W.std().item()) - 12, math.log(W.std().item()) + 4
    for _ in range(40):
        mid = (lo + hi) / 2
        if rtn_H(mid) > target:
            lo = mid
        else:
            hi = mid
    logc = (lo + hi) / 2
    for _ in range(2):
        C = gptq(W, Hinv, math.exp(logc) * base)
        logc += (entropy_bits(C) - target) * math.log(2)
    steps = math.exp(logc) * base
    C = gptq(W, Hinv, steps)
    h = entropy_bits(C)
    return C, steps, dict(bpw=h + side, code_entropy=h, levels=int(torch.unique(C).numel()))


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
    ref = json.load(open(REF_RESULTS))["infos"]
    out = {"bits": BITS, "method": "ecsq_wf (restated), synthetic random-init layer", "groups": {}}
    fixture = None
    for g, (rows, cols, kurt, ratio) in GROUPS.items():
        t0 = time.time()
        W, H = synth_layer(rows, cols, kurt, ratio, gen)
        dh = torch.diag(H)
        C, steps, info = ecsq_wf(W, H, BITS)
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
