"""torch.nn.Linear drop-in whose weight stays rANS-coded in HBM.

The reference names model integration as its next step (README.md:39) and
stops at the kernel.  RansLinear is that step: forward(x) runs the fused
decode+GEMV kernel for decode-sized batches (up to 8 or 16 rows) and, for larger
batches (prefill), decodes the weight to bf16 once and calls the dense GEMM,
which is then the faster path.  Inference only: the weight is not a
parameter.

Projections that read the same activations (a decoder layer's q, k, v, or
its gate and up) can be linked into a LinearGroup: the first member called
computes all members' products in one grouped launch, and the others return
theirs when called with the same input.  replace_linears links them by name.

quantize_uniform is a plain uniform quantiser (one step per tensor, chosen
for a target code entropy) so that ordinary nn.Linear layers can be
converted in tests and demos; the reference's ECSQ-GPTQ quantiser
(exp/quant.py) is outside this repository.
"""
import weakref

import numpy as np
import torch

import rans

# Batches above a matrix's fused_rows_limit decode the weight to bf16 and
# use the dense GEMM.  The fused GEMV runs up to 8 vectors per launch (4
# where tiles are taller than 8 rows, the launch splits over column groups,
# or matrices share a grouped launch), so its time grows with the batch
# while decode+GEMM stays flat: on MI355X the fused path wins up to 16 rows
# with the batch-8 kernel and up to 8 without it (rans.fused_rows_limit).


def _entropy(codes):
    _, counts = np.unique(codes, return_counts=True)
    p = counts / counts.sum()
    return float(-(p * np.log2(p)).sum())


def quantize_uniform(weight, bits, iters=40, sample=1 << 22, seed=0):
    """codes = round(W / delta) with one delta per tensor, bisected on a
    sample of W (all of it when small) so that the codes' empirical entropy
    is `bits`.  Returns (int32 codes, f32 step vector of one value per
    input column)."""
    w = torch.as_tensor(weight).detach().float().cpu().numpy()
    flat = w.ravel()
    if flat.size > sample:
        flat = np.random.default_rng(seed).choice(flat, sample, replace=False)
    scale = float(np.abs(flat).max()) or 1.0
    lo, hi = np.log(scale) - 20.0, np.log(scale) + 1.0
    for _ in range(iters):
        mid = (lo + hi) / 2
        h = _entropy(np.round(flat / np.exp(mid)).astype(np.int64))
        lo, hi = (mid, hi) if h > bits else (lo, mid)
    delta = float(np.exp((lo + hi) / 2))
    codes = np.round(w / delta).astype(np.int32)
    return codes, np.full(w.shape[1], delta, np.float32)


class LinearGroup:
    """RansLinear modules that read the same input: a decoder layer's q, k
    and v projections, or its gate and up.  When a member is called, every
    member's product is computed at once: for decode-sized inputs in one
    grouped launch (rans.gemv_group), for larger ones by decoding all
    members into one bf16 weight and one dense GEMM.  The other members'
    results are kept and returned when those members are called with the
    same input tensor, unmodified, so Hugging Face's q_proj(h), k_proj(h),
    v_proj(h) costs one launch (or one GEMM).  A member called with any
    other input computes afresh.  The members need the same tiling
    (rans.pick_group_tiling) for the grouped launch."""

    def __init__(self, members):
        self.members = list(members)
        self._x = None        # weak reference to the input of the last launch
        self._version = None  # its version counter then (in-place writes bump it)
        self._pending = {}    # member index -> its product, not yet returned

    def product(self, member, x, xd):
        """member's x @ W^T (no bias) for the module input x, flattened and
        converted to xd (rows x in_features, f32 or bf16); f32."""
        i = next(j for j, m in enumerate(self.members) if m is member)
        if (self._x is not None and self._x() is x and self._version == x._version
                and i in self._pending):
            return self._pending.pop(i)
        m0 = self.members[0].matrix
        if xd.shape[0] > rans.fused_rows_limit(m0._desc, m0.lib, grouped=True):
            # all members decoded into row slices of one bf16 weight, one GEMM
            w = torch.empty(sum(m.out_features for m in self.members), xd.shape[1],
                            device="cuda", dtype=torch.bfloat16)
            ys, off = [], 0
            for m in self.members:
                m.matrix.decode(w[off:off + m.out_features])
                off += m.out_features
            yall = torch.nn.functional.linear(xd.to(torch.bfloat16), w).float()
            off = 0
            for m in self.members:
                ys.append(yall[:, off:off + m.out_features])
                off += m.out_features
        else:
            ys = rans.gemv_group([m.matrix for m in self.members], xd)
        self._x, self._version = weakref.ref(x), x._version
        self._pending = {j: y for j, y in enumerate(ys) if j != i}
        return ys[i]


class RansLinear(torch.nn.Module):
    """y = x @ W^T + b with W = code * step held as a rans.RansMatrix."""

    def __init__(self, matrix, bias=None):
        super().__init__()
        self.matrix = matrix
        self.group = None  # a LinearGroup this module belongs to, if any
        self.in_features = matrix.cols
        self.out_features = matrix.rows
        if bias is not None:
            b = torch.as_tensor(bias).detach().float().reshape(self.out_features)
            self.register_buffer("bias", b.to("cuda"))
        else:
            self.bias = None

    @classmethod
    def from_codes(cls, codes, step, bias=None, lib=None, tiling=None, tune=True):
        """codes (out x in ints), step (in,) f32.  tiling: (R, C, S) or None
        for rans.pick_tiling; tune: pick the word-fetch policy by timing."""
        codes = np.ascontiguousarray(codes, dtype=np.int32)
        rows, cols = codes.shape
        if tiling is None:
            R, C = rans.pick_tiling(rows, cols)
            S = 1
        else:
            R, C, S = tiling
        lib = lib or rans.build()
        m = rans.RansMatrix(rans.encode(codes, R, C, S), torch.as_tensor(step), lib)
        if tune:
            m.tune()
        return cls(m, bias)

    @classmethod
    def from_linear(cls, linear, bits=3.25, lib=None, tiling=None, tune=True):
        """Quantise an nn.Linear with quantize_uniform and encode it."""
        codes, step = quantize_uniform(linear.weight, bits)
        bias = None if linear.bias is None else linear.bias.detach()
        return cls.from_codes(codes, step, bias, lib, tiling, tune)

    def forward(self, x):
        if x.shape[-1] != self.in_features:
            raise ValueError(f"expected last dim {self.in_features}, got {x.shape[-1]}")
        lead = x.shape[:-1]
        xd = x.reshape(-1, self.in_features)
        if xd.dtype not in (torch.bfloat16, torch.float32):
            xd = xd.float()
        if self.group is not None:
            y = self.group.product(self, x, xd.contiguous())
        elif xd.shape[0] > self.matrix.fused_rows_limit:
            w = self.matrix.decode()  # bf16 code*step, then the dense GEMM
            y = torch.nn.functional.linear(xd.to(torch.bfloat16), w).float()
        else:
            y = self.matrix.gemv(xd.contiguous())
        if self.bias is not None:
            y = y + self.bias
        out_dtype = x.dtype if x.dtype in (torch.bfloat16, torch.float16, torch.float32) \
            else torch.float32
        return y.to(out_dtype).reshape(*lead, self.out_features)

    def extra_repr(self):
        m = self.matrix
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, tiles={m.R}x{m.C}x{m.S}, "
                f"bits_per_weight={8 * m.nbytes / (m.rows * m.cols):.3f}, "
                f"grouped={self.group is not None}")


# sibling projections that read the same activations (Hugging Face names)
GROUPS = (("q_proj", "k_proj", "v_proj"), ("gate_proj", "up_proj"))


def replace_linears(module, bits=3.25, lib=None, skip=("lm_head",), tune=True, groups=GROUPS):
    """Swap every nn.Linear of `module` (except names containing an entry of
    `skip`) for a RansLinear quantised at `bits`.  Returns the names swapped.
    Layers whose in_features is not a multiple of 32 (the reference's
    column granularity) are left dense.  Siblings named in one entry of `groups` (same parent,
    same in_features) are encoded with one tiling and linked into a
    LinearGroup; groups=() links none."""
    lib = lib or rans.build()
    done = []
    for name, child in list(module.named_modules()):
        children = dict(child.named_children())

        def eligible(cname):
            sub = children.get(cname)
            full = f"{name}.{cname}" if name else cname
            return (isinstance(sub, torch.nn.Linear) and not any(s in full for s in skip)
                    and sub.in_features % 32 == 0)

        tilings, links = {}, []
        for names_ in groups or ():
            if not all(eligible(n) for n in names_):
                continue
            subs = [children[n] for n in names_]
            if len({s.in_features for s in subs}) != 1:
                continue
            try:
                R, C = rans.pick_group_tiling([s.out_features for s in subs], subs[0].in_features)
            except AssertionError:  # no compiled tile height divides every member
                continue
            for n in names_:
                tilings[n] = (R, C, 1)
            links.append(names_)
        for cname in list(children):
            if not eligible(cname):
                continue
            full = f"{name}.{cname}" if name else cname
            new = RansLinear.from_linear(children[cname], bits, lib, tiling=tilings.get(cname),
                                         tune=tune)
            setattr(child, cname, new)
            done.append(full)
        for names_ in links:
            group = LinearGroup([getattr(child, n) for n in names_])
            for m in group.members:
                m.group = group
    return done
