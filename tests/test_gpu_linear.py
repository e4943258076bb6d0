"""RansLinear on the GPU: the nn.Linear drop-in against a dense fp32
reference, and a tiny random-init Qwen2 model with every projection
replaced (fp32 model: attention stays out of bf16 batched products)."""
import copy

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).norm() / b.norm())


def test_ranslinear_matches_dense(rans, lib):
    import rans_linear as L
    print("case RansLinear 512x1536", flush=True)
    g = torch.Generator().manual_seed(0)
    w = torch.randn(512, 1536, generator=g) * 0.02
    b = torch.randn(512, generator=g)
    codes, step = L.quantize_uniform(w, 4.0)
    codes[7, 9] = 400  # an escape
    lin = L.RansLinear.from_codes(codes, step, b, lib)
    assert lin.matrix.fused_rows_limit == 16  # 8-row tiles: the batch-8 kernel
    wd = torch.from_numpy(codes).double() * torch.from_numpy(step).double()
    tol = {torch.float32: 1e-3, torch.bfloat16: 8e-3, torch.float16: 2e-3}
    for shape in [(1536,), (3, 1536), (2, 4, 1536), (12, 1536)]:  # fused GEMV path
        for dt in (torch.float32, torch.bfloat16, torch.float16):
            x = torch.randn(shape, generator=g).to(dt)
            y = lin(x.cuda())
            ref = torch.nn.functional.linear(x.double(), wd) + b.double()
            assert y.dtype == dt and tuple(y.shape) == tuple(ref.shape)
            assert _rel(y, ref) <= tol[dt], (shape, dt, _rel(y, ref))
    # prefill-sized batch: bf16 decode + dense GEMM
    x = torch.randn(32, 1536, generator=g)
    y = lin(x.cuda())
    ref = torch.nn.functional.linear(x.double(), wd) + b.double()
    assert _rel(y, ref) <= 1e-2


def test_tiny_qwen2_with_rans_linears(rans, lib):
    import rans_linear as L
    from transformers import Qwen2Config, Qwen2ForCausalLM
    print("case tiny Qwen2, all projections rANS-coded", flush=True)
    cfg = Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=512,
                      num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                      max_position_embeddings=128)
    torch.manual_seed(0)
    dense = Qwen2ForCausalLM(cfg).eval()
    coded = copy.deepcopy(dense)
    names = L.replace_linears(coded, bits=6.0, lib=lib, tune=False)
    assert len(names) == 2 * 7  # q, k, v, o, gate, up, down per layer; lm_head stays dense
    for layer in coded.model.layers:  # q/k/v and gate/up linked into grouped launches
        att, mlp = layer.self_attn, layer.mlp
        assert att.q_proj.group is att.k_proj.group is att.v_proj.group is not None
        assert mlp.gate_proj.group is mlp.up_proj.group is not None
        assert att.o_proj.group is None and mlp.down_proj.group is None
    # the dense twin gets exactly the dequantised weights code*step (fp32)
    for n in names:
        m = coded.get_submodule(n).matrix
        wq = m.decode_codes().float() * m.step.reshape(1, -1)
        dense.get_submodule(n).weight.data.copy_(wq.cpu())
    dense, coded = dense.cuda(), coded.cuda()
    # an 8-token prompt runs every projection on the fused GEMV (exact code*step)
    ids = torch.randint(0, 512, (1, 8), generator=torch.Generator().manual_seed(1)).cuda()
    with torch.no_grad():
        a = dense(ids).logits
        b = coded(ids).logits
        assert _rel(b, a) <= 1e-3
        # a longer prompt (more rows than any matrix's fused_rows_limit) takes
        # the prefill path (bf16-decoded weights + dense GEMM)
        long_ids = torch.randint(0, 512, (1, 20), generator=torch.Generator().manual_seed(2)).cuda()
        assert _rel(coded(long_ids).logits, dense(long_ids).logits) <= 2e-2
        # one decode step: two grouped launches per layer (q/k/v, gate/up)
        calls = []
        real = rans.gemv_group
        rans.gemv_group = lambda *a, **k: (calls.append(1), real(*a, **k))[1]
        try:
            coded(ids[:, :1])
        finally:
            rans.gemv_group = real
        assert len(calls) == 2 * len(coded.model.layers)
        # greedy token loop with the KV cache: same tokens from both models
        out_d, out_c = dense(ids, use_cache=True), coded(ids, use_cache=True)
        pd, pc = out_d.past_key_values, out_c.past_key_values
        td = tc = ids[:, -1:]
        for _ in range(6):
            td = out_d.logits[:, -1:].argmax(-1)
            tc = out_c.logits[:, -1:].argmax(-1)
            assert torch.equal(td, tc)
            out_d = dense(td, past_key_values=pd, use_cache=True)
            out_c = coded(tc, past_key_values=pc, use_cache=True)
            pd, pc = out_d.past_key_values, out_c.past_key_values
            assert _rel(out_c.logits, out_d.logits) <= 1e-3


def test_linear_group_reuses_one_launch(rans, lib):
    """q, k, v RansLinears linked into a LinearGroup: the three calls with
    one input make one grouped launch, and each output is bitwise that
    module's own GEMV (plus bias).  A second call with the same input, an
    in-place write to it, or another input launch again."""
    import rans_linear as L
    print("case LinearGroup q/k/v 1536+256+256 x 1536", flush=True)
    g = torch.Generator().manual_seed(5)
    R, C = rans.pick_group_tiling([1536, 256, 256], 1536)
    mods = []
    for rows in (1536, 256, 256):
        codes, step = L.quantize_uniform(torch.randn(rows, 1536, generator=g) * 0.02, 3.5)
        mods.append(L.RansLinear.from_codes(codes, step, torch.randn(rows, generator=g), lib,
                                            tiling=(R, C, 1), tune=False))
    group = L.LinearGroup(mods)
    for m in mods:
        m.group = group
    calls = []
    real = rans.gemv_group
    rans.gemv_group = lambda *a, **k: (calls.append(1), real(*a, **k))[1]
    try:
        x = torch.randn(1, 2, 1536, generator=g).bfloat16().cuda()
        ys = [m(x) for m in mods]
        assert len(calls) == 1
        xd = x.reshape(-1, 1536)
        for m, y in zip(mods, ys):
            want = (m.matrix.gemv(xd) + m.bias).to(torch.bfloat16).reshape(1, 2, -1)
            assert torch.equal(y, want)
        mods[1](x)               # k again with the same input: its result was taken
        assert len(calls) == 2
        x.mul_(1.0)              # an in-place write: the kept results are stale
        mods[2](x)
        assert len(calls) == 3
        mods[0](x.clone())       # another tensor
        assert len(calls) == 4
    finally:
        rans.gemv_group = real


def test_linear_group_prefill_one_gemm(rans, lib):
    """Prefill-sized inputs (more than 8 rows) through a LinearGroup: the
    members' weights are decoded into one bf16 matrix and one dense GEMM
    serves all three calls.  Each output is within the prefill bar (1e-2)
    of the float64 product with code*step, and within 5e-3 of the member's
    own decode + GEMM (both round the GEMM's output to bf16, and the two
    GEMM shapes may round an element differently)."""
    import rans_linear as L
    print("case LinearGroup prefill q/k/v 1536+256+256 x 1536, 12 rows", flush=True)
    g = torch.Generator().manual_seed(9)
    R, C = rans.pick_group_tiling([1536, 256, 256], 1536)
    mods = []
    for rows in (1536, 256, 256):
        codes, step = L.quantize_uniform(torch.randn(rows, 1536, generator=g) * 0.02, 3.5)
        mods.append(L.RansLinear.from_codes(codes, step, torch.randn(rows, generator=g), lib,
                                            tiling=(R, C, 1), tune=False))
    group = L.LinearGroup(mods)
    for m in mods:
        m.group = group
    x = torch.randn(12, 1536, generator=g).bfloat16().cuda()
    calls = []
    real = torch.nn.functional.linear
    torch.nn.functional.linear = lambda *a, **k: (calls.append(1), real(*a, **k))[1]
    try:
        ys = [m(x) for m in mods]
    finally:
        torch.nn.functional.linear = real
    assert len(calls) == 1
    for m, y in zip(mods, ys):
        own = torch.nn.functional.linear(x, m.matrix.decode()).float() + m.bias
        wd = m.matrix.decode_codes().double() * m.matrix.step.double().reshape(1, -1)
        ref = x.double() @ wd.t() + m.bias.double()
        assert _rel(y, ref) <= 1e-2
        assert _rel(y.float(), own) <= 5e-3


def test_linears_with_odd_multiple_of_32_inputs(rans, lib):
    """in_features an odd multiple of 32 (96, 1568): RansLinear (GEMV and
    prefill paths) and a grouped pair built by replace_linears match their
    dense twins; the matrices are stored with 32 appended columns."""
    import rans_linear as L
    print("case RansLinear odd-32 in_features", flush=True)
    g = torch.Generator().manual_seed(3)
    for out_f, in_f in ((64, 96), (384, 1568)):
        w = torch.randn(out_f, in_f, generator=g) * 0.02
        codes, step = L.quantize_uniform(w, 4.0)
        lin = L.RansLinear.from_codes(codes, step, None, lib, tune=False)
        assert lin.matrix.stream_cols == in_f + 32
        wd = torch.from_numpy(codes).double() * torch.from_numpy(step).double()
        for shape in [(in_f,), (3, in_f), (20, in_f)]:
            x = torch.randn(shape, generator=g)
            y = lin(x.cuda())
            ref = torch.nn.functional.linear(x.double(), wd)
            assert _rel(y, ref) <= (1e-2 if len(shape) > 1 and shape[0] > 8 else 1e-3), shape

    class Pair(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.gate_proj = torch.nn.Linear(96, 64, bias=False)
            self.up_proj = torch.nn.Linear(96, 64, bias=False)

        def forward(self, x):
            return self.gate_proj(x) * self.up_proj(x)

    torch.manual_seed(4)
    model = Pair()
    # the dense twin holds the same quantised weights (code * step)
    wq = {}
    for n in ("gate_proj", "up_proj"):
        c, st = L.quantize_uniform(getattr(model, n).weight, 4.25)
        wq[n] = torch.from_numpy(c).double() * torch.from_numpy(st).double()
    names = L.replace_linears(model, bits=4.25, lib=lib, tune=False)
    assert sorted(names) == ["gate_proj", "up_proj"]
    assert model.gate_proj.group is not None and model.gate_proj.group is model.up_proj.group
    model.cuda()
    x = torch.randn(2, 96)
    y = model(x.cuda())
    xd = x.double()
    ref = (xd @ wq["gate_proj"].T) * (xd @ wq["up_proj"].T)
    assert _rel(y, ref) <= 2e-3
