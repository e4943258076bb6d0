"""RansLinear host logic (no GPU): the uniform quantiser and the loud
failure without a device."""
import numpy as np
import pytest
import torch


def test_quantize_uniform_hits_entropy(rans):
    import rans_linear as L
    w = torch.from_numpy(np.random.default_rng(0).standard_normal((256, 512)).astype(np.float32))
    for bits in (2.25, 3.25, 4.25):
        codes, step = L.quantize_uniform(w, bits)
        assert codes.shape == (256, 512) and codes.dtype == np.int32
        assert step.shape == (512,) and np.all(step == step[0])
        assert abs(L._entropy(codes) - bits) < 0.02
        # dequantisation error of a uniform quantiser is at most step/2
        assert np.abs(codes * step[0] - w.numpy()).max() <= step[0] / 2 + 1e-6


def test_ranslinear_fails_without_gpu(rans):
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    import rans_linear as L
    codes = np.random.default_rng(1).integers(-5, 6, size=(64, 128)).astype(np.int32)
    with pytest.raises(RuntimeError):
        L.RansLinear.from_codes(codes, np.ones(128, np.float32), tune=False)
