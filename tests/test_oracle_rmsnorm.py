"""Pins oracle/rmsnorm.py against the reference tests' torch formulas and closed forms."""

import numpy as np
import pytest
import torch

from oracle import rmsnorm as R
from oracle.numerics import ulp_distance_bf16

TD = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def torch_reference(x, weight, eps, offset, mode):
    """rmsnorm/tests/test_ops.py:10-21 (llama/gemma) and test_rms_norm.py:27-43 (none)."""
    if mode == "gemma":
        y = x.float() * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + eps)
        if weight is not None:
            y = y * (offset + weight.float())
        return y.to(x.dtype)
    if mode == "none":
        variance = x.pow(2).mean(-1, keepdim=True)
        y = x * torch.rsqrt(variance + eps)
        return (weight * y.to(x.dtype)) if weight is not None else y.to(x.dtype)
    y = x.float() * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + eps)
    y = y.to(x.dtype)
    if weight is not None:
        y = (offset + weight.float()) * y.float()
    return y.to(x.dtype)


@pytest.mark.parametrize("mode,offset", [("llama", 0.0), ("gemma", 1.0), ("llama", 0.5)])
@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("affine", [True, False])
def test_forward_vs_reference_formula(mode, offset, dtype, affine):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 1000, generator=g).to(TD[dtype])
    w = (torch.rand(1000, generator=g) + 0.5).to(TD[dtype]) if affine else None
    y, rstd = R.forward(x.float().numpy(), None if w is None else w.float().numpy(), 1e-6,
                        offset, mode, dtype)
    ref = torch_reference(x, w, 1e-6, offset, mode).float().numpy()
    if dtype == "bf16":
        assert ulp_distance_bf16(y, ref).max() <= 1
    else:
        tol = 1e-5 if dtype == "f32" else 2e-3
        np.testing.assert_allclose(y, ref, rtol=tol, atol=tol)
    ref_rstd = torch.rsqrt(x.double().pow(2).mean(-1) + 1e-6).numpy()
    np.testing.assert_allclose(rstd, ref_rstd, rtol=2e-6)


def test_none_mode_matches_input_dtype_formula():
    # "none": Liger's input-dtype math; the torch BaseRMSNorm formula in f16.
    g = torch.Generator().manual_seed(3)
    x = torch.randn(32, 512, generator=g).half()
    w = (torch.rand(512, generator=g) + 0.5).half()
    y, _ = R.forward(x.float().numpy(), w.float().numpy(), 1e-6, 0.0, "none", "f16")
    ref = torch_reference(x.float(), w.float(), 1e-6, 0.0, "none").half().float().numpy()
    np.testing.assert_allclose(y, ref, rtol=4e-3, atol=4e-3)


def test_closed_forms():
    # A constant row c gives x_hat = c / sqrt(c^2 + eps).
    x = np.full((3, 256), 2.0, dtype=np.float32)
    y, rstd = R.forward(x, None, 0.0, mode="gemma", xdtype="f32")
    np.testing.assert_allclose(rstd, 0.5, rtol=1e-7)
    np.testing.assert_allclose(y, 1.0, rtol=1e-7)
    # A zero row gives rstd = 1/sqrt(eps) and y = 0.
    y, rstd = R.forward(np.zeros((1, 8), np.float32), None, 1e-6, mode="gemma", xdtype="f32")
    np.testing.assert_allclose(rstd, 1000.0, rtol=1e-6)
    assert np.all(y == 0)
    # Scale invariance with eps = 0 (powers of two are exact).
    rng = np.random.default_rng(0)
    x = rng.standard_normal((4, 128)).astype(np.float32)
    y1, _ = R.forward(x, None, 0.0, mode="gemma", xdtype="f32")
    y2, _ = R.forward(8 * x, None, 0.0, mode="gemma", xdtype="f32")
    np.testing.assert_allclose(y1, y2, rtol=1e-6)


@pytest.mark.parametrize("mode,offset", [("llama", 0.0), ("gemma", 1.0), ("none", 0.0)])
@pytest.mark.parametrize("affine", [True, False])
def test_backward_vs_torch_autograd(mode, offset, affine):
    g = torch.Generator().manual_seed(1)
    x = torch.randn(16, 300, generator=g, dtype=torch.float64)
    w = torch.rand(300, generator=g, dtype=torch.float64) + 0.5 if affine else None
    dy = torch.randn(16, 300, generator=g, dtype=torch.float64)
    xg = x.clone().requires_grad_()
    wg = w.clone().requires_grad_() if affine else None
    y = xg * torch.rsqrt(xg.pow(2).mean(-1, keepdim=True) + 1e-6)
    if affine:
        y = y * (offset + wg)
    y.backward(dy)
    _, rstd = R.forward(x.float().numpy(), None, 1e-6, mode="gemma", xdtype="f32")
    dx, dw = R.backward(dy.float().numpy(), x.float().numpy(),
                        None if w is None else w.float().numpy(), rstd, offset, mode, "f32")
    np.testing.assert_allclose(dx, xg.grad.numpy(), rtol=1e-4, atol=1e-5)
    if affine:
        np.testing.assert_allclose(dw, wg.grad.numpy(), rtol=1e-4, atol=1e-4)
