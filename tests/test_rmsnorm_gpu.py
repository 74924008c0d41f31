"""GPU parity of the RMSNorm kernels against oracle/rmsnorm.py, following
rmsnorm/tests/test_ops.py and test_rms_norm.py."""

import numpy as np
import pytest
import torch

from oracle import rmsnorm as R
from oracle.numerics import ulp_distance_bf16, ulp_distance_f16

pytestmark = pytest.mark.gpu

DT = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def ulps(actual, expected, dtype):
    a = actual.float().cpu().numpy()
    if dtype == torch.float32:
        return np.abs(a - expected) / (np.abs(expected) * 2.0**-23 + 1e-30)
    return (ulp_distance_bf16 if dtype == torch.bfloat16 else ulp_distance_f16)(a, expected)


@pytest.mark.parametrize("shape", [(16384 // 16, 4096), (3, 1), (5, 31), (3, 4097), (3, 8192),
                                   (2, 65536), (7, 96), (64, 8200)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("mode,offset", [("llama", 0.0), ("gemma", 1.0), ("none", 0.0)])
def test_forward_parity(shape, dtype, mode, offset):
    g = torch.Generator().manual_seed(1)
    x = torch.randn(shape, generator=g).to(dtype)
    w = (torch.rand(shape[-1], generator=g) + 0.5).to(dtype)
    import rmsnorm

    xd, wd = x.cuda(), w.cuda()
    y = torch.empty_like(xd)
    rstd = torch.empty(shape[:-1], device="cuda")
    rmsnorm.ops.rms_norm_forward(y, rstd, xd, wd, 1e-6, offset, mode)
    ey, er = R.forward(x.float().numpy(), w.float().numpy(), 1e-6, offset, mode, DT[dtype])
    d = ulps(y, ey, dtype)
    if dtype == torch.float32:
        assert d.max() <= 8, d.max()
    elif mode == "gemma":
        # One rounding (f32 math, output rounded): <= 1 ulp, the sum order being
        # the only difference from the oracle.
        assert d.max() <= 1, d.max()
    else:
        # "llama"/"none" round x_hat to X before the weight multiply
        # (device.rs:161-179): a rounding-boundary flip of x_hat (from the sum
        # order of rstd) costs 1 ulp of x_hat before the product's own rounding.
        assert d.max() <= 2, d.max()
        assert (d > 1).mean() < 1e-3
    np.testing.assert_allclose(rstd.cpu().numpy(), er, rtol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("mode,offset", [("llama", 0.0), ("gemma", 1.0)])
def test_float32_weight(dtype, mode, offset):
    """rmsnorm/tests/test_ops.py:33-55: float32 weight with 16-bit x, fwd + bwd."""
    import rmsnorm

    g = torch.Generator().manual_seed(0)
    x = torch.randn(4, 33, 1000, generator=g).to(dtype)
    w = torch.randn(1000, generator=g)
    dy = torch.randn(4, 33, 1000, generator=g).to(dtype)
    xd = x.cuda().requires_grad_()
    wd = w.cuda().requires_grad_()
    y = rmsnorm.rms_norm(xd, wd, 1e-6, offset, mode, in_place=False)
    y.backward(dy.cuda())
    ey, er = R.forward(x.float().numpy(), w.numpy(), 1e-6, offset, mode, DT[dtype], "f32")
    assert ulps(y.detach(), ey, dtype).max() <= (1 if mode == "gemma" else 2)
    edx, edw = R.backward(dy.float().numpy(), x.float().numpy(), w.numpy(), er, offset, mode, DT[dtype])
    # dx = rstd*m - rstd^3/n*dot(m,x)*x cancels; compare like rmsnorm/tests/test_ops.py:49-51
    # and, tighter, against the size of the two terms it subtracts.
    tol = dict(atol=2e-2, rtol=2e-2) if dtype == torch.float16 else dict(atol=2e-1, rtol=2e-2)
    got = xd.grad.float().cpu().numpy()
    np.testing.assert_allclose(got, edx, **tol)
    xn, dyn = x.float().numpy(), dy.float().numpy()
    m = dyn * (w.numpy() + offset)
    scale_terms = np.abs(er[..., None] * m) + np.abs(er[..., None] ** 3 * np.mean(m * xn, -1, keepdims=True) * xn)
    ulp = 2.0**-8 if dtype == torch.bfloat16 else 2.0**-11
    assert np.all(np.abs(got - edx) <= 2 * ulp * (np.abs(edx) + 1e-3 * scale_terms) + 1e-2 * ulp * scale_terms)
    np.testing.assert_allclose(wd.grad.cpu().numpy(), edw, rtol=2e-3, atol=2e-2)
    assert y.dtype == dtype and xd.grad.dtype == dtype and wd.grad.dtype == torch.float32


@pytest.mark.parametrize("hidden", [1, 31, 4097, 8192, 65536])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_hidden_sizes_backward(hidden, dtype):
    """rmsnorm/tests/test_ops.py:58-68 shapes, fwd + bwd against the oracle."""
    import rmsnorm

    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, hidden, generator=g).to(dtype)
    w = torch.randn(hidden, generator=g).to(dtype)
    dy = torch.randn(3, hidden, generator=g).to(dtype)
    xd = x.cuda().requires_grad_()
    wd = w.cuda().requires_grad_()
    rmsnorm.rms_norm(xd, wd, 1e-6).backward(dy.cuda().clone())
    _, er = R.forward(x.float().numpy(), w.float().numpy(), 1e-6, 0.0, "llama", DT[dtype])
    edx, edw = R.backward(dy.float().numpy(), x.float().numpy(), w.float().numpy(), er, 0.0,
                          "llama", DT[dtype])
    tol = dict(atol=1e-4, rtol=1e-5) if dtype == torch.float32 else dict(atol=2e-1, rtol=2e-2)
    torch.testing.assert_close(xd.grad.float().cpu(), torch.from_numpy(edx), **tol)
    torch.testing.assert_close(wd.grad.float().cpu(),
                               torch.from_numpy(edw).to(dtype).float(), **tol)


def test_in_place_overwrites_output_grad():
    """rmsnorm/tests/test_ops.py:71-85."""
    import rmsnorm

    torch.manual_seed(0)
    x = torch.randn(8, 64, device="cuda").requires_grad_()
    w = torch.randn(64, device="cuda").requires_grad_()
    dy = torch.randn_like(x)
    dy_in_place = dy.clone()
    rmsnorm.rms_norm(x, w, 1e-6, in_place=True).backward(dy_in_place)
    dx = x.grad.clone()
    x.grad = None
    rmsnorm.rms_norm(x, w, 1e-6, in_place=False).backward(dy)
    torch.testing.assert_close(dx, x.grad, atol=0.0, rtol=0.0)
    torch.testing.assert_close(dy_in_place, dx, atol=0.0, rtol=0.0)


@pytest.mark.parametrize("with_weight", [True, False])
def test_opcheck(with_weight):
    import rmsnorm

    torch.manual_seed(0)
    x = torch.randn(4, 7, 96, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(96, device="cuda", dtype=torch.bfloat16) if with_weight else None
    _, rstd = rmsnorm.torch_ops.rms_norm_forward(x, w, 1e-6, 0.0, "llama")
    dy = torch.randn_like(x)
    torch.library.opcheck(rmsnorm.torch_ops.rms_norm_forward, (x, w, 1e-6, 0.0, "llama"))
    torch.library.opcheck(rmsnorm.torch_ops.rms_norm_backward, (dy, x, w, rstd, 0.0, "llama"))
    torch.library.opcheck(rmsnorm.torch_ops.rms_norm_backward_, (dy.clone(), x, w, rstd, 0.0, "llama"))


@pytest.mark.parametrize("with_weight", [True, False])
def test_empty_input(with_weight):
    import rmsnorm

    x = torch.empty(0, 64, device="cuda", requires_grad=True)
    w = torch.randn(64, device="cuda", requires_grad=True) if with_weight else None
    y = rmsnorm.rms_norm(x, w, 1e-6)
    y.backward(torch.empty_like(y))
    assert y.shape == (0, 64) and x.grad.shape == (0, 64)
    if with_weight:
        torch.testing.assert_close(w.grad, torch.zeros_like(w))


def test_layers_match_transformers_formula():
    """rmsnorm/tests/test_layers.py: RMSNorm / GemmaRMSNorm layers, fwd + bwd."""
    import rmsnorm

    torch.manual_seed(0)
    hidden = 256
    x = torch.randn(2, 128, hidden, device="cuda")
    w = torch.randn(hidden, device="cuda") * 0.1 + 1.0

    layer = rmsnorm.layers.RMSNorm()
    layer.weight = torch.nn.Parameter(w.clone())
    layer.variance_epsilon = 1e-6
    xk = x.clone().requires_grad_()
    out = layer(xk)
    xr = x.clone().requires_grad_()
    wr = w.clone().requires_grad_()
    ref = wr * (xr * torch.rsqrt(xr.pow(2).mean(-1, keepdim=True) + 1e-6))
    dy = torch.randn_like(x)
    out.backward(dy)
    ref.backward(dy)
    torch.testing.assert_close(out, ref, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(xk.grad, xr.grad, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(layer.weight.grad, wr.grad, atol=1e-4, rtol=1e-4)


def test_large_row_offset():
    """rmsnorm/tests/test_rms_norm.py:130-143: the first row beyond the int32 element range."""
    import rmsnorm

    rows, cols = 2**23 + 16, 256
    x = torch.zeros(rows, cols, dtype=torch.bfloat16, device="cuda")
    x[-1].fill_(1)
    w = torch.ones(cols, dtype=torch.bfloat16, device="cuda")
    y = rmsnorm.RMSNormFunction.apply(x, w, 1e-6, 0.0, "llama", True)
    assert torch.allclose(y[-1], torch.ones_like(y[-1]), atol=1e-2, rtol=1e-2)
    del x, y
