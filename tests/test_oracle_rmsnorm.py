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


def _literal_block_sum(row, vectorized):
    """Thread-by-thread restatement of the reference kernel's sum of squares
    (rmsnorm/src/device.rs:41-63, 113-145): a literal loop per thread, then
    shuffle-xor butterflies over explicit 32-lane arrays, all in f32."""
    f = np.float32
    n = len(row)
    T = R.block_threads(n)
    tail = n // 8 * 8 if vectorized else 0
    partial = []
    for t in range(T):
        s = f(0.0)
        col = 8 * t
        first = True
        while col < tail:
            g = f(0.0)
            for i in range(8):
                g = f(g + f(row[col + i] * row[col + i]))
            s = g if first else f(s + g)
            first = False
            col += 8 * T
        col = tail + t
        while col < n:
            s = f(s + f(row[col] * row[col]))
            col += T
        partial.append(s)

    def warp_reduce(lanes):
        lanes = list(lanes)
        for d in (16, 8, 4, 2, 1):
            lanes = [f(lanes[i] + lanes[i ^ d]) for i in range(32)]
        assert len(set(np.asarray(lanes).view(np.uint32).tolist())) == 1  # every lane agrees
        return lanes[0]

    warps = [warp_reduce(partial[32 * w : 32 * w + 32]) for w in range(T // 32)]
    return warp_reduce(warps + [f(0.0)] * (32 - len(warps)))


@pytest.mark.parametrize("n,vectorized", [(96, True), (1000, True), (1001, False), (4096, True),
                                          (2052, True), (300, False), (8200, True)])
def test_sum_order_matches_literal_thread_loop(n, vectorized):
    g = np.random.default_rng(n)
    x = g.standard_normal((3, n)).astype(np.float32)
    got = R.sum_squares_reference_order(x, vectorized)
    want = np.array([_literal_block_sum(r, vectorized) for r in x], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # and it is a sum of squares to f32 accuracy
    np.testing.assert_allclose(got, (x.astype(np.float64) ** 2).sum(-1), rtol=n * 2.0**-24)


def test_rsqrt_is_correctly_rounded():
    g = np.random.default_rng(0)
    v = np.concatenate([g.uniform(1e-6, 10, 20000), [1.0, 4.0, 0.25, 1e-6, 2.0]]).astype(np.float32)
    r = R.rsqrt_rn(v)
    exact = 1.0 / np.sqrt(v.astype(np.longdouble))
    err = np.abs(r.astype(np.longdouble) - exact) / np.spacing(r).astype(np.longdouble)
    assert err.max() <= 0.5 + 1e-6
    assert r[-5:].tolist() == [1.0, 0.5, 2.0, np.float32(1000.0), np.float32(1 / np.sqrt(2.0))]
