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


def bits_equal(actual, expected):
    """Element count whose bits differ from the oracle (f32 holding X values)."""
    a = actual.float().cpu().numpy().view(np.uint32)
    e = np.asarray(expected, dtype=np.float32).view(np.uint32)
    return int(np.sum(a != e))


@pytest.mark.parametrize("shape", [(1024, 4096), (3, 1), (5, 31), (3, 4097), (3, 8192),
                                   (2, 65536), (7, 96), (64, 8200), (5, 1000), (4, 2052),
                                   (9, 16384), (3, 40000), (200, 512)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("mode,offset", [("llama", 0.0), ("gemma", 1.0), ("none", 0.0)])
def test_forward_parity(shape, dtype, mode, offset):
    """Every kernel (wave per row, block per row with and without 16-byte access)
    sums x^2 in the reference's order and rounds rstd correctly, so y and rstd
    equal the oracle bit for bit."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(shape, generator=g).to(dtype)
    w = (torch.rand(shape[-1], generator=g) + 0.5).to(dtype)
    import rmsnorm

    xd, wd = x.cuda(), w.cuda()
    y = torch.empty_like(xd)
    rstd = torch.empty(shape[:-1], device="cuda")
    rmsnorm.ops.rms_norm_forward(y, rstd, xd, wd, 1e-6, offset, mode)
    ey, er = R.forward(x.float().numpy(), w.float().numpy(), 1e-6, offset, mode, DT[dtype])
    assert bits_equal(rstd, er) == 0
    assert bits_equal(y, ey) == 0, f"max {ulps(y, ey, dtype).max()} ulp"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_forward_unaligned_and_no_weight(dtype):
    """A storage offset of one element takes the block kernel without 16-byte
    access (single columns, ops.rs:108-115); no weight takes the non-affine
    kernels. Both bit-exact."""
    import rmsnorm

    g = torch.Generator().manual_seed(4)
    n = 1024
    base = torch.randn(17 * n + 1, generator=g).to(dtype)
    x = base[1:].view(17, n)
    xd = base.cuda()[1:].view(17, n)
    y = torch.empty(17 * n + 1, dtype=dtype, device="cuda")[1:].view(17, n)
    rstd = torch.empty(17, device="cuda")
    rmsnorm.ops.rms_norm_forward(y, rstd, xd, None, 1e-5, 0.0, "llama")
    ey, er = R.forward(x.float().numpy(), None, 1e-5, 0.0, "llama", DT[dtype], vectorized=False)
    assert bits_equal(rstd, er) == 0
    assert bits_equal(y, ey) == 0
    y2 = torch.empty(17, n, dtype=dtype, device="cuda")
    rmsnorm.ops.rms_norm_forward(y2, rstd, x.cuda(), None, 1e-5, 0.0, "llama")
    ey2, er2 = R.forward(x.float().numpy(), None, 1e-5, 0.0, "llama", DT[dtype])
    assert bits_equal(y2, ey2) == 0 and bits_equal(rstd, er2) == 0


def test_forward_baseline_config():
    """The benchmarked shape in full: x [16384, 4096] bf16 ~N(0,1), w ~U(0.5, 1.5),
    eps 1e-6, llama, seed 1 (the wave kernel's multi-row loop with prefetch).
    Every element of y and rstd against the oracle."""
    import rmsnorm

    g = torch.Generator().manual_seed(1)
    x = torch.randn(16384, 4096, generator=g).bfloat16()
    w = (torch.rand(4096, generator=g) + 0.5).bfloat16()
    xd, wd = x.cuda(), w.cuda()
    y = torch.empty_like(xd)
    rstd = torch.empty(16384, device="cuda")
    rmsnorm.ops.rms_norm_forward(y, rstd, xd, wd, 1e-6, 0.0, "llama")
    ey, er = R.forward(x.float().numpy(), w.float().numpy(), 1e-6, 0.0, "llama", "bf16")
    d = ulps(y, ey, torch.bfloat16)
    print(f"config 2: {int((d > 0).sum())} of {d.size} elements differ, max {int(d.max())} ulp; "
          f"rstd differs in {bits_equal(rstd, er)} rows")
    assert d.max() <= 1
    assert bits_equal(y, ey) == 0 and bits_equal(rstd, er) == 0


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
    assert bits_equal(y.detach(), ey) == 0
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


def assert_dx_close(got, edx, dy, x, w, rstd, offset, dtype):
    """dx = rstd*m - rstd^3/n*dot(m,x)*x is rounded once. The kernel's f32
    dot(m, x) sums in another order than the oracle's; its error is at most
    n * 2^-24 * sum|m*x| (the worst-case bound of a recursive f32 sum), which
    moves dx by rstd^3 / n times that times |x| before the rounding. Beyond
    that, one rounding flip (one ulp of the element type)."""
    m = dy * (1.0 if w is None else (w + offset))
    n = x.shape[-1]
    dot_err = n * 2.0**-24 * np.sum(np.abs(m * x), -1, keepdims=True)
    slack = rstd[..., None] ** 3 / n * dot_err * np.abs(x) * 1.01
    mant = 7 if dtype == torch.bfloat16 else 10
    mag = np.maximum(np.abs(edx), np.abs(got))
    e = np.floor(np.log2(np.maximum(mag, 2.0**-126 if mant == 7 else 2.0**-14)))
    ulp = 2.0 ** (e - mant)  # spacing of the element type at the larger magnitude
    # two values within `slack` round to grid points at most slack + one ulp apart
    bound = ulp + slack
    assert np.all(np.abs(got - edx) <= bound), np.max(np.abs(got - edx) / bound)


@pytest.mark.parametrize("n", [96, 1000, 2048, 4096])
@pytest.mark.parametrize("rows", [48, 1100])
@pytest.mark.parametrize("weight", ["same", "f32", None])
@pytest.mark.parametrize("mode,offset", [("llama", 0.0), ("gemma", 1.0), ("none", 0.0)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_backward_wave_parity(n, rows, weight, mode, offset, dtype):
    """The wave-per-partial-row backward (16-bit x, n % 8 == 0) against the
    oracle: dx per element, dw_partial summed by rms_norm_reduce_weight_grad.
    rows 1100 > 4 waves x 256 CUs runs several rows per wave."""
    import rmsnorm

    g = torch.Generator().manual_seed(n + rows)
    x = torch.randn(rows, n, generator=g).to(dtype)
    dy = torch.randn(rows, n, generator=g).to(dtype)
    wdt = dtype if weight == "same" else torch.float32
    w = None if weight is None else (torch.rand(n, generator=g) + 0.5).to(wdt)
    xd, dyd = x.cuda(), dy.cuda()
    wd = None if w is None else w.cuda()
    y = torch.empty_like(xd)
    rstd = torch.empty(rows, device="cuda")
    rmsnorm.ops.rms_norm_forward(y, rstd, xd, wd, 1e-6, offset, mode)
    blocks = 256
    dwp = torch.empty(blocks, n, device="cuda") if w is not None else None
    dx = torch.empty_like(xd)
    rmsnorm.ops.rms_norm_backward(dx, dwp, dyd, xd, wd, rstd, offset, mode)
    wn = None if w is None else w.float().numpy()
    ey, er = R.forward(x.float().numpy(), wn, 1e-6, offset, mode, DT[dtype],
                       None if w is None else DT[wdt])
    assert bits_equal(rstd, er) == 0
    edx, edw = R.backward(dy.float().numpy(), x.float().numpy(), wn, er, offset, mode, DT[dtype])
    assert_dx_close(dx.float().cpu().numpy(), edx, dy.float().numpy(), x.float().numpy(), wn, er,
                    offset, dtype)
    if w is not None:
        dw = torch.empty(n, dtype=wdt, device="cuda")
        rmsnorm.ops.rms_norm_reduce_weight_grad(dw, dwp)
        rw = torch.from_numpy(edw).to(wdt).float().numpy()
        np.testing.assert_allclose(dw.float().cpu().numpy(), rw, rtol=1e-2 if wdt != torch.float32 else 1e-4,
                                   atol=1e-3 * np.abs(edw).max())
    # in place (dy read from dx): the same bits as out of place
    dx2 = dyd.clone()
    dwp2 = torch.empty_like(dwp) if dwp is not None else None
    rmsnorm.ops.rms_norm_backward(dx2, dwp2, None, xd, wd, rstd, offset, mode)
    assert torch.equal(dx2, dx)
    if dwp is not None:
        assert torch.equal(dwp2, dwp)


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
