"""Pins oracle/activation.py.

The reference tests' oracle is torch CPU/GPU `F.silu`, `F.gelu` and friends
(activation-rs/tests/kernels/test_activation.py:41-83), compared exactly. Here
the numpy restatement is checked against torch CPU on every bf16 bit pattern for
the element-wise maps, on random gated inputs for every dtype, and on closed forms.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import activation as A
from oracle.numerics import ulp_distance_bf16, ulp_distance_f16

TORCH_DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def all_bf16_values():
    bits = (np.arange(1 << 16, dtype=np.uint32) << 16).view(np.float32)
    return bits[np.isfinite(bits)]


def torch_act(name, t, threshold=0.0):
    if name == "silu":
        return F.silu(t)
    if name == "gelu":
        return F.gelu(t)
    if name == "gelu_tanh":
        return F.gelu(t, approximate="tanh")
    if name == "gelu_quick":
        return t * torch.sigmoid(1.702 * t)
    if name == "fatrelu":
        return F.threshold(t, threshold, 0.0)
    raise KeyError(name)


@pytest.mark.parametrize("name", ["silu", "gelu", "gelu_tanh"])
def test_elementwise_all_bf16_values_vs_torch(name):
    x = all_bf16_values()
    # torch evaluates gelu as x * (1 + erf) * 0.5, which overflows above ~1.7e38;
    # the reference evaluates (x * 0.5) * (1 + erf) (activation.rs:57). Compare
    # the range where both orders are finite.
    x = x[np.abs(x) < 1e38]
    # torch's vectorised CPU gelu flushes subnormal results to zero; keep away from them.
    x = x[(np.abs(x) >= 1e-30) | (x == 0)]
    ours = A.act(name, x, "bf16")
    theirs = torch_act(name, torch.from_numpy(x).bfloat16()).float().numpy()
    finite = np.isfinite(theirs) & np.isfinite(ours)
    np.testing.assert_array_equal(np.isfinite(ours), np.isfinite(theirs))
    dist = ulp_distance_bf16(ours[finite], theirs[finite])
    # Exact GELU at x < -4 forms 1 + erf(x / sqrt 2) ~ 1e-5 in f32: the result
    # inherits one f32 ulp of erf near -1 (2^-24), i.e. an absolute error of
    # |x| * 2^-24 that spans several bf16 ulps of the tiny result. Any two f32 erf
    # implementations differ there; allow that bound, nothing more.
    cancel = np.abs(ours[finite] - theirs[finite]) <= np.abs(x[finite]) * 2.0**-23
    assert np.all((dist <= 1) | cancel)
    # Disagreements are rare rounding-boundary cases of the f32 libm result.
    assert (dist > 0).mean() < 1e-3


@pytest.mark.parametrize("op,torch_fn", [
    ("silu_and_mul", lambda x, d: F.silu(x[..., :d]) * x[..., d:]),
    ("mul_and_silu", lambda x, d: x[..., :d] * F.silu(x[..., d:])),
    ("gelu_and_mul", lambda x, d: F.gelu(x[..., :d]) * x[..., d:]),
    ("gelu_tanh_and_mul", lambda x, d: F.gelu(x[..., :d], approximate="tanh") * x[..., d:]),
    ("fatrelu_and_mul", lambda x, d: F.threshold(x[..., :d], 0.25, 0.0) * x[..., d:]),
])
@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_gated_vs_torch(op, torch_fn, dtype):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 2 * 384, generator=g).to(TORCH_DT[dtype])
    ours = A.gated(op, x.float().numpy(), dtype, threshold=0.25)
    theirs = torch_fn(x, 384).float().numpy()
    if dtype == "f32":
        # atol: one f32 ulp of erf near -1 scaled by |x| (cancellation in 1 + erf).
        xa = np.abs(x.float().numpy()).max()
        np.testing.assert_allclose(ours, theirs, rtol=2e-6, atol=xa * 2.0**-22)
    else:
        dist = (ulp_distance_bf16 if dtype == "bf16" else ulp_distance_f16)(ours, theirs)
        assert dist.max() <= 1
        assert (dist > 0).mean() < 5e-3


def test_closed_forms():
    for name in ("silu", "gelu", "gelu_tanh", "gelu_new", "gelu_fast", "gelu_quick"):
        assert A.act(name, np.float32(0.0), "f32") == 0.0
        # act(x) -> x for large x, -> 0 for very negative x
        assert A.act(name, np.float32(60.0), "bf16") == np.float32(60.0)
        assert abs(A.act(name, np.float32(-60.0), "f32")) < 1e-12
    # silu(1) = 1 / (1 + e^-1)
    assert abs(A.act("silu", np.float32(1.0), "f32") - 1.0 / (1.0 + math.exp(-1.0))) < 1e-7
    # gelu(1) = 0.5 * (1 + erf(1/sqrt 2)) = Phi(1)
    assert abs(A.act("gelu", np.float32(1.0), "f32") - 0.8413447460685429) < 1e-7
    # gelu_quick(x) = x * sigmoid(1.702 x)
    assert abs(A.act("gelu_quick", np.float32(2.0), "f32") - 2.0 / (1 + math.exp(-3.404))) < 1e-6
    # FATReLU keeps values strictly above the threshold only
    np.testing.assert_array_equal(
        A.act("fatrelu", np.float32([0.1, 0.5, 0.6, -1.0]), "f32", threshold=0.5), np.float32([0, 0, 0.6, 0])
    )


def _torch_gelu_fast(x):
    # activation-rs/tests/kernels/test_activation.py:41-42
    return 0.5 * x * (1.0 + torch.tanh(x * 0.7978845608 * (1.0 + 0.044715 * x * x)))


def _torch_gelu_new(x):
    # activation-rs/tests/kernels/test_activation.py:45-47
    c = math.sqrt(2.0 / math.pi)
    return 0.5 * x * (1.0 + torch.tanh(c * (x + 0.044715 * torch.pow(x, 3.0))))


@pytest.mark.parametrize("name,fn", [("gelu_new", _torch_gelu_new), ("gelu_fast", _torch_gelu_fast)])
@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_gelu_new_fast_vs_reference_test_formula(name, fn, dtype):
    # The reference tests compare these with torch's default tolerances
    # (allclose_default.py:7-8), since every intermediate is rounded to T.
    atol = {"bf16": 1e-3, "f16": 1e-3, "f32": 1e-5}[dtype]
    rtol = {"bf16": 1.6e-2, "f16": 1e-3, "f32": 1.3e-6}[dtype]
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2048, 512, generator=g).to(TORCH_DT[dtype])
    ours = torch.from_numpy(A.act(name, x.float().numpy(), dtype)).to(TORCH_DT[dtype])
    torch.testing.assert_close(ours, fn(x), atol=atol, rtol=rtol)
    # and a dropped cubic term would not pass:
    wrong = 0.5 * x * (1.0 + torch.tanh(0.7978845608 * x))
    assert not torch.allclose(ours.float(), wrong.float(), atol=atol, rtol=rtol)


def test_fma32_against_exact_rationals():
    """oracle.activation.fma32 equals the correctly rounded a*b + c computed with
    exact rationals, on random triples and on constructed halfway cases where a
    plain f64 evaluation rounds twice."""
    from fractions import Fraction

    from oracle.activation import fma32

    def exact(a, b, c):
        v = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
        lo = np.float32(float(v))  # nearest f64 then f32: candidate neighbourhood
        cands = [np.nextafter(lo, np.float32(-np.inf)), lo, np.nextafter(lo, np.float32(np.inf))]
        best = min(cands, key=lambda r: (abs(Fraction(float(r)) - v),
                                         int(np.float32(r).view(np.uint32)) & 1))
        return np.float32(best)

    g = np.random.default_rng(0)
    a = g.standard_normal(3000).astype(np.float32)
    b = (g.standard_normal(3000) * 10).astype(np.float32)
    c = g.standard_normal(3000).astype(np.float32)
    # halfway cases: c = 1 + 2^-24 (an f32 midpoint offset) with a tiny product
    a2 = np.full(8, 2.0**-30, np.float32)
    b2 = np.array([2.0**-40, -(2.0**-40), 2.0**-50, -(2.0**-50), 1e-20, -1e-20, 2.0**-60, -(2.0**-60)], np.float32)
    c2 = np.full(8, 1.0 + 2.0**-23, np.float32)
    # p = (1 + 2^-23) * 2^-24 (1 - 2^-23) = 2^-24 - 2^-70: p + c is just below
    # (or, negated, above) an f32 midpoint and a plain f64 sum lands on it
    u = 2.0**-23
    a3 = np.array([1 + u, 1 + u, -(1 + u), 1 + u], np.float32)
    b3 = np.array([2.0**-24 * (1 - u), 2.0**-24 * (1 - u), 2.0**-24 * (1 - u), 2.0**-25 * (1 - u)], np.float32)
    c3 = np.array([1 + u, 1.0, -(1 + u), 0.5 + u / 2], np.float32)
    A, B, C = (np.concatenate(t) for t in ((a, a2, a3), (b, b2, b3), (c, c2, c3)))
    got = fma32(A, B, C)
    want = np.array([exact(x, y, z) for x, y, z in zip(A, B, C)], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # a plain f64 evaluation rounds twice on at least one of the constructed cases
    naive = (A.astype(np.float64) * B + C).astype(np.float32)
    assert not np.array_equal(naive.view(np.uint32), want.view(np.uint32))
