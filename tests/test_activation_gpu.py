"""GPU parity of the activation kernels against oracle/activation.py.

Mirrors activation-rs/tests/kernels/test_activation.py. For bf16 / f16 every
op is compared bit for bit with the oracle (the activation of a 16-bit input
comes from a table built from the reference's expression with correctly rounded
exp / erf / tanh, and the product with the other half is rounded once, so the
whole output is defined to the bit); f32 results carry the device libm's error
and are compared within a few f32 ulp. Also the unaligned, empty and
layer/torch-op paths of that file.
"""

import numpy as np
import pytest
import torch

from oracle import activation as A
from oracle.numerics import ulp_distance_bf16, ulp_distance_f16

pytestmark = pytest.mark.gpu

DT = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}
GATED = ["silu_and_mul", "mul_and_silu", "gelu_and_mul", "gelu_tanh_and_mul", "fatrelu_and_mul"]
ELEMENTWISE = ["silu", "gelu", "gelu_tanh", "gelu_new", "gelu_fast", "gelu_quick"]


def assert_within_one_ulp(actual, expected_np, dtype, x_np=None):
    a = actual.float().cpu().numpy()
    if dtype == torch.float32:
        # f32 results: the GPU libm (<= 2 ulp) vs correctly rounded oracle; exact
        # GELU's 1 + erf cancellation below -4 scales with |x| (see the oracle pins).
        atol = 1e-6 if x_np is None else np.abs(x_np).max() * 2.0**-22
        np.testing.assert_allclose(a, expected_np, rtol=4e-6, atol=atol)
        return
    dist = (ulp_distance_bf16 if dtype == torch.bfloat16 else ulp_distance_f16)(a, expected_np)
    ok = dist <= 1
    if x_np is not None:
        ok |= np.abs(a - expected_np) <= np.abs(x_np) * 2.0**-23
    assert ok.all(), f"max ulp distance {dist.max()}, {np.sum(~ok)} elements"


def ulp_of(x, dtype):
    """Spacing of the element type at |x| (as f32)."""
    x = np.abs(np.asarray(x, dtype=np.float32))
    if dtype == torch.float16:
        return np.spacing(x.astype(np.float16)).astype(np.float32)
    if dtype == torch.bfloat16:
        e = np.floor(np.log2(np.maximum(x, 2.0**-126)))
        return (2.0 ** (e - 7)).astype(np.float32)
    return np.spacing(x)


def differing(actual, expected):
    """Count of elements whose bits differ (NaN matches NaN)."""
    a = np.asarray(actual, dtype=np.float32)
    e = np.asarray(expected, dtype=np.float32)
    both_nan = np.isnan(a) & np.isnan(e)
    return int(np.sum((a.view(np.uint32) != e.view(np.uint32)) & ~both_nan))


def assert_gated(out, x, op, dtype, threshold=0.3):
    """16-bit: bit-exact. f32: the activation (device libm, a few ulp) times the
    other half, within 4 f32 ulp of the activation scaled by |other|, plus the
    1 + erf / 1 + tanh cancellation for the GELUs."""
    d = x.shape[-1] // 2
    xn = x.float().numpy()
    expected = A.gated(op, xn, DT[dtype], threshold=threshold)
    a = out.float().cpu().numpy()
    if dtype != torch.float32:
        assert differing(a, expected) == 0, (
            f"{differing(a, expected)} elements differ, max "
            f"{(ulp_distance_bf16 if dtype == torch.bfloat16 else ulp_distance_f16)(a, expected).max()} ulp")
        return
    gate, up = (xn[:, :d], xn[:, d:]) if op != "mul_and_silu" else (xn[:, d:], xn[:, :d])
    name = A.GATED[op][0]
    act = A.act(name, gate, DT[dtype], threshold)
    bound = 4 * (ulp_of(act, dtype) * np.abs(up) + ulp_of(expected, dtype))
    if name == "gelu" or name == "gelu_tanh":
        bound += 4 * np.abs(gate) * np.abs(up) * 2.0**-23
    err = np.abs(a - expected)
    assert np.all(err <= bound), f"{np.sum(err > bound)} elements outside the bound"


@pytest.mark.parametrize("op", GATED)
@pytest.mark.parametrize("num_tokens", [7, 83, 2048])
@pytest.mark.parametrize("d", [512, 13824])
@pytest.mark.parametrize("dtype", [torch.half, torch.bfloat16, torch.float])
def test_act_and_mul(op, num_tokens, d, dtype):
    import activation_rs

    g = torch.Generator().manual_seed(0)
    x = torch.randn(num_tokens, 2 * d, generator=g).to(dtype)
    xd = x.cuda()
    out = torch.empty(num_tokens, d, dtype=dtype, device="cuda")
    fn = getattr(activation_rs, op)
    if op == "fatrelu_and_mul":
        fn(out, xd, 0.3)
    else:
        fn(out, xd)
    assert_gated(out, x, op, dtype)


@pytest.mark.parametrize("op", ELEMENTWISE)
@pytest.mark.parametrize("dtype", [torch.half, torch.bfloat16, torch.float])
def test_elementwise(op, dtype):
    import activation_rs

    g = torch.Generator().manual_seed(1)
    x = torch.randn(83, 13824, generator=g).to(dtype)
    out = getattr(activation_rs, op)(torch.empty(x.shape, dtype=dtype, device="cuda"), x.cuda())
    expected = A.elementwise(op, x.float().numpy(), DT[dtype])
    if dtype != torch.float32:
        assert differing(out.float().cpu().numpy(), expected) == 0
        return
    if op in ("gelu_new", "gelu_fast"):
        # f32 has no rounding between the steps to absorb the libm's tanh error.
        np.testing.assert_allclose(out.float().cpu().numpy(), expected, atol=1e-5, rtol=1.3e-6)
        return
    assert_within_one_ulp(out, expected, dtype, x.float().numpy() if op.startswith("gelu") else None)


def all_16bit_values(dtype):
    n = np.arange(1 << 16, dtype=np.uint32)
    if dtype == torch.bfloat16:
        return (n << 16).view(np.float32)
    return n.astype(np.uint16).view(np.float16).astype(np.float32)


@pytest.mark.parametrize("op", ELEMENTWISE)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.half])
def test_every_16bit_value_elementwise(op, dtype):
    """Element-wise maps over every 16-bit input, NaN and infinities included
    (the exhaustive pin): bit-exact. A 16-bit input has no other values, so
    this covers the op completely."""
    import activation_rs

    x = all_16bit_values(dtype)
    xt = torch.from_numpy(x).to(dtype).cuda()
    out = getattr(activation_rs, op)(torch.empty_like(xt), xt)
    exp = A.elementwise(op, x, DT[dtype])
    got = out.float().cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(exp))
    assert differing(got, exp) == 0, x[(got.view(np.uint32) != exp.view(np.uint32)) & ~np.isnan(exp)][:8]


@pytest.mark.parametrize("op", ["silu_and_mul", "mul_and_silu", "gelu_and_mul", "gelu_tanh_and_mul"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.half])
def test_every_16bit_value_gated(op, dtype):
    """Gated ops over every 16-bit gate value (NaN and infinities included),
    with the other half 1, -3 and 0.7: bit-exact against the oracle on both
    the vector kernel (aligned) and the scalar kernel (odd width)."""
    import activation_rs

    g = all_16bit_values(dtype)
    for other in (1.0, -3.0, 0.7):
        for width in (len(g), len(g) - 1):
            gg = g[:width]
            halves = [gg, np.full_like(gg, other)]
            if op == "mul_and_silu":
                halves.reverse()
            x = np.concatenate(halves)[None, :]
            xt = torch.from_numpy(x).to(dtype).cuda()
            out = torch.empty(1, width, dtype=dtype, device="cuda")
            getattr(activation_rs.ops, op)(out, xt)
            got = out.float().cpu().numpy()[0]
            exp = A.gated(op, torch.from_numpy(x).to(dtype).float().numpy(), DT[dtype])[0]
            assert np.array_equal(np.isnan(got), np.isnan(exp))
            bad = (got.view(np.uint32) != exp.view(np.uint32)) & ~np.isnan(exp)
            assert not bad.any(), (other, width, gg[bad][:8])


@pytest.mark.parametrize("op", ["silu_and_mul", "gelu_and_mul", "gelu_tanh_and_mul"])
def test_gated_baseline_config(op):
    """The benchmarked shape: x [16384, 28672] bf16 ~N(0,1), seed 2, out
    [16384, 14336]. 2048 rows (the first, the last and a seeded sample) of the
    GPU output against the oracle, bit for bit."""
    import activation_rs

    g = torch.Generator().manual_seed(2)
    x = torch.randn(16384, 28672, generator=g).bfloat16()
    xd = x.cuda()
    out = torch.empty(16384, 14336, dtype=torch.bfloat16, device="cuda")
    getattr(activation_rs, op)(out, xd)
    del xd
    rows = np.unique(np.concatenate([[0, 16383], np.random.default_rng(2).choice(16384, 2046, replace=False)]))
    got = out[torch.from_numpy(rows).cuda()].float().cpu().numpy()
    exp = A.gated(op, x[torch.from_numpy(rows)].float().numpy(), "bf16")
    d = ulp_distance_bf16(got, exp)
    print(f"config 3 {op}: {int((d > 0).sum())} of {d.size} sampled elements differ, max {int(d.max())} ulp")
    assert d.max() <= 1
    assert differing(got, exp) == 0


@pytest.mark.parametrize("d", [1, 13, 4097])
@pytest.mark.parametrize("dtype", [torch.half, torch.bfloat16, torch.float])
def test_act_and_mul_unaligned(d, dtype):
    """activation-rs/tests/kernels/test_activation.py:278-294: odd widths and a
    storage offset of one element take the scalar path."""
    import activation_rs

    g = torch.Generator().manual_seed(0)
    num_tokens = 5
    base = torch.randn(num_tokens * 2 * d + 1, generator=g).to(dtype).cuda()
    x = base[1:].view(num_tokens, 2 * d)
    out = activation_rs.silu_and_mul(torch.empty(num_tokens, d, dtype=dtype, device="cuda"), x)
    assert_gated(out, x.cpu(), "silu_and_mul", dtype)


def test_empty_input():
    import activation_rs

    x = torch.empty(0, 128, dtype=torch.bfloat16, device="cuda")
    assert activation_rs.silu_and_mul(torch.empty(0, 64, dtype=x.dtype, device="cuda"), x).shape == (0, 64)
    assert activation_rs.silu(torch.empty(0, 128, dtype=x.dtype, device="cuda"), x).shape == (0, 128)


def test_layers_and_torch_ops_match_functions():
    import activation_rs

    x = torch.randn(33, 1024, device="cuda", dtype=torch.bfloat16)
    for layer, fn in [
        (activation_rs.layers.SiluAndMul(), activation_rs.silu_and_mul),
        (activation_rs.layers.GeluAndMul(), activation_rs.gelu_and_mul),
        (activation_rs.layers.GeluTanhAndMul(), activation_rs.gelu_tanh_and_mul),
        (activation_rs.layers.MulAndSilu(), activation_rs.mul_and_silu),
    ]:
        out = fn(torch.empty(33, 512, dtype=x.dtype, device="cuda"), x)
        torch.testing.assert_close(layer(x), out, atol=0, rtol=0)
    torch.testing.assert_close(activation_rs.layers.FastGELU()(x),
                               activation_rs.gelu_fast(torch.empty_like(x), x), atol=0, rtol=0)


def test_opcheck():
    import activation_rs

    x = torch.randn(7, 512, device="cuda", dtype=torch.half)
    out = torch.empty(7, 256, device="cuda", dtype=torch.half)
    torch.library.opcheck(activation_rs.torch_ops.silu_and_mul, (out, x))
    torch.library.opcheck(activation_rs.torch_ops.fatrelu_and_mul, (out, x, 0.5))
    torch.library.opcheck(activation_rs.torch_ops.gelu, (torch.empty_like(x), x))


def test_repeated_calls_bitwise_equal():
    import activation_rs

    x = torch.randn(16384, 2 * 1024, device="cuda", dtype=torch.bfloat16)
    a = activation_rs.gelu_and_mul(torch.empty(16384, 1024, dtype=x.dtype, device="cuda"), x)
    b = activation_rs.gelu_and_mul(torch.empty(16384, 1024, dtype=x.dtype, device="cuda"), x)
    assert torch.equal(a, b)
