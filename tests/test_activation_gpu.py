"""GPU parity of the activation kernels against oracle/activation.py.

Mirrors activation-rs/tests/kernels/test_activation.py: the gated ops are
compared per element in units of the last place (the bar is <= 1 ulp of the
element type; the reference compares against torch exactly, here torch's f32
libm and the GPU's differ at rare rounding boundaries), plus the unaligned,
empty and layer/torch-op paths of that file.
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


def assert_gated(out, x, op, dtype, threshold=0.3):
    """The gated ops round twice (act(x) to T, then act * y to T). A 1-ulp
    disagreement of the GPU libm in act(x) therefore moves the product by
    ulp(act) * |y| before its own rounding: allow exactly that plus 1 ulp of the
    product; everything else must be within 1 ulp."""
    d = x.shape[-1] // 2
    xn = x.float().numpy()
    gate, up = (xn[:, :d], xn[:, d:]) if op != "mul_and_silu" else (xn[:, d:], xn[:, :d])
    name = A.GATED[op][0]
    act = A.act(name, gate, DT[dtype], threshold)
    expected = A.gated(op, xn, DT[dtype], threshold=threshold)
    a = out.float().cpu().numpy()
    bound = ulp_of(act, dtype) * np.abs(up) + ulp_of(expected, dtype)
    if name == "gelu" or name == "gelu_tanh":
        bound += np.abs(gate) * np.abs(up) * 2.0**-23  # 1 + erf / 1 + tanh cancellation
    if dtype == torch.float32:
        bound *= 4  # f32 results carry the GPU libm error itself (a few ulp)
    err = np.abs(a - expected)
    assert np.all(err <= bound), f"{np.sum(err > bound)} elements outside the bound"
    if dtype != torch.float32:
        dist = (ulp_distance_bf16 if dtype == torch.bfloat16 else ulp_distance_f16)(a, expected)
        assert (dist > 1).mean() < 1e-3, "too many elements beyond 1 ulp"


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
    if op in ("gelu_new", "gelu_fast"):
        # Every intermediate is rounded to T (activation.rs:79-104), so a 1-ulp libm
        # difference in tanh can move the result by several ulp of T; the reference
        # tests compare these with torch's default tolerances (allclose_default.py:7-8).
        atol = {torch.float16: 1e-3, torch.bfloat16: 1e-3, torch.float32: 1e-5}[dtype]
        rtol = {torch.float16: 1e-3, torch.bfloat16: 1.6e-2, torch.float32: 1.3e-6}[dtype]
        np.testing.assert_allclose(out.float().cpu().numpy(), expected, atol=atol, rtol=rtol)
        return
    assert_within_one_ulp(out, expected, dtype, x.float().numpy() if op.startswith("gelu") else None)


def test_every_bf16_value_silu_and_gelu():
    """Element-wise maps over all finite bf16 inputs (the exhaustive pin)."""
    import activation_rs

    bits = (np.arange(1 << 16, dtype=np.uint32) << 16).view(np.float32)
    x = bits[np.isfinite(bits)]
    xt = torch.from_numpy(x).bfloat16().cuda()
    for op in ("silu", "gelu_tanh", "gelu_quick"):
        out = getattr(activation_rs, op)(torch.empty_like(xt), xt)
        assert_within_one_ulp(out, A.elementwise(op, x, "bf16"), torch.bfloat16)


@pytest.mark.parametrize("op", ["silu_and_mul", "gelu_tanh_and_mul"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.half])
def test_every_16bit_value_gated(op, dtype):
    """Gated ops over every finite 16-bit gate value, with up = 1 and up = -3:
    the vectorised kernels' activation forms (including the overflow tails)
    against the oracle. At most 1 ulp anywhere, and under 0.1 % of elements
    off at all."""
    import activation_rs

    n = np.arange(1 << 16, dtype=np.uint32)
    if dtype == torch.bfloat16:
        g = (n << 16).view(np.float32)
    else:
        g = n.astype(np.uint16).view(np.float16).astype(np.float32)
    g = g[np.isfinite(g)]
    g = g[: len(g) // 8 * 8]
    for up_value in (1.0, -3.0):
        x = np.concatenate([g, np.full_like(g, up_value)])[None, :]
        xt = torch.from_numpy(x).to(dtype).cuda()
        out = torch.empty(1, len(g), dtype=dtype, device="cuda")
        getattr(activation_rs.ops, op)(out, xt)
        got = out.float().cpu().numpy()[0]
        exp = A.gated(op, x, DT[dtype])[0]
        finite = np.isfinite(exp)
        assert np.array_equal(np.isnan(got), np.isnan(exp))
        if up_value == 1.0:
            # out = act(gate) rounded once: within 1 ulp of the oracle.
            dist = (ulp_distance_bf16 if dtype == torch.bfloat16 else ulp_distance_f16)(got, exp)
            assert dist[finite].max() <= 1, g[finite][dist[finite] > 1][:8]
            assert (dist[finite] > 0).mean() < 1e-3
        else:
            # Rounded act times up, rounded again: a 1-ulp act difference moves
            # the product by ulp(act) * |up| before its own rounding.
            act = A.act(A.GATED[op][0], g, DT[dtype])
            bound = ulp_of(act, dtype) * abs(up_value) + ulp_of(exp, dtype)
            err = np.abs(got - exp)
            assert np.all(err[finite] <= bound[finite]), g[finite][err[finite] > bound[finite]][:8]


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
