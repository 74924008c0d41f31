"""The HIP kernels against the committed golden fixtures (tests/golden/*.npz),
through the same Python ops a caller of the reference uses.

Bars (the north star's and the reference tests'): attention output max-abs
<= 2e-2 against the fp32 oracle; gradients at the reference's bf16 backward
tolerance (atol 0.06, rtol 0.08, flash-attn2-rs/tests/test_gold.py:267);
RMSNorm and the gated activations bit for bit (the kernels sum mean(x^2) in
the reference's order and round rstd correctly; 16-bit activations come from
exact tables and the product is rounded once).
"""

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.numerics import ulp_distance_bf16

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import make_golden as G  # noqa: E402

pytestmark = pytest.mark.gpu

GRAD_TOL = dict(atol=0.06, rtol=0.08)


def bf16(bits):
    return torch.from_numpy(G.from_bits(bits)).bfloat16().cuda()


def test_golden_fa_dense():
    import flash_attn2_rs

    d = np.load(GOLDEN / "fa_dense_causal_b1_h4_s128_d64.npz")
    q, k, v, do = (bf16(d[n]) for n in ("q", "k", "v", "dout"))
    out, lse, _, _ = flash_attn2_rs.fwd(q, k, v, is_causal=True)
    assert np.abs(out.float().cpu().numpy() - d["out"]).max() <= 2e-2
    np.testing.assert_allclose(lse.cpu().numpy(), d["lse"], atol=1e-3, rtol=1e-4)
    dq, dk, dv, delta = flash_attn2_rs.bwd(do, q, k, v, out, lse, is_causal=True)
    for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        np.testing.assert_allclose(got.float().cpu().numpy(), d[key], err_msg=key, **GRAD_TOL)
    np.testing.assert_allclose(delta[..., :128].cpu().numpy(), d["delta"], atol=2e-2, rtol=2e-2)


def test_golden_fa_varlen():
    import flash_attn2_rs

    d = np.load(GOLDEN / "fa_varlen_causal_l37_96_75_h4_hk2_d64.npz")
    q, k, v, do = (bf16(d[n]) for n in ("q", "k", "v", "dout"))
    cu = torch.from_numpy(d["cu_seqlens"]).cuda()
    mx = int(np.diff(d["cu_seqlens"]).max())
    out, lse, _, _ = flash_attn2_rs.varlen_fwd(q, k, v, cu, cu, max_seqlen_q=mx, max_seqlen_k=mx,
                                               is_causal=True)
    assert np.abs(out.float().cpu().numpy() - d["out"]).max() <= 2e-2
    np.testing.assert_allclose(lse.cpu().numpy(), d["lse"], atol=1e-3, rtol=1e-4)
    dq, dk, dv, delta = flash_attn2_rs.varlen_bwd(do, q, k, v, out, lse, cu, cu, max_seqlen_q=mx,
                                                  max_seqlen_k=mx, is_causal=True)
    for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        np.testing.assert_allclose(got.float().cpu().numpy(), d[key], err_msg=key, **GRAD_TOL)
    # delta of the kernel's own bf16 output vs the oracle's fp32 output.
    np.testing.assert_allclose(delta.cpu().numpy(), d["delta"], atol=2e-2, rtol=2e-2)


def test_golden_rms_norm():
    import rmsnorm

    d = np.load(GOLDEN / "rms_norm_llama_16x4096.npz")
    x, w = bf16(d["x"]), bf16(d["weight"])
    y = torch.empty_like(x)
    rstd = torch.empty(x.shape[0], device="cuda")
    rmsnorm.ops.rms_norm_forward(y, rstd, x, w, G.RMS["eps"], 0.0, "llama")
    assert np.array_equal(y.float().cpu().numpy().view(np.uint32),
                          G.from_bits(d["y"]).view(np.uint32))
    assert np.array_equal(rstd.cpu().numpy().view(np.uint32), d["rstd"].view(np.uint32))


@pytest.mark.parametrize("op", ["silu_and_mul", "gelu_and_mul", "gelu_tanh_and_mul"])
def test_golden_gated(op):
    import activation_rs

    d = np.load(GOLDEN / "gated_act_32x1024.npz")
    x = bf16(d["x"])
    out = torch.empty(x.shape[0], x.shape[1] // 2, dtype=x.dtype, device="cuda")
    getattr(activation_rs.ops, op)(out, x)
    got = out.float().cpu().numpy()
    exp = G.from_bits(d[op])
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), ulp_distance_bf16(got, exp).max()
