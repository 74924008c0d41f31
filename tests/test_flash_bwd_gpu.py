"""GPU parity of the FlashAttention-2 backward (dense and varlen) against the oracle's
gradients, following flash-attn2-rs/tests/test_gold.py:236-460 and 542-569.

Bars: fp16 atol 0.008 / rtol 0.04 and bf16 atol 0.06 / rtol 0.08 (the reference
tests' backward tolerances, test_gold.py:267, 363), delta to 2e-4.
"""

import numpy as np
import pytest
import torch

from attn_cases import PARITY_CASES, make_inputs, oracle_kwargs
from oracle import attention as OA

pytestmark = pytest.mark.gpu

BWD_CASES = [c for c in PARITY_CASES if c[1][3] <= 512]


def grad_tol(dtype):
    return dict(atol=0.008, rtol=0.04) if dtype == torch.float16 else dict(atol=0.06, rtol=0.08)


def run_dense(q, k, v, dout, options, deterministic=False):
    import flash_attn2_rs

    alibi = options.get("alibi_slopes")
    kw = dict(alibi_slopes=None if alibi is None else alibi.cuda(),
              softmax_scale=options.get("softmax_scale"), is_causal=options.get("causal", False),
              window_size_left=options.get("window_left", -1),
              window_size_right=options.get("window_right", -1), softcap=options.get("softcap", 0.0))
    qd, kd, vd, dod = q.cuda(), k.cuda(), v.cuda(), dout.cuda()
    out, lse, _, _ = flash_attn2_rs.fwd(qd, kd, vd, **kw)
    dq, dk, dv, delta = flash_attn2_rs.bwd(dod, qd, kd, vd, out, lse, deterministic=deterministic, **kw)
    return out, lse, dq, dk, dv, delta


@pytest.mark.parametrize("name,shape,options", BWD_CASES, ids=[c[0] for c in BWD_CASES])
def test_backward_parity(name, shape, options):
    q, k, v, options, dtype = make_inputs(shape, options)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(1)).to(dtype)
    out, lse, dq, dk, dv, delta = run_dense(q, k, v, dout, options)
    kw = oracle_kwargs(options)
    # Gradients of the kernel's own (rounded) output, as the reference tests do.
    edq, edk, edv, edelta = OA.backward(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                        out.float().cpu().numpy(), dout.float().numpy(),
                                        lse.cpu().numpy(), **kw)
    tol = grad_tol(dtype)
    for got, exp in ((dq, edq), (dk, edk), (dv, edv)):
        got = got.float().cpu().numpy()
        assert np.isfinite(got).all()
        np.testing.assert_allclose(got, exp, **tol)
    sq = q.shape[1]
    np.testing.assert_allclose(delta[..., :sq].cpu().numpy(), edelta, atol=2e-4, rtol=2e-4)
    assert (delta[..., sq:] == 0).all()


def test_deterministic_matches_default_bitwise():
    q, k, v, options, dtype = make_inputs((2, 8, 2, 300, 300), {"causal": True})
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(1)).to(dtype)
    a = run_dense(q, k, v, dout, options, deterministic=True)
    b = run_dense(q, k, v, dout, options, deterministic=False)
    for x, y in zip(a[2:5], b[2:5]):
        assert torch.equal(x, y)


@pytest.mark.parametrize("sq,sk,causal", [(33, 257, False), (513, 33, False), (257, 513, True),
                                          (1024, 1024, True)])
def test_backward_shapes(sq, sk, causal):
    """test_gold.py:338-364 shapes (no dropout), GQA 8:2."""
    g = torch.Generator().manual_seed(0)
    q = torch.randn(2, sq, 8, 128, generator=g).half()
    k = torch.randn(2, sk, 2, 128, generator=g).half()
    v = torch.randn(2, sk, 2, 128, generator=g).half()
    dout = torch.randn(2, sq, 8, 128, generator=g).half()
    out, lse, dq, dk, dv, _ = run_dense(q, k, v, dout, {"causal": causal})
    edq, edk, edv, _ = OA.backward(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                   out.float().cpu().numpy(), dout.float().numpy(), lse.cpu().numpy(),
                                   causal=causal)
    for got, exp in ((dq, edq), (dk, edk), (dv, edv)):
        np.testing.assert_allclose(got.float().cpu().numpy(), exp, atol=0.008, rtol=0.04)


def test_autograd_flash_attn_func_head_padding():
    """test_gold.py:367-425 without dropout: head size 63 is padded to 64."""
    import flash_attn2_rs

    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, 17, 4, 63, generator=g).half()
    k = torch.randn(1, 23, 2, 63, generator=g).half()
    v = torch.randn(1, 23, 2, 63, generator=g).half()
    qd, kd, vd = (x.cuda().requires_grad_() for x in (q, k, v))
    out = flash_attn2_rs.flash_attn_func(qd, kd, vd, causal=True)
    out.sum().backward()
    eo, el = OA.forward(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal=True)
    np.testing.assert_allclose(out.detach().float().cpu().numpy(), eo, atol=0.005, rtol=0.03)
    edq, edk, edv, _ = OA.backward(q.float().numpy(), k.float().numpy(), v.float().numpy(), eo,
                                   np.ones_like(eo), el, causal=True)
    for got, exp in ((qd.grad, edq), (kd.grad, edk), (vd.grad, edv)):
        np.testing.assert_allclose(got.float().cpu().numpy(), exp, atol=0.008, rtol=0.04)


@pytest.mark.parametrize("packing", ["qkv", "kv"])
def test_autograd_packed(packing):
    import flash_attn2_rs

    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, 40, 4, 64, generator=g).half().cuda()
    k = torch.randn(1, 40, 4, 64, generator=g).half().cuda()
    v = torch.randn(1, 40, 4, 64, generator=g).half().cuda()
    ref_in = [x.clone().requires_grad_() for x in (q, k, v)]
    ref = flash_attn2_rs.flash_attn_func(*ref_in, causal=True)
    ref.sum().backward()
    if packing == "qkv":
        qkv = torch.stack((q, k, v), 2).requires_grad_()
        out = flash_attn2_rs.flash_attn_qkvpacked_func(qkv, causal=True)
        out.sum().backward()
        grads = qkv.grad.unbind(2)
    else:
        qq = q.clone().requires_grad_()
        kv = torch.stack((k, v), 2).requires_grad_()
        out = flash_attn2_rs.flash_attn_kvpacked_func(qq, kv, causal=True)
        out.sum().backward()
        grads = (qq.grad, *kv.grad.unbind(2))
    torch.testing.assert_close(out, ref, atol=0, rtol=0)
    for a, b in zip(grads, (x.grad for x in ref_in)):
        torch.testing.assert_close(a, b, atol=0, rtol=0)


def test_varlen_forward_backward():
    """test_gold.py:542-569 without dropout: three sequences incl. an empty one, GQA."""
    import flash_attn2_rs

    g = torch.Generator().manual_seed(0)
    q = torch.randn(25, 4, 64, generator=g).half()
    k = torch.randn(31, 2, 64, generator=g).half()
    v = torch.randn(31, 2, 64, generator=g).half()
    cu_q = torch.tensor([0, 17, 17, 25], dtype=torch.int32)
    cu_k = torch.tensor([0, 19, 19, 31], dtype=torch.int32)
    opts = dict(max_seqlen_q=17, max_seqlen_k=19, is_causal=True, zero_tensors=True)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    out, lse, _, _ = flash_attn2_rs.varlen_fwd(qd, kd, vd, cu_q.cuda(), cu_k.cuda(), **opts)
    dout = torch.ones_like(qd)
    dq, dk, dv, delta = flash_attn2_rs.varlen_bwd(dout, qd, kd, vd, out, lse, cu_q.cuda(), cu_k.cuda(), **opts)
    assert delta.shape == (4, 25 + 128 * 3)
    edq, edk, edv, edelta = OA.varlen_backward(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                               out.float().cpu().numpy(), dout.float().cpu().numpy(),
                                               lse.cpu().numpy(), cu_q.numpy(), cu_k.numpy(), causal=True)
    np.testing.assert_allclose(delta.cpu().numpy(), edelta, atol=2e-4, rtol=2e-5)
    for got, exp in ((dq, edq), (dk, edk), (dv, edv)):
        np.testing.assert_allclose(got.float().cpu().numpy(), exp, atol=0.008, rtol=0.04)


def test_varlen_autograd_matches_dense_per_sequence():
    import flash_attn2_rs

    g = torch.Generator().manual_seed(0)
    lens = [100, 257, 64]
    cu = torch.tensor(np.cumsum([0] + lens), dtype=torch.int32).cuda()
    q = torch.randn(sum(lens), 8, 128, generator=g).bfloat16().cuda().requires_grad_()
    k = torch.randn(sum(lens), 2, 128, generator=g).bfloat16().cuda().requires_grad_()
    v = torch.randn(sum(lens), 2, 128, generator=g).bfloat16().cuda().requires_grad_()
    out = flash_attn2_rs.flash_attn_varlen_func(q, k, v, cu, cu, max(lens), max(lens), causal=True)
    out.float().square().sum().backward()
    for i in range(3):
        a, b = int(cu[i]), int(cu[i + 1])
        qs, ks, vs = (x.detach()[a:b][None].clone().requires_grad_() for x in (q, k, v))
        o = flash_attn2_rs.flash_attn_func(qs, ks, vs, causal=True)
        o.float().square().sum().backward()
        torch.testing.assert_close(out[a:b], o[0], atol=0, rtol=0)
        torch.testing.assert_close(q.grad[a:b], qs.grad[0], atol=2e-2, rtol=2e-2)
        torch.testing.assert_close(k.grad[a:b], ks.grad[0], atol=2e-2, rtol=2e-2)


def test_baseline_config_backward_subset():
    """BASELINE config 4 shape, causal bf16: full launch; dK/dV of one KV head and dQ
    of its 4 query heads (batch 1) checked against the oracle."""
    import flash_attn2_rs

    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 4096, 32, 128, generator=g).bfloat16()
    k = torch.randn(2, 4096, 8, 128, generator=g).bfloat16()
    v = torch.randn(2, 4096, 8, 128, generator=g).bfloat16()
    dout = torch.randn(2, 4096, 32, 128, generator=g).bfloat16()
    out, lse, dq, dk, dv, _ = run_dense(q, k, v, dout, {"causal": True})
    b, grp = 1, 6
    sl = slice(4 * grp, 4 * grp + 4)
    edq, edk, edv, _ = OA.backward(q[b:b + 1, :, sl].float().numpy(), k[b:b + 1, :, grp:grp + 1].float().numpy(),
                                   v[b:b + 1, :, grp:grp + 1].float().numpy(),
                                   out[b:b + 1, :, sl].float().cpu().numpy(), dout[b:b + 1, :, sl].float().numpy(),
                                   lse[b:b + 1, sl].cpu().numpy(), causal=True)
    np.testing.assert_allclose(dq[b:b + 1, :, sl].float().cpu().numpy(), edq, atol=0.06, rtol=0.08)
    np.testing.assert_allclose(dk[b:b + 1, :, grp:grp + 1].float().cpu().numpy(), edk, atol=0.06, rtol=0.08)
    np.testing.assert_allclose(dv[b:b + 1, :, grp:grp + 1].float().cpu().numpy(), edv, atol=0.06, rtol=0.08)


def test_varlen_baseline_config_backward():
    """BASELINE config 5 backward: 16 sequences with lengths ~U[128, 8192] (seed 5),
    Hq=32, Hkv=8, D=128, causal bf16, dO ~N(0,1): the whole varlen_fwd +
    varlen_bwd launch; dQ of query heads 8-11 and dK/dV of their KV head 2
    (the complete GQA sum of that group) for sequences 0, 7 and 15 against the
    oracle's gradients, at the reference's bf16 backward tolerance
    (test_gold.py:267), and the delta rows of those sequences."""
    import flash_attn2_rs

    lens = torch.randint(128, 8193, (16,), generator=torch.Generator().manual_seed(5)).tolist()
    cu = torch.tensor(np.cumsum([0] + lens), dtype=torch.int32)
    total = int(cu[-1])
    g = torch.Generator().manual_seed(6)
    q = torch.randn(total, 32, 128, generator=g).bfloat16()
    k = torch.randn(total, 8, 128, generator=g).bfloat16()
    v = torch.randn(total, 8, 128, generator=g).bfloat16()
    dout = torch.randn(total, 32, 128, generator=g).bfloat16()
    ops = flash_attn2_rs.ops
    qd, kd, vd, dod, cud = q.cuda(), k.cuda(), v.cuda(), dout.cuda(), cu.cuda()
    mx = max(lens)
    out, lse, _ = ops.varlen_fwd_explicit(qd, kd, vd, cud, cud, None, None, None, None, True, -1, -1,
                                          0.0, 0.0, None, mx, mx, False, False)
    dq, dk, dv, delta = ops.varlen_bwd_explicit(qd, kd, vd, dod, out, lse, cud, cud, None, None, True,
                                                -1, -1, 0.0, 0.0, None, mx, mx, False)
    for t in (dq, dk, dv):
        assert torch.isfinite(t).all()
    hs, grp = slice(8, 12), 2
    for s in (0, 7, 15):
        a, b = int(cu[s]), int(cu[s + 1])
        edq, edk, edv, edelta = OA.backward(
            q[None, a:b, hs].float().numpy(), k[None, a:b, grp:grp + 1].float().numpy(),
            v[None, a:b, grp:grp + 1].float().numpy(), out[a:b, hs][None].float().cpu().numpy(),
            dout[None, a:b, hs].float().numpy(), lse[hs, a:b][None].cpu().numpy(), causal=True)
        np.testing.assert_allclose(dq[a:b, hs].float().cpu().numpy(), edq[0], atol=0.06, rtol=0.08)
        np.testing.assert_allclose(dk[a:b, grp].float().cpu().numpy(), edk[0, :, 0], atol=0.06, rtol=0.08)
        np.testing.assert_allclose(dv[a:b, grp].float().cpu().numpy(), edv[0, :, 0], atol=0.06, rtol=0.08)
        # delta [H, Tq + 128 B]: row qs + 128 b of sequence b (host/varlen/backward.rs:173-178)
        np.testing.assert_allclose(delta[hs, a + 128 * s:b + 128 * s].cpu().numpy(), edelta[0],
                                   atol=2e-3, rtol=2e-4)
        print(f"config 5 seq {s} (L={b - a}): max |dq err| "
              f"{np.abs(dq[a:b, hs].float().cpu().numpy() - edq[0]).max():.3g}, "
              f"|dk err| {np.abs(dk[a:b, grp].float().cpu().numpy() - edk[0, :, 0]).max():.3g}, "
              f"|dv err| {np.abs(dv[a:b, grp].float().cpu().numpy() - edv[0, :, 0]).max():.3g}")


@pytest.mark.parametrize("d", [64, 128, 48, 96, 192, 256])
@pytest.mark.parametrize("mode", ["plain", "alibi", "softcap", "both"])
def test_varlen_scored_forward_backward(mode, d):
    """Packed sequences (one empty, ragged lengths) with [B, H] ALiBi slopes and / or
    softcap: the tiled forward's and v2 backward's scored instances against the
    oracle, at the fp16 tolerances of the dense tests. Head sizes 48 and 96 run
    the backward through zero-padded copies; 192 and 256 the general kernels'
    separate dV and dK passes."""
    import flash_attn2_rs

    g = torch.Generator().manual_seed(31 + d)
    lens_q, lens_k = [70, 0, 129, 33], [90, 5, 129, 200]
    cu_q = torch.tensor(np.cumsum([0] + lens_q), dtype=torch.int32)
    cu_k = torch.tensor(np.cumsum([0] + lens_k), dtype=torch.int32)
    h, hk = 4, 2
    q = torch.randn(sum(lens_q), h, d, generator=g).half()
    k = torch.randn(sum(lens_k), hk, d, generator=g).half()
    v = torch.randn(sum(lens_k), hk, d, generator=g).half()
    dout = torch.randn(sum(lens_q), h, d, generator=g).half()
    slopes = (torch.rand(4, h, generator=g) * 0.2).float() if mode in ("alibi", "both") else None
    cap = 20.0 if mode in ("softcap", "both") else 0.0
    print(f"varlen scored mode={mode} d={d}", flush=True)
    opts = dict(max_seqlen_q=max(lens_q), max_seqlen_k=max(lens_k), is_causal=True, softcap=cap,
                alibi_slopes=None if slopes is None else slopes.cuda())
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    out, lse, _, _ = flash_attn2_rs.varlen_fwd(qd, kd, vd, cu_q.cuda(), cu_k.cuda(), **opts)
    dq, dk, dv, _ = flash_attn2_rs.varlen_bwd(dout.cuda(), qd, kd, vd, out, lse, cu_q.cuda(), cu_k.cuda(), **opts)
    kw = dict(causal=True, softcap=cap, alibi_slopes=None if slopes is None else slopes.numpy())
    eo, el = OA.varlen_forward(q.float().numpy(), k.float().numpy(), v.float().numpy(), cu_q.numpy(),
                               cu_k.numpy(), **kw)
    assert np.abs(out.float().cpu().numpy() - eo).max() <= 2e-2
    np.testing.assert_allclose(lse.cpu().numpy(), el, atol=1e-3, rtol=1e-4)
    edq, edk, edv, _ = OA.varlen_backward(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                          out.float().cpu().numpy(), dout.float().numpy(), lse.cpu().numpy(),
                                          cu_q.numpy(), cu_k.numpy(), **kw)
    for got, exp in ((dq, edq), (dk, edk), (dv, edv)):
        np.testing.assert_allclose(got.float().cpu().numpy(), exp, atol=0.008, rtol=0.04)
