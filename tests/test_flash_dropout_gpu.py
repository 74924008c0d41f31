"""GPU parity of FlashAttention-2 dropout against the oracle's Philox4x32-7 mask
stream (oracle/dropout.py, flash-attn2-rs/src/device/dropout.rs).

The mask itself is checked bit for bit with a readout: Q = 0 makes every visible
key equally likely, and V (or dO) = identity turns the output (or dV) into the
mask divided by the number of keys and the keep probability. The values are
then checked against the oracle's dropped forward / backward at the non-dropout
tolerances (max-abs 2e-2 for the output, the reference's backward tolerance for
the gradients).
"""

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import dropout as DR

pytestmark = pytest.mark.gpu

GRAD_TOL = {torch.float16: dict(atol=0.008, rtol=0.04), torch.bfloat16: dict(atol=0.06, rtol=0.08)}


def ops():
    import flash_attn2_rs

    return flash_attn2_rs.ops


def state_tensor(seed, offset):
    return torch.tensor([seed, offset], dtype=torch.int64, device="cuda")


@pytest.mark.parametrize("d", [64, 128, 96])
@pytest.mark.parametrize("p", [0.17, 0.5])
def test_forward_mask_readout_dense(d, p):
    b, h, s = 2, 3, d if d <= 128 else 128
    q = torch.zeros(b, s, h, d, dtype=torch.bfloat16, device="cuda")
    k = torch.randn(b, s, h, d, generator=torch.Generator().manual_seed(1)).bfloat16().cuda()
    eye = torch.eye(s, d)
    v = eye[None, :, None, :].expand(b, s, h, d).contiguous().bfloat16().cuda()
    out = torch.empty_like(q)
    seed, offset = 0x1234_5678_9ABC, 96
    ops().fwd_lse(q, k, v, None, None, False, -1, -1, 0.0, p, seed, offset, out)
    keep = float(np.float32(1) - np.float32(p))
    got = out.float().cpu().numpy()  # [B, S, H, D]: O[b, q, h, key] = mask / (s * keep)
    mask = DR.dense_mask(seed, offset, b, h, s, s, p)
    readout = np.transpose(got[..., :s], (0, 2, 1, 3)) > 0.5 / (s * keep)
    assert np.array_equal(readout, mask)
    np.testing.assert_allclose(np.transpose(got[..., :s], (0, 2, 1, 3)), mask / (s * keep), rtol=1e-2)


def test_forward_mask_readout_varlen():
    lens = [37, 128, 75]
    h, d = 2, 128
    total = sum(lens)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32, device="cuda")
    q = torch.zeros(total, h, d, dtype=torch.bfloat16, device="cuda")
    k = torch.randn(total, h, d, generator=torch.Generator().manual_seed(2)).bfloat16().cuda()
    v = torch.cat([torch.eye(n, d)[:, None, :].expand(n, h, d) for n in lens]).contiguous().bfloat16().cuda()
    p = 0.3
    state = state_tensor(987654321, 32)
    out, lse, _ = ops().varlen_fwd_explicit(q, k, v, cu, cu, None, None, None, None, False, -1, -1, 0.0,
                                            p, state, max(lens), max(lens), False, False)
    keep = float(np.float32(1) - np.float32(p))
    got = out.float().cpu().numpy()
    for bi, (s0, n) in enumerate(zip(np.cumsum([0] + lens[:-1]), lens)):
        for hi in range(h):
            mask = DR.keep_mask(987654321, 32, bi * h + hi, n, n, p)
            assert np.array_equal(got[s0:s0 + n, hi, :n] > 0.5 / (n * keep), mask)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal,d,alibi", [(True, 128, False), (False, 64, False), (True, 96, False),
                                            (True, 128, True), (True, 256, False), (False, 192, True)])
def test_forward_backward_parity_dense(dtype, causal, d, alibi):
    import flash_attn2_rs

    b, h, hk, s = 2, 4, 2, 200
    g = torch.Generator().manual_seed(3)
    q = torch.randn(b, s, h, d, generator=g).to(dtype)
    k = torch.randn(b, s, hk, d, generator=g).to(dtype)
    v = torch.randn(b, s, hk, d, generator=g).to(dtype)
    dout = torch.randn(b, s, h, d, generator=g).to(dtype)
    slopes = (2.0 ** (-8.0 * (torch.arange(h) + 1) / h)).float() if alibi else None
    p = 0.2
    state = state_tensor(2024, 64)
    qd, kd, vd, dod = q.cuda(), k.cuda(), v.cuda(), dout.cuda()
    out = torch.empty_like(qd)
    lse = flash_attn2_rs.ops.fwd_lse(qd, kd, vd, None if slopes is None else slopes.cuda(), None, causal,
                                     -1, -1, 0.0, p, state, 0, out)
    mask = DR.dense_mask(2024, 64, b, h, s, s, p)
    kw = dict(causal=causal, dropout_mask=mask, p_dropout=p)
    if alibi:
        kw["alibi_slopes"] = slopes.numpy()
    eo, el = OA.forward(q.float().numpy(), k.float().numpy(), v.float().numpy(), **kw)
    assert np.abs(out.float().cpu().numpy() - eo).max() <= 2e-2
    np.testing.assert_allclose(lse.cpu().numpy(), el, atol=1e-3, rtol=1e-4)
    dq, dk, dv, delta = flash_attn2_rs.bwd(dod, qd, kd, vd, out, lse, p_dropout=p, is_causal=causal,
                                           alibi_slopes=None if slopes is None else slopes.cuda(),
                                           rng_state=state)
    edq, edk, edv, edelta = OA.backward(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                        out.float().cpu().numpy(), dout.float().numpy(), lse.cpu().numpy(),
                                        **kw)
    for got, exp in ((dq, edq), (dk, edk), (dv, edv)):
        np.testing.assert_allclose(got.float().cpu().numpy(), exp, **GRAD_TOL[dtype])
    np.testing.assert_allclose(delta[..., :s].cpu().numpy(), edelta, atol=2e-4, rtol=2e-4)


def test_backward_dv_mask_readout():
    """dV = (P * M / keep)^T dO with Q = 0 and dO = identity reads the mask out of
    the dK/dV kernel."""
    import flash_attn2_rs

    b, h, s, d = 1, 2, 128, 128
    q = torch.zeros(b, s, h, d, dtype=torch.bfloat16, device="cuda")
    k = torch.randn(b, s, h, d, generator=torch.Generator().manual_seed(4)).bfloat16().cuda()
    v = torch.randn(b, s, h, d, generator=torch.Generator().manual_seed(5)).bfloat16().cuda()
    dout = torch.eye(s, d)[None, :, None, :].expand(b, s, h, d).contiguous().bfloat16().cuda()
    p = 0.4
    state = state_tensor(55, 0)
    out = torch.empty_like(q)
    lse = flash_attn2_rs.ops.fwd_lse(q, k, v, None, None, False, -1, -1, 0.0, p, state, 0, out)
    _, _, dv, _ = flash_attn2_rs.bwd(dout, q, k, v, out, lse, p_dropout=p, rng_state=state)
    keep = float(np.float32(1) - np.float32(p))
    got = dv.float().cpu().numpy()  # dV[b, key, h, query] = mask[query, key] / (s * keep)
    mask = DR.dense_mask(55, 0, b, h, s, s, p)
    assert np.array_equal(np.transpose(got, (0, 2, 3, 1)) > 0.5 / (s * keep), mask)


def test_varlen_dropout_parity():
    import flash_attn2_rs

    lens = [150, 64, 97]
    h, hk, d = 4, 2, 128
    total = sum(lens)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32, device="cuda")
    g = torch.Generator().manual_seed(6)
    q, dout = (torch.randn(total, h, d, generator=g).bfloat16() for _ in range(2))
    k, v = (torch.randn(total, hk, d, generator=g).bfloat16() for _ in range(2))
    p = 0.25
    state = state_tensor(77, 128)
    out, lse, _ = flash_attn2_rs.ops.varlen_fwd_explicit(
        q.cuda(), k.cuda(), v.cuda(), cu, cu, None, None, None, None, True, -1, -1, 0.0, p, state,
        max(lens), max(lens), False, False)
    cun = cu.cpu().numpy()
    eo, el = OA.varlen_forward(q.float().numpy(), k.float().numpy(), v.float().numpy(), cun, cun,
                               causal=True, dropout=(77, 128, p))
    assert np.abs(out.float().cpu().numpy() - eo).max() <= 2e-2
    dq, dk, dv, delta = flash_attn2_rs.varlen_bwd(dout.cuda(), q.cuda(), k.cuda(), v.cuda(), out, lse, cu, cu,
                                                  max_seqlen_q=max(lens), max_seqlen_k=max(lens),
                                                  p_dropout=p, is_causal=True, rng_state=state)
    edq, edk, edv, _ = OA.varlen_backward(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                          out.float().cpu().numpy(), dout.float().numpy(), lse.cpu().numpy(),
                                          cun, cun, causal=True, dropout=(77, 128, p))
    for got, exp in ((dq, edq), (dk, edk), (dv, edv)):
        np.testing.assert_allclose(got.float().cpu().numpy(), exp, **GRAD_TOL[torch.bfloat16])


def test_state_tensor_equals_explicit_seed_and_is_repeatable():
    b, h, s, d = 1, 4, 256, 128
    g = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(b, s, h, d, generator=g).bfloat16().cuda() for _ in range(3))
    o1, o2, o3 = (torch.empty_like(q) for _ in range(3))
    ops().fwd_lse(q, k, v, None, None, True, -1, -1, 0.0, 0.1, 42, 7, o1)
    ops().fwd_lse(q, k, v, None, None, True, -1, -1, 0.0, 0.1, state_tensor(42, 7), 0, o2)
    ops().fwd_lse(q, k, v, None, None, True, -1, -1, 0.0, 0.1, 42, 7, o3)
    assert torch.equal(o1, o2) and torch.equal(o1, o3)
    o4 = torch.empty_like(q)
    ops().fwd_lse(q, k, v, None, None, True, -1, -1, 0.0, 0.1, 42, 8, o4)
    assert not torch.equal(o1, o4)


def test_flash_attn_func_dropout_autograd_reproducible():
    from flash_attn2_rs import flash_attn_func

    g = torch.Generator().manual_seed(8)
    q, k, v = (torch.randn(2, 128, 4, 64, generator=g).bfloat16().cuda().requires_grad_() for _ in range(3))
    torch.manual_seed(123)
    o1 = flash_attn_func(q, k, v, dropout_p=0.3, causal=True)
    o1.sum().backward()
    g1 = [t.grad.clone() for t in (q, k, v)]
    for t in (q, k, v):
        t.grad = None
    torch.manual_seed(123)
    o2 = flash_attn_func(q, k, v, dropout_p=0.3, causal=True)
    o2.sum().backward()
    assert torch.equal(o1, o2)
    assert all(torch.equal(a, t.grad) for a, t in zip(g1, (q, k, v)))
    o0 = flash_attn_func(q, k, v, dropout_p=0.0, causal=True)
    assert not torch.equal(o0, o1)


def test_dropout_argument_errors():
    q = torch.randn(1, 16, 2, 64, device="cuda").bfloat16()
    out = torch.empty_like(q)
    with pytest.raises(ValueError, match="p_dropout must be finite"):
        ops().fwd_lse(q, q, q, None, None, False, -1, -1, 0.0, 1.0, 1, 0, out)
    with pytest.raises(ValueError, match="softcap with dropout"):
        ops().fwd_lse(q, q, q, None, None, False, -1, -1, 30.0, 0.1, 1, 0, out)
    with pytest.raises(ValueError, match="offset must be zero"):
        ops().fwd_lse(q, q, q, None, None, False, -1, -1, 0.0, 0.1, state_tensor(1, 0), 3, out)
    with pytest.raises(ValueError, match="rng_state must be a contiguous"):
        ops().fwd_lse(q, q, q, None, None, False, -1, -1, 0.0, 0.1,
                      torch.zeros(3, dtype=torch.int64, device="cuda"), 0, out)
