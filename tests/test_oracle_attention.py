"""Pins oracle/attention.py (forward, varlen, backward) against torch CPU library
routines, autograd, finite differences and closed forms."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as OA


def rnd(*shape, seed=0):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def sdpa(q, k, v, causal, scale=None):
    """torch's SDPA on [B,S,H,D] (GQA expanded); causal is top-left aligned, equal to
    FlashAttention's bottom-right alignment when Sq == Sk."""
    g = q.shape[2] // k.shape[2]
    qt = torch.from_numpy(q).double().transpose(1, 2)
    kt = torch.from_numpy(k).double().transpose(1, 2).repeat_interleave(g, 1)
    vt = torch.from_numpy(v).double().transpose(1, 2).repeat_interleave(g, 1)
    o = F.scaled_dot_product_attention(qt, kt, vt, is_causal=causal, scale=scale)
    s = (qt @ kt.transpose(-1, -2)) * (scale if scale is not None else q.shape[-1] ** -0.5)
    if causal:
        s = s.masked_fill(torch.ones_like(s, dtype=torch.bool).triu(1), float("-inf"))
    return o.transpose(1, 2).numpy(), torch.logsumexp(s, -1).numpy()


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("hq,hk", [(4, 4), (8, 2), (4, 1)])
def test_forward_vs_torch_sdpa(causal, hq, hk):
    q, k, v = rnd(2, 97, hq, 64, seed=1), rnd(2, 97, hk, 64, seed=2), rnd(2, 97, hk, 64, seed=3)
    out, lse = OA.forward(q, k, v, causal=causal, dtype=np.float64)
    eo, el = sdpa(q, k, v, causal)
    np.testing.assert_allclose(out, eo, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(lse, el, rtol=1e-10, atol=1e-10)


def test_custom_scale_vs_torch():
    q, k, v = rnd(1, 33, 2, 32, seed=4), rnd(1, 33, 2, 32, seed=5), rnd(1, 33, 2, 32, seed=6)
    out, lse = OA.forward(q, k, v, softmax_scale=0.05, dtype=np.float64)
    eo, el = sdpa(q, k, v, False, scale=0.05)
    np.testing.assert_allclose(out, eo, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(lse, el, rtol=1e-10, atol=1e-10)


def test_bottom_right_causal_alignment():
    # Sq < Sk: row i sees keys 0..i + Sk - Sq (test_fwd.py:64-76). Row 0 of the last
    # query equals full attention of that query over all keys.
    q, k, v = rnd(1, 5, 1, 16, seed=7), rnd(1, 9, 1, 16, seed=8), rnd(1, 9, 1, 16, seed=9)
    out, _ = OA.forward(q, k, v, causal=True, dtype=np.float64)
    full, _ = OA.forward(q[:, -1:], k, v, dtype=np.float64)
    np.testing.assert_allclose(out[:, -1:], full, rtol=1e-12)
    first, _ = OA.forward(q[:, :1], k[:, :5], v[:, :5], dtype=np.float64)
    np.testing.assert_allclose(out[:, :1], first, rtol=1e-12)
    # Sq > Sk: the first Sq - Sk rows see no key: O = 0, LSE = +inf.
    out, lse = OA.forward(rnd(1, 7, 1, 16), k[:, :4], v[:, :4], causal=True)
    assert np.all(out[:, :3] == 0) and np.all(np.isposinf(lse[..., :3]))
    assert np.all(np.isfinite(lse[..., 3:]))


def test_closed_forms():
    q, k, v = rnd(2, 11, 4, 32, seed=1), rnd(2, 1, 2, 32, seed=2), rnd(2, 1, 2, 32, seed=3)
    out, _ = OA.forward(q, k, v)
    np.testing.assert_array_equal(out, np.repeat(v, 11, axis=1).repeat(2, axis=2))  # Sk = 1
    v_const = np.broadcast_to(rnd(1, 1, 1, 32, seed=4), (1, 13, 1, 32)).copy()
    out, _ = OA.forward(rnd(1, 13, 1, 32, seed=5), rnd(1, 13, 1, 32, seed=6), v_const, causal=True)
    np.testing.assert_allclose(out, np.broadcast_to(v_const[:, :1], out.shape), rtol=1e-6)
    # Zero queries: uniform weights, LSE = log(number of visible keys).
    _, lse = OA.forward(np.zeros((1, 6, 1, 8), np.float32), rnd(1, 6, 1, 8), rnd(1, 6, 1, 8), causal=True)
    np.testing.assert_allclose(lse[0, 0], np.log(np.arange(1, 7)), rtol=1e-6)
    # Empty keys: O = 0, LSE = +inf (test_gold.py:136-146).
    out, lse = OA.forward(rnd(1, 3, 2, 8), np.zeros((1, 0, 2, 8), np.float32), np.zeros((1, 0, 2, 8), np.float32))
    assert np.all(out == 0) and np.all(np.isposinf(lse))


def test_windows_match_explicit_masks():
    q, k, v = rnd(1, 40, 2, 16, seed=1), rnd(1, 40, 2, 16, seed=2), rnd(1, 40, 2, 16, seed=3)
    out, _ = OA.forward(q, k, v, window_left=5, window_right=3, dtype=np.float64)
    for i in (0, 7, 39):
        lo, hi = max(0, i - 5), min(40, i + 4)
        exp, _ = OA.forward(q[:, i:i + 1], k[:, lo:hi], v[:, lo:hi], dtype=np.float64)
        np.testing.assert_allclose(out[:, i:i + 1], exp, rtol=1e-12)


def test_softcap_and_alibi_against_direct_formula():
    q, k, v = rnd(1, 16, 2, 8, seed=1), rnd(1, 16, 2, 8, seed=2), rnd(1, 16, 2, 8, seed=3)
    slopes = np.float64([0.5, 0.25])
    out, lse = OA.forward(q, k, v, softcap=3.0, alibi_slopes=slopes, dtype=np.float64)
    for h in range(2):
        raw = q[0, :, h].astype(np.float64) @ k[0, :, h].astype(np.float64).T
        s = 3.0 * np.tanh(raw / math.sqrt(8) / 3.0)
        s -= slopes[h] * np.abs(np.arange(16)[:, None] - np.arange(16)[None, :])
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        np.testing.assert_allclose(out[0, :, h], p @ v[0, :, h], rtol=1e-12)
        np.testing.assert_allclose(lse[0, h], np.log(np.exp(s).sum(1)), rtol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("softcap", [0.0, 2.0])
def test_backward_vs_torch_autograd(causal, softcap):
    hq, hk = 4, 2
    q, k, v = rnd(2, 23, hq, 16, seed=1), rnd(2, 23, hk, 16, seed=2), rnd(2, 23, hk, 16, seed=3)
    dout = rnd(2, 23, hq, 16, seed=4)
    out, lse = OA.forward(q, k, v, causal=causal, softcap=softcap, dtype=np.float64)
    dq, dk, dv, delta = OA.backward(q, k, v, out, dout, lse, causal=causal, softcap=softcap,
                                    dtype=np.float64)
    qt, kt, vt = (torch.from_numpy(x).double().requires_grad_() for x in (q, k, v))
    s = torch.einsum("bqhd,bkhd->bhqk", qt, kt.repeat_interleave(2, 2)) / 4.0
    if softcap:
        s = softcap * torch.tanh(s / softcap)
    if causal:
        s = s.masked_fill(torch.ones(23, 23, dtype=torch.bool).triu(1), float("-inf"))
    o = torch.einsum("bhqk,bkhd->bqhd", s.softmax(-1), vt.repeat_interleave(2, 2))
    o.backward(torch.from_numpy(dout).double())
    np.testing.assert_allclose(out, o.detach().numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dq, qt.grad.numpy(), rtol=1e-8, atol=1e-10)
    np.testing.assert_allclose(dk, kt.grad.numpy(), rtol=1e-8, atol=1e-10)
    np.testing.assert_allclose(dv, vt.grad.numpy(), rtol=1e-8, atol=1e-10)
    np.testing.assert_allclose(delta, np.sum(dout * out, -1).transpose(0, 2, 1), rtol=1e-10)


def test_backward_finite_differences():
    q, k, v = rnd(1, 5, 1, 4, seed=1), rnd(1, 6, 1, 4, seed=2), rnd(1, 6, 1, 4, seed=3)
    dout = rnd(1, 5, 1, 4, seed=4)
    kw = dict(causal=True, window_left=3, dtype=np.float64)
    out, lse = OA.forward(q, k, v, **kw)
    dq, dk, _, _ = OA.backward(q, k, v, out, dout, lse, **kw)
    eps = 1e-6
    for arr, grad in ((q, dq), (k, dk)):
        idx = (0, 2, 0, 1)
        plus, minus = arr.astype(np.float64).copy(), arr.astype(np.float64).copy()
        plus[idx] += eps
        minus[idx] -= eps
        args_p = (plus, k, v) if arr is q else (q, plus, v)
        args_m = (minus, k, v) if arr is q else (q, minus, v)
        fp = np.sum(OA.forward(*args_p, **kw)[0] * dout)
        fm = np.sum(OA.forward(*args_m, **kw)[0] * dout)
        assert abs((fp - fm) / (2 * eps) - grad[idx]) < 1e-6


def test_varlen_equals_per_sequence_dense():
    lens_q, lens_k = [17, 0, 8], [19, 0, 12]
    cu_q, cu_k = np.cumsum([0] + lens_q), np.cumsum([0] + lens_k)
    q, k, v = rnd(25, 4, 16, seed=1), rnd(31, 2, 16, seed=2), rnd(31, 2, 16, seed=3)
    out, lse = OA.varlen_forward(q, k, v, cu_q, cu_k, causal=True)
    for (qs, qe), (ks, ke) in zip(zip(cu_q[:-1], cu_q[1:]), zip(cu_k[:-1], cu_k[1:])):
        if qe == qs:
            continue
        o, l = OA.forward(q[None, qs:qe], k[None, ks:ke], v[None, ks:ke], causal=True)
        np.testing.assert_allclose(out[qs:qe], o[0], rtol=1e-6)
        np.testing.assert_allclose(lse[:, qs:qe], l[0], rtol=1e-6)
    dout = rnd(25, 4, 16, seed=4)
    dq, dk, dv, delta = OA.varlen_backward(q, k, v, out, dout, lse, cu_q, cu_k, causal=True)
    assert delta.shape == (4, 25 + 128 * 3)  # test_gold.py:531
    np.testing.assert_allclose(delta[:, 17 + 256: 25 + 256], np.sum(dout[17:] * out[17:], -1).T, rtol=1e-5)
    assert np.all(delta[:, 17:17 + 256] == 0)


def test_varlen_backward_per_sequence_alibi_and_softcap():
    """[B, H] ALiBi slopes select row b for sequence b in the packed backward, as
    in the packed forward, with softcap on top."""
    lens_q, lens_k = [17, 0, 8], [19, 0, 12]
    cu_q, cu_k = np.cumsum([0] + lens_q), np.cumsum([0] + lens_k)
    q, k, v = rnd(25, 4, 16, seed=5), rnd(31, 2, 16, seed=6), rnd(31, 2, 16, seed=7)
    slopes = np.abs(rnd(3, 4, seed=8)) * 0.1
    kw = dict(causal=True, softcap=5.0, alibi_slopes=slopes)
    out, lse = OA.varlen_forward(q, k, v, cu_q, cu_k, **kw)
    dout = rnd(25, 4, 16, seed=9)
    dq, dk, dv, _ = OA.varlen_backward(q, k, v, out, dout, lse, cu_q, cu_k, **kw)
    for b, ((qs, qe), (ks, ke)) in enumerate(zip(zip(cu_q[:-1], cu_q[1:]), zip(cu_k[:-1], cu_k[1:]))):
        if qe == qs:
            continue
        one = dict(causal=True, softcap=5.0, alibi_slopes=slopes[b])
        o, l = OA.forward(q[None, qs:qe], k[None, ks:ke], v[None, ks:ke], **one)
        np.testing.assert_allclose(out[qs:qe], o[0], rtol=1e-6)
        a, bk, c, _ = OA.backward(q[None, qs:qe], k[None, ks:ke], v[None, ks:ke], o, dout[None, qs:qe], l, **one)
        np.testing.assert_allclose(dq[qs:qe], a[0], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(dk[ks:ke], bk[0], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(dv[ks:ke], c[0], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("causal", [False, True])
def test_probabilities_are_the_attention_matrix(causal):
    """|P| times V is torch's SDPA output (so |P| is the softmax attention matrix),
    rows of visible keys sum to 1, the padding to 128 is +0, and the sign bit is
    set exactly on the visible elements the keep mask drops."""
    from oracle import dropout as DR

    b, s, hq, hk, d = 2, 75, 4, 2, 64
    q, k, v = rnd(b, s, hq, d, seed=11), rnd(b, s, hk, d, seed=12), rnd(b, s, hk, d, seed=13)
    keep = DR.dense_mask(5, 64, b, hq, s, s, 0.3)
    p = OA.probabilities(q, k, keep, causal=causal)
    assert p.shape == (b, hq, 128, 128)
    assert not p[:, :, s:].any() and not p[:, :, :, s:].any() and not np.signbit(p[:, :, s:]).any()
    a = np.abs(p[:, :, :s, :s]).astype(np.float64)
    vt = np.repeat(np.transpose(v, (0, 2, 1, 3)), hq // hk, axis=1)
    o, _ = sdpa(q, k, v, causal)
    np.testing.assert_allclose(np.transpose(a @ vt, (0, 2, 1, 3)), o, atol=2e-5)
    np.testing.assert_allclose(a.sum(-1), 1.0, atol=1e-5)
    visible = ~np.triu(np.ones((s, s), dtype=bool), 1) if causal else np.ones((s, s), dtype=bool)
    np.testing.assert_array_equal(np.signbit(p[:, :, :s, :s]), ~keep & visible)
