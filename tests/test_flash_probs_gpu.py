"""GPU parity of the diagnostic probabilities of a dropout forward (return_softmax,
flash-attn2-rs/src/host/forward/mod.rs:133-199, 382-398, src/device/dropout.rs:
93-112) against oracle/attention.py:probabilities.

The reference's own test (tests/test_gold.py:160-180) compares the shape and the
sign bits (the drop decisions) of the probabilities; those are checked bit for
bit here over the whole padded plane. The magnitudes are the softmax
probabilities, within |got - P| <= 1e-3 + 1e-2 P (a bf16 / fp16 rounding of a
value computed from the forward's fp32 LSE). Output and LSE must equal those of
the same forward without probabilities, bit for bit.
"""

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import dropout as DR

pytestmark = pytest.mark.gpu


def ops():
    import flash_attn2_rs

    return flash_attn2_rs.ops


def _check_plane(got, expect):
    got = got.float().cpu().numpy()
    assert got.shape == expect.shape
    np.testing.assert_array_equal(np.signbit(got), np.signbit(expect))
    assert np.all(np.abs(np.abs(got) - np.abs(expect)) <= 1e-3 + 1e-2 * np.abs(expect))


@pytest.mark.parametrize(
    "dtype,b,sq,sk,h,hk,d,causal,wl,wr,alibi",
    [
        (torch.float16, 1, 33, 33, 2, 2, 64, False, -1, -1, False),  # the reference test's shape
        (torch.bfloat16, 2, 150, 300, 4, 2, 128, True, -1, -1, False),
        (torch.bfloat16, 1, 200, 130, 2, 1, 64, True, -1, -1, False),  # rows with no key
        (torch.float16, 2, 96, 257, 2, 2, 256, False, 40, 7, False),
        (torch.bfloat16, 1, 128, 128, 4, 4, 96, True, -1, -1, True),
    ],
)
def test_dense_probabilities(dtype, b, sq, sk, h, hk, d, causal, wl, wr, alibi):
    print(f"probabilities dense {dtype} b={b} sq={sq} sk={sk} h={h}/{hk} d={d} causal={causal} "
          f"window=({wl},{wr}) alibi={alibi}", flush=True)
    g = torch.Generator().manual_seed(sq + sk + d)
    q = torch.randn(b, sq, h, d, generator=g).to(dtype)
    k = torch.randn(b, sk, hk, d, generator=g).to(dtype)
    v = torch.randn(b, sk, hk, d, generator=g).to(dtype)
    slopes = (torch.rand(h, generator=g) * 0.3).float() if alibi else None
    p, seed, offset = 0.17, 0x5EED_1234_5678, 32
    state = torch.tensor([seed, offset], dtype=torch.int64, device="cuda")
    qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
    sc = slopes.cuda() if alibi else None
    out, lse, probs = ops().fwd(qc, kc, vc, sc, None, causal, wl, wr, 0.0, p, state, 0, None, True)
    ref_out = torch.empty_like(qc)
    ref_lse = ops().fwd_lse(qc, kc, vc, sc, None, causal, wl, wr, 0.0, p, state, 0, ref_out)
    assert torch.equal(out, ref_out) and torch.equal(lse, ref_lse)
    keep = DR.dense_mask(seed, offset, b, h, sq, sk, p)
    expect = OA.probabilities(q.float().numpy(), k.float().numpy(), keep, causal=causal,
                              window_left=wl, window_right=wr,
                              alibi_slopes=slopes.numpy() if alibi else None)
    _check_plane(probs, expect)


def test_varlen_probabilities():
    """Packed sequences (one empty, rows no sequence covers): plane [B, H,
    ceil128(max_q), ceil128(max_k)] with rows and columns local to each sequence."""
    lens_q, lens_k = [37, 0, 200, 64], [90, 33, 150, 64]
    h, hk, d = 4, 2, 128
    g = torch.Generator().manual_seed(21)
    cu_q = torch.tensor(np.cumsum([0] + lens_q), dtype=torch.int32)
    cu_k = torch.tensor(np.cumsum([0] + lens_k), dtype=torch.int32)
    tq = sum(lens_q) + 3
    q = torch.randn(tq, h, d, generator=g).bfloat16()
    k = torch.randn(sum(lens_k), hk, d, generator=g).bfloat16()
    v = torch.randn(sum(lens_k), hk, d, generator=g).bfloat16()
    seed, offset, p = 424242, 64, 0.25
    state = torch.tensor([seed, offset], dtype=torch.int64, device="cuda")
    for causal in (False, True):
        print(f"probabilities varlen causal={causal}", flush=True)
        out, lse, probs = ops().varlen_fwd_explicit(
            q.cuda(), k.cuda(), v.cuda(), cu_q.cuda(), cu_k.cuda(), None, None, None, None, causal, -1, -1,
            0.0, p, state, max(lens_q), max(lens_k), True, True)
        assert probs.shape == (4, h, 256, 256)
        expect = np.zeros((4, h, 256, 256), dtype=np.float32)
        for bi, (qs, ks) in enumerate(zip(cu_q[:-1].tolist(), cu_k[:-1].tolist())):
            nq, nk = lens_q[bi], lens_k[bi]
            keep = np.stack([DR.keep_mask(seed, offset, bi * h + hh, nq, nk, p) for hh in range(h)])[None]
            plane = OA.probabilities(q[None, qs:qs + nq].float().numpy(), k[None, ks:ks + nk].float().numpy(),
                                     keep, causal=causal)
            expect[bi, :, :plane.shape[2], :plane.shape[3]] = plane[0]
        _check_plane(probs, expect)


def test_interface_returns_probabilities():
    """flash_attn_func(return_attn_probs=True) with dropout and fwd(return_softmax)
    return the plane; its sign bits follow the returned RNG state."""
    import flash_attn2_rs

    torch.manual_seed(0)
    q = torch.randn(1, 33, 2, 64, device="cuda", dtype=torch.float16)
    out, lse, probs, state = flash_attn2_rs.fwd(q, q, q, p_dropout=0.17, return_softmax=True)
    assert probs.shape == (1, 2, 128, 128)
    seed, offset = (int(x) for x in state.cpu())
    keep = DR.dense_mask(seed, offset, 1, 2, 33, 33, 0.17)
    np.testing.assert_array_equal(np.signbit(probs[:, :, :33, :33].float().cpu().numpy()), ~keep)
    o2, lse2, p2 = flash_attn2_rs.flash_attn_func(q, q, q, dropout_p=0.17, return_attn_probs=True)
    assert p2.shape == (1, 2, 128, 128) and torch.isfinite(o2).all()
    with pytest.raises(RuntimeError):
        flash_attn2_rs.fwd(q, q, q, return_softmax=True)
