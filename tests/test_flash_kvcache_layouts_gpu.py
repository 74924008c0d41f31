"""KV-cache calls on unusual layouts, mirroring flash-attn2-rs/tests/test_gold.py
:766-1010 with the oracle in place of the CUDA reference: caches that are
interleaved strided views of one storage, odd (unaligned) row strides, sources
that alias the cache allocation, padded head sizes with paged rotary splits,
an ignored sine table, and the grouped decode layout. Each case checks out /
LSE against oracle.kvcache and the whole backing storage against a copy with
only the expected rows written."""

import math

import numpy as np
import pytest
import torch

from oracle import kvcache as KV

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy()


def _expected(q, kc, vc, k, v, lengths, *, causal=False, cos=None, sin=None, interleaved=True, table=None,
              window=(-1, -1), scale=None, dtype="f16"):
    """Oracle result on host copies: (out, lse, k cache, v cache) after the append."""
    qn, kcn, vcn = _np(q), _np(kc), _np(vc)
    cap = kc.shape[1] * (table.shape[1] if table is not None else 1)
    if k is not None and k.shape[1] > 0:
        if cos is not None:
            adv = causal or 0 <= window[0] < cap or 0 <= window[1] < cap
            qn = KV.rotate_q(qn, lengths, _np(cos), _np(sin), interleaved, adv, dtype)
        kcn, vcn = KV.append(kcn, vcn, _np(k), _np(v), lengths, cos=None if cos is None else _np(cos),
                             sin=None if sin is None else _np(sin), interleaved=interleaved,
                             block_table=table, dtype=dtype)
    new = 0 if k is None else k.shape[1]
    used = np.asarray(lengths) + new if lengths is not None else np.full(q.shape[0], cap)
    out, lse = KV.attend(qn, kcn, vcn, used, block_table=table, causal=causal, window_left=window[0],
                         window_right=window[1], softmax_scale=scale)
    return out, lse, kcn, vcn


def _close(out, lse, eo, el):
    assert np.abs(_np(out) - eo).max() <= 7e-3 + 0.04 * np.abs(eo).max()
    fin = np.isfinite(el)
    np.testing.assert_array_equal(np.isfinite(_np(lse)), fin)
    np.testing.assert_allclose(_np(lse)[fin], el[fin], atol=2e-2, rtol=0)


def test_interleaved_axes():
    """test_gold.py:766-786: three interleaved axes with disjoint rows."""
    import flash_attn2_rs

    torch.manual_seed(0)
    storage = torch.randn(2, 80, device="cuda", dtype=torch.float16)
    before = storage.clone()
    q = torch.randn(2, 1, 2, 8, device="cuda", dtype=storage.dtype)
    lengths = torch.ones(2, device="cuda", dtype=torch.int32)
    kc, vc = (row.as_strided((2, 2, 2, 8), (16, 24, 32, 1)) for row in storage)
    ekc = before[0].as_strided((2, 2, 2, 8), (16, 24, 32, 1))
    evc = before[1].as_strided((2, 2, 2, 8), (16, 24, 32, 1))
    eo, el, kcn, vcn = _expected(q, ekc, evc, q, q, [1, 1])
    out, lse = flash_attn2_rs.fwd_kvcache(q, kc, vc, k=q, v=q, seqlens_k=lengths)
    _close(out, lse, eo, el)
    want = before.clone()
    want[0].as_strided((2, 2, 2, 8), (16, 24, 32, 1)).copy_(torch.from_numpy(kcn).half())
    want[1].as_strided((2, 2, 2, 8), (16, 24, 32, 1)).copy_(torch.from_numpy(vcn).half())
    assert torch.equal(storage, want)


def test_padded_batch_strides():
    """test_gold.py:789-815: an odd (unaligned) row stride in a shared storage;
    one appended key per sequence, so O equals the appended V exactly."""
    import flash_attn2_rs

    rows, step, d = 4097, 8192, 8
    batch_stride = (rows * (step + 1) + 135) // 8 * 8
    storage = torch.empty(batch_stride + 8 + (rows - 1) * (step + 1) + 2 * d, device="cuda",
                          dtype=torch.float16)
    kc = storage.as_strided((2, rows, 1, d), (batch_stride, step, d, 1))
    vc = storage.as_strided((2, rows, 1, d), (batch_stride + 8, step + 1, d, 1), d)
    q = torch.ones(2, 1, 1, d, device="cuda", dtype=storage.dtype)
    v = torch.arange(d, device="cuda", dtype=storage.dtype).reshape(1, 1, 1, d).expand_as(q).contiguous()
    lengths = torch.zeros(2, device="cuda", dtype=torch.int32)
    out = flash_attn2_rs.fwd_kvcache(q, kc, vc, k=q, v=v, seqlens_k=lengths)[0]
    torch.testing.assert_close(out, v)
    assert torch.equal(vc[:, 0], v[:, 0]) and torch.equal(kc[:, 0], q[:, 0])


def test_append_reads_same_allocation():
    """test_gold.py:819-841: q / k / v are views of the caches being appended to."""
    import flash_attn2_rs

    torch.manual_seed(0)
    kc = torch.randn(1, 8, 1, 16, device="cuda", dtype=torch.float16)
    vc = torch.randn_like(kc)
    q, k, v = kc[:, :2], kc[:, :1], vc[:, :1]
    eo, el, kcn, vcn = _expected(q.clone(), kc.clone(), vc.clone(), k.clone(), v.clone(), [3])
    out, lse = flash_attn2_rs.fwd_kvcache(q, kc, vc, k=k, v=v,
                                          seqlens_k=torch.tensor([3], device="cuda", dtype=torch.int32))
    _close(out, lse, eo, el)
    assert np.array_equal(_np(kc), kcn) and np.array_equal(_np(vc), vcn)


def test_paged_rotary_padded_head():
    """test_gold.py:844-894: D = 63 (padded), two pages, rotary append, 3 splits;
    a full-capacity window; an empty append leaves Q unrotated and the caches
    unchanged."""
    import flash_attn2_rs

    torch.manual_seed(0)
    q = torch.randn(1, 2, 4, 63, device="cuda", dtype=torch.float16)
    k = torch.randn(1, 2, 2, 63, device="cuda", dtype=q.dtype)
    v = torch.randn_like(k)
    kc = torch.randn(2, 256, 2, 63, device="cuda", dtype=q.dtype)
    vc = torch.randn_like(kc)
    kc0, vc0 = kc.clone(), vc.clone()
    lengths = torch.tensor([255], device="cuda", dtype=torch.int32)
    table = torch.tensor([[1, 0]], device="cuda", dtype=torch.int32)
    angles = torch.randn(512, 32, device="cuda")
    cos, sin = angles.cos().to(q.dtype), angles.sin().to(q.dtype)
    opts = dict(k=k, v=v, rotary_cos=cos, rotary_sin=sin, cache_seqlens=lengths, block_table=table,
                causal=True, num_splits=3, return_softmax_lse=True)
    pad = lambda t: torch.nn.functional.pad(t, (0, 1))
    tab = table.cpu().numpy()
    scale = 1.0 / math.sqrt(63)
    eo, el, kcn, vcn = _expected(pad(q), pad(kc0), pad(vc0), pad(k), pad(v), [255], causal=True, cos=cos,
                                 sin=sin, table=tab, scale=scale)
    out, lse = flash_attn2_rs.flash_attn_with_kvcache(q, kc, vc, **opts)
    _close(out, lse, eo[..., :63], el)
    assert np.array_equal(_np(kc), kcn[..., :63]) and np.array_equal(_np(vc), vcn[..., :63])
    assert lengths.item() == 255

    kc1, vc1 = kc.clone(), vc.clone()
    full = {**opts, "causal": False, "window_size": (512, 512)}
    eo, el, kcn, vcn = _expected(pad(q), pad(kc1), pad(vc1), pad(k), pad(v), [255], causal=False, cos=cos,
                                 sin=sin, table=tab, window=(512, 512), scale=scale)
    out, lse = flash_attn2_rs.flash_attn_with_kvcache(q, kc, vc, **full)
    _close(out, lse, eo[..., :63], el)

    saved = (kc.clone(), vc.clone())
    opts.update(k=k[:, :0], v=v[:, :0])
    eo, el, _, _ = _expected(pad(q), pad(saved[0]), pad(saved[1]), None, None, [255], causal=True, table=tab,
                             scale=scale)
    out, lse = flash_attn2_rs.flash_attn_with_kvcache(q, kc, vc, **opts)
    _close(out, lse, eo[..., :63], el)
    assert torch.equal(kc, saved[0]) and torch.equal(vc, saved[1])


def test_shared_storage_head_strides():
    """test_gold.py:897-936: K/V caches as views with different head strides in
    one storage; a sine table without cosine is ignored; empty caches give O = 0
    and LSE = +inf even with 128 splits."""
    import flash_attn2_rs

    torch.manual_seed(0)
    storage = torch.randn(2, 8, 6, 64, device="cuda", dtype=torch.float16)
    before = storage.clone()
    q = torch.randn(1, 1, 4, 64, device="cuda", dtype=storage.dtype)
    k = torch.randn(1, 1, 2, 64, device="cuda", dtype=storage.dtype)
    v = torch.randn_like(k)
    lengths = torch.tensor([2], device="cuda", dtype=torch.int32)
    eo, el, kcn, vcn = _expected(q, before[:, :, :2], before[:, :, 2::2], k, v, [2])
    out, lse = flash_attn2_rs.fwd_kvcache(q, storage[:, :, :2], storage[:, :, 2::2], k, v, lengths,
                                          rotary_sin=torch.tensor(0.0))
    _close(out, lse, eo, el)
    want = before.clone()
    want[:, :, :2] = torch.from_numpy(kcn).half().cuda()
    want[:, :, 2::2] = torch.from_numpy(vcn).half().cuda()
    assert torch.equal(storage, want)
    out, lse = flash_attn2_rs.fwd_kvcache(q, storage[:, :, :2], storage[:, :, 2::2],
                                          seqlens_k=torch.zeros_like(lengths), num_splits=128)
    assert torch.count_nonzero(out) == 0
    assert torch.isposinf(lse).all()


def test_packed_disjoint_views():
    """test_gold.py:939-955: read-only sources and writable caches as disjoint
    views of one packed storage."""
    import flash_attn2_rs

    torch.manual_seed(0)
    storage = torch.randn(1, 8, 3, 2, 64, device="cuda", dtype=torch.float16)
    before = storage.clone()
    q, k, v = storage[:, :1, 0], storage[:, 1:2, 0], storage[:, 2:3, 0]
    eo, el, kcn, vcn = _expected(before[:, :1, 0], before[:, :, 1], before[:, :, 2], before[:, 1:2, 0],
                                 before[:, 2:3, 0], [4])
    out, lse = flash_attn2_rs.fwd_kvcache(q, storage[:, :, 1], storage[:, :, 2], k, v,
                                          torch.tensor([4], device="cuda", dtype=torch.int32))
    _close(out, lse, eo, el)
    want = before.clone()
    want[:, :, 1] = torch.from_numpy(kcn).half().cuda()
    want[:, :, 2] = torch.from_numpy(vcn).half().cuda()
    assert torch.equal(storage, want)


def test_interleaved_batch_gaps():
    """test_gold.py:958-980: source batches in the gaps of interleaved caches."""
    import flash_attn2_rs

    torch.manual_seed(0)
    storage = torch.randn(256, device="cuda", dtype=torch.float16)
    before = storage.clone()
    views = lambda s: ([s.as_strided((2, 1, 1, 8), (8, 8, 8, 1), o) for o in (16, 48, 80)],
                       [s.as_strided((2, 4, 1, 8), (32, 64, 8, 1), o) for o in (0, 8)])
    (q, k, v), (kc, vc) = views(storage)
    (q0, k0, v0), (kc0, vc0) = views(before)
    eo, el, kcn, vcn = _expected(q0, kc0, vc0, k0, v0, [1, 2])
    out, lse = flash_attn2_rs.fwd_kvcache(q, kc, vc, k, v, torch.tensor([1, 2], device="cuda",
                                                                        dtype=torch.int32))
    _close(out, lse, eo, el)
    want = before.clone()
    views(want)[1][0].copy_(torch.from_numpy(kcn).half())
    views(want)[1][1].copy_(torch.from_numpy(vcn).half())
    assert torch.equal(storage, want)


def test_grouped_decode_layout():
    """test_gold.py:983-1007: decode with an interleaved query layout, and `out`
    in the grouped [B, H / Hk, Hk, D] layout filled in head order."""
    import flash_attn2_rs

    torch.manual_seed(0)
    q = torch.randn(8, 2, 128, device="cuda", dtype=torch.float16).transpose(0, 1).unsqueeze(1)
    kc = torch.randn(2, 1024, 2, 128, device="cuda", dtype=q.dtype)
    vc = torch.randn_like(kc)
    eo, el, _, _ = _expected(q, kc, vc, None, None, None)
    out, lse = flash_attn2_rs.fwd_kvcache(q, kc, vc, num_splits=0)
    _close(out, lse, eo, el)
    grouped = torch.empty((2, 4, 2, 128), device="cuda", dtype=q.dtype)
    out, lse = flash_attn2_rs.fwd_kvcache(q, kc, vc, out=grouped, num_splits=0)
    _close(out, lse, eo, el)
    # Query head h = kvh * 4 + j sits at grouped[:, j, kvh].
    np.testing.assert_allclose(_np(grouped).transpose(0, 2, 1, 3).reshape(2, 8, 128), eo[:, 0],
                               atol=7e-3 + 0.04 * np.abs(eo).max())


@pytest.mark.parametrize("grouped", [True, False])
@pytest.mark.parametrize("splits", [1, 3])
def test_out_views_written_in_place(grouped, splits):
    """`out` as a strided view (padded rows: written in place) and with unaligned
    rows (written through a temporary) gives the same bits as a fresh output,
    and the caller's tensor holds the result."""
    import flash_attn2_rs

    torch.manual_seed(3)
    B, Hk, D = 3, 2, 128
    H, sq = (8, 1) if grouped else (4, 3)
    q = torch.randn(B, sq, H, D + 8, device="cuda", dtype=torch.bfloat16)[..., :D]
    kc = torch.randn(B, 768, Hk, D, device="cuda", dtype=q.dtype)
    vc = torch.randn_like(kc)
    lengths = torch.tensor([5, 300, 767], dtype=torch.int32, device="cuda")
    ref_out, ref_lse = flash_attn2_rs.fwd_kvcache(q, kc, vc, seqlens_k=lengths, is_causal=True,
                                                  num_splits=splits)
    eo, el, _, _ = _expected(q, kc, vc, None, None, lengths.cpu().numpy(), causal=True, dtype="bf16")
    _close(ref_out, ref_lse, eo, el)
    for pad in (8, 4):
        backing = torch.full((B, sq, H, D + pad), 7.0, device="cuda", dtype=q.dtype)
        view = backing[..., :D]
        out, lse = flash_attn2_rs.fwd_kvcache(q, kc, vc, seqlens_k=lengths, is_causal=True,
                                              num_splits=splits, out=view)
        torch.cuda.synchronize()
        assert torch.equal(view, ref_out) and torch.equal(out, ref_out)
        assert torch.equal(lse, ref_lse)
        assert bool((backing[..., D:] == 7.0).all())  # padding columns untouched
