"""flash_attn_with_kvcache on the GPU against oracle.kvcache: the appended cache
bit for bit (rotary included), out within 2e-2 (bf16) of the fp32 oracle and LSE
within 8e-2, over contiguous / indexed / left-padded / paged caches, decode (GQA
rows) and chunked prefill, rotary layouts, key splits and the general kernel.
Cases follow the reference's cache tests (flash-attn2-rs/tests/test_gold.py,
flash_attn_with_kvcache)."""

import numpy as np
import pytest
import torch

from oracle import kvcache as KV

pytestmark = pytest.mark.gpu

DT = {torch.bfloat16: "bf16", torch.float16: "f16"}


def _setup(B, cap, Hk, H, D, snew, sq, dtype, seed, *, batches=None, page=None, cols=None):
    g = torch.Generator().manual_seed(seed)
    nb = batches if batches is not None else B
    if page is not None:
        kc = torch.randn(nb, page, Hk, D, generator=g).to(dtype)
    else:
        kc = torch.randn(nb, cap, Hk, D, generator=g).to(dtype)
    vc = torch.randn(kc.shape, generator=g).to(dtype)
    k = torch.randn(B, snew, Hk, D, generator=g).to(dtype) if snew else None
    v = torch.randn(B, snew, Hk, D, generator=g).to(dtype) if snew else None
    q = torch.randn(B, sq, H, D, generator=g).to(dtype)
    return q, kc, vc, k, v


def _f(t):
    return None if t is None else t.float().numpy()


def _run(q, kc, vc, k, v, lengths, *, causal=False, window=(-1, -1), splits=1, cos=None, sin=None,
         interleaved=True, idx=None, leftpad=None, table=None, softcap=0.0, alibi=None):
    import flash_attn2_rs

    dev = "cuda"
    kcd, vcd = kc.to(dev), vc.to(dev)
    out, lse = flash_attn2_rs.flash_attn_with_kvcache(
        q.to(dev), kcd, vcd, None if k is None else k.to(dev), None if v is None else v.to(dev),
        rotary_cos=None if cos is None else cos.to(dev), rotary_sin=None if sin is None else sin.to(dev),
        cache_seqlens=None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=dev),
        cache_batch_idx=None if idx is None else torch.tensor(idx, dtype=torch.int32, device=dev),
        cache_leftpad=None if leftpad is None else torch.tensor(leftpad, dtype=torch.int32, device=dev),
        block_table=None if table is None else torch.tensor(table, dtype=torch.int32, device=dev),
        causal=causal, window_size=window, softcap=softcap, rotary_interleaved=interleaved,
        alibi_slopes=None if alibi is None else alibi.to(dev), num_splits=splits, return_softmax_lse=True)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu(), kcd.cpu(), vcd.cpu()


def _expect(q, kc, vc, k, v, lengths, *, causal=False, window=(-1, -1), cos=None, sin=None,
            interleaved=True, idx=None, leftpad=None, table=None, softcap=0.0, dtype=torch.bfloat16,
            alibi=None):
    dt = DT[dtype]
    B, sq = q.shape[:2]
    snew = 0 if k is None else k.shape[1]
    cap = kc.shape[1] * (len(table[0]) if table is not None else 1)
    qn = _f(q)
    kcn, vcn = _f(kc), _f(vc)
    if snew:
        if cos is not None:
            advance = causal or 0 <= window[0] < cap or 0 <= window[1] < cap
            qn = KV.rotate_q(qn, lengths, _f(cos), _f(sin), interleaved, advance, dt)
        kcn, vcn = KV.append(kcn, vcn, _f(k), _f(v), lengths, cos=_f(cos), sin=_f(sin),
                             interleaved=interleaved, cache_batch_idx=idx,
                             block_table=None if table is None else np.array(table), dtype=dt)
    used = np.array(lengths) + snew if lengths is not None else np.full(B, cap)
    out, lse = KV.attend(qn, kcn, vcn, used, leftpad=leftpad, cache_batch_idx=idx,
                         block_table=None if table is None else np.array(table), causal=causal,
                         window_left=window[0], window_right=window[1], softcap=softcap,
                         alibi_slopes=None if alibi is None else alibi.numpy())
    return out, lse, kcn, vcn


def _check(got, want, cache_exact=True):
    out, lse, kc, vc = got
    eo, el, ekc, evc = want
    if cache_exact:
        np.testing.assert_array_equal(kc.float().numpy(), ekc)
        np.testing.assert_array_equal(vc.float().numpy(), evc)
    assert np.abs(out.float().numpy() - eo).max() <= 2e-2
    fin = np.isfinite(el)
    np.testing.assert_array_equal(np.isfinite(lse.numpy()), fin)
    np.testing.assert_allclose(lse.numpy()[fin], el[fin], atol=8e-2, rtol=0)


@pytest.mark.parametrize("splits", [1, 0, 4])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_gqa_append(splits, dtype):
    """Sq = 1 decode with GQA (query heads as rows), one appended token."""
    B, cap, Hk, H, D = 3, 1024, 2, 8, 128
    q, kc, vc, k, v = _setup(B, cap, Hk, H, D, 1, 1, dtype, seed=1)
    lengths = [5, 700, 1023]
    got = _run(q, kc, vc, k, v, lengths, causal=True, splits=splits)
    _check(got, _expect(q, kc, vc, k, v, lengths, causal=True, dtype=dtype))


@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("D", [64, 128])
def test_chunked_prefill_causal(splits, D):
    B, cap, Hk, H = 2, 512, 2, 4
    q, kc, vc, k, v = _setup(B, cap, Hk, H, D, 7, 7, torch.bfloat16, seed=2)
    lengths = [0, 300]
    got = _run(q, kc, vc, k, v, lengths, causal=True, splits=splits)
    _check(got, _expect(q, kc, vc, k, v, lengths, causal=True))


@pytest.mark.parametrize("splits", [1, 3])
def test_long_chunk_two_query_tiles(splits):
    """A 200-token chunk (two 128-row query tiles per sequence) appended and
    attended causally, with and without key splits."""
    B, cap, Hk, H, D = 2, 1024, 2, 4, 128
    q, kc, vc, k, v = _setup(B, cap, Hk, H, D, 200, 200, torch.bfloat16, seed=14)
    lengths = [0, 300]
    got = _run(q, kc, vc, k, v, lengths, causal=True, splits=splits)
    _check(got, _expect(q, kc, vc, k, v, lengths, causal=True))


@pytest.mark.parametrize("splits", [1, 2])
@pytest.mark.parametrize("D", [64, 128])
def test_paged_cache(splits, D):
    """Pages of 256 rows in a permuted block table; decode and a 3-token chunk."""
    B, page, cols, Hk, H = 2, 256, 3, 2, 4
    perm = np.random.default_rng(3).permutation(B * cols).reshape(B, cols).tolist()
    for sq in (1, 3):
        q, kc, vc, k, v = _setup(B, None, Hk, H, D, sq, sq, torch.bfloat16, seed=3 + sq,
                                 batches=B * cols, page=page)
        lengths = [255, 600]
        got = _run(q, kc, vc, k, v, lengths, causal=True, splits=splits, table=perm)
        _check(got, _expect(q, kc, vc, k, v, lengths, causal=True, table=perm))


def test_cache_batch_idx_and_leftpad():
    B, cap, Hk, H, D = 3, 256, 1, 2, 128
    q, kc, vc, k, v = _setup(B, cap, Hk, H, D, 2, 2, torch.bfloat16, seed=5, batches=5)
    idx = [4, 0, 2]
    lengths = [100, 30, 250]
    leftpad = [10, 0, 200]
    got = _run(q, kc, vc, k, v, lengths, causal=True, idx=idx, leftpad=leftpad)
    _check(got, _expect(q, kc, vc, k, v, lengths, causal=True, idx=idx, leftpad=leftpad))


@pytest.mark.parametrize("interleaved", [True, False])
@pytest.mark.parametrize("causal", [True, False])
def test_rotary_append(interleaved, causal):
    B, cap, Hk, H, D, rd = 2, 512, 2, 4, 128, 64
    q, kc, vc, k, v = _setup(B, cap, Hk, H, D, 3, 3, torch.bfloat16, seed=6)
    g = torch.Generator().manual_seed(7)
    theta = torch.rand(cap, rd // 2, generator=g) * 6.283
    cos, sin = theta.cos().bfloat16(), theta.sin().bfloat16()
    lengths = [17, 400]
    got = _run(q, kc, vc, k, v, lengths, causal=causal, cos=cos, sin=sin, interleaved=interleaved)
    _check(got, _expect(q, kc, vc, k, v, lengths, causal=causal, cos=cos, sin=sin, interleaved=interleaved))


def test_readonly_full_cache_and_window():
    """No append, no lengths (every row attended), sliding window."""
    B, cap, Hk, H, D = 2, 320, 2, 4, 128
    q, kc, vc, _, _ = _setup(B, cap, Hk, H, D, 0, 4, torch.bfloat16, seed=8)
    got = _run(q, kc, vc, None, None, None, causal=True, window=(64, 0))
    _check(got, _expect(q, kc, vc, None, None, None, causal=True, window=(64, 0)))


@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("mode", ["alibi", "softcap", "both"])
def test_scored_cache(mode, paged, splits):
    """Softcap and / or ALiBi over a contiguous or paged cache, with key splits:
    the tiled kernel's scored instances in cache mode, against the oracle."""
    B, cap, Hk, H, D = 2, 512, 2, 8, 128
    q, kc, vc, k, v = _setup(B, cap, Hk, H, D, 3, 3, torch.bfloat16, seed=21)
    lengths = [100, 400]
    table = None
    if paged:
        # Two sequences of two 256-row pages each, pages in permuted order.
        kc = kc.reshape(B * 2, 256, Hk, D)
        vc = vc.reshape(B * 2, 256, Hk, D)
        table = [[2, 0], [3, 1]]
    alibi = (torch.rand(H, generator=torch.Generator().manual_seed(5)) * 0.2).float() if mode != "softcap" else None
    cap_v = 30.0 if mode != "alibi" else 0.0
    got = _run(q, kc, vc, k, v, lengths, causal=True, splits=splits, table=table, softcap=cap_v, alibi=alibi)
    _check(got, _expect(q, kc, vc, k, v, lengths, causal=True, table=table, softcap=cap_v, alibi=alibi))


@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("mode", ["plain", "both"])
def test_cache_d256(mode, paged):
    """Head size 256 over a contiguous or paged cache, plain or with softcap and
    ALiBi, with key splits: the tiled kernel's D = 256 instances in cache mode
    and the 4-column merge."""
    B, cap, Hk, H, D = 2, 512, 2, 4, 256
    q, kc, vc, k, v = _setup(B, cap, Hk, H, D, 3, 3, torch.bfloat16, seed=23)
    lengths = [130, 400]
    table = None
    if paged:
        kc = kc.reshape(B * 2, 256, Hk, D)
        vc = vc.reshape(B * 2, 256, Hk, D)
        table = [[3, 1], [0, 2]]
    alibi = (torch.rand(H, generator=torch.Generator().manual_seed(6)) * 0.2).float() if mode == "both" else None
    cap_v = 30.0 if mode == "both" else 0.0
    got = _run(q, kc, vc, k, v, lengths, causal=True, splits=3, table=table, softcap=cap_v, alibi=alibi)
    _check(got, _expect(q, kc, vc, k, v, lengths, causal=True, table=table, softcap=cap_v, alibi=alibi))


def test_general_kernel_softcap_d96():
    B, cap, Hk, H, D = 2, 300, 1, 2, 96
    q, kc, vc, k, v = _setup(B, cap, Hk, H, D, 2, 2, torch.bfloat16, seed=9)
    lengths = [50, 290]
    got = _run(q, kc, vc, k, v, lengths, causal=True, softcap=30.0, splits=4)
    _check(got, _expect(q, kc, vc, k, v, lengths, causal=True, softcap=30.0))


def test_empty_cache_row_and_out_of_range_positions():
    """A sequence with no keys gives O = 0, LSE = +inf; appends past the capacity
    are skipped (src/device/cache.rs:190-197)."""
    B, cap, Hk, H, D = 2, 256, 1, 2, 128
    q, kc, vc, k, v = _setup(B, cap, Hk, H, D, 2, 1, torch.bfloat16, seed=10)
    lengths = [255, 100]
    got = _run(q, kc, vc, k, v, lengths, causal=False)
    want = _expect(q, kc, vc, k, v, lengths, causal=False)
    # used = lengths + 2 exceeds the capacity for batch 0: that sequence is skipped
    # (metadata bounds), so only batch 1's output is defined.
    np.testing.assert_array_equal(got[2].float().numpy(), want[2])
    assert np.abs(got[0][1].float().numpy() - want[0][1]).max() <= 2e-2
    q2, kc2, vc2, _, _ = _setup(1, cap, Hk, H, D, 0, 1, torch.bfloat16, seed=11)
    out, lse, _, _ = _run(q2, kc2, vc2, None, None, [0])
    assert torch.count_nonzero(out) == 0 and torch.isinf(lse).all() and (lse > 0).all()


@pytest.mark.parametrize("H", [8, 2])
def test_split_invalid_sequence_is_empty(H):
    """Key splits with a sequence whose cache batch index is out of range: its
    blocks write nothing but "unseen" partials, so the merge gives O = 0 and
    LSE = +inf for it; the other sequence is unaffected."""
    B, cap, Hk, D = 2, 1024, 2, 128
    q, kc, vc, _, _ = _setup(B, cap, Hk, H, D, 0, 1, torch.bfloat16, seed=13)
    lengths = [700, 300]
    out, lse, _, _ = _run(q, kc, vc, None, None, lengths, idx=[1, 7], splits=3)
    eo, el, _, _ = _expect(q[:1], kc, vc, None, None, lengths[:1], idx=[1])
    _check((out[:1], lse[:1], kc, vc), (eo, el, kc.float().numpy(), vc.float().numpy()))
    assert torch.count_nonzero(out[1]) == 0
    assert torch.isinf(lse[1]).all() and (lse[1] > 0).all()


def test_split_merge_matches_unsplit():
    """Key splits (explicit counts) reproduce the unsplit result within fp32 merge
    rounding."""
    B, cap, Hk, H, D = 2, 2048, 2, 8, 128
    q, kc, vc, k, v = _setup(B, cap, Hk, H, D, 1, 1, torch.bfloat16, seed=12)
    lengths = [1500, 2047]
    base = _run(q, kc, vc, k, v, lengths, causal=True, splits=1)
    for s in (2, 5, 16):
        got = _run(q, kc, vc, k, v, lengths, causal=True, splits=s)
        assert (got[0].float() - base[0].float()).abs().max() <= 1e-2
        assert (got[1] - base[1]).abs().max() <= 1e-4


def test_paged_varlen_func_forward():
    """flash_attn_varlen_func with a block table (paged K/V, forward only): packed
    queries of 3 sequences over keys read through the table."""
    import flash_attn2_rs

    g = torch.Generator().manual_seed(13)
    page, cols, Hk, H, D = 256, 2, 2, 4, 128
    lens_q, lens_k = [65, 0, 17], [300, 17, 512]  # an empty query sequence, as test_gold.py:636-652
    B = len(lens_q)
    kp = torch.randn(B * cols, page, Hk, D, generator=g).bfloat16()
    vp = torch.randn(B * cols, page, Hk, D, generator=g).bfloat16()
    q = torch.randn(sum(lens_q), H, D, generator=g).bfloat16()
    table = np.random.default_rng(14).permutation(B * cols).reshape(B, cols).astype(np.int32)
    cu_q = torch.tensor(np.cumsum([0] + lens_q), dtype=torch.int32)
    cu_k = torch.tensor(np.cumsum([0] + lens_k), dtype=torch.int32)
    out = flash_attn2_rs.flash_attn_varlen_func(
        q.cuda(), kp.cuda(), vp.cuda(), cu_q.cuda(), cu_k.cuda(), max(lens_q), max(lens_k), causal=True,
        block_table=torch.from_numpy(table).cuda())
    torch.cuda.synchronize()
    qs = np.cumsum([0] + lens_q)
    for b in range(B):
        if lens_q[b] == 0:
            continue
        qb = q[qs[b]:qs[b + 1]].float().numpy()[None]
        eo, _ = KV.attend(qb, _f(kp), _f(vp), np.array([lens_k[b]]), block_table=table[b:b + 1], causal=True)
        assert np.abs(out[qs[b]:qs[b + 1]].float().cpu().numpy() - eo[0]).max() <= 2e-2


def test_rejected_append_preserves_cache():
    """A rejected append (V of another dtype) raises before writing anything
    (test_gold.py:655-672)."""
    import flash_attn2_rs

    q = torch.randn(1, 1, 1, 16, device="cuda", dtype=torch.float16)
    kc = torch.randn(1, 4, 1, 16, device="cuda", dtype=q.dtype)
    vc = torch.randn_like(kc)
    saved = (kc.clone(), vc.clone(), kc._version, vc._version)
    with pytest.raises(RuntimeError):
        flash_attn2_rs.flash_attn_with_kvcache(q, kc, vc, k=q, v=q.float(), cache_seqlens=1)
    assert torch.equal(kc, saved[0]) and torch.equal(vc, saved[1])
    assert (kc._version, vc._version) == saved[2:]


def test_append_bumps_cache_versions():
    """Native cache writes bump the tensors' versions, so a graph that saved the
    old cache fails in backward (test_gold.py:675-689)."""
    import flash_attn2_rs

    q = torch.randn(1, 1, 1, 16, device="cuda", dtype=torch.float16)
    kc = torch.randn(1, 4, 1, 16, device="cuda", dtype=q.dtype, requires_grad=True)
    vc = torch.randn_like(kc, requires_grad=True)
    loss = kc.square().float().sum() + vc.square().float().sum()
    versions = (kc._version, vc._version)
    with torch.no_grad():
        flash_attn2_rs.flash_attn_with_kvcache(q, kc, vc, k=q, v=q, cache_seqlens=1)
    assert kc._version > versions[0] and vc._version > versions[1]
    with pytest.raises(RuntimeError, match="modified by an inplace operation"):
        loss.backward()


@pytest.mark.parametrize("D", [7, 20])
def test_unpadded_head_size(D):
    """Head sizes that are not a multiple of 8 run on padded copies; the appended
    rows land in the caller's caches (flash_attn_interface.py:1562-1642)."""
    B, cap, Hk, H = 2, 64, 1, 2
    q, kc, vc, k, v = _setup(B, cap, Hk, H, D, 2, 2, torch.float16, seed=15)
    lengths = [3, 40]
    got = _run(q, kc, vc, k, v, lengths, causal=True)
    _check(got, _expect(q, kc, vc, k, v, lengths, causal=True, dtype=torch.float16))


def test_decode_step_in_cuda_graph():
    """A decode step (append + split attention + merge) captured in a CUDA graph
    and replayed several times, with eager work in between, matches the eager
    call each time."""
    import flash_attn2_rs

    B, cap, Hk, H, D = 4, 2048, 2, 8, 128
    q, kc, vc, k, v = _setup(B, cap, Hk, H, D, 1, 1, torch.bfloat16, seed=16)
    q, kc, vc, k, v = (t.cuda() for t in (q, kc, vc, k, v))
    lengths = torch.tensor([100, 900, 1500, 2000], dtype=torch.int32, device="cuda")

    def step():
        return flash_attn2_rs.flash_attn_with_kvcache(q, kc, vc, k, v, cache_seqlens=lengths, causal=True,
                                                      num_splits=4, return_softmax_lse=True)

    eager_out, eager_lse = (t.clone() for t in step())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_out, g_lse = step()
    for i in range(3):
        torch.randn(1000, device="cuda").sum().item()  # eager work between replays
        g_out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(g_out, eager_out), f"replay {i}"
        assert torch.equal(g_lse, eager_lse), f"replay {i}"


def test_cached_forward_opcheck():
    """torch.library.opcheck of the custom ops behind flash_attn_with_kvcache
    (schema, fake tensors, declared cache mutation)."""
    import flash_attn2_rs  # noqa: F401

    B, cap, Hk, H, D = 2, 256, 1, 2, 64
    q, kc, vc, k, v = (t.cuda() if t is not None else None
                       for t in _setup(B, cap, Hk, H, D, 1, 1, torch.bfloat16, seed=17))
    lengths = torch.tensor([10, 100], dtype=torch.int32, device="cuda")
    rest = (None, None, None, None, None, None, None, True, -1, -1, 0.0, True, 1)
    ns = torch.ops.kcr_flash_attn2
    torch.library.opcheck(ns._cached_forward, (q, kc, vc, k, v, lengths, *rest))
    torch.library.opcheck(ns._cached_forward_readonly, (q, kc, vc, None, None, lengths, *rest))
