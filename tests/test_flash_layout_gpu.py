"""Layouts the attention kernels cannot read directly, handled inside the C ABI
(flash-attn2-rs/src/host/layout.rs:46-125 and host/forward/mod.rs:349-376):
tensors whose base is not 16-byte aligned or whose outer strides are not
multiples of 8 elements are staged through packed copies, an output that
cannot be written in place (or that overlaps an input) is written to a packed
buffer and copied out, and a self-overlapping output is refused with the
reference's message. Checked against the oracle, and against the same call
with contiguous tensors bit for bit (the kernels then see identical data)."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import attention as OA

pytestmark = pytest.mark.gpu


def misaligned(shape, dtype, seed, pad_last=0):
    """A tensor of `shape` whose data starts 2 bytes past a 16-byte boundary and,
    with pad_last, whose rows are pad_last elements longer than D (odd strides)."""
    g = torch.Generator().manual_seed(seed)
    full = list(shape[:-1]) + [shape[-1] + pad_last]
    n = int(np.prod(full))
    base = torch.randn(n + 1, generator=g).to(dtype).cuda()
    t = base[1:].view(full)[..., : shape[-1]]
    assert t.data_ptr() % 16 != 0
    return t


def call_fwd(q, k, v, out, lse, causal):
    import kcr_native
    from kcr_native import describe, ref, stream_of

    descs = [describe(t) for t in (q, k, v)]
    return kcr_native.lib.kcr_flash_fwd(*(ref(d) for d in descs), None, 0, ctypes.c_double(0.0),
                                        int(causal), ctypes.c_int64(-1), ctypes.c_int64(-1),
                                        ctypes.c_double(0.0), None, ref(describe(out)),
                                        ref(describe(lse)), stream_of(q))


@pytest.mark.parametrize("causal", [False, True])
def test_c_abi_fwd_misaligned_odd_strides(causal):
    """kcr_flash_fwd over ctypes: q 2 bytes off alignment, k with an odd head
    stride (D + 3), v broadcast over the batch (stride 0), out misaligned."""
    import kcr_native

    B, S, H, Hk, D = 2, 200, 4, 2, 64
    q = misaligned((B, S, H, D), torch.bfloat16, 0)
    k = misaligned((B, S, Hk, D), torch.bfloat16, 1, pad_last=3)
    assert k.stride(2) % 8 != 0
    v0 = torch.randn(1, S, Hk, D, generator=torch.Generator().manual_seed(2)).bfloat16().cuda()
    v = v0.expand(B, S, Hk, D)
    out = misaligned((B, S, H, D), torch.bfloat16, 3)
    lse = torch.empty(B, H, S, device="cuda")
    kcr_native.check(call_fwd(q, k, v, out, lse, causal))
    eo, el = OA.forward(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                        causal=causal)
    assert np.abs(out.float().cpu().numpy() - eo).max() <= 2e-2
    np.testing.assert_allclose(lse.cpu().numpy(), el, atol=2e-3, rtol=1e-4)
    # the same call on contiguous copies gives the same bits
    out2 = torch.empty(B, S, H, D, dtype=torch.bfloat16, device="cuda")
    lse2 = torch.empty_like(lse)
    kcr_native.check(call_fwd(q.contiguous(), k.contiguous(), v.contiguous(), out2, lse2, causal))
    assert torch.equal(out, out2) and torch.equal(lse, lse2)


def test_c_abi_fwd_out_overlapping_input_and_self_overlap():
    import kcr_native

    B, S, H, D = 1, 130, 4, 128
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B, S, H, D, generator=g).half().cuda()
    k = torch.randn(B, S, H, D, generator=g).half().cuda()
    v = torch.randn(B, S, H, D, generator=g).half().cuda()
    ref_out = torch.empty_like(q)
    lse = torch.empty(B, H, S, device="cuda")
    kcr_native.check(call_fwd(q, k, v, ref_out, lse, True))
    qa = q.clone()
    kcr_native.check(call_fwd(qa, k, v, qa, lse, True))  # out aliases q: written after the reads
    assert torch.equal(qa, ref_out)
    bad = torch.empty(1, 1, H, D, dtype=q.dtype, device="cuda").expand(B, S, H, D)
    status = call_fwd(q, k, v, bad, lse, True)
    assert status == 1
    assert "nonoverlapping" in kcr_native.lib.kcr_last_error().decode()


def test_varlen_and_backward_misaligned_match_contiguous():
    """varlen forward and backward, dense backward and bwd_preprocess with
    misaligned q / k / v / dout / out: the same bits as contiguous inputs."""
    import flash_attn2_rs

    ops = flash_attn2_rs.ops
    lens = [70, 133, 1]
    cu = torch.tensor(np.cumsum([0] + lens), dtype=torch.int32).cuda()
    T, H, Hk, D = sum(lens), 4, 2, 64
    q = misaligned((T, H, D), torch.bfloat16, 10, pad_last=5)
    k = misaligned((T, Hk, D), torch.bfloat16, 11)
    v = misaligned((T, Hk, D), torch.bfloat16, 12, pad_last=1)
    dout = misaligned((T, H, D), torch.bfloat16, 13)
    args = (None, None, None, None, True, -1, -1, 0.0, 0.0, None, max(lens), max(lens), False, False)
    o1, l1, _ = ops.varlen_fwd_explicit(q, k, v, cu, cu, *args)
    o2, l2, _ = ops.varlen_fwd_explicit(q.contiguous(), k.contiguous(), v.contiguous(), cu, cu, *args)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    bargs = (None, None, True, -1, -1, 0.0, 0.0, None, max(lens), max(lens), False)
    om = misaligned((T, H, D), torch.bfloat16, 14)
    om.copy_(o1)
    g1 = ops.varlen_bwd_explicit(q, k, v, dout, om, l1, cu, cu, *bargs)
    g2 = ops.varlen_bwd_explicit(q.contiguous(), k.contiguous(), v.contiguous(), dout.contiguous(), o2,
                                 l2, cu, cu, *bargs)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)
    # dense backward and preprocess
    B, S = 2, 96
    qd = misaligned((B, S, H, D), torch.float16, 20)
    kd = misaligned((B, S, Hk, D), torch.float16, 21, pad_last=7)
    vd = misaligned((B, S, Hk, D), torch.float16, 22)
    dod = misaligned((B, S, H, D), torch.float16, 23, pad_last=2)
    od, lsed = ops.fwd(qd.contiguous(), kd.contiguous(), vd.contiguous(), None, None, True, -1, -1, 0.0)
    om = misaligned((B, S, H, D), torch.float16, 24)
    om.copy_(od)
    d1 = ops.bwd_preprocess(dod, om, 0.0)
    d2 = ops.bwd_preprocess(dod.contiguous(), od, 0.0)
    assert torch.equal(d1, d2)
    a = ops.bwd_all(qd, kd, vd, dod, lsed, d1, None, None, True, -1, -1, 0.0, 0.0, None)
    b = ops.bwd_all(qd.contiguous(), kd.contiguous(), vd.contiguous(), dod.contiguous(), lsed, d2, None,
                    None, True, -1, -1, 0.0, 0.0, None)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_padded_head_size_from_strided_views():
    """Head size 72 (run through zero-padded 128-wide copies) with q and dout
    as transposed [B, H, S, D] views and k, v with a size-1 batch dimension of
    odd stride: the padded copies read the views in 16-byte chunks; forward and
    backward give the same bits as contiguous inputs."""
    import flash_attn2_rs

    B, S, H, Hk, D = 1, 150, 4, 2, 72
    g = torch.Generator().manual_seed(21)
    q = torch.randn(B, H, S, D, generator=g).bfloat16().cuda().transpose(1, 2)
    dout = torch.randn(B, H, S, D, generator=g).bfloat16().cuda().transpose(1, 2)
    kv = torch.randn(2, S, Hk, D, generator=g).bfloat16().cuda()
    k = kv[0].as_strided((1, S, Hk, D), (7, Hk * D, D, 1))
    v = kv[1].as_strided((1, S, Hk, D), (13, Hk * D, D, 1))
    assert not q.is_contiguous() and k.stride(0) % 8 != 0
    o1, l1, _, _ = flash_attn2_rs.fwd(q, k, v, is_causal=True)
    o2, l2, _, _ = flash_attn2_rs.fwd(q.contiguous(), k.contiguous(), v.contiguous(), is_causal=True)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    g1 = flash_attn2_rs.bwd(dout, q, k, v, o1, l1, is_causal=True)
    g2 = flash_attn2_rs.bwd(dout.contiguous(), q.contiguous(), k.contiguous(), v.contiguous(), o2, l2,
                            is_causal=True)
    for a, b in zip(g1[:3], g2[:3]):
        assert torch.equal(a, b)
