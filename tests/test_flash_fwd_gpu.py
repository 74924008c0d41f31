"""GPU parity of the FlashAttention-2 forward (dense and varlen) against
oracle/attention.py, on the reference's parity cases (flash-attn2-rs/tests/
test_gold.py:872-1270 and test_fwd.py:88-168) plus BASELINE.json-sized checks.

Bars: the reference tests' tolerances (bf16: atol 1e-2, rtol 5e-2, mean 8e-3, LSE
8e-2; fp16: 2e-3 / 2.5e-2 / 3e-3 / 3e-2) and the north-star bound, max abs error
<= 2e-2 against the fp32 softmax(QK^T)V oracle.
"""

import math

import numpy as np
import pytest
import torch

from attn_cases import PARITY_CASES, make_inputs, oracle_kwargs, tolerances
from oracle import attention as OA

pytestmark = pytest.mark.gpu


def run_fwd(q, k, v, options):
    import flash_attn2_rs

    alibi = options.get("alibi_slopes")
    out, lse = flash_attn2_rs.ops.fwd(
        q.cuda(), k.cuda(), v.cuda(), None if alibi is None else alibi.cuda(),
        options.get("softmax_scale"), options.get("causal", False), options.get("window_left", -1),
        options.get("window_right", -1), options.get("softcap", 0.0))
    return out.float().cpu().numpy(), lse.cpu().numpy()


def check(out, lse, eo, el, dtype):
    tol = tolerances(dtype)
    assert np.isfinite(out).all()
    np.testing.assert_allclose(out, eo, atol=tol["atol"], rtol=tol["rtol"])
    assert np.abs(out - eo).mean() < tol["mean"]
    assert np.abs(out - eo).max() <= 2e-2
    inf = np.isposinf(el)
    np.testing.assert_array_equal(np.isposinf(lse), inf)
    np.testing.assert_allclose(lse[~inf], el[~inf], atol=tol["lse"], rtol=0)


@pytest.mark.parametrize("name,shape,options", PARITY_CASES, ids=[c[0] for c in PARITY_CASES])
def test_forward_parity(name, shape, options):
    q, k, v, options, dtype = make_inputs(shape, options)
    out, lse = run_fwd(q, k, v, options)
    eo, el = OA.forward(q.float().numpy(), k.float().numpy(), v.float().numpy(), **oracle_kwargs(options))
    check(out, lse, eo, el, dtype)


def test_sk1_returns_v_exactly():
    """test_gold.py:259-266 / test_forward_batch_and_heads_grid."""
    import flash_attn2_rs

    g = torch.Generator().manual_seed(0)
    q = torch.randn(257, 1, 256, 8, generator=g).half().cuda()
    kv = torch.randn(257, 1, 1, 8, generator=g).half().cuda()
    out = flash_attn2_rs.fwd(q, kv, kv)[0]
    torch.testing.assert_close(out, kv.expand_as(q), atol=0, rtol=0)


def test_empty_keys_and_fully_masked_rows():
    import flash_attn2_rs

    q = torch.randn(2, 33, 4, 64, device="cuda", dtype=torch.bfloat16)
    empty = torch.empty(2, 0, 4, 64, device="cuda", dtype=torch.bfloat16)
    out = torch.full_like(q, 7.0)
    o, lse = flash_attn2_rs.ops.fwd(q, empty, empty, None, None, False, -1, -1, 0.0, out)
    assert o.data_ptr() == out.data_ptr()
    assert (o == 0).all() and torch.isposinf(lse).all()
    # Sq > Sk causal: the first Sq - Sk rows see no key.
    k = torch.randn(2, 20, 4, 64, device="cuda", dtype=torch.bfloat16)
    o, lse = flash_attn2_rs.ops.fwd(q, k, k, None, None, True, -1, -1, 0.0)
    assert (o[:, :13] == 0).all() and torch.isposinf(lse[:, :, :13]).all()
    assert torch.isfinite(lse[:, :, 13:]).all()


def test_strided_views_and_unaligned_out():
    """test_gold.py:1270-1284 (zero-copy [B,H,S,D] transposes) and an output at a
    2-byte offset (test_output_layout)."""
    import flash_attn2_rs

    g = torch.Generator().manual_seed(0)
    q = torch.randn(2, 8, 256, 128, generator=g).half().cuda().transpose(1, 2)
    k = torch.randn(2, 2, 256, 128, generator=g).half().cuda().transpose(1, 2)
    v = torch.randn(2, 2, 256, 128, generator=g).half().cuda().transpose(1, 2)
    storage = torch.full((q.numel() + 1,), 123, device="cuda", dtype=q.dtype)
    out_buf = storage[1:].view(q.shape)
    out, lse = flash_attn2_rs.ops.fwd(q, k, v, None, None, True, -1, -1, 0.0, out_buf)
    assert out.data_ptr() == out_buf.data_ptr() and storage[0] == 123
    eo, el = OA.forward(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(), causal=True)
    np.testing.assert_allclose(out.float().cpu().numpy(), eo, atol=2e-2, rtol=0)
    np.testing.assert_allclose(lse.cpu().numpy(), el, atol=3e-2, rtol=0)


def test_repeated_calls_bitwise_equal():
    import flash_attn2_rs

    q = torch.randn(2, 512, 8, 128, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(2, 512, 2, 128, device="cuda", dtype=torch.bfloat16)
    a = flash_attn2_rs.ops.fwd(q, k, k, None, None, True, -1, -1, 0.0)
    b = flash_attn2_rs.ops.fwd(q, k, k, None, None, True, -1, -1, 0.0)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("causal", [True, False])
def test_baseline_config_subset(causal):
    """BASELINE config 4 (B=4, Hq=32, Hkv=8, S=4096, D=128, bf16): the full launch,
    checked against the oracle on one batch entry x one GQA group (4 query heads)."""
    import flash_attn2_rs

    g = torch.Generator().manual_seed(3)
    q = torch.randn(4, 4096, 32, 128, generator=g).bfloat16()
    k = torch.randn(4, 4096, 8, 128, generator=g).bfloat16()
    v = torch.randn(4, 4096, 8, 128, generator=g).bfloat16()
    out, lse = flash_attn2_rs.ops.fwd(q.cuda(), k.cuda(), v.cuda(), None, None, causal, -1, -1, 0.0)
    b, grp = 3, 5
    eo, el = OA.forward(q[b:b + 1, :, 4 * grp:4 * grp + 4].float().numpy(),
                        k[b:b + 1, :, grp:grp + 1].float().numpy(),
                        v[b:b + 1, :, grp:grp + 1].float().numpy(), causal=causal)
    o = out[b:b + 1, :, 4 * grp:4 * grp + 4].float().cpu().numpy()
    assert np.abs(o - eo).max() <= 2e-2
    np.testing.assert_allclose(lse[b:b + 1, 4 * grp:4 * grp + 4].cpu().numpy(), el, atol=8e-2, rtol=0)
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()


def varlen_setup(lens_q, lens_k, hq, hk, d, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    cu_q = torch.tensor(np.cumsum([0] + lens_q), dtype=torch.int32)
    cu_k = torch.tensor(np.cumsum([0] + lens_k), dtype=torch.int32)
    q = torch.randn(sum(lens_q), hq, d, generator=g).to(dtype)
    k = torch.randn(sum(lens_k), hk, d, generator=g).to(dtype)
    v = torch.randn(sum(lens_k), hk, d, generator=g).to(dtype)
    return q, k, v, cu_q, cu_k


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("lens_q,lens_k", [([17, 0, 8], [19, 0, 12]), ([130, 300, 1, 257], [130, 300, 1, 257]),
                                           ([64, 128], [200, 128])])
def test_varlen_forward(causal, lens_q, lens_k):
    """test_gold.py:542-569: packed sequences, GQA, an empty sequence."""
    import flash_attn2_rs

    q, k, v, cu_q, cu_k = varlen_setup(lens_q, lens_k, 4, 2, 64, torch.float16)
    out, lse, _ = flash_attn2_rs.ops.varlen_fwd_explicit(
        q.cuda(), k.cuda(), v.cuda(), cu_q.cuda(), cu_k.cuda(), None, None, None, None, causal, -1, -1,
        0.0, 0.0, None, max(lens_q), max(lens_k), False, True)
    eo, el = OA.varlen_forward(q.float().numpy(), k.float().numpy(), v.float().numpy(), cu_q.numpy(),
                               cu_k.numpy(), causal=causal)
    check(out.float().cpu().numpy(), lse.cpu().numpy(), eo, el, torch.float16)


def test_varlen_baseline_config():
    """16 sequences with lengths ~U[128, 8192] (seed 5), Hq=32,
    Hkv=8, D=128, causal bf16; the whole launch, checked on 3 sequences x 1 group."""
    import flash_attn2_rs

    lens = torch.randint(128, 8193, (16,), generator=torch.Generator().manual_seed(5)).tolist()
    q, k, v, cu_q, cu_k = varlen_setup(lens, lens, 32, 8, 128, torch.bfloat16, seed=6)
    out, lse, _ = flash_attn2_rs.ops.varlen_fwd_explicit(
        q.cuda(), k.cuda(), v.cuda(), cu_q.cuda(), cu_k.cuda(), None, None, None, None, True, -1, -1,
        0.0, 0.0, None, max(lens), max(lens), False, False)
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    for s in (0, 7, 15):
        a, bnd = int(cu_q[s]), int(cu_q[s + 1])
        eo, el = OA.forward(q[None, a:bnd, 8:12].float().numpy(), k[None, a:bnd, 2:3].float().numpy(),
                            v[None, a:bnd, 2:3].float().numpy(), causal=True)
        assert np.abs(out[a:bnd, 8:12].float().cpu().numpy() - eo[0]).max() <= 2e-2
        np.testing.assert_allclose(lse[8:12, a:bnd].cpu().numpy(), el[0], atol=8e-2, rtol=0)


def test_varlen_grouped_decode_lse():
    """test_gold.py:600-617: one query per sequence with GQA (the grouped decode
    path); out against the oracle and LSE against a float64 logsumexp, LSE
    contiguous [H, B]."""
    import flash_attn2_rs

    g = torch.Generator().manual_seed(0)
    q = torch.randn(16, 8, 128, generator=g).half()
    k = torch.randn(16, 1024, 2, 128, generator=g).half()
    v = torch.randn(16, 1024, 2, 128, generator=g).half()
    cu_q = torch.arange(17, dtype=torch.int32)
    out, lse, _ = flash_attn2_rs.ops.varlen_fwd_explicit(
        q.cuda(), k.flatten(0, 1).cuda(), v.flatten(0, 1).cuda(), cu_q.cuda(), (cu_q * 1024).cuda(), None,
        None, None, None, True, -1, -1, 0.0, 0.0, None, 1, 1024, False, False)
    eo, _ = OA.varlen_forward(q.float().numpy(), k.flatten(0, 1).float().numpy(), v.flatten(0, 1).float().numpy(),
                              cu_q.numpy(), (cu_q * 1024).numpy(), causal=True)
    assert np.abs(out.float().cpu().numpy() - eo).max() <= 2e-2
    scores = torch.einsum("bhd,bkhd->bhk", q.double(), k.double().repeat_interleave(4, 2)) / math.sqrt(128)
    np.testing.assert_allclose(lse.cpu().numpy(), scores.logsumexp(-1).T.numpy(), atol=5e-3, rtol=0)
    assert lse.is_contiguous() and lse.shape == (8, 16)


def test_attention_custom_ops_opcheck():
    """torch.library.opcheck of the custom ops behind flash_attn_func and
    flash_attn_varlen_func (schema, fake tensors incl. the probabilities shape,
    AOT dispatch), mirroring tvm-ffi-ext/flash_attn2_rs/_torch_interface.py:19-555."""
    import flash_attn2_rs  # noqa: F401

    ns = torch.ops.kcr_flash_attn2
    g = torch.Generator().manual_seed(23)
    q = torch.randn(2, 70, 4, 64, generator=g).bfloat16().cuda()
    k = torch.randn(2, 90, 2, 64, generator=g).bfloat16().cuda()
    v = torch.randn(2, 90, 2, 64, generator=g).bfloat16().cuda()
    scale = 64 ** -0.5
    torch.library.opcheck(ns._dense_forward, (q, k, v, scale, True, -1, -1, 0.0, None, 0.0, False))
    out, lse, _, state = ns._dense_forward(q, k, v, scale, True, -1, -1, 0.0, None, 0.0, False)
    torch.library.opcheck(ns._dense_backward,
                          (torch.randn_like(out), q, k, v, out, lse, scale, True, -1, -1, 0.0, None, False,
                           0.0, None))
    cu = torch.tensor([0, 30, 70], dtype=torch.int32, device="cuda")
    cuk = torch.tensor([0, 50, 90], dtype=torch.int32, device="cuda")
    qv, kv, vv = q[0], k[0], v[0]
    torch.library.opcheck(ns._varlen_forward, (qv, kv, vv, cu, cuk, 40, 50, scale, True, -1, -1, 0.0, None,
                                               0.0, False))
    out, lse, _, _ = ns._varlen_forward(qv, kv, vv, cu, cuk, 40, 50, scale, True, -1, -1, 0.0, None, 0.0, False)
    torch.library.opcheck(ns._varlen_backward,
                          (torch.randn_like(out), qv, kv, vv, out, lse, cu, cuk, 40, 50, scale, True, -1, -1,
                           0.0, None, 0.0, None))
