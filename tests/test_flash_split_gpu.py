"""Key-split forward for underfilled grids: few query tiles against long keys.

When B * H * ceil(Sq / 128) cannot fill the chip, `kcr_flash_fwd` and
`kcr_flash_varlen_fwd` split the keys over blocks and merge fp32 partials (the
reference plans the same trade, flash-attn2-rs/src/host/forward/dispatch.rs:
127-238). The results must match the unsplit oracle to the north-star bound:
max abs error <= 2e-2 against the fp32 softmax(QK^T)V of oracle/attention.py,
LSE within the reference tests' bf16 bound (8e-2, test_gold.py:1267).
"""

import numpy as np
import pytest
import torch

from oracle import attention as OA

pytestmark = pytest.mark.gpu


def _inputs(b, sq, sk, hq, hk, d, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, sq, hq, d, generator=g).bfloat16()
    k = torch.randn(b, sk, hk, d, generator=g).bfloat16()
    v = torch.randn(b, sk, hk, d, generator=g).bfloat16()
    return q, k, v


def _check(out, lse, eo, el):
    assert np.isfinite(out).all()
    assert np.abs(out - eo).max() <= 2e-2
    inf = np.isposinf(el)
    np.testing.assert_array_equal(np.isposinf(lse), inf)
    np.testing.assert_allclose(lse[~inf], el[~inf], atol=8e-2, rtol=0)


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sq", [1, 64, 128])
def test_dense_split_long_keys(sq, causal, d):
    """B=1, Hq=8, Hkv=2, Sk=32k: 8 blocks of 128 query rows without splits."""
    import flash_attn2_rs

    q, k, v = _inputs(1, sq, 32768, 8, 2, d, seed=sq + d)
    print(f"dense split case sq={sq} causal={causal} d={d}", flush=True)
    out, lse = flash_attn2_rs.ops.fwd(q.cuda(), k.cuda(), v.cuda(), None, None, causal, -1, -1, 0.0)
    eo, el = OA.forward(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal=causal)
    _check(out.float().cpu().numpy(), lse.cpu().numpy(), eo, el)


def test_dense_split_rows_without_keys():
    """Causal with Sq > Sk: rows before Sq - Sk see no key (O = 0, LSE = +inf)
    in every split, and the merge keeps that."""
    import flash_attn2_rs

    q, k, v = _inputs(1, 2048, 1024, 8, 2, 128, seed=3)
    out, lse = flash_attn2_rs.ops.fwd(q.cuda(), k.cuda(), v.cuda(), None, None, True, -1, -1, 0.0)
    eo, el = OA.forward(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal=True)
    assert np.isposinf(el[:, :, :1024]).all()
    _check(out.float().cpu().numpy(), lse.cpu().numpy(), eo, el)
    assert (out[:, :1024].float() == 0).all()


def test_dense_split_sliding_window():
    """A local window on an underfilled grid: splits past the window see no key."""
    import flash_attn2_rs

    q, k, v = _inputs(2, 64, 8192, 4, 4, 128, seed=4)
    out, lse = flash_attn2_rs.ops.fwd(q.cuda(), k.cuda(), v.cuda(), None, None, False, 700, 50, 0.0)
    eo, el = OA.forward(q.float().numpy(), k.float().numpy(), v.float().numpy(), window_left=700,
                        window_right=50)
    _check(out.float().cpu().numpy(), lse.cpu().numpy(), eo, el)


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_varlen_split_long_keys(causal, d):
    """Packed sequences with short queries and long keys (one of them empty); a
    query row no sequence covers keeps the cleared output (zero_tensors)."""
    import flash_attn2_rs

    lens_q, lens_k = [3, 64, 0, 100], [8192, 20000, 4096, 4100]
    hq, hk = 8, 2
    g = torch.Generator().manual_seed(11)
    cu_q = torch.tensor(np.cumsum([0] + lens_q), dtype=torch.int32)
    cu_k = torch.tensor(np.cumsum([0] + lens_k), dtype=torch.int32)
    tq = sum(lens_q) + 5  # 5 trailing rows outside every sequence
    q = torch.randn(tq, hq, d, generator=g).bfloat16()
    k = torch.randn(sum(lens_k), hk, d, generator=g).bfloat16()
    v = torch.randn(sum(lens_k), hk, d, generator=g).bfloat16()
    out, lse, _ = flash_attn2_rs.ops.varlen_fwd_explicit(
        q.cuda(), k.cuda(), v.cuda(), cu_q.cuda(), cu_k.cuda(), None, None, None, None, causal, -1, -1,
        0.0, 0.0, None, max(lens_q), max(lens_k), False, True)
    n = sum(lens_q)
    eo, el = OA.varlen_forward(q[:n].float().numpy(), k.float().numpy(), v.float().numpy(), cu_q.numpy(),
                               cu_k.numpy(), causal=causal)
    _check(out[:n].float().cpu().numpy(), lse[:, :n].cpu().numpy(), eo, el)
    assert (out[n:].float() == 0).all()
    assert torch.isneginf(lse[:, n:]).all()
