"""kcr_flash_fwd_kvcache_noalloc (split partials in the library's fixed scratch)
against kcr_flash_fwd_kvcache (split partials in a caller workspace), both
called through the C ABI: the same kernels over the same inputs, so the outputs
must agree bit for bit, on two calls in a row (the second smaller, over the
scratch the first left behind), for the batched decode form and the packed
form, and sizes beyond the scratch must be refused."""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _c_args(q, kc, vc, cu, used, splits, causal):
    from kcr_native import describe

    return [describe(t) for t in (q, kc, vc, cu, used)], splits, causal


def _run(entry, q, kc, vc, cu, used, splits, causal, out, lse, workspace=None):
    import kcr_native
    from kcr_native import describe, ref, stream_of

    descs = [describe(t) for t in (q, kc, vc, cu, used)]
    common = [*(ref(d) for d in descs), ctypes.c_int64(0), None, None, None, None, 0,
              ctypes.c_double(0.0), int(causal), ctypes.c_int64(-1), ctypes.c_int64(-1),
              ctypes.c_double(0.0), ctypes.c_int64(q.shape[1] if cu is None else int((cu[1:] - cu[:-1]).max())),
              ctypes.c_int64(splits)]
    tail = [ref(describe(out)), ref(describe(lse)), stream_of(q)]
    if entry == "kcr_flash_fwd_kvcache":
        ws = workspace
        common += [ctypes.c_void_p(ws.data_ptr()), ctypes.c_int64(ws.numel())]
    return getattr(kcr_native.lib, entry)(*common, *tail)


def _case(batch, rows, heads, kv_heads, cap, d, packed, seed):
    g = torch.Generator().manual_seed(seed)
    kc = torch.randn(batch, cap, kv_heads, d, generator=g).bfloat16().cuda()
    vc = torch.randn(batch, cap, kv_heads, d, generator=g).bfloat16().cuda()
    used = torch.randint(1, cap + 1, (batch,), generator=g).to(torch.int32).cuda()
    if packed:
        q = torch.randn(batch * rows, heads, d, generator=g).bfloat16().cuda()
        cu = torch.arange(0, batch * rows + 1, rows, dtype=torch.int32).cuda()
        lse_shape = (heads, batch * rows)
    else:
        q = torch.randn(batch, rows, heads, d, generator=g).bfloat16().cuda()
        cu = None
        lse_shape = (batch, heads, rows)
    return q, kc, vc, cu, used, lse_shape


@pytest.mark.parametrize("packed", [False, True])
def test_noalloc_matches_workspace_entry(packed):
    import kcr_native

    lib = kcr_native.lib
    lib.kcr_flash_fwd_kvcache_noalloc_scratch_bytes.restype = ctypes.c_int64
    assert lib.kcr_flash_fwd_kvcache_noalloc_scratch_bytes() == 64 << 20
    # each call smaller than the one before, over the scratch it left behind
    # (head size 256: four columns per lane in the split merge)
    for batch, rows, heads, kv_heads, cap, d, splits, seed in ((8, 4, 32, 8, 3000, 128, 16, 0),
                                                              (4, 4, 16, 4, 2000, 256, 8, 2),
                                                              (3, 2, 8, 2, 700, 64, 5, 1)):
        q, kc, vc, cu, used, lse_shape = _case(batch, rows, heads, kv_heads, cap, d, packed, seed)
        tq = batch * rows
        need = lib.kcr_flash_fwd_kvcache_workspace_bytes(splits, heads, tq, d)
        assert 0 < need <= 64 << 20
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        out_ws, out_na = torch.empty_like(q), torch.empty_like(q)
        lse_ws = torch.empty(lse_shape, device="cuda")
        lse_na = torch.empty(lse_shape, device="cuda")
        kcr_native.check(_run("kcr_flash_fwd_kvcache", q, kc, vc, cu, used, splits, True, out_ws, lse_ws, ws))
        kcr_native.check(_run("kcr_flash_fwd_kvcache_noalloc", q, kc, vc, cu, used, splits, True, out_na, lse_na))
        torch.cuda.synchronize()
        assert torch.isfinite(out_ws.float()).all()
        assert torch.equal(out_na, out_ws), (batch, packed)
        assert torch.equal(lse_na, lse_ws), (batch, packed)
        # and the split result is the unsplit one within the split merge's rounding
        out1 = torch.empty_like(q)
        lse1 = torch.empty(lse_shape, device="cuda")
        kcr_native.check(_run("kcr_flash_fwd_kvcache_noalloc", q, kc, vc, cu, used, 1, True, out1, lse1))
        torch.testing.assert_close(out_na.float(), out1.float(), atol=2e-2, rtol=0)
        torch.testing.assert_close(lse_na, lse1, atol=1e-4, rtol=1e-5)


def test_noalloc_refuses_sizes_beyond_scratch():
    import kcr_native

    q, kc, vc, cu, used, lse_shape = _case(64, 64, 32, 8, 256, 128, False, 2)
    out = torch.empty_like(q)
    lse = torch.empty(lse_shape, device="cuda")
    status = _run("kcr_flash_fwd_kvcache_noalloc", q, kc, vc, cu, used, 64, True, out, lse)
    assert status == 1
    msg = kcr_native.lib.kcr_last_error().decode()
    assert "kcr_flash_fwd_kvcache_noalloc holds at most 67108864" in msg, msg
