"""The __tvm_ffi_* packed exports on the GPU, called as a tvm-ffi runtime calls
them (packed TVMFFIAny arguments, DLTensor pointers), against the same ops
through the Python `ops` modules: results must be identical bit for bit, the
Array results must hold the reference's items in order, and every object the
adapters return must be released by one reference drop (no leak)."""

import ctypes

import pytest
import torch

import tvm_ffi_util as T

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def runtime():
    T.install_torch_allocator()
    return T.mock()


def _ok(rc, m):
    assert rc == 0, (m.mock_error_kind(), m.mock_error_message())


def _release(m, *objs):
    for o in objs:
        m.TVMFFIObjectDecRef(ctypes.c_void_p(o))


def test_activations(runtime):
    import activation_rs

    g = torch.Generator().manual_seed(0)
    x = torch.randn(33, 2 * 1000, generator=g).bfloat16().cuda()
    for op in ("silu_and_mul", "mul_and_silu", "gelu_and_mul", "gelu_tanh_and_mul"):
        out = torch.empty(33, 1000, dtype=x.dtype, device="cuda")
        _ok(T.call(op, out, x)[0], runtime)
        ref = torch.empty_like(out)
        getattr(activation_rs.ops, op)(ref, x)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), op
    out = torch.empty(33, 1000, dtype=x.dtype, device="cuda")
    _ok(T.call("fatrelu_and_mul", out, x, 0.25)[0], runtime)
    ref = torch.empty_like(out)
    activation_rs.ops.fatrelu_and_mul(ref, x, 0.25)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    for op in ("gelu", "gelu_tanh", "gelu_new", "gelu_fast", "gelu_quick", "silu"):
        out = torch.empty_like(x)
        _ok(T.call(op, out, x)[0], runtime)
        ref = torch.empty_like(x)
        getattr(activation_rs.ops, op)(ref, x)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), op


@pytest.mark.parametrize("mode,offset,with_weight", [("llama", 0.0, True), ("gemma", 1.0, True),
                                                      ("none", 0.0, False)])
def test_rms_norm(runtime, mode, offset, with_weight):
    import rmsnorm

    g = torch.Generator().manual_seed(1)
    x = torch.randn(300, 4096, generator=g).bfloat16().cuda()
    w = (torch.rand(4096, generator=g) + 0.5).bfloat16().cuda() if with_weight else None
    y, rstd = torch.empty_like(x), torch.empty(300, device="cuda")
    _ok(T.call("rms_norm_forward", y, rstd, x, w, 1e-6, offset, mode)[0], runtime)
    y2, rstd2 = torch.empty_like(x), torch.empty(300, device="cuda")
    rmsnorm.ops.rms_norm_forward(y2, rstd2, x, w, 1e-6, offset, mode)
    torch.cuda.synchronize()
    assert torch.equal(y, y2) and torch.equal(rstd, rstd2)

    dy = torch.randn(300, 4096, generator=g).bfloat16().cuda()
    parts = 16
    dx, dxr = torch.empty_like(x), torch.empty_like(x)
    dwp = torch.empty(parts, 4096, device="cuda") if with_weight else None
    dwpr = torch.empty(parts, 4096, device="cuda") if with_weight else None
    _ok(T.call("rms_norm_backward", dx, dwp, dy, x, w, rstd, offset, mode)[0], runtime)
    rmsnorm.ops.rms_norm_backward(dxr, dwpr, dy, x, w, rstd, offset, mode)
    if with_weight:
        dw, dwr = torch.empty_like(w), torch.empty_like(w)
        _ok(T.call("rms_norm_reduce_weight_grad", dw, dwp)[0], runtime)
        rmsnorm.ops.rms_norm_reduce_weight_grad(dwr, dwpr)
    torch.cuda.synchronize()
    assert torch.equal(dx, dxr)
    if with_weight:
        assert torch.equal(dw, dwr)


def _attn(b=2, s=200, h=8, hk=2, d=128, seed=2):
    g = torch.Generator().manual_seed(seed)
    mk = lambda *sh: torch.randn(*sh, generator=g).bfloat16().cuda()  # noqa: E731
    return mk(b, s, h, d), mk(b, s, hk, d), mk(b, s, hk, d), mk(b, s, h, d)


def test_forward_and_backward(runtime):
    import flash_attn2_rs

    ops = flash_attn2_rs.ops
    q, k, v, do = _attn()
    live = runtime.mock_live_objects()
    base = (q, k, v, None, None, True, -1, -1, 0.0)

    # fwd -> [out, lse]
    rc, res = T.call("fwd", *base)
    _ok(rc, runtime)
    items = T.array_items(res)
    assert len(items) == 2
    out, lse = T.tensor_of(items[0]), T.tensor_of(items[1])
    out_r, lse_r = ops.fwd(*base)
    torch.cuda.synchronize()
    assert torch.equal(out, out_r) and torch.equal(lse, lse_r)
    assert lse.shape == (2, 8, 200) and out.shape == q.shape

    # fwd_lse(..., out) -> lse, writing out
    out2 = torch.empty_like(q)
    rc, res2 = T.call("fwd_lse", *base, out2)
    _ok(rc, runtime)
    assert res2.type_index == T.TENSOR
    torch.cuda.synchronize()
    assert torch.equal(T.tensor_of(res2.p), lse_r) and torch.equal(out2, out_r)

    # dropout by explicit (seed, offset): arity 12
    rc, res3 = T.call("fwd", *base, 0.2, 1234, 8)
    _ok(rc, runtime)
    o3 = T.tensor_of(T.array_items(res3)[0])
    o3r, _ = ops.fwd(*base, 0.2, 1234, 8)
    torch.cuda.synchronize()
    assert torch.equal(o3, o3r)

    # return_softmax: arity 14 (..., p, state, offset, out | None, True) -> [out, lse, probabilities]
    state = torch.tensor([99, 4], dtype=torch.int64, device="cuda")
    rc, res4 = T.call("fwd", *base, 0.2, state, 0, None, True)
    _ok(rc, runtime)
    items4 = T.array_items(res4)
    assert len(items4) == 3
    o4, l4, p4 = (T.tensor_of(x) for x in items4)
    o4r, l4r, p4r = ops.fwd(*base, 0.2, state, 0, None, True)
    torch.cuda.synchronize()
    assert p4.shape == (2, 8, 256, 256)
    assert torch.equal(o4, o4r) and torch.equal(l4, l4r) and torch.equal(p4, p4r)

    # bwd_preprocess -> delta; bwd_all -> [dq, dk, dv]; bwd_dkv; bwd_dq
    rc, rd = T.call("bwd_preprocess", do, out_r, 0.0)
    _ok(rc, runtime)
    delta = T.tensor_of(rd.p)
    delta_r = ops.bwd_preprocess(do, out_r, 0.0)
    torch.cuda.synchronize()
    assert torch.equal(delta, delta_r)
    bargs = (q, k, v, do, lse_r, delta_r, None, None, True, -1, -1, 0.0, 0.0, None)
    rc, rb = T.call("bwd_all", *bargs)
    _ok(rc, runtime)
    grads = [T.tensor_of(p) for p in T.array_items(rb)]
    grads_r = ops.bwd_all(*bargs)
    rc, rkv = T.call("bwd_dkv", *bargs)
    _ok(rc, runtime)
    rc, rq = T.call("bwd_dq", *bargs)
    _ok(rc, runtime)
    torch.cuda.synchronize()
    assert len(grads) == 3 and all(torch.equal(a, b) for a, b in zip(grads, grads_r))
    dk, dv = (T.tensor_of(p) for p in T.array_items(rkv))
    assert torch.equal(dk, grads_r[1]) and torch.equal(dv, grads_r[2])
    assert torch.equal(T.tensor_of(rq.p), grads_r[0])

    # Every returned object goes away with one reference drop.
    _release(runtime, res.p, res2.p, res3.p, res4.p, rd.p, rb.p, rkv.p, rq.p)
    assert runtime.mock_live_objects() == live


def test_varlen(runtime):
    import flash_attn2_rs

    ops = flash_attn2_rs.ops
    lens = [37, 200, 1, 129]
    g = torch.Generator().manual_seed(3)
    cu = torch.tensor([0, 37, 237, 238, 367], dtype=torch.int32).cuda()
    t = sum(lens)
    q = torch.randn(t, 8, 128, generator=g).bfloat16().cuda()
    k = torch.randn(t, 2, 128, generator=g).bfloat16().cuda()
    v = torch.randn(t, 2, 128, generator=g).bfloat16().cuda()
    do = torch.randn(t, 8, 128, generator=g).bfloat16().cuda()
    live = runtime.mock_live_objects()
    fargs = (q, k, v, cu, cu, None, None, None, None, True, -1, -1, 0.0, 0.0, None, 200, 200, False, False)
    rc, rf = T.call("varlen_fwd_explicit", *fargs)
    _ok(rc, runtime)
    items = T.array_items(rf)
    assert len(items) == 3
    out, lse = T.tensor_of(items[0]), T.tensor_of(items[1])
    out_r, lse_r, _ = ops.varlen_fwd_explicit(*fargs)
    torch.cuda.synchronize()
    assert torch.equal(out, out_r) and torch.equal(lse, lse_r)
    bargs = (q, k, v, do, out_r, lse_r, cu, cu, None, None, True, -1, -1, 0.0, 0.0, None, 200, 200, False)
    rc, rb = T.call("varlen_bwd_explicit", *bargs)
    _ok(rc, runtime)
    grads = [T.tensor_of(p) for p in T.array_items(rb)]
    grads_r = ops.varlen_bwd_explicit(*bargs)
    torch.cuda.synchronize()
    assert len(grads) == 4
    for a, b in zip(grads[:3], grads_r[:3]):
        assert torch.equal(a, b)
    _release(runtime, rf.p, rb.p)
    assert runtime.mock_live_objects() == live


def test_rng_descriptors(runtime):
    """rng_state and fwd at arities 16 (reserve Function returning a Shape) and
    18 (explicit descriptor) equal the explicit-seed forward bit for bit."""
    import flash_attn2_rs

    ops = flash_attn2_rs.ops
    q, k, v, _ = _attn(d=64)
    live = runtime.mock_live_objects()
    base = (q, k, v, None, None, True, -1, -1, 0.0)
    seed, offset = 4242, 96
    ref_out, ref_lse = ops.fwd(*base, 0.2, seed, offset)

    rc, rs = T.call("rng_state", q, seed, offset, 0, False)
    _ok(rc, runtime)
    torch.cuda.synchronize()
    assert T.tensor_of(rs.p).tolist() == [seed, offset]

    state = torch.empty(2, dtype=torch.int64, device="cuda")
    rc, r18 = T.call("fwd", *base, 0.2, state, 0, None, False, seed, offset, 0, False)
    _ok(rc, runtime)
    o18, l18, p18 = (T.tensor_of(x) for x in T.array_items(r18))
    torch.cuda.synchronize()
    assert torch.equal(o18, ref_out) and torch.equal(l18, ref_lse) and p18.numel() == 0
    assert state.tolist() == [seed, offset]

    reserve = T.make_reserve(seed, offset, 0, 0)
    state2 = torch.empty(2, dtype=torch.int64, device="cuda")
    rc, r16 = T.call("fwd", *base, 0.2, state2, 0, None, False, reserve, 3)
    _ok(rc, runtime)
    o16 = T.tensor_of(T.array_items(r16)[0])
    torch.cuda.synchronize()
    assert torch.equal(o16, ref_out) and state2.tolist() == [seed, offset]
    assert [runtime.mock_reserve_arg(reserve.ptr, i) for i in range(3)] == [3, q.device.index, 2 * 8 * 32]

    _release(runtime, rs.p, r18.p, r16.p)
    assert runtime.mock_live_objects() == live
