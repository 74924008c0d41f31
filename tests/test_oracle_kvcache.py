"""Pins oracle.kvcache (CPU): rotary against an independent complex rotation,
identity / norm invariants, append-then-attend against attention over the
concatenated keys, and paged == contiguous."""

import numpy as np
import pytest

from oracle import attention as OA
from oracle import kvcache as KV
from oracle.numerics import round_bf16


def _tables(positions, rd, seed=0):
    rng = np.random.default_rng(seed)
    theta = rng.uniform(0, 2 * np.pi, size=(positions, rd // 2)).astype(np.float32)
    return round_bf16(np.cos(theta)), round_bf16(np.sin(theta))


@pytest.mark.parametrize("interleaved", [True, False])
def test_rotary_matches_complex_rotation(interleaved):
    rng = np.random.default_rng(1)
    D, rd, P = 64, 32, 50
    cos, sin = _tables(P, rd)
    x = round_bf16(rng.standard_normal((20, D)).astype(np.float32))
    pos = rng.integers(0, P, size=20)
    got = KV.rotate_rows(x, pos, cos, sin, interleaved, "bf16")
    # Independent statement: each pair is a complex number multiplied by e^{i theta}.
    if interleaved:
        z = x[:, 0:rd:2].astype(np.float64) + 1j * x[:, 1:rd:2]
    else:
        z = x[:, :rd // 2].astype(np.float64) + 1j * x[:, rd // 2:rd]
    w = z * (cos[pos].astype(np.float64) + 1j * sin[pos].astype(np.float64))
    want = x.astype(np.float64).copy()
    if interleaved:
        want[:, 0:rd:2], want[:, 1:rd:2] = w.real, w.imag
    else:
        want[:, :rd // 2], want[:, rd // 2:rd] = w.real, w.imag
    # Two f32 roundings plus one bf16 rounding: within 1 bf16 ulp of the exact value.
    ulp = np.spacing(np.abs(want).astype(np.float32) * 1.0001).astype(np.float64) * 2 ** 16
    assert np.all(np.abs(got - want) <= ulp + 1e-30)
    assert np.array_equal(got[:, rd:], x[:, rd:])  # columns past rotary_dim untouched


@pytest.mark.parametrize("interleaved", [True, False])
def test_rotary_identity_and_norm(interleaved):
    rng = np.random.default_rng(2)
    D, rd = 32, 32
    cos = np.ones((4, rd // 2), np.float32)
    sin = np.zeros((4, rd // 2), np.float32)
    x = round_bf16(rng.standard_normal((8, D)).astype(np.float32))
    assert np.array_equal(KV.rotate_rows(x, np.zeros(8, int), cos, sin, interleaved, "bf16"), x)
    c, s = _tables(4, rd, seed=3)
    y = KV.rotate_rows(x.astype(np.float32), np.full(8, 2), c.astype(np.float32), s.astype(np.float32),
                       interleaved, "f32")
    # |e^{i theta}| = 1 up to the bf16 rounding of the tables.
    np.testing.assert_allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x, axis=1), rtol=2e-2)


def test_append_then_attend_equals_concatenated_attention():
    rng = np.random.default_rng(4)
    B, cap, Hk, H, D, snew, sq = 2, 40, 2, 4, 16, 3, 3
    kc = rng.standard_normal((B, cap, Hk, D)).astype(np.float32)
    vc = rng.standard_normal((B, cap, Hk, D)).astype(np.float32)
    k = rng.standard_normal((B, snew, Hk, D)).astype(np.float32)
    v = rng.standard_normal((B, snew, Hk, D)).astype(np.float32)
    q = rng.standard_normal((B, sq, H, D)).astype(np.float32)
    lengths = np.array([10, 25])
    kc2, vc2 = KV.append(kc, vc, k, v, lengths, dtype="f32")
    out, lse = KV.attend(q, kc2, vc2, lengths + snew, causal=True)
    for b in range(B):
        kk = np.concatenate([kc[b, :lengths[b]], k[b]])[None]
        vv = np.concatenate([vc[b, :lengths[b]], v[b]])[None]
        eo, el = OA.forward(q[b:b + 1], kk, vv, causal=True)
        np.testing.assert_allclose(out[b], eo[0], rtol=1e-6, atol=1e-6)
        np.testing.assert_allclose(lse[b], el[0], rtol=1e-6, atol=1e-6)
    # Rows outside the append are untouched.
    assert np.array_equal(kc2[0, 13:], kc[0, 13:]) and np.array_equal(kc2[1, :25], kc[1, :25])


def test_paged_equals_contiguous():
    rng = np.random.default_rng(5)
    B, page, cols, Hk, H, D = 2, 4, 3, 1, 2, 8
    cap = page * cols
    kc = rng.standard_normal((B, cap, Hk, D)).astype(np.float32)
    vc = rng.standard_normal((B, cap, Hk, D)).astype(np.float32)
    table = rng.permutation(B * cols).reshape(B, cols).astype(np.int32)
    kp = np.zeros((B * cols, page, Hk, D), np.float32)
    vp = np.zeros_like(kp)
    for b in range(B):
        for c in range(cols):
            kp[table[b, c]] = kc[b, c * page:(c + 1) * page]
            vp[table[b, c]] = vc[b, c * page:(c + 1) * page]
    q = rng.standard_normal((B, 2, H, D)).astype(np.float32)
    k = rng.standard_normal((B, 2, Hk, D)).astype(np.float32)
    v = rng.standard_normal((B, 2, Hk, D)).astype(np.float32)
    lengths = np.array([3, 7])
    kc2, vc2 = KV.append(kc, vc, k, v, lengths, dtype="f32")
    kp2, vp2 = KV.append(kp, vp, k, v, lengths, block_table=table, dtype="f32")
    a = KV.attend(q, kc2, vc2, lengths + 2, causal=True)
    p = KV.attend(q, kp2, vp2, lengths + 2, block_table=table, causal=True)
    np.testing.assert_array_equal(a[0], p[0])
    np.testing.assert_array_equal(a[1], p[1])
