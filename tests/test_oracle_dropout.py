"""Pins of the dropout mask stream oracle (oracle/dropout.py)."""

import numpy as np

from oracle import dropout as DR


def test_philox_round_function_matches_random123_known_answers():
    # Random123 kat_vectors, philox4x32 with 10 rounds (the reference uses the
    # same round function and key schedule with 7 rounds).
    cases = [
        ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
        ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
        ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
         (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
    ]
    for ctr, key, expected in cases:
        got = DR.philox4x32(*ctr, *key, rounds=10)
        assert tuple(int(x) for x in got) == expected


def test_keep_rate_and_threshold():
    assert DR.threshold(0.0) == 255
    assert DR.threshold(0.5) == 127
    assert DR.threshold(0.1) == int(np.float32(np.float32(0.9) * 255))
    m = DR.dense_mask(1234, 0, 2, 4, 256, 256, 0.25)
    rate = m.mean()
    expected = (DR.threshold(0.25) + 1) / 256
    assert abs(rate - expected) < 0.005


def test_mask_depends_on_head_seed_offset_and_is_reproducible():
    a = DR.keep_mask(7, 0, 0, 64, 96, 0.5)
    assert np.array_equal(a, DR.keep_mask(7, 0, 0, 64, 96, 0.5))
    assert not np.array_equal(a, DR.keep_mask(7, 0, 1, 64, 96, 0.5))
    assert not np.array_equal(a, DR.keep_mask(8, 0, 0, 64, 96, 0.5))
    # Head bh at offset o reads the same counters as head bh + 1 at offset o - 32.
    assert np.array_equal(DR.keep_mask(7, 64, 0, 64, 96, 0.5), DR.keep_mask(7, 32, 1, 64, 96, 0.5))


def test_dropout_attention_gradients_match_torch_autograd():
    import torch

    from oracle import attention as OA

    rng = np.random.default_rng(3)
    B, S, H, Hk, D = 1, 40, 4, 2, 16
    q, k, v, do = (rng.standard_normal(sh).astype(np.float64) for sh in
                   [(B, S, H, D), (B, S, Hk, D), (B, S, Hk, D), (B, S, H, D)])
    p = 0.3
    mask = DR.dense_mask(99, 64, B, H, S, S, p)
    out, lse = OA.forward(q, k, v, causal=True, dtype=np.float64, dropout_mask=mask, p_dropout=p)
    dq, dk, dv, delta = OA.backward(q, k, v, out, do, lse, causal=True, dtype=np.float64,
                                    dropout_mask=mask, p_dropout=p)
    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    kk = tk.repeat_interleave(H // Hk, dim=2)
    vv = tv.repeat_interleave(H // Hk, dim=2)
    s = torch.einsum("bqhd,bkhd->bhqk", tq, kk) / np.sqrt(D)
    s = s.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
    keep = float(np.float32(1) - np.float32(p))
    pm = torch.softmax(s, -1) * torch.tensor(mask) / keep
    o = torch.einsum("bhqk,bkhd->bqhd", pm, vv)
    o.backward(torch.tensor(do))
    np.testing.assert_allclose(out, o.detach().numpy(), rtol=1e-10, atol=1e-12)
    for got, ref in ((dq, tq.grad), (dk, tk.grad), (dv, tv.grad)):
        np.testing.assert_allclose(got, ref.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(delta, keep * np.einsum("bqhd,bqhd->bhq", do, out), rtol=1e-12)


def test_varlen_dropout_equals_per_sequence_dense():
    from oracle import attention as OA

    rng = np.random.default_rng(4)
    lens = [13, 40, 7]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T, H, D = sum(lens), 2, 8
    q, k, v = (rng.standard_normal((T, H, D)).astype(np.float32) for _ in range(3))
    out, lse = OA.varlen_forward(q, k, v, cu, cu, causal=True, dropout=(5, 0, 0.5))
    for b, (s0, s1) in enumerate(zip(cu[:-1], cu[1:])):
        n = s1 - s0
        mask = np.stack([DR.keep_mask(5, 0, b * H + h, n, n, 0.5) for h in range(H)])[None]
        o, l = OA.forward(q[None, s0:s1], k[None, s0:s1], v[None, s0:s1], causal=True,
                          dropout_mask=mask, p_dropout=0.5)
        np.testing.assert_allclose(out[s0:s1], o[0], rtol=1e-6, atol=1e-6)
