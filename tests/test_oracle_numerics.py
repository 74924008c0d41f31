"""Pins oracle/numerics.py against torch's own dtype conversions."""

import numpy as np
import torch

from oracle.numerics import round_bf16, round_f16, ulp_distance_bf16


def test_round_bf16_matches_torch_on_random_f32():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(1 << 16).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 1 << 16)
    x = x.astype(np.float32)
    ours = round_bf16(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(ours, theirs)


def test_round_bf16_ties_to_even():
    # 1 + 2^-8 is exactly halfway between bf16 1.0 and 1 + 2^-7: rounds to even (1.0).
    assert round_bf16(np.float32(1 + 2.0**-8)) == np.float32(1.0)
    # 1 + 3 * 2^-8 is halfway between 1 + 2^-7 (odd) and 1 + 2^-6 (even): rounds up.
    assert round_bf16(np.float32(1 + 3 * 2.0**-8)) == np.float32(1 + 2.0**-6)
    assert np.isnan(round_bf16(np.float32(np.nan)))
    assert round_bf16(np.float32(np.inf)) == np.inf


def test_round_bf16_is_identity_on_every_bf16_value():
    bits = np.arange(1 << 16, dtype=np.uint32) << 16
    x = bits.view(np.float32)
    finite = np.isfinite(x)
    np.testing.assert_array_equal(round_bf16(x)[finite], x[finite])


def test_round_f16_matches_torch():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(4096) * 100).astype(np.float32)
    np.testing.assert_array_equal(round_f16(x), torch.from_numpy(x).half().float().numpy())


def test_ulp_distance():
    a = np.float32([1.0, -1.0, 0.0])
    b = np.float32([1.0 + 2.0**-7, -1.0 - 2.0**-7, -0.0])
    np.testing.assert_array_equal(ulp_distance_bf16(a, b), [1, 1, 0])
