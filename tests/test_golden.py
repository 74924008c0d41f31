"""The committed golden fixtures (tests/golden/*.npz) against the generator recipe
and the oracle: the seeded inputs regenerate bit for bit, and the oracle
reproduces the stored outputs. A change to the oracle or to the input recipe
that moves a result shows up here before any GPU test runs."""

import sys
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))

import make_golden as G  # noqa: E402


@pytest.mark.parametrize("name", sorted(G.FIXTURES))
def test_fixture_regenerates(name):
    stored = np.load(GOLDEN / name)
    fresh = G.FIXTURES[name]()
    assert sorted(stored.files) == sorted(fresh)
    for key in stored.files:
        a, b = stored[key], fresh[key]
        assert a.shape == b.shape and a.dtype == b.dtype, key
        if a.dtype == np.float32:
            np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-7, err_msg=key)
        else:
            np.testing.assert_array_equal(a, b, err_msg=key)


def test_fixture_known_answers():
    d = np.load(GOLDEN / "fa_dense_causal_b1_h4_s128_d64.npz")
    v = G.from_bits(d["v"])
    # Causal row 0 sees key 0 only: O[0] == V[0] exactly, LSE = scale * q0.k0.
    np.testing.assert_allclose(d["out"][0, 0], v[0, 0], rtol=0, atol=1e-6)
    q, k = G.from_bits(d["q"]), G.from_bits(d["k"])
    s00 = (q[0, 0] * k[0, 0]).sum(-1) / np.sqrt(64.0)
    np.testing.assert_allclose(d["lse"][0, :, 0], s00, rtol=1e-5)
    r = np.load(GOLDEN / "rms_norm_llama_16x4096.npz")
    x = G.from_bits(r["x"])
    np.testing.assert_allclose(r["rstd"], 1.0 / np.sqrt((x * x).mean(-1) + 1e-6), rtol=1e-5)
