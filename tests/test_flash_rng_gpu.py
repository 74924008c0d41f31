"""GPU checks of the generator-descriptor paths of dropout
(flash-attn2-rs/src/host/rng.rs:13-98, src/device/rng.rs, host/forward/mod.rs:
132-178, 492-523): the `rng_state` op, fwd at arities 16 (reserve callback) and
18 (explicit descriptor), and the generator reservation of the Python interface
(tvm-ffi-ext/flash_attn2_rs/flash_attn_interface.py:20-73).

A descriptor (seed, offset, intragraph, captured) resolves to [seed, offset]
(captured = 0) or to [*seed, *offset + intragraph] (captured = 1, device
addresses); a forward that takes it must equal, bit for bit, the forward with
that explicit (seed, offset), and leave the values in its state tensor.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def ops():
    import flash_attn2_rs

    return flash_attn2_rs.ops


def _inputs(d=64, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(2, 100, 4, d, generator=g).bfloat16().cuda()
    k = torch.randn(2, 120, 2, d, generator=g).bfloat16().cuda()
    v = torch.randn(2, 120, 2, d, generator=g).bfloat16().cuda()
    return q, k, v


def test_rng_state_values_and_captured_pointers():
    q = torch.zeros(1, device="cuda")
    st = ops().rng_state(q, 0x1234_5678_9ABC_DEF0, 96, 5, False)
    assert st.tolist() == [0x1234_5678_9ABC_DEF0, 96]
    seed_t = torch.tensor([-7], dtype=torch.int64, device="cuda")
    off_t = torch.tensor([1000], dtype=torch.int64, device="cuda")
    st = ops().rng_state(q, seed_t.data_ptr(), off_t.data_ptr(), 24, True)
    assert st.tolist() == [-7, 1024]
    # The pointers are read at launch time, on the stream.
    off_t.fill_(2000)
    st = ops().rng_state(q, seed_t.data_ptr(), off_t.data_ptr(), 24, True)
    assert st.tolist() == [-7, 2024]
    with pytest.raises(ValueError, match="aligned non-null"):
        ops().rng_state(q, 0, 8, 0, True)


def test_fwd_descriptor_arities_equal_explicit_seed():
    q, k, v = _inputs()
    base = (q, k, v, None, None, True, -1, -1, 0.0)
    seed, offset, p = 31337, 64, 0.2
    ref_out, ref_lse = ops().fwd(*base, p, seed, offset)
    # Arity 18: explicit descriptor.
    state = torch.empty(2, dtype=torch.int64, device="cuda")
    out, lse, probs = ops().fwd(*base, p, state, 0, None, False, seed, offset, 0, False)
    assert torch.equal(out, ref_out) and torch.equal(lse, ref_lse) and probs.numel() == 0
    assert state.tolist() == [seed, offset]
    # Arity 18 with captured pointers: offset = *offset + intragraph.
    seed_t = torch.tensor([seed], dtype=torch.int64, device="cuda")
    off_t = torch.tensor([offset - 32], dtype=torch.int64, device="cuda")
    state2 = torch.empty(2, dtype=torch.int64, device="cuda")
    out2, _, _ = ops().fwd(*base, p, state2, 0, None, False, seed_t.data_ptr(), off_t.data_ptr(), 32, True)
    assert torch.equal(out2, ref_out) and state2.tolist() == [seed, offset]
    # Arity 16: the reserve callback gets (generator, device, B * H * 32).
    calls = []

    def reserve(generator, device, increment):
        calls.append((generator, device, increment))
        return (seed, offset, 0, 0)

    state3 = torch.empty(2, dtype=torch.int64, device="cuda")
    out3, lse3, _ = ops().fwd(*base, p, state3, 0, None, False, reserve, 5)
    assert calls == [(5, q.device.index, 2 * 4 * 32)]
    assert torch.equal(out3, ref_out) and torch.equal(lse3, ref_lse) and state3.tolist() == [seed, offset]
    # Arity 16 with return_softmax: probabilities follow the reserved state.
    out4, _, probs4 = ops().fwd(*base, p, state3, 0, None, True, reserve, 5)
    ref4 = ops().fwd(*base, p, ops().rng_state(q, seed, offset, 0, False), 0, None, True)
    assert torch.equal(out4, ref_out) and torch.equal(probs4, ref4[2])
    with pytest.raises(ValueError, match="D64"):
        qq, kk, vv = _inputs(d=128)
        ops().fwd(qq, kk, vv, None, None, True, -1, -1, 0.0, p, state, 0, None, False, seed, offset, 0, False)


def test_generator_reservation_matches_philox_offsets():
    """fwd(gen=...) reserves [initial seed, current Philox offset] and advances
    the offset by B * H * 32, so two generators in the same state give the same
    state tensor, mask and output."""
    import flash_attn2_rs

    q, k, v = _inputs()
    g1 = torch.Generator(device="cuda").manual_seed(17)
    g2 = torch.Generator(device="cuda").manual_seed(17)
    before = g1.get_offset()
    out1, _, _, st1 = flash_attn2_rs.fwd(q, k, v, p_dropout=0.17, gen=g1)
    assert st1.tolist() == [17 & 0xFFFF_FFFF_FFFF_FFFF, before]
    assert g1.get_offset() == before + 2 * 4 * 32
    out2, _, _, st2 = flash_attn2_rs.fwd(q, k, v, p_dropout=0.17, gen=g2)
    assert torch.equal(st1, st2) and torch.equal(out1, out2)
    st3 = flash_attn2_rs.reserve_rng_state(q, g1)
    assert st3.tolist() == [17, before + 2 * 4 * 32] and g1.get_offset() == before + 4 * 4 * 32
    with pytest.raises(TypeError):
        flash_attn2_rs.reserve_rng_state(q, torch.Generator())
