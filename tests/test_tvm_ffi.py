"""The __tvm_ffi_* packed exports on the CPU: argument decoding and error
raising through the caller's tvm-ffi runtime (a mock of its entry points, since
no tvm-ffi runtime exists in this image). Validation happens before any device
work, so nothing here touches a GPU."""

import ctypes

import pytest
import torch

import tvm_ffi_util as T


@pytest.fixture(autouse=True)
def runtime():
    return T.mock()


def _err(m):
    return m.mock_error_kind().decode(), m.mock_error_message().decode()


def test_wrong_argument_type_raises_type_error(runtime):
    rc, _ = T.call("silu_and_mul", 1.5, None)
    assert rc == -1
    kind, msg = _err(runtime)
    assert kind == "TypeError" and "argument #0: expected a Tensor" in msg


def test_fwd_arity_is_the_reference_table(runtime):
    x = torch.zeros(1, 4, 1, 8, dtype=torch.half)
    rc, _ = T.call("fwd", x, x, x, None, None, False, -1, -1, 0.0, 0.0, 1)
    assert rc == -1
    kind, msg = _err(runtime)
    assert kind == "ValueError" and "fwd expects 9 positional arguments" in msg
    rc, _ = T.call("fwd", *([x] * 3), None, None, False, -1, -1, 0.0, 0.0, 1, 2, None, True, 5)
    assert rc == -1 and "fwd expects 9 positional arguments" in _err(runtime)[1]


def test_fwd_return_softmax_validation(runtime):
    """Arity 14 (..., p, state, offset, out, return_softmax): probabilities need
    dropout and an RNG-state tensor, and fwd_lse cannot return them
    (host/forward/mod.rs:181-199)."""
    x = torch.zeros(1, 4, 1, 8, dtype=torch.half)
    state = torch.zeros(2, dtype=torch.int64)
    rc, _ = T.call("fwd", *([x] * 3), None, None, False, -1, -1, 0.0, 0.0, state, 0, None, True)
    assert rc == -1
    kind, msg = _err(runtime)
    assert kind == "ValueError" and "return_softmax requires nonzero dropout" in msg
    rc, _ = T.call("fwd", *([x] * 3), None, None, False, -1, -1, 0.0, 0.2, 7, 0, None, True)
    assert rc == -1 and "RNG-state tensor" in _err(runtime)[1]
    rc, _ = T.call("fwd_lse", *([x] * 3), None, None, False, -1, -1, 0.0, 0.2, state, 0, x, True)
    assert rc == -1 and "cannot return diagnostic probabilities" in _err(runtime)[1]


def test_fwd_lse_requires_an_output(runtime):
    x = torch.zeros(1, 4, 1, 8, dtype=torch.half)
    rc, _ = T.call("fwd_lse", x, x, x, None, None, False, -1, -1, 0.0)
    assert rc == -1 and "requires a supplied output" in _err(runtime)[1]


def test_host_tensors_are_refused_by_the_c_abi(runtime):
    import kcr_native

    x = torch.randn(7, 512, dtype=torch.half)
    rc, _ = T.call("silu_and_mul", torch.empty(7, 256, dtype=torch.half), x)
    assert rc == -1
    kind, msg = _err(runtime)
    assert kind == "ValueError" and "GPU tensor" in msg
    assert "GPU tensor" in kcr_native.lib.kcr_last_error().decode()


def test_rms_norm_string_arguments(runtime):
    """casting_mode arrives as a small string (<= 7 bytes inline) or a C string;
    an unknown mode raises the reference's error."""
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    rstd = torch.zeros(4)
    rc, _ = T.call("rms_norm_forward", x, rstd, x, None, 1e-6, 0.0, "llama2")
    assert rc == -1 and "casting mode" in _err(runtime)[1]
    rc, _ = T.call("rms_norm_forward", x, rstd, x, None, 1e-6, 0.0, "not-a-casting-mode")
    assert rc == -1 and "casting mode" in _err(runtime)[1]


def test_backward_needs_fourteen_arguments(runtime):
    x = torch.zeros(1, 4, 1, 8, dtype=torch.half)
    rc, _ = T.call("bwd_all", x, x, x)
    assert rc == -1 and "backward component expects" in _err(runtime)[1]


def test_fwd_descriptor_arities_validation(runtime):
    """Arity 16 calls reserve(generator, device, B*H*32) and needs a 4-element
    Shape; arity 18 needs nonempty D64 dropout and aligned capture pointers
    (host/forward/mod.rs:132-178, 492-523). All fail before any device work."""
    x = torch.zeros(2, 4, 3, 64, dtype=torch.half)
    state = torch.zeros(2, dtype=torch.int64)
    base = (x, x, x, None, None, False, -1, -1, 0.0)
    reserve = T.make_reserve(1, 2, 3)  # three values: invalid
    rc, _ = T.call("fwd", *base, 0.0, state, 0, None, False, reserve, 7)
    assert rc == -1 and "native reservation requires dropout" in _err(runtime)[1]
    rc, _ = T.call("fwd", *base, 0.2, state, 0, None, False, reserve, 7)
    assert rc == -1 and "invalid reserved RNG descriptor" in _err(runtime)[1]
    assert runtime.mock_reserve_calls(reserve.ptr) == 1
    assert [runtime.mock_reserve_arg(reserve.ptr, i) for i in range(3)] == [7, 0, 2 * 3 * 32]
    rc, _ = T.call("fwd", *base, 0.2, state, 0, None, False, T.make_reserve(8, 0, 0, 1), 7)
    assert rc == -1 and "invalid reserved capture pointers" in _err(runtime)[1]
    rc, _ = T.call("fwd", *base, 0.2, state, 0, None, False, 1, 2, 0, True)
    assert rc == -1 and "invalid capture descriptor pointers" in _err(runtime)[1]
    rc, _ = T.call("fwd", *base, 0.2, state, 0, None, True, 1, 2, 0, False)
    assert rc == -1 and "does not support diagnostic probabilities" in _err(runtime)[1]
    y = torch.zeros(1, 4, 1, 128, dtype=torch.half)
    rc, _ = T.call("fwd", y, y, y, None, None, False, -1, -1, 0.0, 0.2, state, 0, None, False, 1, 2, 0, False)
    assert rc == -1 and "RNG descriptor requires nonempty D64 dropout" in _err(runtime)[1]
    rc, _ = T.call("fwd", *base, 0.2, state, 3, None, False, 1, 2, 0, False)
    assert rc == -1 and "offset must be zero" in _err(runtime)[1]


def test_rng_state_export_validation(runtime):
    x = torch.zeros(4)
    rc, _ = T.call("rng_state", x, 1, 2, 3)
    assert rc == -1 and "rng_state expects reference" in _err(runtime)[1]
    rc, _ = T.call("rng_state", x, 1, 2, 3, False)
    assert rc == -1 and "CUDA reference tensor" in _err(runtime)[1]
