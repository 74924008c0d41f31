"""`ops` of activation-rs: the 11 exports of activation-rs/src/ops.rs:255-265 with
their positional signatures, backed by libkcr_hip.so.

Each op writes into the preallocated `out` and returns None, like the tvm-ffi
exports (`silu_and_mul(out, input)`, ops.rs:200).
"""

import ctypes
from types import SimpleNamespace

from kcr_native import call, describe, op_namespace_prefixer, ref, stream_of

torch_add_op_namespace_prefix = op_namespace_prefixer("activation")


def _unary(symbol):
    def op(out, input):
        o, i = describe(out), describe(input)
        call(symbol, ref(o), ref(i), stream_of(input, out))

    op.__name__ = symbol[len("kcr_"):]
    return op


def fatrelu_and_mul(out, input, threshold):
    o, i = describe(out), describe(input)
    call("kcr_fatrelu_and_mul", ref(o), ref(i), ctypes.c_double(float(threshold)),
         stream_of(input, out))


ops = SimpleNamespace(
    silu_and_mul=_unary("kcr_silu_and_mul"),
    mul_and_silu=_unary("kcr_mul_and_silu"),
    gelu_and_mul=_unary("kcr_gelu_and_mul"),
    gelu_tanh_and_mul=_unary("kcr_gelu_tanh_and_mul"),
    fatrelu_and_mul=fatrelu_and_mul,
    gelu=_unary("kcr_gelu"),
    gelu_tanh=_unary("kcr_gelu_tanh"),
    gelu_new=_unary("kcr_gelu_new"),
    gelu_fast=_unary("kcr_gelu_fast"),
    gelu_quick=_unary("kcr_gelu_quick"),
    silu=_unary("kcr_silu"),
)
