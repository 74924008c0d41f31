"""`ops` of rmsnorm: the three exports of rmsnorm/src/ops.rs:442-444 with their
positional signatures, backed by libkcr_hip.so. Every op writes into
preallocated outputs and returns None."""

import ctypes
from types import SimpleNamespace

from kcr_native import call, describe, op_namespace_prefixer, ref, stream_of

torch_add_op_namespace_prefix = op_namespace_prefixer("rmsnorm")


def rms_norm_forward(y, rstd, x, weight, eps, offset, casting_mode):
    """rmsnorm/src/ops.rs:237-265."""
    d = [describe(t) for t in (y, rstd, x, weight)]
    call(
        "kcr_rms_norm_forward",
        *(ref(t) for t in d),
        ctypes.c_double(float(eps)),
        ctypes.c_double(float(offset)),
        ctypes.c_char_p(str(casting_mode).encode()),
        stream_of(x, y),
    )


def rms_norm_backward(dx, dw_partial, dy, x, weight, rstd, offset, casting_mode):
    """rmsnorm/src/ops.rs:326-380; dy=None reads the gradient from dx in place."""
    d = [describe(t) for t in (dx, dw_partial, dy, x, weight, rstd)]
    call(
        "kcr_rms_norm_backward",
        *(ref(t) for t in d),
        ctypes.c_double(float(offset)),
        ctypes.c_char_p(str(casting_mode).encode()),
        stream_of(x, dx),
    )


def rms_norm_reduce_weight_grad(dw, dw_partial):
    """rmsnorm/src/ops.rs:383-440."""
    a, b = describe(dw), describe(dw_partial)
    call("kcr_rms_norm_reduce_weight_grad", ref(a), ref(b), stream_of(dw, dw_partial))


ops = SimpleNamespace(
    rms_norm_forward=rms_norm_forward,
    rms_norm_backward=rms_norm_backward,
    rms_norm_reduce_weight_grad=rms_norm_reduce_weight_grad,
)
