"""torch.library registration of the activation ops, in the namespace
`kcr_activation`, for `torch.compile` and `torch.library.opcheck`.

Interface kept from the reference (activation-rs/tvm-ffi-ext/activation_rs/
torch_ops.py): the eleven op names, `(out, input)` arguments (plus `threshold`
for fatrelu_and_mul), that each op writes `out` and returns nothing. Here the
ops come from one table of names and schemas, declared on a
`torch.library.Library` with a CUDA entry that calls the C ABI shim and a fake
entry with no outputs.
"""

from __future__ import annotations

import torch

from ._ops import ops, torch_add_op_namespace_prefix

NAMESPACE = torch_add_op_namespace_prefix("silu").split("::")[0]
_lib = torch.library.Library(NAMESPACE, "DEF")

_UNARY = "(Tensor(a!) out, Tensor input) -> ()"
_SCHEMAS = {
    "silu_and_mul": _UNARY,
    "mul_and_silu": _UNARY,
    "gelu_and_mul": _UNARY,
    "gelu_tanh_and_mul": _UNARY,
    "fatrelu_and_mul": "(Tensor(a!) out, Tensor input, float threshold) -> ()",
    "gelu_new": _UNARY,
    "gelu_fast": _UNARY,
    "gelu_quick": _UNARY,
    "gelu_tanh": _UNARY,
    "silu": _UNARY,
    "gelu": _UNARY,
}


def _no_outputs(*args):
    return None


for _name, _schema in _SCHEMAS.items():
    _lib.define(_name + _schema)
    _lib.impl(_name, getattr(ops, _name), "CUDA")
    torch.library.register_fake(f"{NAMESPACE}::{_name}", _no_outputs, lib=_lib)
    globals()[_name] = getattr(getattr(torch.ops, NAMESPACE), _name).default

__all__ = sorted(_SCHEMAS)
