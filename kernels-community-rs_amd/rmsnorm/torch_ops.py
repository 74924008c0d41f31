"""torch.library registration of the RMSNorm ops, in the namespace `kcr_rmsnorm`.

The op names, their argument order and types, the returned tensors and the
in-place variant's write into `dy` are the reference package's interface
(rmsnorm/tvm-ffi-ext/rmsnorm/torch_ops.py). Here each op is declared by an
explicit schema on a `torch.library.Library`, with a CUDA kernel entry and a
fake (meta) entry for tracing; the backward chooses its partial weight-gradient
row count from the row count (`partial_rows`).
"""

from __future__ import annotations

import functools

import torch

from ._ops import ops, torch_add_op_namespace_prefix

_QUALIFIED = torch_add_op_namespace_prefix("rms_norm_forward")
NAMESPACE = _QUALIFIED.split("::")[0]
_lib = torch.library.Library(NAMESPACE, "DEF")

_SCHEMAS = {
    "rms_norm_forward":
        "(Tensor x, Tensor? weight, float eps, float offset, str casting_mode) -> (Tensor, Tensor)",
    "rms_norm_backward":
        "(Tensor dy, Tensor x, Tensor? weight, Tensor rstd, float offset, str casting_mode)"
        " -> (Tensor, Tensor)",
    "rms_norm_backward_":
        "(Tensor(a!) dy, Tensor x, Tensor? weight, Tensor rstd, float offset, str casting_mode)"
        " -> Tensor",
}


@functools.lru_cache(maxsize=None)
def _compute_units(index: int) -> int:
    return torch.cuda.get_device_properties(index).multi_processor_count


def partial_rows(rows: int, device: torch.device) -> int:
    """Rows of the float32 weight-gradient partials: one per backward wave, at
    most four per CU (the measured best at 16384 x 4096), never more than there
    are rows, at least one (the op requires a non-empty partial buffer)."""
    return max(1, min(int(rows), 4 * _compute_units(device.index or 0)))


def _rstd_like(x: torch.Tensor) -> torch.Tensor:
    return torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)


def _weight_grad_of(x, weight, fill):
    """The weight gradient: `fill(dw_partial)` runs the backward kernel into the
    partials, which are then reduced into dw (empty without a weight)."""
    if weight is None:
        fill(None)
        return x.new_empty(0)
    rows = x.numel() // max(x.shape[-1], 1)
    dw_partial = torch.empty(partial_rows(rows, x.device), x.shape[-1], dtype=torch.float32,
                             device=x.device)
    fill(dw_partial)
    dw = torch.empty_like(weight)
    ops.rms_norm_reduce_weight_grad(dw, dw_partial)
    return dw


def _forward_cuda(x, weight, eps, offset, casting_mode):
    y, rstd = torch.empty_like(x), _rstd_like(x)
    ops.rms_norm_forward(y, rstd, x, weight, eps, offset, casting_mode)
    return y, rstd


def _backward_cuda(dy, x, weight, rstd, offset, casting_mode):
    dx = torch.empty_like(dy)
    dw = _weight_grad_of(
        x, weight, lambda part: ops.rms_norm_backward(dx, part, dy, x, weight, rstd, offset, casting_mode))
    return dx, dw


def _backward_inplace_cuda(dy, x, weight, rstd, offset, casting_mode):
    return _weight_grad_of(
        x, weight, lambda part: ops.rms_norm_backward(dy, part, None, x, weight, rstd, offset, casting_mode))


def _forward_fake(x, weight, eps, offset, casting_mode):
    return torch.empty_like(x), _rstd_like(x)


def _backward_fake(dy, x, weight, rstd, offset, casting_mode):
    return torch.empty_like(dy), (x.new_empty(0) if weight is None else torch.empty_like(weight))


def _backward_inplace_fake(dy, x, weight, rstd, offset, casting_mode):
    return x.new_empty(0) if weight is None else torch.empty_like(weight)


for _name, _cuda, _fake in (
    ("rms_norm_forward", _forward_cuda, _forward_fake),
    ("rms_norm_backward", _backward_cuda, _backward_fake),
    ("rms_norm_backward_", _backward_inplace_cuda, _backward_inplace_fake),
):
    _lib.define(_name + _SCHEMAS[_name])
    _lib.impl(_name, _cuda, "CUDA")
    torch.library.register_fake(f"{NAMESPACE}::{_name}", _fake, lib=_lib)

_namespace = getattr(torch.ops, NAMESPACE)
rms_norm_forward = _namespace.rms_norm_forward.default
rms_norm_backward = _namespace.rms_norm_backward.default
rms_norm_backward_ = _namespace.rms_norm_backward_.default
