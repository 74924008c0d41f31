"""Autograd entry points of RMSNorm: `RMSNormFunction` and `rms_norm`.

Interface kept from the reference (rmsnorm/tvm-ffi-ext/rmsnorm/functional.py):
the class and function names, `RMSNormFunction.apply(x, weight, eps, offset,
casting_mode, in_place)`, the accepted casting modes and the ValueError text for
others, the float32-weight option, the in-place backward, and that
tensor-parallel (DTensor) inputs and gradients are gathered to full tensors so
every rank normalises whole rows.
"""

from __future__ import annotations

import functools
from typing import NamedTuple, Optional

import torch

from . import torch_ops

CASTING_MODES = ("llama", "gemma", "none")


@functools.lru_cache(maxsize=None)
def _dtensor_type():
    """torch's DTensor class, or None for a torch built without distributed."""
    try:
        from torch.distributed.tensor import DTensor
    except ImportError:
        return None
    return DTensor


def _as_local(t: torch.Tensor) -> torch.Tensor:
    """A whole, contiguous tensor: DTensor shards are gathered first."""
    dtensor = _dtensor_type()
    if dtensor is not None and isinstance(t, dtensor):
        t = t.full_tensor()
    return t.contiguous()


class _Saved(NamedTuple):
    offset: float
    casting_mode: str
    in_place: bool


class RMSNormFunction(torch.autograd.Function):
    """RMSNorm over the last dimension: `x / rms(x) * (offset + weight)`.

    `casting_mode` picks the rounding points: "llama" (inverse RMS in float32,
    x / rms rounded to x's dtype before the weight), "gemma" (all float32, one
    rounding at the end; Gemma also uses offset = 1) or "none" (input-dtype
    arithmetic). `weight` may be None or, for 16-bit x, float32. With `in_place`
    the backward pass overwrites the incoming gradient with the input gradient,
    so the caller must not reuse that gradient tensor.
    """

    @staticmethod
    def forward(ctx, x, weight, eps, offset=0.0, casting_mode="llama", in_place=True):
        if casting_mode not in CASTING_MODES:
            raise ValueError(f"Invalid casting mode {casting_mode!r}, expected one of {CASTING_MODES}")
        x = _as_local(x)
        weight = None if weight is None else weight.contiguous()
        y, rstd = torch_ops.rms_norm_forward(x, weight, float(eps), float(offset), casting_mode)
        ctx.saved = _Saved(float(offset), casting_mode, bool(in_place))
        ctx.save_for_backward(x, weight, rstd)
        return y

    @staticmethod
    def backward(ctx, grad_y):
        x, weight, rstd = ctx.saved_tensors
        saved = ctx.saved
        grad_y = _as_local(grad_y)
        if saved.in_place:
            dw = torch_ops.rms_norm_backward_(grad_y, x, weight, rstd, saved.offset, saved.casting_mode)
            dx = grad_y
        else:
            dx, dw = torch_ops.rms_norm_backward(grad_y, x, weight, rstd, saved.offset, saved.casting_mode)
        # gradients of (x, weight, eps, offset, casting_mode, in_place)
        return dx, None if weight is None else dw, None, None, None, None


def rms_norm(
    x: torch.Tensor,
    weight: Optional[torch.Tensor],
    eps: float,
    offset: float = 0.0,
    casting_mode: str = "llama",
    in_place: bool = True,
) -> torch.Tensor:
    """RMSNorm of `x` (see `RMSNormFunction`), differentiable in x and weight."""
    return RMSNormFunction.apply(x, weight, eps, offset, casting_mode, in_place)
