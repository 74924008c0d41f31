"""`RMSNormFunction` / `rms_norm`, mirroring rmsnorm/tvm-ffi-ext/rmsnorm/functional.py:15-89."""

from typing import Optional

import torch

from . import torch_ops

try:
    from torch.distributed.tensor import DTensor
except ImportError:  # torch built without distributed support
    DTensor = None

CASTING_MODES = ("llama", "gemma", "none")


def _full_tensor(tensor: torch.Tensor) -> torch.Tensor:
    # Tensor-parallel inputs are gathered so every rank normalises full rows.
    if DTensor is not None and isinstance(tensor, DTensor):
        return tensor.full_tensor()
    return tensor


class RMSNormFunction(torch.autograd.Function):
    """RMSNorm: `x / rms(x) * (offset + weight)` over the last dimension of `x`.

    `casting_mode` selects where values are rounded: "llama" (inverse RMS in f32,
    normalised x rounded to x's dtype before the weight), "gemma" (everything in
    f32, output rounded) or "none" (input-dtype math). `weight` may be None or,
    for 16-bit x, float32. With `in_place` the backward pass overwrites the output
    gradient with the input gradient.
    """

    @staticmethod
    def forward(ctx, x, weight, eps, offset=0.0, casting_mode="llama", in_place=True):
        if casting_mode not in CASTING_MODES:
            raise ValueError(
                f"Invalid casting mode {casting_mode!r}, expected one of {CASTING_MODES}"
            )
        x = _full_tensor(x).contiguous()
        if weight is not None:
            weight = weight.contiguous()
        y, rstd = torch_ops.rms_norm_forward(x, weight, float(eps), float(offset), casting_mode)
        ctx.offset = float(offset)
        ctx.casting_mode = casting_mode
        ctx.in_place = in_place
        ctx.save_for_backward(x, weight, rstd)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, weight, rstd = ctx.saved_tensors
        dy = _full_tensor(dy).contiguous()
        args = (x, weight, rstd, ctx.offset, ctx.casting_mode)
        if ctx.in_place:
            dw = torch_ops.rms_norm_backward_(dy, *args)
            dx = dy
        else:
            dx, dw = torch_ops.rms_norm_backward(dy, *args)
        return dx, (dw if weight is not None else None), None, None, None, None


def rms_norm(
    x: torch.Tensor,
    weight: Optional[torch.Tensor],
    eps: float,
    offset: float = 0.0,
    casting_mode: str = "llama",
    in_place: bool = True,
) -> torch.Tensor:
    """RMSNorm of `x`, see `RMSNormFunction`."""
    return RMSNormFunction.apply(x, weight, eps, offset, casting_mode, in_place)
