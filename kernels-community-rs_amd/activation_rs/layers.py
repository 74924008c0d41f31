"""nn.Module wrappers of the activation ops, mirroring
activation-rs/tvm-ffi-ext/activation_rs/layers.py:7-201 (same class names,
same shape rules: gated layers halve the last dimension)."""

import torch
import torch.nn as nn

from . import torch_ops as ops


def _gated(x: torch.Tensor, op) -> torch.Tensor:
    if not x.is_contiguous():
        x = x.contiguous()
    d = x.shape[-1] // 2
    out = torch.empty(x.shape[:-1] + (d,), dtype=x.dtype, device=x.device)
    op(out, x)
    return out


def _elementwise(x: torch.Tensor, op) -> torch.Tensor:
    if not x.is_contiguous():
        x = x.contiguous()
    out = torch.empty_like(x)
    op(out, x)
    return out


class SiluAndMul(nn.Module):
    """x -> silu(x[..., :d]) * x[..., d:] with d = x.shape[-1] // 2."""

    can_torch_compile: bool = True

    def forward(self, x: torch.Tensor):
        return _gated(x, ops.silu_and_mul)


class MulAndSilu(nn.Module):
    """x -> x[..., :d] * silu(x[..., d:])."""

    can_torch_compile: bool = True

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _gated(x, ops.mul_and_silu)


class GeluAndMul(nn.Module):
    """x -> gelu(x[..., :d]) * x[..., d:] (exact erf GELU)."""

    can_torch_compile: bool = True

    def forward(self, x: torch.Tensor):
        return _gated(x, ops.gelu_and_mul)


class GeluTanhAndMul(nn.Module):
    can_torch_compile: bool = True

    def forward(self, x: torch.Tensor):
        return _gated(x, ops.gelu_tanh_and_mul)


class FatreluAndMul(nn.Module):
    """x -> FATReLU(x[..., :d], threshold) * x[..., d:]."""

    can_torch_compile: bool = True

    def __init__(self, threshold: float = 0.0):
        super().__init__()
        self.threshold = threshold

    def forward(self, x: torch.Tensor):
        if not x.is_contiguous():
            x = x.contiguous()
        d = x.shape[-1] // 2
        out = torch.empty(x.shape[:-1] + (d,), dtype=x.dtype, device=x.device)
        ops.fatrelu_and_mul(out, x, self.threshold)
        return out


class Silu(nn.Module):
    can_torch_compile: bool = True

    def forward(self, x: torch.Tensor):
        return _elementwise(x, ops.silu)


class Gelu(nn.Module):
    can_torch_compile: bool = True

    def forward(self, x: torch.Tensor):
        return _elementwise(x, ops.gelu)


class GeluTanh(nn.Module):
    can_torch_compile: bool = True

    def forward(self, x: torch.Tensor):
        return _elementwise(x, ops.gelu_tanh)


class FastGELU(nn.Module):
    can_torch_compile: bool = True

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _elementwise(x, ops.gelu_fast)


class NewGELU(nn.Module):
    can_torch_compile: bool = True

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _elementwise(x, ops.gelu_new)


class QuickGELU(nn.Module):
    can_torch_compile: bool = True

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _elementwise(x, ops.gelu_quick)
