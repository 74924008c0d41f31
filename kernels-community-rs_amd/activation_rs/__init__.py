"""activation-rs on MI355X: gated and element-wise activations.

Mirrors activation-rs/tvm-ffi-ext/activation_rs/__init__.py:21-89: every function
writes into `out` (same shape rules as the reference) and returns it.
"""

from __future__ import annotations

import torch

from . import layers, torch_ops
from ._ops import ops

_impl = torch_ops


def silu_and_mul(out: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    _impl.silu_and_mul(out, x)
    return out


def mul_and_silu(out: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    _impl.mul_and_silu(out, x)
    return out


def gelu_and_mul(out: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    _impl.gelu_and_mul(out, x)
    return out


def gelu_tanh_and_mul(out: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    _impl.gelu_tanh_and_mul(out, x)
    return out


def fatrelu_and_mul(out: torch.Tensor, x: torch.Tensor, threshold: float = 0.0) -> torch.Tensor:
    _impl.fatrelu_and_mul(out, x, threshold)
    return out


def gelu(out: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    _impl.gelu(out, x)
    return out


def silu(out: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    _impl.silu(out, x)
    return out


def gelu_tanh(out: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    _impl.gelu_tanh(out, x)
    return out


def gelu_fast(out: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    _impl.gelu_fast(out, x)
    return out


def gelu_new(out: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    _impl.gelu_new(out, x)
    return out


def gelu_quick(out: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    _impl.gelu_quick(out, x)
    return out


__all__ = [
    "silu_and_mul",
    "mul_and_silu",
    "gelu_and_mul",
    "gelu_tanh_and_mul",
    "fatrelu_and_mul",
    "gelu_fast",
    "gelu_new",
    "gelu_quick",
    "gelu_tanh",
    "silu",
    "gelu",
    "layers",
    "torch_ops",
    "ops",
]
