"""Drop-in forwards for transformers' RMSNorm modules, mirroring
rmsnorm/tvm-ffi-ext/rmsnorm/layers.py:7-51."""

import torch
import torch.nn as nn

from .functional import RMSNormFunction


class RMSNorm(nn.Module):
    """Llama-style RMSNorm: `weight * (x / rms(x)).to(x.dtype)`."""

    weight: nn.Parameter
    variance_epsilon: float

    can_torch_compile = True

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        # Not in place: dY can be shared with other branches (a residual add).
        return RMSNormFunction.apply(
            hidden_states, self.weight, self.variance_epsilon, 0.0, "llama", False
        )

    def extra_repr(self):
        return f"{tuple(self.weight.shape)}, eps={self.variance_epsilon}"


class GemmaRMSNorm(nn.Module):
    """Gemma-style RMSNorm: `(x / rms(x) * (1 + weight)).to(x.dtype)` in float32."""

    weight: nn.Parameter
    eps: float

    can_torch_compile = True

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return RMSNormFunction.apply(x, self.weight, self.eps, 1.0, "gemma", False)

    def extra_repr(self):
        return f"{tuple(self.weight.shape)}, eps={self.eps}"
