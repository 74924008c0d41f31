"""rmsnorm on MI355X, mirroring rmsnorm/tvm-ffi-ext/rmsnorm/__init__.py."""

from . import layers, torch_ops
from ._ops import ops
from .functional import RMSNormFunction, rms_norm

__all__ = ["ops", "RMSNormFunction", "rms_norm", "layers", "torch_ops"]
