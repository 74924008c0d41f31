"""flash-attn2-rs on MI355X: FlashAttention-2 forward (dense, varlen) and backward.

Mirrors flash-attn2-rs/tvm-ffi-ext/flash_attn2_rs/__init__.py, including the
KV-cache entry points (ops.fwd_kvcache, flash_attn_with_kvcache) and dropout.
"""

from ._ops import ops
from .flash_attn_interface import (
    bwd,
    flash_attn_func,
    flash_attn_kvpacked_func,
    flash_attn_qkvpacked_func,
    flash_attn_varlen_func,
    flash_attn_varlen_kvpacked_func,
    flash_attn_varlen_qkvpacked_func,
    flash_attn_with_kvcache,
    fwd,
    fwd_explicit,
    fwd_kvcache,
    reserve_rng_state,
    varlen_bwd,
    varlen_fwd,
)
from . import _torch_interface  # noqa: F401  (registers the torch custom ops)

__all__ = [
    "ops",
    "fwd",
    "bwd",
    "varlen_fwd",
    "varlen_bwd",
    "fwd_explicit",
    "fwd_kvcache",
    "reserve_rng_state",
    "flash_attn_func",
    "flash_attn_qkvpacked_func",
    "flash_attn_kvpacked_func",
    "flash_attn_varlen_func",
    "flash_attn_varlen_qkvpacked_func",
    "flash_attn_varlen_kvpacked_func",
    "flash_attn_with_kvcache",
]
