"""Rounding helpers for the oracle -- test infrastructure only.

bf16 rounding is round-to-nearest-even on the f32 bit pattern, which is what the
reference's `f32_to_bf16_rne` / `cvt.rn.bf16x2.f32` compute
(activation-rs/src/element.rs:83-98) and what torch's CPU `.to(torch.bfloat16)`
computes. Pinned in tests/test_oracle_numerics.py against torch's conversion on
every bf16 bit pattern and on random f32 values (including ties and NaN).
"""

from __future__ import annotations

import numpy as np


def round_bf16(x) -> np.ndarray:
    """f32 -> nearest-even bf16, returned as f32."""
    a = np.atleast_1d(np.asarray(x, dtype=np.float32))
    scalar = np.ndim(x) == 0
    u = a.view(np.uint32).astype(np.uint64)
    nan = np.isnan(a)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = (r << 16).astype(np.uint32)
    out = r.view(np.float32).copy()
    out[nan] = np.float32(np.nan)
    return out[0] if scalar else out


def round_f16(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def rounder(dtype: str):
    """Rounding function of an element type name ("bf16", "f16", "f32")."""
    if dtype == "bf16":
        return round_bf16
    if dtype == "f16":
        return round_f16
    if dtype == "f32":
        return lambda x: np.asarray(x, dtype=np.float32)
    raise ValueError(f"unknown dtype {dtype}")


def bf16_bits(x) -> np.ndarray:
    """The 16-bit patterns of f32 values that are exact bf16 numbers."""
    return (np.asarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def ulp_distance_bf16(a, b) -> np.ndarray:
    """Distance in bf16 units in the last place between two arrays of bf16 values
    (held as f32), on the monotone integer line of the bit patterns."""

    def ordered(x):
        bits = bf16_bits(x).astype(np.int32)
        return np.where(bits & 0x8000, 0x8000 - (bits & 0x7FFF), bits + 0x8000)

    return np.abs(ordered(a) - ordered(b))


def ulp_distance_f16(a, b) -> np.ndarray:
    def ordered(x):
        bits = np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16).astype(np.int32)
        return np.where(bits & 0x8000, 0x8000 - (bits & 0x7FFF), bits + 0x8000)

    return np.abs(ordered(a) - ordered(b))
