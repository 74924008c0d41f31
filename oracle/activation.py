"""activation-rs oracle (numpy) -- test infrastructure only.

Restates activation-rs/src/activation.rs:34-122 and the gated kernel
activation-rs/src/device.rs:18-41: the activation is computed in f32 and rounded
to the element type T, then multiplied by the other half in f32 and rounded to
T again (`mul`, element.rs:103-106). The transcendental functions (exp, erf,
tanh) are evaluated in float64 and rounded once to f32, i.e. the correctly
rounded f32 value the GPU's libm approximates.

Pins (tests/test_oracle_activation.py):
  * the reference tests' own oracle, torch CPU `F.silu(x[..., :d]) * x[..., d:]`
    and `F.gelu(..., approximate="none"|"tanh")`
    (activation-rs/tests/kernels/test_activation.py:41-83), on every bf16 bit
    pattern for the element-wise maps and on random gated inputs;
  * closed forms: silu(0) = gelu(0) = 0, act(x) -> x for large x, act(x) -> 0 for
    very negative x, FATReLU's threshold rule, gelu_quick(x) = x*sigmoid(1.702x).
"""

from __future__ import annotations

import math

import numpy as np

from .numerics import rounder

try:
    from scipy.special import erf as _erf64
except ImportError:  # pragma: no cover - scipy is part of the image
    _erf64 = np.vectorize(math.erf)

F32 = np.float32


def _f32(x):
    return np.asarray(x, dtype=np.float32)


def _exp(x):
    return np.exp(np.asarray(x, dtype=np.float64)).astype(F32)


def _tanh(x):
    return np.tanh(np.asarray(x, dtype=np.float64)).astype(F32)


def _erf(x):
    return _erf64(np.asarray(x, dtype=np.float64)).astype(F32)


def fma32(a, b, c) -> np.ndarray:
    """Correctly rounded f32 a*b + c (one rounding), for f32 arrays.

    a*b is exact in f64; the f64 sum s = a*b + c is rounded, and TwoSum gives
    its exact error e. Rounding s to f32 is then correct except when s lies
    exactly halfway between two floats and e != 0, where the tie is broken
    toward the side of e (no other f64 value can sit between the exact sum and
    s across an f32 midpoint, as every such midpoint is an f64 number).
    """
    a64 = np.asarray(a, dtype=np.float32).astype(np.float64)
    b64 = np.asarray(b, dtype=np.float32).astype(np.float64)
    c64 = np.asarray(c, dtype=np.float32).astype(np.float64)
    p = a64 * b64
    with np.errstate(over="ignore", invalid="ignore"):
        s = p + c64
        bb = s - p
        e = (p - (s - bb)) + (c64 - bb)
        r = s.astype(F32)
        up = np.nextafter(r, np.float32(np.inf))
        down = np.nextafter(r, np.float32(-np.inf))
        other = np.where(s > r.astype(np.float64), up, down)
        tie = (np.isfinite(s) & np.isfinite(e) & (e != 0)
               & ((r.astype(np.float64) + other.astype(np.float64)) * 0.5 == s))
        # at a tie the exact sum lies on the side of e: pick the float on that side
        toward = np.where(e > 0, np.maximum(r, other), np.minimum(r, other))
    return np.where(tie, toward, r).astype(F32)


def act(name: str, x, dtype: str, threshold: float = 0.0) -> np.ndarray:
    """act(x) rounded to `dtype`, for x holding values of that dtype."""
    R = rounder(dtype)
    f = _f32(x)
    with np.errstate(over="ignore", invalid="ignore"):
        if name == "silu":  # activation.rs:42-46
            return R(f / (F32(1.0) + _exp(-f)))
        if name == "gelu":  # activation.rs:53-58
            alpha = F32(1.0 / math.sqrt(2.0))
            return R(f * F32(0.5) * (F32(1.0) + _erf(f * alpha)))
        if name == "gelu_tanh":  # activation.rs:64-76
            beta = F32(math.sqrt(2.0) * (2.0 / math.sqrt(math.pi)) * 0.5)
            kappa = F32(0.044715)
            x_cube = f * f * f
            # fused multiply-add: one rounding of kappa * x^3 + f
            inner = beta * fma32(np.broadcast_to(kappa, np.shape(f)), x_cube, f)
            return R(F32(0.5) * f * (F32(1.0) + _tanh(inner)))
        if name == "gelu_new":  # activation.rs:79-90
            x3 = R(R(f * f) * f)
            inner = R(f + R(F32(0.044715) * x3))
            t = R(_tanh(R(F32(0.79788456) * inner)))
            return R(R(R(F32(0.5)) * f) * R(R(F32(1.0)) + t))
        if name == "gelu_fast":  # activation.rs:92-104
            scaled = R(f * F32(0.79788456))
            cubic = R(R(F32(1.0)) + R(R(F32(0.044715) * f) * f))
            t = R(_tanh(R(scaled * cubic)))
            return R(R(R(F32(0.5)) * f) * R(R(F32(1.0)) + t))
        if name == "gelu_quick":  # activation.rs:106-115
            return R(f / (F32(1.0) + _exp(F32(-1.702) * f)))
        if name == "fatrelu":  # activation.rs:117-122
            return R(np.where(f > F32(threshold), f, F32(0.0)))
    raise ValueError(f"unknown activation {name}")


GATED = {
    "silu_and_mul": ("silu", True),
    "mul_and_silu": ("silu", False),
    "gelu_and_mul": ("gelu", True),
    "gelu_tanh_and_mul": ("gelu_tanh", True),
    "fatrelu_and_mul": ("fatrelu", True),
}


def gated(op: str, x, dtype: str, threshold: float = 0.0) -> np.ndarray:
    """Gated op over the last dimension: activation-rs/src/device.rs:18-41."""
    name, act_first = GATED[op]
    R = rounder(dtype)
    x = _f32(x)
    d = x.shape[-1] // 2
    a, b = x[..., :d], x[..., d:]
    if act_first:
        return R(act(name, a, dtype, threshold) * b)
    return R(a * act(name, b, dtype, threshold))


def elementwise(op: str, x, dtype: str) -> np.ndarray:
    """Element-wise op: activation-rs/src/device.rs:62-79."""
    return act(op, x, dtype)
