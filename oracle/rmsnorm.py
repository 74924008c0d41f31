"""rmsnorm oracle (numpy) -- test infrastructure only.

Restates rmsnorm/src/device.rs:75-358 with the casting modes of
rmsnorm/src/casting.rs:44-60:
  forward   rstd = 1/sqrt(mean(x^2) + eps) (f32; "none" rounds mean, eps and rstd
            to X), y = X(x_hat * (offset + w)) with x_hat rounded to X in
            "llama"/"none" (device.rs:147-179)
  backward  m = dy*(offset+w); dx = rstd*m + rstd*(-(rstd^2/n)*dot(m,x)*x);
            dw = sum_rows dy*x_hat, each term rounded to X in "llama"
            (device.rs:228-335)
Sums are accumulated in float64 and rounded to f32 once (the GPU sums in f32 in
a different order; the difference is far below the output rounding).

Pins (tests/test_oracle_rmsnorm.py): the reference tests' torch formulas
(rmsnorm/tests/test_ops.py:10-21, test_rms_norm.py:27-90) for every mode and
dtype; torch autograd of those formulas for dx/dw; closed forms (constant rows,
x -> c*x invariance, zero rows give rstd = eps^-1/2).
"""

from __future__ import annotations

import numpy as np

from .numerics import rounder

F32 = np.float32
MODES = ("llama", "gemma", "none")


def _flags(mode):
    if mode == "llama":
        return False, True, True  # input_dtype_math, round_x_hat, round_weight_grad
    if mode == "gemma":
        return False, False, False
    if mode == "none":
        return True, True, False
    raise ValueError(mode)


def forward(x, weight, eps, offset=0.0, mode="llama", xdtype="bf16", wdtype=None):
    """Returns (y, rstd); x [..., n] values of xdtype, weight [n] of wdtype or None."""
    RX = rounder(xdtype)
    RW = rounder(wdtype or xdtype)
    idm, round_x_hat, _ = _flags(mode)
    x = np.asarray(x, dtype=F32)
    n = x.shape[-1]
    sum_sq = np.sum(x.astype(np.float64) ** 2, axis=-1).astype(F32)
    ms = sum_sq * F32(1.0 / n)
    if idm:
        rstd = RX(F32(1.0) / np.sqrt(RX(ms) + RX(F32(eps))))
    else:
        rstd = (1.0 / np.sqrt(ms.astype(np.float64) + np.float64(F32(eps)))).astype(F32)
    xr = x * rstd[..., None]
    x_hat = RX(xr) if round_x_hat else xr
    if weight is None:
        return RX(x_hat), rstd
    w = np.asarray(weight, dtype=F32)
    factor = RW(RX(F32(offset)) + w) if idm else F32(offset) + w
    return RX(x_hat * factor), rstd


def backward(dy, x, weight, rstd, offset=0.0, mode="llama", xdtype="bf16", wdtype=None):
    """Returns (dx, dw) with dw in f32 before the final rounding to the weight
    dtype (rms_norm_reduce_weight_grad rounds it, device.rs:339-358)."""
    RX = rounder(xdtype)
    _, _, round_wg = _flags(mode)
    dy = np.asarray(dy, dtype=F32)
    x = np.asarray(x, dtype=F32)
    n = x.shape[-1]
    r = np.asarray(rstd, dtype=F32)[..., None]
    g = dy if weight is None else dy * (np.asarray(weight, dtype=F32) + F32(offset))
    dot = np.sum(g.astype(np.float64) * x, axis=-1, keepdims=True).astype(F32)
    correction = F32(-1.0 / n) * r * r * dot
    dx = RX(r * g + r * (correction * x))
    if weight is None:
        return dx, None
    x_hat = x * r
    if round_wg:
        terms = RX(dy * RX(x_hat))
    else:
        terms = dy * x_hat
    dw = np.sum(terms.reshape(-1, n).astype(np.float64), axis=0).astype(F32)
    return dx, dw
