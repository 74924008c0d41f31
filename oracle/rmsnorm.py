"""rmsnorm oracle (numpy) -- test infrastructure only.

Restates rmsnorm/src/device.rs:75-358 with the casting modes of
rmsnorm/src/casting.rs:44-60:
  forward   rstd = 1/sqrt(mean(x^2) + eps) (f32; "none" rounds mean, eps and rstd
            to X), y = X(x_hat * (offset + w)) with x_hat rounded to X in
            "llama"/"none" (device.rs:147-179)
  backward  m = dy*(offset+w); dx = rstd*m + rstd*(-(rstd^2/n)*dot(m,x)*x);
            dw = sum_rows dy*x_hat, each term rounded to X in "llama"
            (device.rs:228-335)
The forward sum of squares follows the reference kernel's f32 order exactly
(`sum_squares_reference_order`, device.rs:41-63 and 113-145 with the block sizes
of ops.rs:98-115), and rstd is the correctly rounded f32 inverse square root of
the f32 value mean + eps (the reference's libdevice `rsqrtf` approximates it), so
y and rstd are defined to the bit. The warp reduction of the third-party
`cuda_device::warp::reduce_sum_f32` (cuda-oxide, git rev d9d4e379, not vendored)
is taken to be the butterfly with lane distances 16, 8, 4, 2, 1; that choice is
parity unpinned against the reference's own bits. The backward sums are
accumulated in float64 and rounded to f32 once (dx is rounded once at the end,
so the summation order moves it by at most one rounding flip).

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


def block_threads(n: int) -> int:
    """Threads per row of the reference kernels (rmsnorm/src/ops.rs:98-106)."""
    if n < 2048:
        return 128
    if n < 8192:
        return 256
    if n < 32768:
        return 512
    return 1024


def _butterfly32(v):
    """Lane-0 value of a 32-lane xor butterfly (distances 16..1) over the last axis."""
    v = v.astype(F32)
    d = 16
    while d >= 1:
        v = v[..., :d] + v[..., d : 2 * d]
        d //= 2
    return v[..., 0]


def sum_squares_reference_order(x, vectorized=True):
    """Row sums of x*x in the reference kernel's f32 order (device.rs:113-145).

    Thread t of T = block_threads(n) owns the 8-element groups t, t+T, ... of the
    first floor(n/8)*8 columns (vectorized) and then the single columns
    tail+t, tail+t+T, ...; each group is summed left to right from its first
    square, the thread adds its groups and columns in order, the 32-thread warps
    reduce by butterfly and the T/32 warp sums by the same butterfly over 32
    slots (device.rs:41-63). Zero padding is exact: every partial is >= +0.
    """
    x = np.asarray(x, dtype=F32)
    lead, n = x.shape[:-1], x.shape[-1]
    x = x.reshape(-1, n)
    rows = x.shape[0]
    T = block_threads(n)
    sq = x * x
    part = np.zeros((rows, T), dtype=F32)
    tail = n // 8 * 8 if vectorized else 0
    if tail:
        grp = sq[:, :tail].reshape(rows, tail // 8, 8)
        s = grp[..., 0].copy()
        for i in range(1, 8):
            s = s + grp[..., i]
        k = -(-s.shape[1] // T)
        s = np.concatenate([s, np.zeros((rows, k * T - s.shape[1]), F32)], axis=1).reshape(rows, k, T)
        for j in range(k):
            part = part + s[:, j]
    if n > tail:
        rest = sq[:, tail:]
        k = -(-rest.shape[1] // T)
        rest = np.concatenate([rest, np.zeros((rows, k * T - rest.shape[1]), F32)], axis=1)
        rest = rest.reshape(rows, k, T)
        for j in range(k):
            part = part + rest[:, j]
    warp = _butterfly32(part.reshape(rows, T // 32, 32))
    slots = np.zeros((rows, 32), dtype=F32)
    slots[:, : T // 32] = warp
    return _butterfly32(slots).reshape(lead)


def rsqrt_rn(v):
    """Correctly rounded f32 1/sqrt(v) of f32 values (via float64)."""
    return (1.0 / np.sqrt(np.asarray(v, dtype=F32).astype(np.float64))).astype(F32)


def forward(x, weight, eps, offset=0.0, mode="llama", xdtype="bf16", wdtype=None, vectorized=None):
    """Returns (y, rstd); x [..., n] values of xdtype, weight [n] of wdtype or None.

    `vectorized`: the reference's 16-byte access rule (ops.rs:108-115); None
    takes it from the row width (16-byte aligned tensors), False is the path of
    a misaligned tensor."""
    RX = rounder(xdtype)
    RW = rounder(wdtype or xdtype)
    idm, round_x_hat, _ = _flags(mode)
    x = np.asarray(x, dtype=F32)
    n = x.shape[-1]
    if vectorized is None:
        vectorized = (n * (4 if xdtype == "f32" else 2)) % 16 == 0
    sum_sq = sum_squares_reference_order(x, vectorized)
    ms = sum_sq * (F32(1.0) / F32(n))
    if idm:
        rstd = RX(rsqrt_rn(RX(ms) + RX(F32(eps))))
    else:
        rstd = rsqrt_rn(ms + F32(eps))
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
