"""FlashAttention-2 oracle (numpy) -- test infrastructure only.

Restates the reference tests' fp32 attention, flash-attn2-rs/tests/test_fwd.py:36-85
(`reference_attention`), with FlashAttention's conventions for rows that see no
key: output 0 and LSE +inf (tests/test_fwd.py:158-168, host/forward/mod.rs:548-572).
  scores = q k^T * scale, or softcap * tanh(q k^T * scale / softcap)
  ALiBi:  + slope * col (pure causal), else - slope * |row + Sk - Sq - col|
  masks:  col > row + (Sk - Sq) + wr (causal: wr = 0), col < row + (Sk - Sq) - wl
  out = softmax(scores) v, lse = logsumexp(scores)
GQA: KV head = query head // (Hq / Hk). Varlen runs the dense formula on each
sequence slice given by cu_seqlens (device/varlen/mod.rs:79-136).

Backward (device/backward/common.rs:121-152, dq.rs, dkv.rs, reduce.rs:40-108):
  P = exp(scores - lse), dP = dO V^T, delta = rowsum(dO * O),
  dS = P * (dP - delta) [* (1 - tanh^2) with softcap],
  dV = P^T dO, dK = scale * dS^T Q, dQ = scale * dS K, with dK/dV summed over the
  query heads of each KV head.

Pins (tests/test_oracle_attention.py): torch's scaled_dot_product_attention and
logsumexp on the CPU (a library routine), torch autograd of the same formula for
the gradients, finite differences on tiny float64 cases, and closed forms:
Sk = 1 gives O = V exactly, constant V rows give O = that row, all-zero Q gives
LSE = log(#visible keys), empty / fully masked rows give O = 0 and LSE = +inf.
"""

from __future__ import annotations

import math

import numpy as np


def _scores(q, k, scale, softcap, alibi_slopes, causal, wl, wr):
    """q [B,Sq,H,D], k [B,Sk,Hk,D] -> scores [B,H,Sq,Sk] (masked entries -inf), and the
    tanh values used by softcap (for the backward)."""
    B, Sq, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    g = H // Hk
    qh = np.transpose(q, (0, 2, 1, 3))  # B H Sq D
    kh = np.repeat(np.transpose(k, (0, 2, 1, 3)), g, axis=1)  # B H Sk D
    raw = qh @ np.swapaxes(kh, -1, -2)
    t = None
    if softcap and softcap > 0:
        t = np.tanh(raw * (scale / softcap))
        s = softcap * t
    else:
        s = raw * scale
    off = Sk - Sq
    rows = np.arange(Sq).reshape(Sq, 1)
    cols = np.arange(Sk).reshape(1, Sk)
    if alibi_slopes is not None:
        slopes = np.asarray(alibi_slopes, dtype=s.dtype).reshape(-1, H, 1, 1)
        if causal and wl < 0:
            s = s + slopes * cols
        else:
            s = s - slopes * np.abs(rows + off - cols)
    mask = np.zeros((Sq, Sk), dtype=bool)
    if causal or wr >= 0:
        mask |= cols > rows + off + (0 if causal else wr)
    if wl >= 0:
        mask |= cols < rows + off - wl
    s = np.where(mask, -np.inf, s)
    return s, t, mask


def forward(q, k, v, *, softmax_scale=None, causal=False, window_left=-1, window_right=-1,
            softcap=0.0, alibi_slopes=None, dtype=np.float32, dropout_mask=None, p_dropout=0.0):
    """Dense attention. q [B,Sq,H,D], k/v [B,Sk,Hk,D] -> out [B,Sq,H,D], lse [B,H,Sq].
    With dropout (mask [B,H,Sq,Sk] of kept elements, oracle.dropout): out =
    ((P * mask) / keep) V, keep = 1 - p (device/forward/mod.rs:1353, 1404); the LSE
    is that of the undropped scores."""
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    B, Sq, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else softmax_scale
    if Sk == 0:
        return np.zeros_like(q), np.full((B, H, Sq), np.inf, dtype=dtype)
    s, _, _ = _scores(q, k, scale, softcap, alibi_slopes, causal, window_left, window_right)
    m = np.max(s, axis=-1, keepdims=True)
    empty = ~np.isfinite(m)
    m = np.where(empty, 0, m)
    e = np.exp(s - m)
    l = np.sum(e, axis=-1, keepdims=True)
    p = np.where(l > 0, e / np.where(l > 0, l, 1), 0)
    if dropout_mask is not None:
        p = p * dropout_mask / (np.float32(1.0) - np.float32(p_dropout))
    vh = np.repeat(np.transpose(v, (0, 2, 1, 3)), H // Hk, axis=1)
    out = np.transpose(p @ vh, (0, 2, 1, 3))
    lse = np.where(l[..., 0] > 0, m[..., 0] + np.log(np.where(l[..., 0] > 0, l[..., 0], 1)), np.inf)
    return out.astype(dtype), lse.astype(dtype)


def backward(q, k, v, out, dout, lse, *, softmax_scale=None, causal=False, window_left=-1,
             window_right=-1, softcap=0.0, alibi_slopes=None, dtype=np.float32, dropout_mask=None,
             p_dropout=0.0):
    """Gradients of `forward`: returns dq [B,Sq,H,D], dk/dv [B,Sk,Hk,D] (GQA-summed)
    and delta [B,H,Sq]. With dropout, delta is keep * rowsum(dO * O) as the
    reference's preprocess writes it (device/backward/reduce.rs:40-108), and the
    gradients are those of the dropped forward: dV = (P*M/keep)^T dO,
    dS = P * (dP*M/keep - rowsum(dO * O))."""
    q, k, v, out, dout = (np.asarray(x, dtype=dtype) for x in (q, k, v, out, dout))
    lse = np.asarray(lse, dtype=dtype)
    B, Sq, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    g = H // Hk
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else softmax_scale
    keep = np.float32(1.0) - np.float32(p_dropout) if dropout_mask is not None else np.float32(1.0)
    delta = np.sum(dout * out, axis=-1).transpose(0, 2, 1)  # B H Sq
    if Sk == 0 or Sq == 0:
        return np.zeros_like(q), np.zeros_like(k), np.zeros_like(v), keep * delta
    s, t, mask = _scores(q, k, scale, softcap, alibi_slopes, causal, window_left, window_right)
    finite = np.isfinite(lse)[..., None]
    p = np.where(finite & ~mask, np.exp(s - np.where(finite, lse[..., None], 0)), 0)
    doh = np.transpose(dout, (0, 2, 1, 3))  # B H Sq D
    qh = np.transpose(q, (0, 2, 1, 3))
    kh = np.repeat(np.transpose(k, (0, 2, 1, 3)), g, axis=1)
    vh = np.repeat(np.transpose(v, (0, 2, 1, 3)), g, axis=1)
    dp = doh @ np.swapaxes(vh, -1, -2)
    pv = p
    if dropout_mask is not None:
        dp = dp * dropout_mask / keep
        pv = p * dropout_mask / keep
    ds = p * (dp - delta[..., None])
    if t is not None:
        ds = ds * (1 - t * t)
    dqh = scale * (ds @ kh)
    dkh = scale * (np.swapaxes(ds, -1, -2) @ qh)
    dvh = np.swapaxes(pv, -1, -2) @ doh
    dk = dkh.reshape(B, Hk, g, Sk, D).sum(axis=2)
    dv = dvh.reshape(B, Hk, g, Sk, D).sum(axis=2)
    return (np.transpose(dqh, (0, 2, 1, 3)).astype(dtype), np.transpose(dk, (0, 2, 1, 3)).astype(dtype),
            np.transpose(dv, (0, 2, 1, 3)).astype(dtype), (keep * delta).astype(dtype))


def probabilities(q, k, keep_mask, *, softmax_scale=None, causal=False, window_left=-1, window_right=-1,
                  alibi_slopes=None, dtype=np.float32):
    """Diagnostic probabilities of a dropout forward (return_softmax): float32
    [B, H, ceil128(Sq), ceil128(Sk)]. Element (q, k) the mask leaves visible holds
    P = exp(score - lse), negated (sign bit set, -0.0 for P = 0) where keep_mask
    [B, H, Sq, Sk] is False; padding and masked elements are +0. The reference
    encodes the drop decision in the same sign bit (src/device/dropout.rs:93-112,
    host/forward/mod.rs:382-398); its magnitudes are scaled by the running row
    maximum of its key tile instead of the final LSE."""
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    rq, rk = (Sq + 127) // 128 * 128, (Sk + 127) // 128 * 128
    out = np.zeros((B, H, rq, rk), dtype=np.float32)
    if Sq == 0 or Sk == 0:
        return out
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else softmax_scale
    s, _, mask = _scores(q, k, scale, 0.0, alibi_slopes, causal, window_left, window_right)
    m = np.max(s, axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0)
    with np.errstate(divide="ignore"):  # rows without a visible key: lse = -inf, every entry masked
        lse = m + np.log(np.sum(np.exp(s - m), axis=-1, keepdims=True))
    p = np.where(mask, 0.0, np.exp(s - np.where(np.isfinite(lse), lse, 0.0))).astype(np.float32)
    dropped = ~np.asarray(keep_mask, dtype=bool) & ~mask
    out[:, :, :Sq, :Sk] = np.where(dropped, -p, p)
    out[:, :, :Sq, :Sk][dropped & (p == 0)] = -0.0
    return out


def _slices(cu):
    cu = np.asarray(cu).tolist()
    return [(cu[i], cu[i + 1]) for i in range(len(cu) - 1)]


def _varlen_dropout(kw, b, H, sq, sk):
    """Per-sequence keep mask for `dropout=(seed, offset, p)`: head bh = b*H + h,
    rows and columns counted from the sequence start."""
    from oracle import dropout as DR

    drop = kw.get("dropout")
    if drop is None:
        return {}
    seed, offset, p = drop
    mask = np.stack([DR.keep_mask(seed, offset, b * H + h, sq, sk, p) for h in range(H)])[None]
    return {"dropout_mask": mask, "p_dropout": p}


def varlen_forward(q, k, v, cu_q, cu_k, **kw):
    """Packed attention: q [Tq,H,D], k/v [Tk,Hk,D] -> out [Tq,H,D], lse [H,Tq].
    `dropout=(seed, offset, p)` applies the reference's mask stream per sequence."""
    kw = dict(kw)
    dtype = kw.get("dtype", np.float32)
    q = np.asarray(q, dtype=dtype)
    Tq, H, D = q.shape
    out = np.zeros_like(q)
    lse = np.full((H, Tq), np.inf, dtype=dtype)
    alibi = kw.pop("alibi_slopes", None)
    for b, ((qs, qe), (ks, ke)) in enumerate(zip(_slices(cu_q), _slices(cu_k))):
        if qe == qs:
            continue
        slopes = None if alibi is None else (np.asarray(alibi)[b] if np.ndim(alibi) == 2 else alibi)
        extra = _varlen_dropout(kw, b, H, qe - qs, ke - ks)
        rest = {key: val for key, val in kw.items() if key != "dropout"}
        o, l = forward(q[None, qs:qe], np.asarray(k)[None, ks:ke], np.asarray(v)[None, ks:ke],
                       alibi_slopes=slopes, **rest, **extra)
        out[qs:qe] = o[0]
        lse[:, qs:qe] = l[0]
    return out, lse


def varlen_backward(q, k, v, out, dout, lse, cu_q, cu_k, **kw):
    """Packed gradients: dq [Tq,H,D], dk/dv [Tk,Hk,D], delta [H, Tq + 128*B]: row r of
    sequence b sits at column cu_q[b] + 128*b + r (device/varlen/backward.rs:126-131,
    host/varlen/backward.rs:173-178); the padding columns are 0."""
    dtype = kw.get("dtype", np.float32)
    q, k, v, out, dout = (np.asarray(x, dtype=dtype) for x in (q, k, v, out, dout))
    Tq, H, D = q.shape
    nb = len(cu_q) - 1
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    delta = np.zeros((H, Tq + 128 * nb), dtype=dtype)
    kw = dict(kw)
    alibi = kw.pop("alibi_slopes", None)
    for b, ((qs, qe), (ks, ke)) in enumerate(zip(_slices(cu_q), _slices(cu_k))):
        if qe == qs:
            continue
        slopes = None if alibi is None else (np.asarray(alibi)[b] if np.ndim(alibi) == 2 else alibi)
        extra = _varlen_dropout(kw, b, H, qe - qs, ke - ks)
        rest = {key: val for key, val in kw.items() if key != "dropout"}
        a, b_, c, d = backward(q[None, qs:qe], k[None, ks:ke], v[None, ks:ke], out[None, qs:qe],
                               dout[None, qs:qe], np.asarray(lse)[None, :, qs:qe], alibi_slopes=slopes,
                               **rest, **extra)
        dq[qs:qe] = a[0]
        dk[ks:ke] += b_[0]
        dv[ks:ke] += c[0]
        delta[:, qs + 128 * b: qe + 128 * b] = d[0]
    return dq, dk, dv, delta
