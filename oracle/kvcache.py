"""KV-cache oracle (numpy) -- test infrastructure only.

Restates flash_attn_with_kvcache of flash-attn2-rs:
  * the append (src/device/cache.rs:142-260): new row r of batch b goes to cache
    position lengths[b] + r of cache batch cache_batch_idx[b] (or b), or of page
    block_table[b, position // page] at row position % page; positions past the
    capacity (or the rotary table) and invalid batch / page indices are skipped;
  * rotary embedding (src/device/cache.rs:26-62): column d < rotary_dim pairs with
    d ^ 1 (interleaved) or d +- rotary_dim / 2, frequency d // 2 or d % (rotary_dim
    / 2), angle row position; out = x_d * cos + x_other * (first ? -sin : sin),
    two rounded fp32 products and a rounded fp32 sum, then rounded to the element
    type. K rotates at its cache position, Q at lengths[b] + (advance_q ? r : 0);
  * attention (device/varlen/mod.rs:79-136 with CACHED): sequence b attends to cache
    rows [leftpad[b], lengths[b] + new) with the dense formula of oracle.attention
    (bottom-right causal alignment, windows, softcap, ALiBi).

Pins (tests/test_oracle_kvcache.py): the rotary step against an independent
complex-number rotation (interleaved pairs as x_even + i x_odd, the other layout
as halves), with rounding bounded by one element ulp; rotation by angle 0 is the
identity; rotation is norm-preserving; appending then attending equals attending
over the concatenated keys computed with oracle.attention; a paged cache with a
permuted block table gives the same result as the contiguous cache.
"""

from __future__ import annotations

import numpy as np

from . import attention as OA
from .numerics import rounder


def rotate_rows(x, positions, cos, sin, interleaved, dtype):
    """x [..., D] (exact element values as f32), positions broadcast to x.shape[:-1];
    cos/sin [P, rotary_dim / 2]. Returns the rotated rows rounded to `dtype`."""
    rnd = rounder(dtype)
    x = np.asarray(x, dtype=np.float32)
    out = x.copy()
    rd = 2 * cos.shape[1]
    half = rd // 2
    pos = np.asarray(positions)
    for d in range(rd):
        if interleaved:
            first, other, freq = d % 2 == 0, d ^ 1, d // 2
        else:
            first = d < half
            other = d + half if first else d - half
            freq = d % half
        c = cos[pos, freq].astype(np.float32)
        s = sin[pos, freq].astype(np.float32)
        s = -s if first else s
        prod_a = (x[..., d] * c).astype(np.float32)
        prod_b = (x[..., other] * s).astype(np.float32)
        out[..., d] = rnd((prod_a + prod_b).astype(np.float32))
    return out


def append(kcache, vcache, k, v, lengths, *, cos=None, sin=None, interleaved=False,
           cache_batch_idx=None, block_table=None, dtype="bf16"):
    """Returns updated copies of kcache/vcache [batches | pages, rows, Hk, D]."""
    kc = np.array(kcache, dtype=np.float32, copy=True)
    vc = np.array(vcache, dtype=np.float32, copy=True)
    B, snew = k.shape[0], k.shape[1]
    page = kc.shape[1]
    capacity = page * block_table.shape[1] if block_table is not None else page
    rows_rot = cos.shape[0] if cos is not None else None
    for b in range(B):
        start = int(lengths[b])
        for r in range(snew):
            pos = start + r
            if start < 0 or pos >= capacity or (rows_rot is not None and pos >= rows_rot):
                continue
            if block_table is not None:
                col = pos // page
                if col >= block_table.shape[1]:
                    continue
                pg = int(block_table[b, col])
                if pg < 0 or pg >= kc.shape[0]:
                    continue
                cb, row = pg, pos % page
            else:
                cb = int(cache_batch_idx[b]) if cache_batch_idx is not None else b
                if cb < 0 or cb >= kc.shape[0]:
                    continue
                row = pos
            kr = k[b, r]
            if cos is not None:
                kr = rotate_rows(kr, np.full(kr.shape[:-1], pos), cos, sin, interleaved, dtype)
            kc[cb, row] = kr
            vc[cb, row] = v[b, r]
    return kc, vc


def rotate_q(q, lengths, cos, sin, interleaved, advance_q, dtype="bf16"):
    """Q [B, Sq, H, D] rotated at lengths[b] + (advance_q ? r : 0); rows whose
    position has no table entry keep their values."""
    B, Sq, H, _ = q.shape
    out = np.array(q, dtype=np.float32, copy=True)
    for b in range(B):
        for r in range(Sq):
            pos = int(lengths[b]) + (r if advance_q else 0)
            if int(lengths[b]) < 0 or pos >= cos.shape[0]:
                continue
            out[b, r] = rotate_rows(out[b, r], np.full((H,), pos), cos, sin, interleaved, dtype)
    return out


def cache_rows(kc, b, lo, hi, *, cache_batch_idx=None, block_table=None):
    """Rows [lo, hi) of sequence b's cache view [rows, Hk, D]."""
    if block_table is not None:
        page = kc.shape[1]
        rows = []
        for pos in range(lo, hi):
            pg = int(block_table[b, pos // page])
            rows.append(kc[pg, pos % page] if 0 <= pg < kc.shape[0] else np.zeros_like(kc[0, 0]))
        return np.stack(rows) if rows else np.zeros((0,) + kc.shape[2:], dtype=kc.dtype)
    cb = int(cache_batch_idx[b]) if cache_batch_idx is not None else b
    return kc[cb, lo:hi]


def attend(q, kc, vc, used, *, leftpad=None, cache_batch_idx=None, block_table=None, **kw):
    """q [B, Sq, H, D] over cache rows [leftpad[b], used[b]) -> out [B, Sq, H, D],
    lse [B, H, Sq]; kw as oracle.attention.forward."""
    B = q.shape[0]
    outs, lses = [], []
    for b in range(B):
        lo = int(leftpad[b]) if leftpad is not None else 0
        hi = int(used[b])
        kb = cache_rows(kc, b, lo, hi, cache_batch_idx=cache_batch_idx, block_table=block_table)
        vb = cache_rows(vc, b, lo, hi, cache_batch_idx=cache_batch_idx, block_table=block_table)
        o, l = OA.forward(q[b:b + 1], kb[None], vb[None], **kw)
        outs.append(o[0])
        lses.append(l[0])
    return np.stack(outs), np.stack(lses)
