"""FlashAttention-2 dropout mask stream (numpy) -- test infrastructure only.

Restates flash-attn2-rs/src/device/dropout.rs:31-51 (`random`: Philox4x32 with 7
rounds; counter [offset lo, offset hi, row, col], key [seed lo, seed hi]) and the
element mapping of `apply` (dropout.rs:53-121) / `transposed_keep`
(device/backward/common.rs:168-185): element (query q, key k) of head bh = b*H + h
reads byte ((q % 16) / 8 * 2 + k % 2) of word (k % 32) / 8 of

    philox(seed, offset + bh * 32 + (q % 8) * 4 + (k % 8) / 2, row = q / 16, col = k / 32)

and is kept when that byte <= threshold = floor(keep * 255) (varlen: b is the
sequence index and q, k count from the sequence start, device/varlen/mod.rs).

Pinned by tests/test_oracle_dropout.py: the same Philox4x32 round function run
for 10 rounds reproduces the published Random123 known-answer vectors, and the
keep rate of a large mask matches (threshold + 1) / 256.
"""

from __future__ import annotations

import numpy as np

M32 = np.uint64(0xFFFFFFFF)


def philox4x32(c0, c1, c2, c3, k0, k1, rounds=7):
    """Philox4x32 on broadcastable uint arrays; returns four uint32 arrays."""
    c = [np.asarray(x, dtype=np.uint64) & M32 for x in (c0, c1, c2, c3)]
    k0 = np.asarray(k0, dtype=np.uint64) & M32
    k1 = np.asarray(k1, dtype=np.uint64) & M32
    for _ in range(rounds):
        a = c[0] * np.uint64(0xD2511F53)
        b = c[2] * np.uint64(0xCD9E8D57)
        c = [(b >> np.uint64(32)) ^ c[1] ^ k0, b & M32, (a >> np.uint64(32)) ^ c[3] ^ k1, a & M32]
        k0 = (k0 + np.uint64(0x9E3779B9)) & M32
        k1 = (k1 + np.uint64(0xBB67AE85)) & M32
    return [x.astype(np.uint32) for x in c]


def threshold(p_dropout: float) -> int:
    keep = np.float32(1.0) - np.float32(p_dropout)
    return int(np.float32(keep * np.float32(255.0)))


def keep_mask(seed: int, offset: int, bh: int, sq: int, sk: int, p_dropout: float) -> np.ndarray:
    """Boolean [sq, sk]: True where element (q, k) of head bh is kept."""
    q = np.arange(sq, dtype=np.uint64)[:, None]
    k = np.arange(sk, dtype=np.uint64)[None, :]
    lane = (q % 8) * 4 + (k % 8) // 2
    off = (np.uint64(offset) + np.uint64(bh) * np.uint64(32) + lane) & np.uint64(0xFFFFFFFFFFFFFFFF)
    words = philox4x32(off & M32, off >> np.uint64(32), q // 16, k // 32,
                       np.uint64(seed) & M32, np.uint64(seed) >> np.uint64(32))
    w = np.stack(words)  # [4, sq, sk]
    word = np.take_along_axis(w, ((k % 32) // 8).astype(np.int64)[None].repeat(sq, axis=1), axis=0)[0]
    shift = (((q % 16) // 8) * 2 + k % 2) * 8
    byte = (word.astype(np.uint64) >> shift) & np.uint64(255)
    return byte <= np.uint64(threshold(p_dropout))


def dense_mask(seed, offset, batch, heads, sq, sk, p_dropout):
    """[B, H, Sq, Sk] keep mask of a dense call."""
    out = np.empty((batch, heads, sq, sk), dtype=bool)
    for b in range(batch):
        for h in range(heads):
            out[b, h] = keep_mask(seed, offset, b * heads + h, sq, sk, p_dropout)
    return out
