"""Writes the golden fixtures of this directory from the CPU oracle.

The reference's tests hold no golden vectors (they draw torch.randn on the
device, e.g. flash-attn2-rs/tests/test_fwd.py:145-148), so the fixtures are
made here: seeded inputs from torch's CPU generator, expected outputs from the
oracle (pinned by tests/test_oracle_*.py). bf16 tensors are stored as their
uint16 bit patterns.

    python tests/golden/make_golden.py          # rewrites tests/golden/*.npz
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import activation as A  # noqa: E402
from oracle import attention as OA  # noqa: E402
from oracle import rmsnorm as R  # noqa: E402
from oracle.numerics import bf16_bits, round_bf16  # noqa: E402


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def attention_inputs(seed, b, sq, sk, hq, hk, d):
    """BASELINE.json configs[0] recipe: bf16 ~N(0,1) from a fixed CPU seed."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, sq, hq, d, generator=g).bfloat16()
    k = torch.randn(b, sk, hk, d, generator=g).bfloat16()
    v = torch.randn(b, sk, hk, d, generator=g).bfloat16()
    do = torch.randn(b, sq, hq, d, generator=g).bfloat16()
    return q, k, v, do


def varlen_inputs(seed, lens, hq, hk, d):
    g = torch.Generator().manual_seed(seed)
    t = sum(lens)
    q = torch.randn(t, hq, d, generator=g).bfloat16()
    k = torch.randn(t, hk, d, generator=g).bfloat16()
    v = torch.randn(t, hk, d, generator=g).bfloat16()
    do = torch.randn(t, hq, d, generator=g).bfloat16()
    return q, k, v, do


FA_DENSE = dict(seed=0, b=1, sq=128, sk=128, hq=4, hk=4, d=64)
FA_VARLEN = dict(seed=7, lens=[37, 96, 75], hq=4, hk=2, d=64)
RMS = dict(seed=1, rows=16, n=4096, eps=1e-6)
ACT = dict(seed=2, rows=32, d=512)


def rms_inputs(seed, rows, n):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, n, generator=g).bfloat16()
    w = (torch.rand(n, generator=g) + 0.5).bfloat16()
    return x, w


def act_inputs(seed, rows, d):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(rows, 2 * d, generator=g).bfloat16()


def make_fa_dense():
    c = FA_DENSE
    q, k, v, do = attention_inputs(c["seed"], c["b"], c["sq"], c["sk"], c["hq"], c["hk"], c["d"])
    qn, kn, vn, don = (t.float().numpy() for t in (q, k, v, do))
    out, lse = OA.forward(qn, kn, vn, causal=True)
    dq, dk, dv, delta = OA.backward(qn, kn, vn, out, don, lse, causal=True)
    return dict(q=bits(q), k=bits(k), v=bits(v), dout=bits(do), out=out.astype(np.float32),
                lse=lse.astype(np.float32), dq=dq.astype(np.float32), dk=dk.astype(np.float32),
                dv=dv.astype(np.float32), delta=np.asarray(delta, np.float32))


def make_fa_varlen():
    c = FA_VARLEN
    q, k, v, do = varlen_inputs(c["seed"], c["lens"], c["hq"], c["hk"], c["d"])
    cu = np.concatenate([[0], np.cumsum(c["lens"])]).astype(np.int32)
    qn, kn, vn, don = (t.float().numpy() for t in (q, k, v, do))
    out, lse = OA.varlen_forward(qn, kn, vn, cu, cu, causal=True)
    dq, dk, dv, delta = OA.varlen_backward(qn, kn, vn, out, don, lse, cu, cu, causal=True)
    return dict(q=bits(q), k=bits(k), v=bits(v), dout=bits(do), cu_seqlens=cu,
                out=out.astype(np.float32), lse=lse.astype(np.float32), dq=dq.astype(np.float32),
                dk=dk.astype(np.float32), dv=dv.astype(np.float32), delta=np.asarray(delta, np.float32))


def make_rms():
    c = RMS
    x, w = rms_inputs(c["seed"], c["rows"], c["n"])
    y, rstd = R.forward(x.float().numpy(), w.float().numpy(), c["eps"], 0.0, "llama", "bf16")
    return dict(x=bits(x), weight=bits(w), y=bf16_bits(y), rstd=np.asarray(rstd, np.float32))


def make_act():
    c = ACT
    x = act_inputs(c["seed"], c["rows"], c["d"])
    xn = x.float().numpy()
    res = dict(x=bits(x))
    for op in ("silu_and_mul", "gelu_and_mul", "gelu_tanh_and_mul"):
        res[op] = bf16_bits(A.gated(op, xn, "bf16"))
    return res


FIXTURES = {
    "fa_dense_causal_b1_h4_s128_d64.npz": make_fa_dense,
    "fa_varlen_causal_l37_96_75_h4_hk2_d64.npz": make_fa_varlen,
    "rms_norm_llama_16x4096.npz": make_rms,
    "gated_act_32x1024.npz": make_act,
}


def main():
    for name, fn in FIXTURES.items():
        arrays = fn()
        np.savez_compressed(HERE / name, **arrays)
        print(name, {k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    main()
