"""Shared attention test cases (shapes follow flash-attn2-rs/tests/test_gold.py:872-1230)."""

import numpy as np
import torch

from oracle import attention as OA


def case(name, batch, hq, hk, sq, sk, **options):
    return (name, (batch, hq, hk, sq, sk), options)


PARITY_CASES = [
    case("full-mha", 2, 4, 4, 256, 256),
    case("causal-mha", 2, 4, 4, 256, 256, causal=True),
    case("causal-gqa-h8-hk2", 2, 8, 2, 256, 256, causal=True),
    case("full-mqa-h4-hk1", 1, 4, 1, 192, 192),
    case("causal-sq256-sk512", 1, 4, 4, 256, 512, causal=True),
    case("causal-sq320-sk256", 1, 4, 4, 320, 256, causal=True),
    case("full-sq128-sk256", 1, 4, 4, 128, 256),
    case("custom-scale", 2, 4, 4, 256, 256, causal=True, softmax_scale=0.05),
    case("local-causal-wl64", 2, 4, 4, 256, 256, causal=True, window_left=64),
    case("window-wl64-wr64", 1, 4, 4, 256, 256, window_left=64, window_right=64),
    case("softcap30-causal", 2, 4, 4, 256, 256, causal=True, softcap=30.0),
    case("softcap50-full", 1, 4, 4, 192, 192, softcap=50.0),
    case("alibi-causal", 2, 4, 4, 256, 256, causal=True, alibi=True),
    case("alibi-full", 1, 4, 4, 192, 192, alibi=True),
    case("alibi-local-wl64", 1, 4, 4, 256, 256, causal=True, window_left=64, alibi=True),
    case("softcap-alibi-gqa-causal", 2, 8, 2, 256, 256, causal=True, softcap=20.0, alibi=True),
    case("long-causal-s2048", 1, 8, 8, 2048, 2048, causal=True),
    case("window-wr32", 1, 4, 4, 256, 256, window_right=32),
    case("window-wl32", 1, 4, 4, 256, 256, window_left=32),
    case("zero-window-causal-wl0", 1, 4, 4, 256, 256, causal=True, window_left=0),
    case("window-wl200-wr8", 1, 4, 4, 512, 512, window_left=200, window_right=8),
    case("window-sq128-sk384-wl64", 1, 4, 4, 128, 384, causal=True, window_left=64),
    case("window-sq384-sk256-wl64", 1, 4, 4, 384, 256, causal=True, window_left=64),
    case("odd-causal-s333", 2, 4, 4, 333, 333, causal=True),
    case("odd-full-s200", 2, 4, 4, 200, 200),
    case("odd-full-gqa-sq600-sk700", 1, 8, 2, 600, 700),
    case("odd-gqa-causal-s130", 2, 8, 2, 130, 130, causal=True),
    case("odd-sq100-sk250", 1, 4, 4, 100, 250, causal=True),
    case("odd-window-softcap-s300", 1, 4, 4, 300, 300, causal=True, window_left=100, softcap=30.0),
    *[case(f"d{d}-causal-gqa", 2, 8, 2, 256, 256, causal=True, head_dim=d) for d in (32, 64, 96, 256)],
    *[case(f"d{d}-causal-mha", 2, 4, 4, 256, 256, causal=True, head_dim=d) for d in (8, 48, 72, 160, 200, 224)],
    case("d64-softcap-causal", 1, 4, 4, 192, 192, causal=True, softcap=30.0, head_dim=64),
    case("d256-softcap-alibi-gqa-causal", 2, 8, 2, 256, 256, causal=True, softcap=20.0, alibi=True, head_dim=256),
    case("d256-window-odd-s300", 1, 4, 4, 300, 300, window_left=64, window_right=16, head_dim=256),
    case("bf16-full-mha", 2, 4, 4, 256, 256, dtype=torch.bfloat16),
    case("bf16-causal-gqa", 2, 8, 2, 256, 256, causal=True, dtype=torch.bfloat16),
    case("bf16-softcap-causal", 2, 4, 4, 256, 256, causal=True, softcap=30.0, dtype=torch.bfloat16),
    case("bf16-alibi-causal", 2, 4, 4, 256, 256, causal=True, alibi=True, dtype=torch.bfloat16),
    case("bf16-local-wl64", 2, 4, 4, 256, 256, causal=True, window_left=64, dtype=torch.bfloat16),
    case("bf16-odd-causal-s333", 2, 4, 4, 333, 333, causal=True, dtype=torch.bfloat16),
    case("bf16-long-causal-s2048", 1, 8, 8, 2048, 2048, causal=True, dtype=torch.bfloat16),
    case("bf16-d64-causal", 2, 4, 4, 256, 256, causal=True, dtype=torch.bfloat16, head_dim=64),
    case("bf16-d256-causal", 1, 4, 4, 256, 256, causal=True, dtype=torch.bfloat16, head_dim=256),
]


def make_inputs(shape, options, seed=0, device="cuda"):
    batch, hq, hk, sq, sk = shape
    options = dict(options)
    dtype = options.pop("dtype", torch.float16)
    d = options.pop("head_dim", 128)
    alibi = options.pop("alibi", False)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, sq, hq, d, generator=g).to(dtype)
    k = torch.randn(batch, sk, hk, d, generator=g).to(dtype)
    v = torch.randn(batch, sk, hk, d, generator=g).to(dtype)
    if alibi:
        heads = torch.arange(hq).float()
        options["alibi_slopes"] = 2.0 ** (-8.0 * (heads + 1) / hq)
    return q, k, v, options, dtype


def oracle_kwargs(options):
    kw = {}
    for key in ("softmax_scale", "causal", "window_left", "window_right", "softcap"):
        if key in options:
            kw[key] = options[key]
    if "alibi_slopes" in options:
        kw["alibi_slopes"] = options["alibi_slopes"].numpy()
    return kw


def tolerances(dtype):
    # flash-attn2-rs/tests/test_gold.py:1265-1268
    if dtype == torch.float16:
        return dict(atol=2e-3, rtol=2.5e-2, mean=3e-3, lse=3e-2)
    return dict(atol=1e-2, rtol=5e-2, mean=8e-3, lse=8e-2)
