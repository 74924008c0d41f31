"""Benchmark of the kernels-community-rs hot paths on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--headline OP] [--only OP,...]

A "step" is one call of an op over its BASELINE.json configuration with inputs
already resident in HBM. The headline op (default: FA2 forward, causal, B=4
Hq=32 Hkv=8 S=4096 D=128 bf16) gives `value`; every op
measured is listed under "ops" with its own throughput and roofline fraction.
Timing: W untimed warmup steps, then untimed steps for at least --warm-ms of
wall time (the GPU's clocks settle under sustained load), then HIP events
recorded on the stream the kernels are launched on (torch's current stream,
which the ops pass to the C ABI) around exactly K steps, bracketed by
torch.cuda.synchronize().

Prints ONE JSON line.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "kernels-community-rs_amd"))

import torch  # noqa: E402

PEAK_HBM_GBS = 8000.0  # MI355X HBM3E, GB/s
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, TFLOP/s

METRIC = "FA2 fwd/bwd TFLOP/s (% bf16 MFMA peak) at S=4k D=128; RMSNorm/act HBM GB/s"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# --------------------------------------------------------------------------
# Workloads. Each returns (run, work, unit, bound, sample_fn).
# --------------------------------------------------------------------------


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def wl_rmsnorm():
    import rmsnorm

    g = _gen(1)
    rows, n = 16384, 4096
    x = torch.randn(rows, n, generator=g).bfloat16().cuda()
    w = (torch.rand(n, generator=g) + 0.5).bfloat16().cuda()
    y = torch.empty_like(x)
    rstd = torch.empty(rows, device="cuda")

    def run():
        rmsnorm.ops.rms_norm_forward(y, rstd, x, w, 1e-6, 0.0, "llama")

    bytes_ = rows * n * 2 * 2 + n * 2 + rows * 4  # read x, w; write y, rstd
    return dict(run=run, work=bytes_, bound="hbm", kernel="rms_fwd_wave",
                config={"x": [rows, n], "dtype": "bf16", "eps": 1e-6, "casting_mode": "llama"},
                cpu=lambda: cpu_rmsnorm(x, w))


def wl_rmsnorm_bwd():
    """RMSNorm backward at the forward's shape: dx and the per-block fp32 weight
    gradient partials, then their fixed-order reduction into dw."""
    import rmsnorm

    g = _gen(3)
    rows, n = 16384, 4096
    x = torch.randn(rows, n, generator=g).bfloat16().cuda()
    dy = torch.randn(rows, n, generator=g).bfloat16().cuda()
    w = (torch.rand(n, generator=g) + 0.5).bfloat16().cuda()
    rstd = torch.empty(rows, device="cuda")
    rmsnorm.ops.rms_norm_forward(torch.empty_like(x), rstd, x, w, 1e-6, 0.0, "llama")
    dx = torch.empty_like(x)
    dw = torch.empty_like(w)
    blocks = 4 * torch.cuda.get_device_properties(0).multi_processor_count
    dw_partial = torch.empty(blocks, n, dtype=torch.float32, device="cuda")

    def run():
        rmsnorm.ops.rms_norm_backward(dx, dw_partial, dy, x, w, rstd, 0.0, "llama")
        rmsnorm.ops.rms_norm_reduce_weight_grad(dw, dw_partial)

    # Algorithmic: read x, dy, w, rstd; write dx, dw (the partials are overhead).
    bytes_ = rows * n * 2 * 3 + n * 2 * 2 + rows * 4
    return dict(run=run, work=bytes_, bound="hbm", kernel="rms_bwd_split",
                config={"x": [rows, n], "dtype": "bf16", "casting_mode": "llama"}, cpu=None)


def wl_silu():
    """Elementwise silu (one of the non-gated activations) on the gated
    workload's output shape."""
    import activation_rs

    g = _gen(4)
    x = torch.randn(16384, 14336, generator=g).bfloat16().cuda()
    out = torch.empty_like(x)

    def run():
        activation_rs.ops.silu(out, x)

    return dict(run=run, work=2 * x.numel() * 2, bound="hbm", kernel="activation_lut",
                config={"x": list(x.shape), "dtype": "bf16"}, cpu=None)


def _wl_gated(op):
    def make():
        import activation_rs

        g = _gen(2)
        tokens, d2 = 16384, 28672
        x = torch.randn(tokens, d2, generator=g).bfloat16().cuda()
        out = torch.empty(tokens, d2 // 2, dtype=x.dtype, device="cuda")
        fn = getattr(activation_rs.ops, op)

        def run():
            fn(out, x)

        bytes_ = tokens * d2 * 2 + tokens * (d2 // 2) * 2
        return dict(run=run, work=bytes_, bound="hbm", kernel="act_and_mul_lut",
                    config={"x": [tokens, d2], "out": [tokens, d2 // 2], "dtype": "bf16"},
                    cpu=lambda: cpu_gated(op, x))

    return make


def _attn_inputs(seed, b=4, hq=32, hkv=8, s=4096, d=128):
    g = _gen(seed)
    q = torch.randn(b, s, hq, d, generator=g).bfloat16().cuda()
    k = torch.randn(b, s, hkv, d, generator=g).bfloat16().cuda()
    v = torch.randn(b, s, hkv, d, generator=g).bfloat16().cuda()
    return q, k, v


def _score_options(hq, alibi, softcap):
    """ALiBi slopes (the usual 2^(-8 (h + 1) / H) ladder) and the softcap, for the
    scored-kernel workloads; none by default."""
    slopes = (2.0 ** (-8.0 * (torch.arange(hq) + 1) / hq)).float().cuda() if alibi else None
    extra = {**({"alibi": True} if alibi else {}), **({"softcap": softcap} if softcap else {})}
    return slopes, float(softcap), extra


def _wl_fa_fwd(causal, p_dropout=0.0, d=128, alibi=False, softcap=0.0):
    def make():
        import flash_attn2_rs

        b, hq, hkv, s = 4, 32, 8, 4096
        q, k, v = _attn_inputs(3, b, hq, hkv, s, d)
        out = torch.empty_like(q)
        ops = flash_attn2_rs.ops
        drop = (p_dropout, 1234, 0) if p_dropout > 0 else ()
        slopes, cap, extra = _score_options(hq, alibi, softcap)

        def run():
            ops.fwd_lse(q, k, v, slopes, None, causal, -1, -1, cap, *drop, out)

        flops = 4.0 * b * hq * s * s * d * (0.5 if causal else 1.0)
        plain = not (alibi or softcap) and d == 128
        return dict(run=run, work=flops, bound="mfma", kernel="flash_fwd",
                    config={"B": b, "Hq": hq, "Hkv": hkv, "S": s, "D": d, "causal": causal,
                            "dtype": "bf16", **({"p_dropout": p_dropout} if p_dropout else {}), **extra},
                    cpu=(lambda: cpu_attention(q, k, v, causal)) if plain else None)

    return make


def _wl_fa_bwd(causal, p_dropout=0.0, d=128, alibi=False, softcap=0.0):
    def make():
        import flash_attn2_rs

        b, hq, hkv, s = 4, 32, 8, 4096
        q, k, v = _attn_inputs(3, b, hq, hkv, s, d)
        g = _gen(4)
        dout = torch.randn(b, s, hq, d, generator=g).bfloat16().cuda()
        out = torch.empty_like(q)
        ops = flash_attn2_rs.ops
        state = torch.tensor([1234, 0], dtype=torch.int64, device="cuda") if p_dropout > 0 else None
        drop = (p_dropout, state, 0) if p_dropout > 0 else ()
        slopes, cap, extra = _score_options(hq, alibi, softcap)
        lse = ops.fwd_lse(q, k, v, slopes, None, causal, -1, -1, cap, *drop, out)
        args = (slopes, None, causal, -1, -1, cap, p_dropout, state)

        def run():
            delta = ops.bwd_preprocess(dout, out, p_dropout)
            ops.bwd_all(q, k, v, dout, lse, delta, *args)

        flops = 2.5 * 4.0 * b * hq * s * s * d * (0.5 if causal else 1.0)
        return dict(run=run, work=flops, bound="mfma", kernel="flash_bwd_dkv",
                    config={"B": b, "Hq": hq, "Hkv": hkv, "S": s, "D": d, "causal": causal,
                            "dtype": "bf16", **({"p_dropout": p_dropout} if p_dropout else {}), **extra},
                    cpu=None)

    return make


def varlen_lengths(seed=5, count=16, lo=128, hi=8192):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (count,), generator=g).tolist()


def _wl_fa_varlen(kind):
    def make():
        import flash_attn2_rs

        lens = varlen_lengths()
        hq, hkv, d = 32, 8, 128
        total = sum(lens)
        cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int32).cuda()
        g = _gen(6)
        q = torch.randn(total, hq, d, generator=g).bfloat16().cuda()
        k = torch.randn(total, hkv, d, generator=g).bfloat16().cuda()
        v = torch.randn(total, hkv, d, generator=g).bfloat16().cuda()
        ops = flash_attn2_rs.ops
        mx = max(lens)
        fwd_args = (q, k, v, cu, cu, None, None, None, None, True, -1, -1, 0.0, 0.0, None, mx, mx,
                    False, False)
        sum_sq = sum(l * l for l in lens)
        fwd_flops = 4.0 * hq * d * sum_sq * 0.5
        if kind == "fwd":
            def run():
                ops.varlen_fwd_explicit(*fwd_args)

            work = fwd_flops
        else:
            out, lse, _ = ops.varlen_fwd_explicit(*fwd_args)
            dout = torch.randn(total, hq, d, generator=g).bfloat16().cuda()

            def run():
                ops.varlen_bwd_explicit(q, k, v, dout, out, lse, cu, cu, None, None, True, -1, -1,
                                        0.0, 0.0, None, mx, mx, False)

            work = 2.5 * fwd_flops
        return dict(run=run, work=work, bound="mfma", kernel="flash_fwd" if kind == "fwd" else "flash_bwd_dkv",
                    config={"seqs": len(lens), "sum_L": total, "sum_L2": sum_sq, "Hq": hq,
                            "Hkv": hkv, "D": d, "causal": True, "dtype": "bf16"},
                    cpu=None)

    return make


def wl_fa_kvcache_decode(graph=False):
    """flash_attn_with_kvcache decode step (an inference path with no benchmark
    config of its own): B=16 sequences with 8191 cached tokens each, one new
    token appended, Hq=32, Hkv=8, D=128 bf16, causal, automatic key splits.
    HBM-bound: the step reads the whole K/V cache once,
    16 x 8192 x 8 x 128 x 2 x 2 = 536,870,912 B."""
    import flash_attn2_rs

    b, hq, hkv, d, cap = 16, 32, 8, 128, 8192
    g = _gen(7)
    kc = torch.randn(b, cap, hkv, d, generator=g).bfloat16().cuda()
    vc = torch.randn(b, cap, hkv, d, generator=g).bfloat16().cuda()
    q = torch.randn(b, 1, hq, d, generator=g).bfloat16().cuda()
    kn = torch.randn(b, 1, hkv, d, generator=g).bfloat16().cuda()
    vn = torch.randn(b, 1, hkv, d, generator=g).bfloat16().cuda()
    lengths = torch.full((b,), cap - 1, dtype=torch.int32, device="cuda")

    def run():
        flash_attn2_rs.flash_attn_with_kvcache(q, kc, vc, kn, vn, cache_seqlens=lengths, causal=True,
                                               num_splits=0)

    if graph:
        # The same step captured once and replayed: no Python or launch cost
        # per step (the append position is fixed, as in the eager run).
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            run()
        torch.cuda.current_stream().wait_stream(side)
        captured = torch.cuda.CUDAGraph()
        with torch.cuda.graph(captured):
            run()
        run = captured.replay
    return dict(run=run, work=2 * b * cap * hkv * d * 2, bound="hbm", kernel="flash_fwd_tiled",
                config={"B": b, "Hq": hq, "Hkv": hkv, "D": d, "cache_len": cap, "new_tokens": 1,
                        "causal": True, "dtype": "bf16", **({"cuda_graph": True} if graph else {})}, cpu=None)


def wl_hbm_copy():
    """Plain device copy (torch `copy_`) of the activation input size
    (939,524,096 B read and written), for comparison with the streaming probe."""
    g = _gen(2)
    x = torch.randn(16384, 28672, generator=g).bfloat16().cuda()
    y = torch.empty_like(x)

    def run():
        y.copy_(x)

    return dict(run=run, work=2 * x.numel() * 2, bound="hbm", kernel="elementwise_kernel",
                config={"x": list(x.shape), "dtype": "bf16"}, cpu=None)


def wl_gemm_ceiling():
    """The MFMA rate a GEMM reaches under the board's power cap: torch.matmul
    (hipBLASLt) of two 8192 x 8192 bf16 matrices, 2 * 8192^3 FLOP per call."""
    g = _gen(4)
    n = 8192
    a = torch.randn(n, n, generator=g).bfloat16().cuda()
    b = torch.randn(n, n, generator=g).bfloat16().cuda()
    c = torch.empty(n, n, dtype=torch.bfloat16, device="cuda")

    def run():
        torch.matmul(a, b, out=c)

    return dict(run=run, work=2 * n ** 3, bound="mfma", kernel="Cijk",
                config={"m": n, "n": n, "k": n, "dtype": "bf16"}, cpu=None)


def _wl_hbm_stream(reads):
    """The HBM ceiling the bandwidth-bound ops can reach: `kcr_hbm_stream_probe`,
    the gated kernel's memory shape with no arithmetic. reads=1 copies the
    RMSNorm-sized 134,217,728 B (1:1 read:write, like RMSNorm forward); reads=2
    reads the gated input's 939,524,096 B and writes half of it (2:1, like
    silu_and_mul)."""

    def make():
        import kcr_native

        if reads == 1:
            words = 16384 * 4096 * 2 // 16
        else:
            words = 16384 * 14336 * 2 // 16
        src = torch.empty(reads * words * 16, dtype=torch.uint8, device="cuda").random_(0, 256)
        dst = torch.empty(words * 16, dtype=torch.uint8, device="cuda")
        fn = kcr_native.lib.kcr_hbm_stream_probe

        def run():
            stream = kcr_native.stream_of(dst)
            kcr_native.check(fn(ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(src.data_ptr()),
                                ctypes.c_int64(words), ctypes.c_int32(reads), stream))

        return dict(run=run, work=(reads + 1) * words * 16, bound="hbm", kernel="hbm_stream_kernel",
                    config={"read_bytes": reads * words * 16, "write_bytes": words * 16,
                            "read_write": f"{reads}:1"}, cpu=None)

    return make


def wl_fa_split():
    """Short queries against long keys (an underfilled grid without key splits):
    B=1, Hq=8, Hkv=2, Sq=128, Sk=32768, D=128, causal bf16. 8 query tiles alone
    would occupy 8 of the 256 CUs."""
    import flash_attn2_rs

    b, hq, hkv, sq, sk, d = 1, 8, 2, 128, 32768, 128
    g = _gen(8)
    q = torch.randn(b, sq, hq, d, generator=g).bfloat16().cuda()
    k = torch.randn(b, sk, hkv, d, generator=g).bfloat16().cuda()
    v = torch.randn(b, sk, hkv, d, generator=g).bfloat16().cuda()
    out = torch.empty_like(q)
    ops = flash_attn2_rs.ops

    def run():
        ops.fwd_lse(q, k, v, None, None, True, -1, -1, 0.0, out)

    # Causal with Sk > Sq: row i sees Sk - Sq + i + 1 keys.
    pairs = sum(sk - sq + i + 1 for i in range(sq))
    return dict(run=run, work=4.0 * b * hq * d * pairs, bound="mfma", kernel="flash_fwd_tiled",
                config={"B": b, "Hq": hq, "Hkv": hkv, "Sq": sq, "Sk": sk, "D": d, "causal": True,
                        "dtype": "bf16"}, cpu=None)


def wl_fa_config1():
    """BASELINE.json configs[0], the reference's CPU-runnable case: B=1,
    Hq=Hkv=4, S=128, D=64, causal bf16. On the GPU it is launch-bound; the CPU
    baseline times it in full."""
    import flash_attn2_rs

    b, h, s, d = 1, 4, 128, 64
    q, k, v = _attn_inputs(0, b, h, h, s, d)
    out = torch.empty_like(q)
    ops = flash_attn2_rs.ops

    def run():
        ops.fwd_lse(q, k, v, None, None, True, -1, -1, 0.0, out)

    flops = 4.0 * b * h * s * s * d * 0.5
    return dict(run=run, work=flops, bound="mfma", kernel="flash_fwd",
                config={"B": b, "Hq": h, "Hkv": h, "S": s, "D": d, "causal": True, "dtype": "bf16"},
                cpu=lambda: cpu_attention(q, k, v, True, full=True))


WORKLOADS = {
    "fa_fwd_causal": _wl_fa_fwd(True),
    "fa_fwd": _wl_fa_fwd(False),
    "fa_bwd_causal": _wl_fa_bwd(True),
    "fa_bwd": _wl_fa_bwd(False),
    "fa_fwd_causal_dropout": _wl_fa_fwd(True, 0.1),
    "fa_bwd_causal_dropout": _wl_fa_bwd(True, 0.1),
    # Opt-in (not in the default run): the scored (ALiBi / softcap) and padded
    # (head sizes 96 / 112) attention paths at the BASELINE shape.
    "fa_fwd_causal_alibi": _wl_fa_fwd(True, alibi=True),
    "fa_fwd_causal_softcap": _wl_fa_fwd(True, softcap=30.0),
    "fa_bwd_causal_alibi": _wl_fa_bwd(True, alibi=True),
    "fa_bwd_causal_softcap": _wl_fa_bwd(True, softcap=30.0),
    "fa_fwd_causal_d112": _wl_fa_fwd(True, d=112),
    "fa_bwd_causal_d96": _wl_fa_bwd(True, d=96),
    "fa_fwd_causal_d256": _wl_fa_fwd(True, d=256),
    "fa_bwd_causal_d256": _wl_fa_bwd(True, d=256),
    "fa_varlen_fwd": _wl_fa_varlen("fwd"),
    "fa_varlen_bwd": _wl_fa_varlen("bwd"),
    "rms_norm": wl_rmsnorm,
    "rms_norm_bwd": wl_rmsnorm_bwd,
    "silu_and_mul": _wl_gated("silu_and_mul"),
    "gelu_and_mul": _wl_gated("gelu_and_mul"),
    "gelu_tanh_and_mul": _wl_gated("gelu_tanh_and_mul"),
    "silu": wl_silu,
    "fa_kvcache_decode": wl_fa_kvcache_decode,
    "fa_kvcache_decode_graph": lambda: wl_fa_kvcache_decode(graph=True),
    "fa_fwd_split": wl_fa_split,
    "fa_fwd_config1": wl_fa_config1,
    "hbm_stream_1to1": _wl_hbm_stream(1),
    "hbm_stream_2to1": _wl_hbm_stream(2),
    "hbm_copy": wl_hbm_copy,
    "gemm_ceiling": wl_gemm_ceiling,
}
OPT_IN = ("hbm_copy", "gemm_ceiling", "fa_fwd_causal_alibi", "fa_fwd_causal_softcap", "fa_bwd_causal_alibi",
          "fa_bwd_causal_softcap", "fa_fwd_causal_d112", "fa_bwd_causal_d96",
          "fa_fwd_causal_d256", "fa_bwd_causal_d256", "fa_kvcache_decode_graph")
DEFAULT_ORDER = [n for n in WORKLOADS if n not in OPT_IN]
# Ops whose CPU baseline is timed in every default run (bounded samples).
CPU_OPS = ("fa_fwd_causal", "fa_fwd_config1", "rms_norm", "silu_and_mul")

# --------------------------------------------------------------------------
# CPU baselines: the oracle (the tests' formulas restated in numpy), timed on a
# bounded sample on this host, scaled to the metric's unit.
# --------------------------------------------------------------------------


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _timed(fn, min_runs=3, budget_s=8.0):
    fn()  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_runs or (time.perf_counter() < t_end and len(times) < 7):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2]


def _blas_threads():
    """Threads numpy's BLAS uses (the attention oracle's matmuls run on them)."""
    try:
        from threadpoolctl import threadpool_info

        return max([p["num_threads"] for p in threadpool_info() if p.get("user_api") == "blas"] or [1])
    except Exception:
        return 1


def cpu_gated(op, x):
    from oracle import activation as A

    rows = 256
    sample = x[:rows].float().cpu().numpy()
    t = _timed(lambda: A.gated(op, sample, "bf16"))
    bytes_ = rows * x.shape[1] * 2 * 1.5
    return {"value": bytes_ / t / 1e9, "unit": "GB/s", "cores": 1,
            "sample": f"oracle.activation.gated on {rows} of {x.shape[0]} rows (numpy, element-wise)"}


def cpu_rmsnorm(x, w):
    from oracle import rmsnorm as R

    rows = 1024
    sample = x[:rows].float().cpu().numpy()
    wn = w.float().cpu().numpy()
    t = _timed(lambda: R.forward(sample, wn, 1e-6, 0.0, "llama", "bf16"))
    bytes_ = rows * x.shape[1] * 2 * 2
    return {"value": bytes_ / t / 1e9, "unit": "GB/s", "cores": 1,
            "sample": f"oracle.rmsnorm.forward on {rows} of {x.shape[0]} rows (numpy, element-wise)"}


def cpu_attention(q, k, v, causal, full=False):
    from oracle import attention as OA

    if full:
        qs, ks, vs = (t.float().cpu().numpy() for t in (q, k, v))
        sample = f"oracle.attention.forward (numpy f32) on the whole call {list(q.shape)}"
        heads = q.shape[0] * q.shape[2]
    else:
        # One (batch, kv-group) slice: 4 query heads sharing one KV head, all rows.
        qs = q[:1, :, :4].float().cpu().numpy()
        ks = k[:1, :, :1].float().cpu().numpy()
        vs = v[:1, :, :1].float().cpu().numpy()
        sample = (f"oracle.attention.forward (numpy f32) on batch 0, query heads 0-3 / KV head 0, "
                  f"S={q.shape[1]}")
        heads = 4
    t = _timed(lambda: OA.forward(qs, ks, vs, causal=causal), min_runs=2, budget_s=15.0)
    s, d = q.shape[1], q.shape[3]
    flops = 4.0 * heads * s * s * d * (0.5 if causal else 1.0)
    return {"value": flops / t / 1e12, "unit": "TFLOP/s", "cores": _blas_threads(), "sample": sample}


# --------------------------------------------------------------------------


def measure(name, steps, warmup, warm_ms):
    wl = WORKLOADS[name]()
    run = wl["run"]
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    # Then untimed steps for at least warm_ms of wall time, so the timed steps
    # see the GPU's sustained clocks rather than the ramp after input set-up.
    t_end = time.perf_counter() + warm_ms * 1e-3
    while time.perf_counter() < t_end:
        for _ in range(max(1, steps // 4)):
            run()
        torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        run()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    if wl["bound"] == "hbm":
        achieved = wl["work"] / (ms * 1e-3) / 1e9
        peak, unit = PEAK_HBM_GBS, "GB/s"
    else:
        achieved = wl["work"] / (ms * 1e-3) / 1e12
        peak, unit = PEAK_BF16_TFLOPS, "TFLOP/s"
    return wl, ms, achieved, peak, unit


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--warm-ms", type=float, default=300.0,
                    help="after the warmup steps, keep stepping untimed for this long (ms)")
    ap.add_argument("--headline", default="fa_fwd_causal")
    ap.add_argument("--only", default=None, help="comma-separated workloads (default: all)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (every box in this run has one); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py is single-GPU; launch it without torch.distributed.run", file=sys.stderr)
        sys.exit(2)

    names = args.only.split(",") if args.only else list(DEFAULT_ORDER)
    if args.headline not in names:
        names.insert(0, args.headline)
    results = {}
    headline = None
    for name in names:
        log(f"[bench] {name} ...")
        try:
            wl, ms, achieved, peak, unit = measure(name, args.steps, args.warmup, args.warm_ms)
        except Exception as e:  # an op that is not built yet is reported, not fatal
            log(f"[bench] {name} failed: {type(e).__name__}: {e}")
            results[name] = {"error": f"{type(e).__name__}: {e}"}
            continue
        results[name] = {"value": round(achieved, 2), "unit": unit, "ms": round(ms, 4),
                         "frac_of_peak": round(achieved / peak, 4), "config": wl["config"]}
        log(f"[bench] {name}: {ms:.4f} ms, {achieved:.1f} {unit} ({achieved / peak:.1%} of peak)")
        if not args.no_cpu and wl.get("cpu") is not None and (name in CPU_OPS or name == args.headline):
            log(f"[bench] {name} cpu baseline ...")
            cpu = wl["cpu"]()
            cpu["kind"] = "port"
            cpu["cpu"] = cpu_model()
            cpu["value"] = round(cpu["value"], 4)
            results[name]["cpu_baseline"] = cpu
            log(f"[bench] {name} cpu: {cpu['value']} {cpu['unit']} on {cpu['cores']} thread(s)")
        if name == args.headline:
            headline = (wl, ms, achieved, peak, unit)
        del wl

    if headline is None:
        print(json.dumps({"metric": METRIC, "value": None, "error": results.get(args.headline)}))
        sys.exit(1)
    wl, ms, achieved, peak, unit = headline
    cpu = results[args.headline].get("cpu_baseline")
    traffic = None
    tfile = ROOT / "profiles" / "traffic.json"
    if tfile.exists():
        entry = json.loads(tfile.read_text()).get(args.headline)
        traffic = entry.get("hbm_bytes_per_launch") if entry else None
    line = {
        "metric": METRIC,
        "value": round(achieved, 2),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded torch.randn, BASELINE.json shapes)",
        "config": {"workload": args.headline, **wl["config"]},
        "roofline": {"bound": wl["bound"], "achieved": round(achieved, 2), "peak": peak,
                     "unit": unit, "frac": round(achieved / peak, 4), "traffic": traffic},
        "cpu_baseline": cpu,
        "ops": results,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
