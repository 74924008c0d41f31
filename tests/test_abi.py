"""The C ABI: libkcr_hip.so loads, exports every symbol include/*.h
declares, and validates arguments (with the reference's error texts) before
touching any device memory -- so these run on the CPU."""

import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    text = "".join(h.read_text() for h in sorted((ROOT / "include").glob("*.h")))
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(re.findall(r"\b(kcr_[a-z0-9_]+)\s*\(", text))
    # KCR_TVM_FFI_EXPORT(name) declares __tvm_ffi_<name>.
    names |= {"__tvm_ffi_" + n for n in re.findall(r"^KCR_TVM_FFI_EXPORT\((\w+)\)", text, flags=re.M)}
    return sorted(names)


def test_library_exports_every_declared_symbol():
    import kcr_native

    names = declared_symbols()
    assert "kcr_silu_and_mul" in names and "kcr_rms_norm_forward" in names
    assert "__tvm_ffi_fwd_lse" in names and "kcr_hbm_stream_probe" in names
    missing = [n for n in names if not hasattr(kcr_native.lib, n)]
    assert not missing, missing
    assert "gfx950" in kcr_native.version()


@pytest.mark.parametrize(
    "out_shape, x_shape, match",
    [
        ((7, 512), (7, 512), "out must have shape"),
        ((7, 256), (7, 513), "must be even"),
        ((6, 256), (7, 512), "out must have shape"),
        ((7, 256), (), "at least one dimension"),
    ],
)
def test_act_and_mul_rejects_bad_shapes(out_shape, x_shape, match):
    # activation-rs/tests/kernels/test_activation.py:308-329
    import activation_rs

    x = torch.randn(x_shape, dtype=torch.half)
    out = torch.empty(out_shape, dtype=torch.half)
    with pytest.raises(ValueError, match=match):
        activation_rs.ops.silu_and_mul(out, x)


def test_activation_rejects_bad_shape_and_dtypes():
    import activation_rs

    x = torch.randn(7, 512, dtype=torch.half)
    with pytest.raises(ValueError, match="out must have shape"):
        activation_rs.ops.gelu(torch.empty(7, 256, dtype=torch.half), x)
    with pytest.raises(ValueError, match="same dtype"):
        activation_rs.ops.silu(torch.empty(7, 512, dtype=torch.float), x)
    x = torch.randn(7, 512, dtype=torch.double)
    with pytest.raises(ValueError, match="unsupported dtype"):
        activation_rs.ops.silu(torch.empty_like(x), x)
    x = torch.randn(512, 14, dtype=torch.half).t()
    with pytest.raises(ValueError, match="contiguous"):
        activation_rs.ops.silu_and_mul(torch.empty(14, 256, dtype=torch.half), x)


def test_host_tensors_never_reach_a_kernel():
    import activation_rs

    x = torch.randn(7, 512, dtype=torch.half)
    with pytest.raises(ValueError, match="GPU tensor"):
        activation_rs.ops.silu_and_mul(torch.empty(7, 256, dtype=torch.half), x)
    # Empty inputs are accepted and do nothing (test_activation.py:297-305).
    activation_rs.ops.silu_and_mul(torch.empty(0, 64, dtype=torch.half), torch.empty(0, 128, dtype=torch.half))


@pytest.mark.parametrize(
    "x_shape, weight_shape, weight_dtype, casting_mode, match",
    [
        ((4, 64), (64,), torch.bfloat16, "llama2", "casting mode"),
        ((4, 64), (32,), torch.bfloat16, "llama", "weight must have shape"),
        ((4, 64), (64,), torch.float16, "llama", "dtype of x or be float32"),
        ((2, 65537), (65537,), torch.bfloat16, "llama", "at most 65536"),
        ((), (1,), torch.bfloat16, "llama", "at least one dimension"),
    ],
)
def test_rms_norm_rejects_bad_arguments(x_shape, weight_shape, weight_dtype, casting_mode, match):
    # rmsnorm/tests/test_ops.py:102-124
    import rmsnorm

    x = torch.randn(x_shape, dtype=torch.bfloat16)
    w = torch.randn(weight_shape, dtype=weight_dtype)
    with pytest.raises(ValueError, match=match):
        rmsnorm.ops.rms_norm_forward(torch.empty_like(x), torch.empty(x.shape[:-1]), x, w, 1e-6,
                                     0.0, casting_mode)


def test_rms_norm_rejects_unsupported_dtype():
    import rmsnorm

    x = torch.randn(4, 64, dtype=torch.float64)
    with pytest.raises(ValueError, match="unsupported dtype"):
        rmsnorm.ops.rms_norm_forward(torch.empty_like(x), torch.empty(4), x, None, 1e-6, 0.0, "llama")


def test_rms_norm_backward_requires_partials_with_weight():
    import rmsnorm

    x = torch.randn(4, 64, dtype=torch.bfloat16)
    w = torch.randn(64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="dw_partial is required"):
        rmsnorm.ops.rms_norm_backward(torch.empty_like(x), None, x, x, w, torch.empty(4), 0.0, "llama")
    with pytest.raises(ValueError, match=r"dw_partial must have shape \[blocks, 64\]"):
        rmsnorm.ops.rms_norm_backward(torch.empty_like(x), torch.empty(4, 32), x, x, w,
                                      torch.empty(4), 0.0, "llama")
