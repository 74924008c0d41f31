"""ctypes binding of libkcr_hip.so (the C ABI in include/kcr_hip.h).

This module plays the role of the tvm-ffi runtime in the reference: it turns
torch tensors into the plain `kcr_tensor` descriptors the C ABI takes (the DLPack
fields a tvm-ffi `Tensor` carries), passes the current HIP stream (the reference
reads `TVMFFIEnvGetStream`, flash-attn2-rs/src/host/forward/mod.rs:612) and maps
the returned status to the Python exception kind the reference raises
(ValueError / TypeError / RuntimeError, as tvm-ffi does for `Error::set_raised`).

There is no fallback: if the library is missing the import fails loudly.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

PKG_DIR = Path(__file__).resolve().parent.parent
LIB_PATH = Path(os.environ.get("KCR_HIP_LIB", PKG_DIR / "libkcr_hip.so"))

KCR_MAX_DIMS = 8

DTYPE_CODES = {
    torch.float32: 0,
    torch.float16: 1,
    torch.bfloat16: 2,
    torch.int32: 3,
    torch.int64: 4,
    torch.float64: 5,
}
DTYPE_OTHER = 99


class KcrTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("device", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("shape", ctypes.c_int64 * KCR_MAX_DIMS),
        ("strides", ctypes.c_int64 * KCR_MAX_DIMS),
    ]


class KcrDropout(ctypes.Structure):
    """`kcr_dropout`: dropout probability and the Philox (seed, offset), or a
    device int64 [2] RNG-state tensor holding them."""

    _fields_ = [
        ("p", ctypes.c_double),
        ("seed", ctypes.c_uint64),
        ("offset", ctypes.c_uint64),
        ("rng_state", ctypes.POINTER(KcrTensor)),
    ]


def dropout_arg(p, seed=0, offset=0, state=None):
    """A `kcr_dropout` reference (kept alive by the returned tuple's first item),
    or None when p is 0."""
    if not float(p) > 0.0:
        return None, None
    d = KcrDropout()
    d.p = float(p)
    d.seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    d.offset = int(offset) & 0xFFFFFFFFFFFFFFFF
    keep = None
    if state is not None:
        keep = describe(state)
        d.rng_state = ctypes.pointer(keep)
    return (d, keep), ctypes.byref(d)


_ERRORS = {1: ValueError, 2: TypeError, 3: RuntimeError}


def _load():
    if not LIB_PATH.exists():
        raise ImportError(
            f"libkcr_hip.so not found at {LIB_PATH}; build it with "
            "`python kernels-community-rs_amd/build.py` (hipcc, gfx950)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.kcr_last_error.restype = ctypes.c_char_p
    lib.kcr_version.restype = ctypes.c_char_p
    for name in ("kcr_flash_bwd_workspace_bytes", "kcr_flash_varlen_bwd_workspace_bytes",
                 "kcr_flash_fwd_kvcache_workspace_bytes"):
        if hasattr(lib, name):
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int64
            fn.argtypes = [ctypes.c_int64] * 4
    return lib


lib = _load()


_DIMS = ctypes.c_int64 * KCR_MAX_DIMS


def describe(t):
    """A `kcr_tensor` for a torch tensor (or a null pointer for None). Built in
    one constructor call: it runs for every tensor of every op call."""
    if t is None:
        return None
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"expected a Tensor, got {type(t).__name__}")
    nd = t.dim()
    if nd > KCR_MAX_DIMS:
        raise ValueError(f"tensors of rank {nd} are not supported (at most {KCR_MAX_DIMS})")
    # get_device(): the CUDA device index, -1 for host tensors.
    return KcrTensor(t.data_ptr(), DTYPE_CODES.get(t.dtype, DTYPE_OTHER), nd, t.get_device(), 0,
                     _DIMS(*t.shape), _DIMS(*t.stride()))


def ref(desc):
    return None if desc is None else ctypes.byref(desc)


def stream_of(*tensors):
    """The current HIP stream of the device the tensors live on."""
    for t in tensors:
        if isinstance(t, torch.Tensor) and t.is_cuda:
            return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)
    return ctypes.c_void_p(0)


def check(status):
    if status != 0:
        message = lib.kcr_last_error().decode()
        raise _ERRORS.get(status, RuntimeError)(message)


def call(name, *args):
    """Calls a C entry point and raises on failure."""
    check(getattr(lib, name)(*args))


def op_namespace_prefixer(package: str):
    """`torch_add_op_namespace_prefix` of one package, like kernel-builder's
    generated `_ops` module: every package registers its torch ops in its own
    namespace."""

    def torch_add_op_namespace_prefix(name: str) -> str:
        return f"kcr_{package}::{name}"

    return torch_add_op_namespace_prefix


def version() -> str:
    return lib.kcr_version().decode()
