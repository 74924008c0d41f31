"""Calls the __tvm_ffi_* exports of libkcr_hip.so the way a tvm-ffi runtime
would: packed TVMFFIAny arguments (DLTensor pointers for tensors), with the
runtime entry points the adapters need provided by tests/tvm_ffi_mock (built
here with gcc and loaded globally, so the library finds it by dlsym)."""

import ctypes
import os
import subprocess
import tempfile
from pathlib import Path

import torch

MOCK_SRC = Path(__file__).resolve().parent / "tvm_ffi_mock" / "mock_runtime.c"

NONE, INT, BOOL, FLOAT, DLTENSOR_PTR, RAW_STR, SMALL_STR, FUNCTION, TENSOR, ARRAY = 0, 1, 2, 3, 7, 8, 11, 68, 70, 71
DL_ROCM = 10


class Any(ctypes.Structure):
    class _V(ctypes.Union):
        _fields_ = [("i", ctypes.c_int64), ("f", ctypes.c_double), ("p", ctypes.c_void_p),
                    ("b", ctypes.c_char * 8)]

    _anonymous_ = ("v",)
    _fields_ = [("type_index", ctypes.c_int32), ("small", ctypes.c_uint32), ("v", _V)]


class DLDataType(ctypes.Structure):
    _fields_ = [("code", ctypes.c_uint8), ("bits", ctypes.c_uint8), ("lanes", ctypes.c_uint16)]


class DLDevice(ctypes.Structure):
    _fields_ = [("device_type", ctypes.c_int32), ("device_id", ctypes.c_int32)]


class DLTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("device", DLDevice), ("ndim", ctypes.c_int32),
                ("dtype", DLDataType), ("shape", ctypes.POINTER(ctypes.c_int64)),
                ("strides", ctypes.POINTER(ctypes.c_int64)), ("byte_offset", ctypes.c_uint64)]


DL_DTYPES = {torch.float16: (2, 16), torch.float32: (2, 32), torch.bfloat16: (4, 16), torch.int32: (0, 32),
             torch.int64: (0, 64), torch.float64: (2, 64)}
TORCH_DTYPES = {v: k for k, v in DL_DTYPES.items()}

_mock = None
_keep = []


def mock():
    """The mock runtime (built once per process, loaded with RTLD_GLOBAL)."""
    global _mock
    if _mock is None:
        out = Path(tempfile.mkdtemp()) / "libtvm_ffi_mock.so"
        subprocess.run(["gcc", "-shared", "-fPIC", "-O2", "-o", str(out), str(MOCK_SRC)], check=True)
        _mock = ctypes.CDLL(str(out), mode=ctypes.RTLD_GLOBAL)
        _mock.mock_error_kind.restype = ctypes.c_char_p
        _mock.mock_error_message.restype = ctypes.c_char_p
        _mock.mock_live_objects.restype = ctypes.c_int64
        _mock.mock_array_size.restype = ctypes.c_int64
        _mock.mock_array_size.argtypes = [ctypes.c_void_p]
        _mock.mock_array_item.restype = ctypes.c_void_p
        _mock.mock_array_item.argtypes = [ctypes.c_void_p, ctypes.c_int64]
        _mock.mock_tensor.restype = ctypes.POINTER(DLTensor)
        _mock.mock_tensor.argtypes = [ctypes.c_void_p]
        _mock.mock_refs.restype = ctypes.c_uint64
        _mock.mock_refs.argtypes = [ctypes.c_void_p]
        _mock.TVMFFIObjectDecRef.argtypes = [ctypes.c_void_p]
        _mock.mock_set_stream.argtypes = [ctypes.c_void_p]
        _mock.mock_make_reserve.restype = ctypes.c_void_p
        _mock.mock_make_reserve.argtypes = [ctypes.POINTER(ctypes.c_int64), ctypes.c_int64]
        _mock.mock_reserve_calls.restype = ctypes.c_int64
        _mock.mock_reserve_calls.argtypes = [ctypes.c_void_p]
        _mock.mock_reserve_arg.restype = ctypes.c_int64
        _mock.mock_reserve_arg.argtypes = [ctypes.c_void_p, ctypes.c_int]
    return _mock


class Function:
    """A tvm-ffi Function object argument (the mock's reserve function)."""

    def __init__(self, ptr):
        self.ptr = ptr


def make_reserve(*values):
    """A reserve Function returning Shape(values) and recording its arguments."""
    arr = (ctypes.c_int64 * max(len(values), 1))(*values)
    return Function(mock().mock_make_reserve(arr, len(values)))


_ALLOC_T = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32)
_allocated = []


@_ALLOC_T
def _torch_alloc(nbytes, device_id):
    t = torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=f"cuda:{device_id}")
    _allocated.append(t)
    return t.data_ptr()


def install_torch_allocator():
    m = mock()
    m.mock_set_alloc(_torch_alloc)
    m.mock_set_stream(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def dltensor(t):
    shape = (ctypes.c_int64 * max(t.dim(), 1))(*t.shape)
    strides = (ctypes.c_int64 * max(t.dim(), 1))(*t.stride())
    code, bits = DL_DTYPES[t.dtype]
    dev = DLDevice(DL_ROCM if t.is_cuda else 1, t.get_device() if t.is_cuda else 0)
    d = DLTensor(t.data_ptr(), dev, t.dim(), DLDataType(code, bits, 1), shape, strides, 0)
    _keep.append((shape, strides, d, t))
    return d


def pack(*values):
    arr = (Any * max(len(values), 1))()
    for i, x in enumerate(values):
        a = arr[i]
        if x is None:
            a.type_index = NONE
        elif isinstance(x, bool):
            a.type_index, a.i = BOOL, int(x)
        elif isinstance(x, int):
            a.type_index, a.i = INT, x
        elif isinstance(x, float):
            a.type_index, a.f = FLOAT, x
        elif isinstance(x, str):
            raw = x.encode()
            if len(raw) <= 7:
                a.type_index, a.small = SMALL_STR, len(raw)
                a.b = raw
            else:
                buf = ctypes.create_string_buffer(raw)
                _keep.append(buf)
                a.type_index, a.p = RAW_STR, ctypes.addressof(buf)
        elif isinstance(x, torch.Tensor):
            d = dltensor(x)
            a.type_index, a.p = DLTENSOR_PTR, ctypes.addressof(d)
        elif isinstance(x, Function):
            a.type_index, a.p = FUNCTION, x.ptr
        else:
            raise TypeError(type(x))
    return arr


def call(name, *values):
    """(return code, result Any) of __tvm_ffi_<name>(values...)."""
    import kcr_native

    fn = getattr(kcr_native.lib, "__tvm_ffi_" + name)
    fn.restype = ctypes.c_int32
    args = pack(*values)
    result = Any()
    rc = fn(None, args, len(values), ctypes.byref(result))
    return rc, result


def tensor_of(obj_ptr):
    """A torch view of a Tensor object the adapters returned (contiguous)."""
    d = mock().mock_tensor(obj_ptr).contents
    shape = [d.shape[i] for i in range(d.ndim)]
    dtype = TORCH_DTYPES[(d.dtype.code, d.dtype.bits)]
    n = 1
    for s in shape:
        n *= s
    for t in _allocated:
        if t.data_ptr() == d.data:
            return t[: n * torch.tensor([], dtype=dtype).element_size()].view(dtype).view(shape)
    raise LookupError("tensor not allocated by the mock")


def array_items(any_result):
    m = mock()
    assert any_result.type_index == ARRAY
    return [m.mock_array_item(any_result.p, i) for i in range(m.mock_array_size(any_result.p))]
