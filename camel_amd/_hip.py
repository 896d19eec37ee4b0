"""ctypes binding of libcamel_hip.so (the C-ABI declared in include/camel_hip.h).

The binding fails loudly: importing it without the built library raises, and
every non-zero status raises :class:`CamelHipError` carrying the library's
message (the same text the reference's ``std::invalid_argument`` carries,
e.g. ``"Division by zero"``).  There is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libcamel_hip.so")

# enum camel_hip_status
OK, ERR_ARG, ERR_SHAPE, ERR_DIV_ZERO, ERR_LOG_DOMAIN, ERR_DTYPE, ERR_OOM, ERR_RUNTIME, \
    ERR_NO_DEVICE = range(9)
# enum camel_hip_dtype
DT_F32, DT_I64, DT_BOOL = 0, 1, 2
# BinaryOp / CompareOp (modules/tensor/runtime.h:39-53)
OP_ADD, OP_SUB, OP_MUL, OP_DIV, OP_POW = range(5)
CMP_LT, CMP_LE, CMP_GT, CMP_GE, CMP_EQ = range(5)
EPI_NONE, EPI_BIAS, EPI_RELU = 0, 1, 2
GEMM_A_T = 0x10
CONV_X_NHWC, CONV_Y_NHWC, CONV_W_PACKED = 0x100, 0x200, 0x400
CONV_X_NCHW4, CONV_Y_NCHW4 = 0x800, 0x1000

NP_DTYPE = {DT_F32: np.float32, DT_I64: np.int64, DT_BOOL: np.uint8}
DT_OF_NP = {np.dtype(np.float32): DT_F32, np.dtype(np.int64): DT_I64,
            np.dtype(np.uint8): DT_BOOL, np.dtype(np.bool_): DT_BOOL}


class CamelHipError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


_P = C.c_void_p
_I64 = C.c_int64
_I = C.c_int
_D = C.c_double

# name -> argtypes (restype is int unless listed in _RESTYPES)
_SIGNATURES = {
    "camel_hip_init": [_I],
    "camel_hip_device_count": [C.POINTER(_I)],
    "camel_hip_current_device": [C.POINTER(_I)],
    "camel_hip_last_error": [],
    "camel_hip_sync": [],
    "camel_hip_device_sync": [],
    "camel_hip_stream": [],
    "camel_hip_malloc": [C.POINTER(_P), C.c_size_t],
    "camel_hip_free": [_P],
    "camel_hip_free_shared": [_P],
    "camel_hip_pool_trim": [],
    "camel_hip_pool_stats": [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)],
    "camel_hip_h2d": [_P, _P, C.c_size_t],
    "camel_hip_d2h": [_P, _P, C.c_size_t],
    "camel_hip_d2d": [_P, _P, C.c_size_t],
    "camel_hip_fill": [_I, _P, _I64, _D],
    "camel_hip_eye": [_P, _I64],
    "camel_hip_arange": [_P, _I64, _I64, _I64],
    "camel_hip_sgemm": [_P, _P, _P, _I64, _I64, _I64, _P, _I],
    "camel_hip_sgemm_noalloc": [_P, _P, _P, _I64, _I64, _I64, _P, _I],
    "camel_hip_matmul_generic": [_I, _P, _I, _P, _I, _P, _I64, _I64, _I64],
    "camel_hip_conv2d": [_P, _P, _P, _P] + [_I64] * 9 + [_I],
    "camel_hip_conv2d_pool2": [_P, _P, _P, _P] + [_I64] * 9 + [_I],
    "camel_hip_conv2d_pair_pool2": [_P] * 6 + [_I64] * 5 + [_I, _I],
    "camel_hip_conv2d_pack_weights": [_P, _P] + [_I64] * 4,
    "camel_hip_dense_softmax": [_P, _P, _P, _P, _I64, _I64, _I64, _I],
    "camel_hip_dense_head": [_P, _P, _P, _P, _P, _P] + [_I64] * 4 + [_I, _I, _I],
    "camel_hip_maxpool2d": [_P, _P] + [_I64] * 7,
    "camel_hip_binary": [_I, _I, _P, _I, _P, _I, _P, _I64],
    "camel_hip_binary_scalar": [_I, _I, _I, _P, _D, _I, _P, _I64],
    "camel_hip_compare": [_I, _I, _P, _I, _P, _P, _I64],
    "camel_hip_compare_scalar": [_I, _I, _I, _P, _D, _P, _I64],
    "camel_hip_relu": [_P, _P, _I64],
    "camel_hip_exp": [_P, _P, _I64],
    "camel_hip_log": [_P, _P, _I64],
    "camel_hip_softmax_rows": [_P, _P, _I64, _I64],
    "camel_hip_sum_axis": [_I, _P, _I64, _I64, _I64, _P],
    "camel_hip_max_axis": [_I, _P, _I64, _I64, _I64, _P],
    "camel_hip_argmax_axis": [_I, _P, _I64, _I64, _I64, _P],
    "camel_hip_sum": [_I, _P, _I64, C.POINTER(_D)],
    "camel_hip_transpose2d": [_I, _P, _P, _I64, _I64],
    "camel_hip_concat": [_I, _P, _P, _P, _I64, _I64, _I64, _I64],
    "camel_hip_event_create": [C.POINTER(_P)],
    "camel_hip_event_record": [_P],
    "camel_hip_event_elapsed_ms": [_P, _P, C.POINTER(C.c_float)],
    "camel_hip_event_destroy": [_P],
}
_RESTYPES = {"camel_hip_last_error": C.c_char_p, "camel_hip_stream": _P}

_lib = None


def load(path: str = LIB_PATH) -> C.CDLL:
    """Loads libcamel_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build it with `python -m camel_amd.build`")
    lib = C.CDLL(path)
    for name, args in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPES.get(name, _I)
    _lib = lib
    return lib


def exported_symbols() -> list[str]:
    return sorted(_SIGNATURES)


def check(status: int) -> None:
    if status != OK:
        msg = load().camel_hip_last_error()
        raise CamelHipError(status, msg.decode() if msg else f"status {status}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))


class DeviceBuffer:
    """A block from the library's device pool, freed with the object."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        ptr = _P()
        call("camel_hip_malloc", C.byref(ptr), C.c_size_t(max(self.nbytes, 1)))
        self.ptr = ptr.value

    @property
    def handle(self) -> int:
        return self.ptr

    def free(self) -> None:
        if self.ptr:
            call("camel_hip_free", _P(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def upload(self, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        call("camel_hip_h2d", _P(self.ptr), arr.ctypes.data_as(_P), C.c_size_t(arr.nbytes))
        return self

    def download(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        assert out.nbytes <= self.nbytes
        call("camel_hip_d2h", out.ctypes.data_as(_P), _P(self.ptr), C.c_size_t(out.nbytes))
        return out


def to_device(arr: np.ndarray) -> DeviceBuffer:
    arr = np.ascontiguousarray(arr)
    return DeviceBuffer(arr.nbytes).upload(arr)


def sync() -> None:
    call("camel_hip_sync")


class Timer:
    """HIP events recorded on the library stream (the stream every kernel runs on)."""

    def __init__(self):
        self.start, self.stop = _P(), _P()
        call("camel_hip_event_create", C.byref(self.start))
        call("camel_hip_event_create", C.byref(self.stop))

    def begin(self) -> None:
        call("camel_hip_event_record", self.start)

    def end(self) -> float:
        call("camel_hip_event_record", self.stop)
        ms = C.c_float()
        call("camel_hip_event_elapsed_ms", self.start, self.stop, C.byref(ms))
        return float(ms.value)

    def __del__(self):
        try:
            load().camel_hip_event_destroy(self.start)
            load().camel_hip_event_destroy(self.stop)
        except Exception:
            pass
