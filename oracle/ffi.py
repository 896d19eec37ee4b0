"""ctypes loader of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker / CPU baseline.  The product
never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, I64, BOOL = 0, 1, 2
ADD, SUB, MUL, DIV, POW = range(5)
LT, LE, GT, GE, EQ = range(5)
OK, ERR_DIV_ZERO, ERR_LOG_DOMAIN, ERR_SHAPE, ERR_DTYPE = range(5)

NP = {F32: np.float32, I64: np.int64, BOOL: np.uint8}

_P, _I, _I64, _U64, _D = C.c_void_p, C.c_int, C.c_int64, C.c_uint64, C.c_double
_SIG = {
    "ot_promote": ([_I, _I], _I),
    "ot_get": ([_I, _P, _U64], _D),
    "ot_binary": ([_I, _I, _P, _I, _P, _I, _P, _U64], _I),
    "ot_binary_scalar_right": ([_I, _I, _P, _D, _I, _P, _U64], _I),
    "ot_binary_scalar_left": ([_I, _D, _I, _P, _I, _P, _U64], _I),
    "ot_compare": ([_I, _I, _P, _I, _P, _P, _U64], None),
    "ot_compare_scalar_right": ([_I, _I, _P, _D, _P, _U64], None),
    "ot_compare_scalar_left": ([_I, _D, _I, _P, _P, _U64], None),
    "ot_matmul": ([_I, _P, _I, _P, _I, _P, _I64, _I64, _I64], _I),
    "ot_matmul_rows": ([_P, _P, _P, _I64, _I64, _I64, _I64, _I64], _I64),
    "ot_sum": ([_I, _P, _U64], _D),
    "ot_sum_axis": ([_I, _P, _I64, _I64, _I64, _P], _I),
    "ot_max_axis": ([_I, _P, _I64, _I64, _I64, _P], _I),
    "ot_argmax_axis": ([_I, _P, _I64, _I64, _I64, _P], _I),
    "ot_exp": ([_I, _P, _P, _U64], _I),
    "ot_log": ([_I, _P, _P, _U64], _I),
    "ot_transpose2d": ([_I, _P, _P, _I64, _I64], None),
    "ot_concat": ([_I, _P, _P, _P, _U64, _U64, _U64, _U64], None),
    "ot_relu": ([_P, _P, _U64], None),
    "ot_softmax_rows": ([_P, _P, _I64, _I64], _I),
    "ot_dense": ([_P, _P, _P, _I, _P, _I64, _I64, _I64], _I),
    "ot_conv2d": ([_P, _P, _P, _I, _P] + [_I64] * 9, _I),
    "ot_conv2d_images": ([_P, _P, _P, _I, _P] + [_I64] * 10, _I64),
    "ot_maxpool2d": ([_P, _P] + [_I64] * 7, _I),
    "ot_splitmix64": ([_U64, _U64], _U64),
    "ot_fill_uniform": ([_P, _U64, _U64, C.c_float, C.c_float], None),
}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = C.CDLL(LIB_PATH)
        for name, (args, res) in _SIG.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(_P)


def dt_of(a: np.ndarray) -> int:
    return {np.dtype(np.float32): F32, np.dtype(np.int64): I64,
            np.dtype(np.uint8): BOOL, np.dtype(np.bool_): BOOL}[a.dtype]


class OracleError(ValueError):
    def __init__(self, code: int):
        super().__init__({ERR_DIV_ZERO: "Division by zero",
                          ERR_LOG_DOMAIN: "log: input must be positive",
                          ERR_SHAPE: "shape error", ERR_DTYPE: "dtype error"}.get(code, str(code)))
        self.code = code


def _check(rc: int) -> None:
    if rc != OK:
        raise OracleError(rc)


def promote(l: int, r: int) -> int:
    return lib().ot_promote(l, r)


def binary_out_dtype(op: int, l: int, r: int) -> int:
    """tensorBinary output dtype (runtime.cpp:780-783)."""
    return F32 if op in (DIV, POW) else promote(l, r)


def binary(op: int, l: np.ndarray, r: np.ndarray) -> np.ndarray:
    odt = binary_out_dtype(op, dt_of(l), dt_of(r))
    out = np.empty(l.shape, dtype=NP[odt])
    _check(lib().ot_binary(op, dt_of(l), ptr(np.ascontiguousarray(l)), dt_of(r),
                           ptr(np.ascontiguousarray(r)), odt, ptr(out), l.size))
    return out


def binary_scalar(op: int, t: np.ndarray, s: float, scalar_dt: int, side: int = 0) -> np.ndarray:
    """side 0: t (op) s; side 1: s (op) t.  scalar_dt: normalised scalar dtype."""
    odt = binary_out_dtype(op, dt_of(t), scalar_dt)
    out = np.empty(t.shape, dtype=NP[odt])
    t = np.ascontiguousarray(t)
    if side == 0:
        rc = lib().ot_binary_scalar_right(op, dt_of(t), ptr(t), float(s), odt, ptr(out), t.size)
    else:
        rc = lib().ot_binary_scalar_left(op, float(s), dt_of(t), ptr(t), odt, ptr(out), t.size)
    _check(rc)
    return out


def compare(op: int, l: np.ndarray, r: np.ndarray) -> np.ndarray:
    out = np.empty(l.shape, dtype=np.uint8)
    lib().ot_compare(op, dt_of(l), ptr(np.ascontiguousarray(l)), dt_of(r),
                     ptr(np.ascontiguousarray(r)), ptr(out), l.size)
    return out


def compare_scalar(op: int, t: np.ndarray, s: float, side: int = 0) -> np.ndarray:
    out = np.empty(t.shape, dtype=np.uint8)
    t = np.ascontiguousarray(t)
    if side == 0:
        lib().ot_compare_scalar_right(op, dt_of(t), ptr(t), float(s), ptr(out), t.size)
    else:
        lib().ot_compare_scalar_left(op, float(s), dt_of(t), ptr(t), ptr(out), t.size)
    return out


def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    M, K = a.shape
    K2, N = b.shape
    assert K == K2
    odt = promote(dt_of(a), dt_of(b))
    out = np.empty((M, N), dtype=NP[odt])
    _check(lib().ot_matmul(dt_of(a), ptr(np.ascontiguousarray(a)), dt_of(b),
                           ptr(np.ascontiguousarray(b)), odt, ptr(out), M, K, N))
    return out


def matmul_rows(a: np.ndarray, b: np.ndarray, r0: int, r1: int) -> np.ndarray:
    """Rows [r0, r1) of an fp32 matmul (the timed slab of the CPU baseline)."""
    M, K = a.shape
    N = b.shape[1]
    out = np.zeros((M, N), dtype=np.float32)
    lib().ot_matmul_rows(ptr(a), ptr(b), ptr(out), M, K, N, r0, r1)
    return out[r0:r1]


def sum_all(x: np.ndarray) -> float:
    return lib().ot_sum(dt_of(x), ptr(np.ascontiguousarray(x)), x.size)


def _axis_out(x: np.ndarray, axis: int) -> int:
    rows, cols = x.shape
    a = axis + 2 if axis < 0 else axis
    if a not in (0, 1):
        raise OracleError(ERR_SHAPE)
    return cols if a == 0 else rows


def sum_axis(x: np.ndarray, axis: int) -> np.ndarray:
    out = np.empty(_axis_out(x, axis), dtype=np.float32)
    _check(lib().ot_sum_axis(dt_of(x), ptr(np.ascontiguousarray(x)), x.shape[0], x.shape[1],
                             axis, ptr(out)))
    return out


def max_axis(x: np.ndarray, axis: int) -> np.ndarray:
    out = np.empty(_axis_out(x, axis), dtype=np.float32)
    _check(lib().ot_max_axis(dt_of(x), ptr(np.ascontiguousarray(x)), x.shape[0], x.shape[1],
                             axis, ptr(out)))
    return out


def argmax_axis(x: np.ndarray, axis: int) -> np.ndarray:
    out = np.empty(_axis_out(x, axis), dtype=np.int64)
    _check(lib().ot_argmax_axis(dt_of(x), ptr(np.ascontiguousarray(x)), x.shape[0], x.shape[1],
                                axis, ptr(out)))
    return out


def exp(x: np.ndarray) -> np.ndarray:
    out = np.empty(x.shape, dtype=np.float32)
    _check(lib().ot_exp(dt_of(x), ptr(np.ascontiguousarray(x)), ptr(out), x.size))
    return out


def log(x: np.ndarray) -> np.ndarray:
    out = np.empty(x.shape, dtype=np.float32)
    _check(lib().ot_log(dt_of(x), ptr(np.ascontiguousarray(x)), ptr(out), x.size))
    return out


def transpose2d(x: np.ndarray) -> np.ndarray:
    rows, cols = x.shape
    out = np.empty((cols, rows), dtype=x.dtype)
    lib().ot_transpose2d(dt_of(x), ptr(np.ascontiguousarray(x)), ptr(out), rows, cols)
    return out


def concat(l: np.ndarray, r: np.ndarray, axis: int) -> np.ndarray:
    shape = list(l.shape)
    shape[axis] += r.shape[axis]
    out = np.empty(shape, dtype=l.dtype)
    outer = int(np.prod(l.shape[:axis])) if axis > 0 else 1
    inner = int(np.prod(l.shape[axis + 1:])) if axis + 1 < l.ndim else 1
    lib().ot_concat(dt_of(l), ptr(np.ascontiguousarray(l)), ptr(np.ascontiguousarray(r)),
                    ptr(out), outer, l.shape[axis], r.shape[axis], inner)
    return out


def relu(x: np.ndarray) -> np.ndarray:
    out = np.empty(x.shape, dtype=np.float32)
    lib().ot_relu(ptr(np.ascontiguousarray(x)), ptr(out), x.size)
    return out


def softmax_rows(x: np.ndarray) -> np.ndarray:
    n, k = x.shape
    out = np.empty((n, k), dtype=np.float32)
    _check(lib().ot_softmax_rows(ptr(np.ascontiguousarray(x)), ptr(out), n, k))
    return out


def dense(x: np.ndarray, w: np.ndarray, b: np.ndarray | None, relu_: bool) -> np.ndarray:
    M, K = x.shape
    N = w.shape[1]
    out = np.empty((M, N), dtype=np.float32)
    _check(lib().ot_dense(ptr(np.ascontiguousarray(x)), ptr(np.ascontiguousarray(w)),
                          ptr(b), int(relu_), ptr(out), M, K, N))
    return out


def conv2d(x, w, b, relu_: bool, stride: int = 1, pad: int = 0) -> np.ndarray:
    N, Cin, H, W = x.shape
    Co, Cw, KH, KW = w.shape
    assert Cw == Cin
    OH = (H + 2 * pad - KH) // stride + 1
    OW = (W + 2 * pad - KW) // stride + 1
    y = np.empty((N, Co, OH, OW), dtype=np.float32)
    _check(lib().ot_conv2d(ptr(np.ascontiguousarray(x)), ptr(np.ascontiguousarray(w)), ptr(b),
                           int(relu_), ptr(y), N, Cin, H, W, Co, KH, KW, stride, pad))
    return y


def conv2d_images(x, w, b, relu_: bool, n0: int, n1: int, stride: int = 1, pad: int = 0):
    """Images [n0, n1) of conv2d (the timed slab of the CPU baseline)."""
    N, Cin, H, W = x.shape
    Co, _, KH, KW = w.shape
    OH = (H + 2 * pad - KH) // stride + 1
    OW = (W + 2 * pad - KW) // stride + 1
    y = np.zeros((N, Co, OH, OW), dtype=np.float32)
    lib().ot_conv2d_images(ptr(x), ptr(w), ptr(b), int(relu_), ptr(y), n0, n1, Cin, H, W, Co,
                           KH, KW, stride, pad)
    return y[n0:n1]


def maxpool2d(x: np.ndarray, k: int = 2, stride: int = 2, kw: int | None = None) -> np.ndarray:
    """Window k x kw (kw defaults to k), NCHW."""
    kw = k if kw is None else kw
    N, Cc, H, W = x.shape
    OH, OW = (H - k) // stride + 1, (W - kw) // stride + 1
    y = np.empty((N, Cc, OH, OW), dtype=np.float32)
    _check(lib().ot_maxpool2d(ptr(np.ascontiguousarray(x)), ptr(y), N, Cc, H, W, k, kw, stride))
    return y
