"""ctypes binding of libcamel_tensor.so (include/camel_tensor.h): the tensor
module's operators, driven the way the reference's executors drive them.

    from camel_amd import tensor as T
    a = T.Tensor.from_numpy(x)                 # host tensor, uploaded on first use
    c = T.call("tensor:matmul", a, b)          # -> Tensor (device-resident)
    s = T.call("sum", c)                       # -> float (Float64 result)
    y = T.call("dense_relu", x, with_=(w, b))  # dense<w, b> bind arguments
    c.numpy()                                  # one D2H copy

Arguments map to the reference's type codes: Tensor -> Tensor, bool -> Bool,
int -> Int64, float -> Float64, T.Int32 / T.Float32 wrap the narrow scalars,
lists / tuples -> Array (nested lists -> nested arrays), None -> Void.
Operator errors raise :class:`CamelError` with the reference's message
("matmul dimension mismatch", "Division by zero", ...).  There is no CPU
fallback: every operator runs on the GPU through libcamel_hip.so.
"""
from __future__ import annotations

import ctypes as C
import os
import struct

import numpy as np

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libcamel_tensor.so")

TC_INT32, TC_INT64, TC_FLOAT32, TC_FLOAT64, TC_BOOL = 0x0, 0x1, 0x2, 0x3, 0x4
TC_VOID, TC_ARRAY, TC_TENSOR = 0x6, 0x60000008, 0xE0000001
OK, ERR_RUNTIME, ERR_URI, ERR_ARG, ERR_RESOLVE = range(5)

NP_OF_TC = {TC_FLOAT32: np.float32, TC_INT64: np.int64, TC_BOOL: np.uint8}
TC_OF_NP = {np.dtype(np.float32): TC_FLOAT32, np.dtype(np.int64): TC_INT64,
            np.dtype(np.uint8): TC_BOOL, np.dtype(np.bool_): TC_BOOL}


class CamelError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class Value(C.Structure):
    _fields_ = [("code", C.c_uint32), ("slot", C.c_uint64)]


_U64, _I64, _U32, _P = C.c_uint64, C.c_int64, C.c_uint32, C.c_void_p


# DLPack v0.8 structs (include/camel_dlpack.h)
class DLDevice(C.Structure):
    _fields_ = [("device_type", C.c_int32), ("device_id", C.c_int32)]


class DLDataType(C.Structure):
    _fields_ = [("code", C.c_uint8), ("bits", C.c_uint8), ("lanes", C.c_uint16)]


class DLTensor(C.Structure):
    _fields_ = [("data", _P), ("device", DLDevice), ("ndim", C.c_int32), ("dtype", DLDataType),
                ("shape", C.POINTER(_I64)), ("strides", C.POINTER(_I64)),
                ("byte_offset", C.c_uint64)]


class DLManagedTensor(C.Structure):
    pass


_DELETER = C.CFUNCTYPE(None, C.POINTER(DLManagedTensor))
DLManagedTensor._fields_ = [("dl_tensor", DLTensor), ("manager_ctx", _P), ("deleter", _DELETER)]
KDL_CPU, KDL_ROCM = 1, 10

_SIG = {
    "camel_tensor_last_error": ([], C.c_char_p),
    "camel_module_abi_version": ([], C.c_int),
    "camel_tensor_type_string": ([_U32, _I64, C.POINTER(_I64), C.c_int, C.c_char_p, C.c_size_t,
                                  C.POINTER(C.c_size_t)], C.c_int),
    "camel_tensor_type_relation": ([_U32, _I64, C.POINTER(_I64), _U32, _I64, C.POINTER(_I64),
                                    C.POINTER(C.c_int), C.POINTER(C.c_int)], C.c_int),
    "camel_tensor_from_host": ([_U32, _I64, C.POINTER(_I64), _P, C.POINTER(_U64)], C.c_int),
    "camel_tensor_to_host": ([_U64, _P, C.c_size_t], C.c_int),
    "camel_tensor_meta": ([_U64, C.POINTER(_U32), C.POINTER(_I64), C.POINTER(_I64), _I64], C.c_int),
    "camel_tensor_residency": ([_U64, C.POINTER(C.c_int), C.POINTER(C.c_int)], C.c_int),
    "camel_tensor_device_ptr": ([_U64, C.POINTER(_U64)], C.c_int),
    "camel_tensor_release": ([_U64], C.c_int),
    "camel_tensor_release_all": ([], _I64),
    "camel_tensor_mark": ([], _U64),
    "camel_tensor_release_since": ([_U64, _I64, C.POINTER(_U64), C.POINTER(_I64)], C.c_int),
    "camel_tensor_live_count": ([], _I64),
    "camel_tensor_format": ([_U64, C.c_char_p, C.c_size_t, C.POINTER(C.c_size_t)], C.c_int),
    "camel_tensor_equals": ([_U64, _U64, C.POINTER(C.c_int)], C.c_int),
    "camel_tensor_clone": ([_U64, C.POINTER(_U64)], C.c_int),
    "camel_array_create": ([_U32, _I64, C.POINTER(_U64), C.POINTER(_U64)], C.c_int),
    "camel_array_read": ([_U64, C.POINTER(_U32), C.POINTER(_I64), C.POINTER(_U64), _I64], C.c_int),
    "camel_array_release": ([_U64], C.c_int),
    "camel_tensor_invoke": ([C.c_char_p, _I64, C.POINTER(Value), _I64, C.POINTER(Value),
                             C.POINTER(Value)], C.c_int),
    "camel_tensor_resolve": ([C.c_char_p, _I64, C.POINTER(_U32), _I64, C.POINTER(_U32), C.c_char_p,
                              C.c_size_t, C.POINTER(_U32), C.POINTER(_U32)], C.c_int),
    "camel_tensor_op_count": ([], _I64),
    "camel_tensor_op_name": ([_I64], C.c_char_p),
    "camel_tensor_group_count": ([], _I64),
    "camel_tensor_group_name": ([_I64], C.c_char_p),
    "camel_tensor_to_dlpack": ([_U64, C.c_int, C.POINTER(C.POINTER(DLManagedTensor))], C.c_int),
    "camel_tensor_from_dlpack": ([C.POINTER(DLManagedTensor), C.POINTER(_U64)], C.c_int),
    "camel_chain_create": ([C.POINTER(_U64)], C.c_int),
    "camel_chain_append": ([_U64, C.c_char_p, _I64, C.POINTER(Value)], C.c_int),
    "camel_chain_apply": ([_U64, _U64, C.POINTER(_U64)], C.c_int),
    "camel_chain_plan": ([_U64, _I64, C.POINTER(_I64), C.c_uint32, C.c_char_p, C.c_size_t,
                          C.POINTER(C.c_size_t)], C.c_int),
    "camel_chain_release": ([_U64], C.c_int),
}

# PyCapsule plumbing of the DLPack Python protocol: a capsule named
# "dltensor" owns its managed tensor until a consumer renames it
# "used_dltensor" (and then calls the deleter itself).
_capsule_new = C.PYFUNCTYPE(C.py_object, _P, C.c_char_p, _P)(("PyCapsule_New", C.pythonapi))
_capsule_get = C.PYFUNCTYPE(_P, C.py_object, C.c_char_p)(("PyCapsule_GetPointer", C.pythonapi))
_capsule_set_name = C.PYFUNCTYPE(C.c_int, C.py_object, C.c_char_p)(("PyCapsule_SetName",
                                                                     C.pythonapi))
# Raw-pointer forms for the destructor, which receives the dying capsule.
_capsule_valid_raw = C.PYFUNCTYPE(C.c_int, _P, C.c_char_p)(("PyCapsule_IsValid", C.pythonapi))
_capsule_get_raw = C.PYFUNCTYPE(_P, _P, C.c_char_p)(("PyCapsule_GetPointer", C.pythonapi))


@C.CFUNCTYPE(None, _P)
def _capsule_destructor(capsule):
    if _capsule_valid_raw(capsule, b"dltensor"):
        managed = C.cast(_capsule_get_raw(capsule, b"dltensor"), C.POINTER(DLManagedTensor))
        if managed and managed.contents.deleter:
            managed.contents.deleter(managed)

_lib = None


def load(path: str = LIB_PATH) -> C.CDLL:
    """Loads libcamel_tensor.so (and with it libcamel_hip.so); raises if unbuilt."""
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise ImportError(f"{path} is missing: build it with `python -m camel_amd.build`")
        lib = C.CDLL(path)
        for name, (args, res) in _SIG.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def exported_symbols() -> list[str]:
    return sorted(_SIG)


def _check(status: int) -> None:
    if status != OK:
        msg = load().camel_tensor_last_error()
        raise CamelError(status, msg.decode() if msg else f"status {status}")


class Int32(int):
    """An Int32 scalar argument."""


class Float32(float):
    """A Float32 scalar argument."""


class Tensor:
    """A handle to a TensorObject of the operator layer."""

    def __init__(self, handle: int):
        self.handle = int(handle)

    @staticmethod
    def from_numpy(arr: np.ndarray) -> "Tensor":
        arr = np.ascontiguousarray(arr)
        if arr.dtype == np.bool_:
            arr = arr.astype(np.uint8)
        code = TC_OF_NP.get(arr.dtype)
        if code is None:
            raise TypeError(f"unsupported dtype {arr.dtype}")
        shape = (_I64 * max(arr.ndim, 1))(*arr.shape)
        h = _U64()
        _check(load().camel_tensor_from_host(code, arr.ndim, shape,
                                             arr.ctypes.data_as(_P) if arr.size else None, C.byref(h)))
        return Tensor(h.value)

    def meta(self):
        dt, rank = _U32(), _I64()
        dims = (_I64 * 16)()
        _check(load().camel_tensor_meta(self.handle, C.byref(dt), C.byref(rank), dims, 16))
        return dt.value, tuple(dims[i] for i in range(rank.value))

    @property
    def dtype_code(self) -> int:
        return self.meta()[0]

    @property
    def shape(self) -> tuple:
        return self.meta()[1]

    def numpy(self) -> np.ndarray:
        dt, shape = self.meta()
        out = np.empty(shape, dtype=NP_OF_TC[dt])
        _check(load().camel_tensor_to_host(self.handle, out.ctypes.data_as(_P) if out.size else None,
                                           out.nbytes))
        return out

    def residency(self) -> tuple[bool, bool]:
        h, d = C.c_int(), C.c_int()
        _check(load().camel_tensor_residency(self.handle, C.byref(h), C.byref(d)))
        return bool(h.value), bool(d.value)

    def device_ptr(self) -> int:
        p = _U64()
        _check(load().camel_tensor_device_ptr(self.handle, C.byref(p)))
        return p.value

    def format(self) -> str:
        need = C.c_size_t()
        _check(load().camel_tensor_format(self.handle, None, 0, C.byref(need)))
        buf = C.create_string_buffer(need.value)
        _check(load().camel_tensor_format(self.handle, buf, need.value, None))
        return buf.value.decode()

    def equals(self, other: "Tensor") -> bool:
        eq = C.c_int()
        _check(load().camel_tensor_equals(self.handle, other.handle, C.byref(eq)))
        return bool(eq.value)

    def clone(self) -> "Tensor":
        """A deep copy with its own handle (TensorObject::clone)."""
        h = _U64()
        _check(load().camel_tensor_clone(self.handle, C.byref(h)))
        return Tensor(h.value)

    def release(self) -> None:
        if self.handle:
            _check(load().camel_tensor_release(self.handle))
            self.handle = 0

    # ---- DLPack -------------------------------------------------------------
    def to_dlpack(self, on_device: bool = True):
        """A "dltensor" capsule: the device payload itself (kDLROCM, no copy)
        or a host copy (kDLCPU).  The payload is complete when this returns."""
        m = C.POINTER(DLManagedTensor)()
        _check(load().camel_tensor_to_dlpack(self.handle, 1 if on_device else 0, C.byref(m)))
        return _capsule_new(C.cast(m, _P), b"dltensor", C.cast(_capsule_destructor, _P))

    def __dlpack__(self, stream=None, max_version=None, dl_device=None, copy=None):
        # Exports are synchronised with the library stream, so any consumer
        # stream may read them.
        return self.to_dlpack(on_device=True)

    def __dlpack_device__(self):
        dev = C.c_int()
        from camel_amd import _hip
        _hip.call("camel_hip_current_device", C.byref(dev))
        return (KDL_ROCM, dev.value)

    @staticmethod
    def from_dlpack(obj) -> "Tensor":
        """A copy of a DLPack tensor (an object with __dlpack__, or a
        "dltensor" capsule), from host memory or from this device.

        For a device producer the copy is ordered after its pending writes:
        the library stream is passed as the DLPack ``stream`` argument (the
        producer makes that stream wait for its own), and a producer that
        takes no stream argument is waited for with a whole-device
        synchronisation.  A bare capsule must already be complete."""
        from camel_amd import _hip
        if hasattr(obj, "__dlpack__"):
            on_device = (hasattr(obj, "__dlpack_device__")
                         and int(obj.__dlpack_device__()[0]) == KDL_ROCM)
            if on_device:
                stream = _hip.load().camel_hip_stream()
                if not stream:
                    raise RuntimeError(_hip.load().camel_hip_last_error().decode())
                try:
                    cap = obj.__dlpack__(stream=int(stream))
                except TypeError:
                    cap = obj.__dlpack__()
                    _hip.call("camel_hip_device_sync")
            else:
                cap = obj.__dlpack__()
        else:
            cap = obj
        managed = C.cast(_capsule_get(cap, b"dltensor"), C.POINTER(DLManagedTensor))
        h = _U64()
        _check(load().camel_tensor_from_dlpack(managed, C.byref(h)))
        _capsule_set_name(cap, b"used_dltensor")
        if managed.contents.deleter:
            managed.contents.deleter(managed)
        return Tensor(h.value)


class Array:
    """A handle to an Array value (shape arguments, array operands)."""

    def __init__(self, handle: int):
        self.handle = int(handle)

    @staticmethod
    def from_list(values, elem: int | None = None) -> "Array":
        values = list(values)
        if elem is None:
            elem = _elem_code(values)
        slots = []
        keep = []
        for v in values:
            if elem == TC_ARRAY:
                child = v if isinstance(v, Array) else Array.from_list(v)
                keep.append(child)
                slots.append(child.handle)
            else:
                slots.append(_scalar_slot(elem, v))
        arr = (_U64 * max(len(slots), 1))(*slots)
        h = _U64()
        _check(load().camel_array_create(elem, len(slots), arr, C.byref(h)))
        return Array(h.value)

    def to_list(self) -> list:
        elem, n = _U32(), _I64()
        _check(load().camel_array_read(self.handle, C.byref(elem), C.byref(n), None, 0))
        slots = (_U64 * max(n.value, 1))()
        _check(load().camel_array_read(self.handle, None, None, slots, n.value))
        if elem.value == TC_ARRAY:
            return [Array(slots[i]).to_list() for i in range(n.value)]
        return [_slot_value(elem.value, slots[i]) for i in range(n.value)]


def _elem_code(values) -> int:
    if not values:
        return TC_INT64
    if all(isinstance(v, (list, tuple, Array)) for v in values):
        return TC_ARRAY
    if all(isinstance(v, bool) for v in values):
        return TC_BOOL
    if all(isinstance(v, Int32) for v in values):
        return TC_INT32
    if all(isinstance(v, int) and not isinstance(v, bool) for v in values):
        return TC_INT64
    return TC_FLOAT64


def _scalar_slot(code: int, v) -> int:
    if code == TC_INT32:
        return struct.unpack("<I", struct.pack("<i", int(v)))[0]
    if code == TC_INT64:
        return struct.unpack("<Q", struct.pack("<q", int(v)))[0]
    if code == TC_FLOAT32:
        return struct.unpack("<I", struct.pack("<f", float(v)))[0]
    if code == TC_FLOAT64:
        return struct.unpack("<Q", struct.pack("<d", float(v)))[0]
    if code == TC_BOOL:
        return 1 if v else 0
    raise TypeError(f"not a scalar code: {code:#x}")


def _slot_value(code: int, slot: int):
    if code == TC_INT32:
        return struct.unpack("<i", struct.pack("<I", slot & 0xFFFFFFFF))[0]
    if code == TC_INT64:
        return struct.unpack("<q", struct.pack("<Q", slot))[0]
    if code == TC_FLOAT32:
        return struct.unpack("<f", struct.pack("<I", slot & 0xFFFFFFFF))[0]
    if code == TC_FLOAT64:
        return struct.unpack("<d", struct.pack("<Q", slot))[0]
    if code == TC_BOOL:
        return bool(slot & 0xFF)
    if code == TC_VOID:
        return None
    if code == TC_TENSOR:
        return Tensor(slot)
    if code == TC_ARRAY:
        return Array(slot).to_list()
    raise TypeError(f"unsupported result code {code:#x}")


def to_value(x, keep: list) -> Value:
    """Maps a Python argument to a {code, slot} pair (keeps temporaries alive)."""
    if isinstance(x, Tensor):
        return Value(TC_TENSOR, x.handle)
    if isinstance(x, Array):
        return Value(TC_ARRAY, x.handle)
    if x is None:
        return Value(TC_VOID, 0)
    if isinstance(x, (list, tuple)):
        a = Array.from_list(x)
        keep.append(a)
        return Value(TC_ARRAY, a.handle)
    if isinstance(x, bool):
        return Value(TC_BOOL, _scalar_slot(TC_BOOL, x))
    if isinstance(x, Int32):
        return Value(TC_INT32, _scalar_slot(TC_INT32, x))
    if isinstance(x, (int, np.integer)):
        return Value(TC_INT64, _scalar_slot(TC_INT64, x))
    if isinstance(x, Float32):
        return Value(TC_FLOAT32, _scalar_slot(TC_FLOAT32, x))
    if isinstance(x, (float, np.floating)):
        return Value(TC_FLOAT64, _scalar_slot(TC_FLOAT64, x))
    raise TypeError(f"unsupported argument {x!r}")


def call(uri: str, *norm, with_=()):
    """Invokes operator `uri` ("tensor:matmul" or "matmul") like an executor."""
    keep: list = []
    nv = [to_value(x, keep) for x in norm]
    wv = [to_value(x, keep) for x in with_]
    na = (Value * max(len(nv), 1))(*nv)
    wa = (Value * max(len(wv), 1))(*wv)
    out = Value()
    _check(load().camel_tensor_invoke(uri.encode(), len(wv), wa, len(nv), na, C.byref(out)))
    return _slot_value(out.code, out.slot)


def resolve(group: str, norm_codes, with_codes=()) -> tuple[str, int]:
    """Overload resolution of an operator group: (uri, result type code)."""
    uri, code, _ = resolve_type(group, norm_codes, with_codes)
    return uri, code


def resolve_type(group: str, norm_codes, with_codes=()) -> tuple[str, int, int]:
    """(uri, result type code, element type): the element type is a Tensor
    result's dtype, an Array result's element type, else the code itself."""
    n = (_U32 * max(len(norm_codes), 1))(*norm_codes)
    w = (_U32 * max(len(with_codes), 1))(*with_codes)
    buf = C.create_string_buffer(128)
    rc, re = _U32(), _U32()
    _check(load().camel_tensor_resolve(group.encode(), len(with_codes), w, len(norm_codes), n, buf,
                                       128, C.byref(rc), C.byref(re)))
    return buf.value.decode(), rc.value, re.value


def _shape_arg(shape):
    shape = tuple(int(d) for d in shape)
    return len(shape), (_I64 * max(len(shape), 1))(*shape)


def tensor_type_string(dtype: int = TC_FLOAT32, shape=(), mangled: bool = False) -> str:
    """TensorType::toString / mangle of Tensor<shape, dtype> (shape () = dynamic)."""
    rank, dims = _shape_arg(shape)
    need = C.c_size_t()
    _check(load().camel_tensor_type_string(dtype, rank, dims, int(mangled), None, 0, C.byref(need)))
    buf = C.create_string_buffer(need.value)
    _check(load().camel_tensor_type_string(dtype, rank, dims, int(mangled), buf, need.value, None))
    return buf.value.decode()


def tensor_type_relation(dst, src) -> tuple[bool, bool]:
    """(dst.assignableFrom(src), dst.equals(src)) for (dtype, shape) pairs."""
    dr, dd = _shape_arg(dst[1])
    sr, sd = _shape_arg(src[1])
    a, e = C.c_int(), C.c_int()
    _check(load().camel_tensor_type_relation(dst[0], dr, dd, src[0], sr, sd, C.byref(a), C.byref(e)))
    return bool(a.value), bool(e.value)


def op_names() -> list[str]:
    L = load()
    return [L.camel_tensor_op_name(i).decode() for i in range(L.camel_tensor_op_count())]


def group_names() -> list[str]:
    L = load()
    return [L.camel_tensor_group_name(i).decode() for i in range(L.camel_tensor_group_count())]


def live_count() -> int:
    return int(load().camel_tensor_live_count())


def release_all() -> int:
    return int(load().camel_tensor_release_all())


def mark() -> int:
    """A mark for release_since: objects made after it have larger serials."""
    return int(load().camel_tensor_mark())


def release_since(mark_: int, keep=()) -> int:
    """Releases every tensor / array made after mark_ except those in keep
    (Tensor objects or raw handles); returns how many were released."""
    handles = [k.handle if hasattr(k, "handle") else int(k) for k in keep]
    arr = (_U64 * max(len(handles), 1))(*handles)
    n = _I64()
    _check(load().camel_tensor_release_since(mark_, len(handles), arr, C.byref(n)))
    return int(n.value)


class Chain:
    """A composed layer chain, `dense<w1, b1>..relu..softmax` (README.md:40-46):
    layers appended with their bind arguments, then applied to a tensor
    (`x->chain`).  Adjacent layers run as one fused kernel where that computes
    the same values."""

    def __init__(self, *layers):
        h = _U64()
        _check(load().camel_chain_create(C.byref(h)))
        self.handle = h.value
        for layer in layers:
            if isinstance(layer, str):
                self.append(layer)
            else:
                self.append(layer[0], *layer[1:])

    def append(self, uri: str, *with_) -> "Chain":
        keep: list = []
        wv = [to_value(x, keep) for x in with_]
        wa = (Value * max(len(wv), 1))(*wv)
        _check(load().camel_chain_append(self.handle, uri.encode(), len(wv), wa))
        return self

    def __call__(self, x: "Tensor") -> "Tensor":
        out = _U64()
        _check(load().camel_chain_apply(self.handle, x.handle, C.byref(out)))
        return Tensor(out.value)

    def plan(self, shape, dtype: int = TC_FLOAT32) -> list[str]:
        dims = (_I64 * max(len(shape), 1))(*shape)
        need = C.c_size_t()
        L = load()
        _check(L.camel_chain_plan(self.handle, len(shape), dims, dtype, None, 0, C.byref(need)))
        buf = C.create_string_buffer(need.value)
        _check(L.camel_chain_plan(self.handle, len(shape), dims, dtype, buf, need.value, None))
        return [line for line in buf.value.decode().split("\n") if line]

    def release(self) -> None:
        if self.handle:
            _check(load().camel_chain_release(self.handle))
            self.handle = 0
