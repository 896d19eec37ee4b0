"""CPU tests of the operator layer (libcamel_tensor.so) and of the C-ABI.

Everything here runs without a GPU: the libraries load, export what the
headers declare, the operator map and overload resolution mirror the
reference's (modules/tensor/operators.cpp:160-583), and the argument and
shape errors the reference raises before touching data are raised with the
same text.  Host tensors stay on the host until a device operator needs them,
so these error paths never reach libcamel_hip's device code.
"""
import ctypes as C
import os
import re

import numpy as np
import pytest

from camel_amd import _hip as H
from camel_amd import tensor as T

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# modules/tensor/operators.cpp:160-194
REFERENCE_OPS = {"add", "subtract", "multiply", "divide", "pow", "matmul", "idx", "idx2d", "lt",
                 "le", "gt", "ge", "eq", "empty", "zeros", "ones", "full", "random", "range", "eye",
                 "shape", "sum", "sum_axis", "max_axis", "argmax_axis", "exp", "log", "transpose",
                 "concat", "reshape", "show"}
LAYER_OPS = {"relu", "softmax", "dense", "dense_relu", "conv2d", "conv2d_relu", "maxpool2d"}


def declared_functions(header: str) -> set[str]:
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(camel_\w+)\s*\(", text))


@pytest.fixture(autouse=True)
def _release():
    yield
    T.release_all()


def test_hip_abi_exports_every_declared_symbol():
    lib = H.load()
    declared = declared_functions("camel_hip.h")
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(lib, name), name
    assert declared == set(H.exported_symbols())


def test_hip_abi_rejects_extents_whose_products_overflow():
    # Shape checks run before the library touches the device, so these calls
    # need no GPU.  Each case's element count wraps around int64 (or around
    # to a small value) if multiplied unchecked.
    lib = H.load()
    big = 2**32
    conv = lib.camel_hip_conv2d
    assert conv(None, None, None, None, 1, 2**31 - 1, 2**31 - 1, 2**31 - 1, 8, 1, 1, 1, 0,
                0) == H.ERR_SHAPE
    assert conv(None, None, None, None, 1, 8, 8, 8, big, 1, 1, 1, 0, 0) == H.ERR_SHAPE
    assert conv(None, None, None, None, 1, 8, 8, 8, 8, 3, 3, 1, 2**62, 0) == H.ERR_SHAPE
    assert lib.camel_hip_conv2d_pool2(None, None, None, None, big, big, 8, 8, 8, 3, 3, 1, 0,
                                      0) == H.ERR_SHAPE
    # Co * C = 2**64 wraps to 0: a wrapped product would pass as an empty tensor.
    assert lib.camel_hip_conv2d_pack_weights(None, None, big, big, 1, 1) == H.ERR_SHAPE
    assert lib.camel_hip_conv2d_pack_weights(None, None, 2**31, 1, 1, 1) == H.ERR_SHAPE
    assert b"too large" in lib.camel_hip_last_error()
    assert lib.camel_hip_maxpool2d(None, None, big, big, 8, 8, 2, 2, 2) == H.ERR_SHAPE
    assert lib.camel_hip_concat(H.DT_I64, None, None, None, big, big, 1, 2) == H.ERR_SHAPE
    assert lib.camel_hip_concat(H.DT_I64, None, None, None, 2, 1, 2**62, 1) == H.ERR_SHAPE
    assert b"too large" in lib.camel_hip_last_error()
    assert lib.camel_hip_sum_axis(H.DT_F32, None, big, big, 0, None) == H.ERR_SHAPE
    assert lib.camel_hip_argmax_axis(H.DT_I64, None, 2**61, 2, 1, None) == H.ERR_SHAPE
    assert lib.camel_hip_softmax_rows(None, None, 2**62, 4) == H.ERR_SHAPE
    assert b"too large" in lib.camel_hip_last_error()
    # The generic (Int64 / Bool) matmul: an extent past INT32_MAX is legal (the
    # kernel indexes in int64), but byte counts that overflow are refused.
    gm = lib.camel_hip_matmul_generic
    assert gm(H.DT_I64, None, H.DT_I64, None, H.DT_I64, None, 2**31, 2**31, 2**31) == H.ERR_SHAPE
    assert gm(H.DT_I64, None, H.DT_I64, None, H.DT_I64, None, 2**60, 1, 4) == H.ERR_SHAPE
    assert gm(H.DT_BOOL, None, H.DT_BOOL, None, H.DT_BOOL, None, 4, 2**61, 1) == H.ERR_SHAPE
    assert b"too large" in lib.camel_hip_last_error()


def test_conv_pair_pool_refuses_shapes_it_does_not_serve():
    # Checked before any device work: the pointers are never dereferenced.
    lib = H.load()
    p = [C.c_void_p(256)] * 6
    pair = lib.camel_hip_conv2d_pair_pool2
    assert pair(*p, 2, 28, 30, 32, 64, 0, 0) == H.ERR_SHAPE     # W != 28
    assert pair(*p, 2, 28, 28, 16, 64, 0, 0) == H.ERR_SHAPE     # C1 != 32
    assert pair(*p, 2, 28, 28, 32, 32, 0, 0) == H.ERR_SHAPE     # Co2 % 64 != 0
    assert pair(*p, 2, 26, 28, 32, 64, 0, 0) == H.ERR_SHAPE     # (H - 4) % 8 != 0
    assert b"shape not served" in lib.camel_hip_last_error()
    assert pair(*p, 2, 28, 28, 32, 64, 0x400, 0) == H.ERR_ARG   # packing is conv2's flag
    assert pair(*p, -1, 28, 28, 32, 64, 0, 0) == H.ERR_SHAPE


def test_tensor_abi_exports_every_declared_symbol():
    lib = T.load()
    declared = declared_functions("camel_tensor.h")
    for name in declared:
        assert hasattr(lib, name), name
    assert declared == set(T.exported_symbols())
    # The version the reference's loader checks (dynamic.h:29,38).
    assert lib.camel_module_abi_version() == 1
    assert not hasattr(lib, "camel_tensor_abi_version")


def test_ops_map_keeps_reference_suffixes():
    names = set(T.op_names())
    assert REFERENCE_OPS <= names
    assert names == REFERENCE_OPS | LAYER_OPS


def test_groups_keep_reference_names():
    groups = set(T.group_names())
    for g in ["__add__", "__sub__", "__mul__", "__div__", "__pow__", "__mat__", "__idx__", "__lt__",
              "__le__", "__gt__", "__ge__", "__eq__", "empty", "zeros", "ones", "full", "random",
              "range", "eye", "shape", "sum", "max", "argmax", "exp", "log", "transpose", "concat",
              "reshape", "show", "add", "subtract", "multiply", "divide", "pow", "matmul"]:
        assert g in groups, g
    assert LAYER_OPS <= groups


@pytest.mark.parametrize("group,norm,with_,uri,result", [
    ("__mat__", [T.TC_TENSOR, T.TC_TENSOR], [], "tensor:matmul", T.TC_TENSOR),
    ("__add__", [T.TC_TENSOR, T.TC_FLOAT64], [], "tensor:add", T.TC_TENSOR),
    ("__add__", [T.TC_INT32, T.TC_TENSOR], [], "tensor:add", T.TC_TENSOR),
    ("__idx__", [T.TC_TENSOR, T.TC_INT64], [], "tensor:idx", T.TC_FLOAT64),
    ("__idx__", [T.TC_TENSOR, T.TC_INT64, T.TC_INT64], [], "tensor:idx2d", T.TC_FLOAT64),
    ("sum", [T.TC_TENSOR], [], "tensor:sum", T.TC_FLOAT64),
    ("sum", [T.TC_TENSOR, T.TC_INT32], [], "tensor:sum_axis", T.TC_TENSOR),
    ("__eq__", [T.TC_ARRAY, T.TC_FLOAT32], [], "tensor:eq", T.TC_TENSOR),
    ("__lt__", [T.TC_ARRAY, T.TC_FLOAT64], [], "tensor:lt", T.TC_TENSOR),
    ("range", [T.TC_INT64, T.TC_INT64, T.TC_INT32], [], "tensor:range", T.TC_TENSOR),
    ("shape", [T.TC_TENSOR], [], "tensor:shape", T.TC_ARRAY),
    ("show", [T.TC_ARRAY], [], "tensor:show", T.TC_VOID),
    ("dense", [T.TC_TENSOR], [T.TC_TENSOR, T.TC_TENSOR], "tensor:dense", T.TC_TENSOR),
    ("dense_relu", [T.TC_TENSOR, T.TC_TENSOR], [], "tensor:dense_relu", T.TC_TENSOR),
    ("conv2d", [T.TC_TENSOR], [T.TC_TENSOR, T.TC_TENSOR, T.TC_INT64, T.TC_INT64], "tensor:conv2d",
     T.TC_TENSOR),
    ("maxpool2d", [T.TC_TENSOR], [T.TC_INT64], "tensor:maxpool2d", T.TC_TENSOR),
])
def test_resolution(group, norm, with_, uri, result):
    assert T.resolve(group, norm, with_) == (uri, result)


F32, I64, BOOL, F64, VOID = T.TC_FLOAT32, T.TC_INT64, T.TC_BOOL, T.TC_FLOAT64, T.TC_VOID
TEN, ARR = T.TC_TENSOR, T.TC_ARRAY


@pytest.mark.parametrize("group,norm,with_,code,elem", [
    # tensorType() = TensorType::Dynamic(Float32) by default (operators.cpp:41-43)
    ("__add__", [TEN, TEN], [], TEN, F32),
    ("__div__", [TEN, T.TC_INT32], [], TEN, F32),
    ("__pow__", [TEN, F64], [], TEN, F32),
    ("__mat__", [TEN, TEN], [], TEN, F32),
    ("zeros", [ARR], [], TEN, F32),
    ("full", [ARR, F64], [], TEN, F32),
    ("eye", [I64], [], TEN, F32),
    ("sum", [TEN, I64], [], TEN, F32),
    ("max", [TEN, I64], [], TEN, F32),
    ("exp", [TEN], [], TEN, F32),
    ("transpose", [TEN], [], TEN, F32),
    ("concat", [TEN, ARR, I64], [], TEN, F32),
    ("reshape", [TEN, ARR], [], TEN, F32),
    ("softmax", [TEN], [], TEN, F32),
    ("dense", [TEN], [TEN, TEN], TEN, F32),
    # comparisons: tensorType(Type::Bool()) (operators.cpp:137), every form
    ("__lt__", [TEN, TEN], [], TEN, BOOL),
    ("__le__", [TEN, F64], [], TEN, BOOL),
    ("__gt__", [F32, TEN], [], TEN, BOOL),
    ("__ge__", [ARR, I64], [], TEN, BOOL),
    ("__eq__", [T.TC_INT32, ARR], [], TEN, BOOL),
    # range and argmax: tensorType(Type::Int64()) (operators.cpp:382, 458)
    ("range", [I64], [], TEN, I64),
    ("range", [I64, I64, T.TC_INT32], [], TEN, I64),
    ("argmax", [TEN, I64], [], TEN, I64),
    # scalars, arrays and void keep their own codes
    ("sum", [TEN], [], F64, F64),
    ("__idx__", [TEN, I64], [], F64, F64),
    ("shape", [TEN], [], ARR, I64),
    ("show", [TEN], [], VOID, VOID),
])
def test_resolution_carries_the_reference_result_dtype(group, norm, with_, code, elem):
    _, got_code, got_elem = T.resolve_type(group, norm, with_)
    assert (got_code, got_elem) == (code, elem)


@pytest.mark.parametrize("dtype,shape,text,mangled", [
    (F32, (), "Tensor", "T_;f32"),
    (BOOL, (), "Tensor<bool>", "T_;b"),
    (I64, (), "Tensor<i64>", "T_;i"),
    (F32, (2, 3), "Tensor<[2, 3]>", "T2,3;f32"),
    (I64, (4,), "Tensor<[4], i64>", "T4;i"),
    (F64, (1, 0, 5), "Tensor<[1, 0, 5], f64>", "T1,0,5;f"),
])
def test_tensor_type_strings(dtype, shape, text, mangled):
    # TensorType::toString and mangle (modules/tensor/type.cpp:64-98)
    assert T.tensor_type_string(dtype, shape) == text
    assert T.tensor_type_string(dtype, shape, mangled=True) == mangled


@pytest.mark.parametrize("dst,src,assignable,equal", [
    ((F32, ()), (F32, ()), True, True),
    ((F32, ()), (BOOL, (2, 2)), True, False),        # Float32 target takes any dtype / shape
    ((BOOL, ()), (F32, ()), False, False),           # not the other way round
    ((I64, ()), (I64, (7,)), True, False),           # dynamic target shape
    ((I64, (7,)), (I64, ()), True, False),           # dynamic source shape
    ((F32, (2, 3)), (F32, (3, 2)), False, False),    # static shapes must match
    ((F32, (2, 3)), (I64, (2, 3)), True, False),
    ((BOOL, (2, 3)), (BOOL, (2, 3)), True, True),
    ((I64, (2,)), (BOOL, (2,)), False, False),
])
def test_tensor_type_assignability(dst, src, assignable, equal):
    # TensorType::assignableFrom / equals (modules/tensor/type.cpp:105-131)
    assert T.tensor_type_relation(dst, src) == (assignable, equal)


@pytest.mark.parametrize("group,norm", [
    ("__mat__", [T.TC_TENSOR, T.TC_FLOAT64]),     # matmul takes two tensors only
    ("__add__", [T.TC_FLOAT64, T.TC_FLOAT64]),    # no tensor operand
    ("__pow__", [T.TC_FLOAT64, T.TC_TENSOR]),     # base must be a tensor
    ("__lt__", [T.TC_ARRAY, T.TC_ARRAY]),         # two arrays: not a compare overload
])
def test_resolution_rejects(group, norm):
    with pytest.raises(T.CamelError, match="no overload"):
        T.resolve(group, norm)


def host(a):
    return T.Tensor.from_numpy(np.asarray(a))


@pytest.mark.parametrize("uri,args,msg", [
    ("add", lambda: (host(np.zeros((2, 3), np.float32)), host(np.zeros((3, 2), np.float32))),
     "Tensor binary operation requires matching shapes"),
    ("lt", lambda: (host(np.zeros(3, np.float32)), host(np.zeros(4, np.float32))),
     "Tensor comparison requires matching shapes"),
    ("matmul", lambda: (host(np.zeros(3, np.float32)), host(np.zeros((3, 2), np.float32))),
     "matmul currently only supports rank-2 tensors"),
    ("matmul", lambda: (host(np.zeros((2, 3), np.float32)), host(np.zeros((2, 2), np.float32))),
     "matmul dimension mismatch"),
    ("transpose", lambda: (host(np.zeros(3, np.float32)),),
     "transpose currently only supports rank-2 tensors"),
    ("concat", lambda: (host(np.zeros((2, 2), np.float32)), host(np.zeros(2, np.float32)), 0),
     "concat requires tensors with the same rank"),
    ("concat", lambda: (host(np.zeros((2, 2), np.float32)), host(np.zeros((2, 2), np.float32)), 2),
     "concat axis out of range"),
    ("concat", lambda: (host(np.zeros((2, 2), np.float32)), host(np.zeros((2, 2), np.int64)), 0),
     "concat currently requires matching dtypes"),
    ("concat", lambda: (host(np.zeros((2, 2), np.float32)), host(np.zeros((2, 3), np.float32)), 0),
     "concat requires equal non-axis dimensions"),
    ("reshape", lambda: (host(np.zeros((2, 3), np.float32)), [4, 2]),
     "reshape changes tensor element count"),
    ("reshape", lambda: (host(np.zeros((2, 3), np.float32)), [-1, 6]),
     "Shape cannot contain negative values"),
    ("reshape", lambda: (host(np.zeros((2, 3), np.float32)), [2.0, 3.0]),
     "Shape array must contain integers"),
    ("idx", lambda: (host(np.zeros((2, 2), np.float32)), 0),
     "Single-index tensor access requires rank-1 tensor"),
    ("idx", lambda: (host(np.zeros(3, np.float32)), 3), "Tensor index out of bounds"),
    ("idx2d", lambda: (host(np.zeros((2, 2), np.float32)), 0, -1), "Tensor index out of bounds"),
    ("range", lambda: (0, 5, 0), "range step cannot be zero"),
    ("eye", lambda: (-1,), "eye size cannot be negative"),
    ("sum_axis", lambda: (host(np.zeros(3, np.float32)), 0),
     r"sum\(axis\) currently only supports rank-2 tensors"),
    ("max_axis", lambda: (host(np.zeros((2, 2), np.float32)), 2),
     r"max\(axis\): axis must be 0 or 1 for rank-2 tensors"),
    ("argmax_axis", lambda: (host(np.zeros((2, 2), np.float32)), -3),
     r"argmax\(axis\): axis must be 0 or 1 for rank-2 tensors"),
    ("exp", lambda: (host(np.zeros(3, np.int64)),), "exp requires floating-point tensor"),
    ("log", lambda: (host(np.zeros(3, np.uint8)),), "log requires floating-point tensor"),
    ("eq", lambda: ([[1, 2], [3]], 1.0), "Nested array shape or dtype mismatch"),
    ("softmax", lambda: (host(np.zeros(3, np.float32)),), "softmax currently only supports rank-2"),
])
def test_reference_errors_before_any_device_work(uri, args, msg):
    with pytest.raises(T.CamelError, match=msg) as info:
        T.call(uri, *args())
    assert info.value.status == T.ERR_RUNTIME


def test_dense_and_conv_argument_errors():
    x = host(np.zeros((4, 3), np.float32))
    w = host(np.zeros((2, 5), np.float32))
    with pytest.raises(T.CamelError, match="dense dimension mismatch"):
        T.call("dense", x, with_=(w,))
    with pytest.raises(T.CamelError, match="no overload of tensor:dense") as info:
        T.call("dense", x)  # the group's resolver wants weights
    assert info.value.status == T.ERR_RESOLVE
    x4 = host(np.zeros((1, 3, 4, 4), np.float32))
    w4 = host(np.zeros((2, 2, 3, 3), np.float32))
    with pytest.raises(T.CamelError, match="conv2d channel mismatch"):
        T.call("conv2d", x4, with_=(w4,))
    with pytest.raises(T.CamelError, match="maxpool2d window larger than input"):
        T.call("maxpool2d", x4, with_=(5,))


def test_ill_typed_calls_fail_resolution():
    # As in the reference, the group's resolver decides which argument types
    # reach an operator; anything else is rejected before the operator runs.
    for uri, args in [("transpose", (1.0,)), ("matmul", (host(np.zeros((1, 1), np.float32)), 1.0)),
                      ("range", (1.5,))]:
        with pytest.raises(T.CamelError, match="no overload") as info:
            T.call(uri, *args)
        assert info.value.status == T.ERR_RESOLVE


def test_unknown_uri_and_bad_handles():
    with pytest.raises(T.CamelError, match="Unrecognized operator URI") as info:
        T.call("tensor:conv3d", host(np.zeros(1, np.float32)))
    assert info.value.status == T.ERR_URI
    bogus = T.Tensor(0xDEAD0)
    with pytest.raises(T.CamelError, match="not a live tensor"):
        T.call("transpose", bogus)


def test_host_only_values_need_no_device():
    a = host(np.arange(6, dtype=np.float32).reshape(2, 3))
    assert a.residency() == (True, False)
    assert T.call("shape", a) == [2, 3]
    assert T.call("idx2d", a, 1, 2) == 5.0
    assert a.residency() == (True, False)
    b = T.call("reshape", a, [3, 2])  # a view: shares the payload, no copy
    assert b.shape == (3, 2)
    assert np.array_equal(b.numpy(), np.arange(6, dtype=np.float32).reshape(3, 2))
    assert b.residency() == (True, False)
    assert a.equals(a) and not a.equals(b)


def test_print_format_matches_reference():
    # TensorObject::print (modules/tensor/runtime.cpp:422-528).
    eye = host(np.eye(2, dtype=np.float32))
    assert eye.format() == ("tensor([[      1.,       0.],\n"
                            "        [      0.,       1.]], dtype=float32)")
    assert host(np.array([1.5, -0.25], np.float32)).format() == \
        "tensor([    1.5,   -0.25], dtype=float32)"
    assert host(np.array([3, -4], np.int64)).format() == "tensor([      3,      -4], dtype=int64)"
    assert host(np.array([1, 0], np.uint8)).format() == "tensor([  true,  false], dtype=bool)"
    long_row = host(np.arange(20, dtype=np.int64)).format()
    assert long_row.startswith("tensor([      0,") and ",\n        " in long_row


def test_array_round_trip_and_tensor_from_nested_array():
    arr = T.Array.from_list([[1, 2], [3, 4]])
    assert arr.to_list() == [[1, 2], [3, 4]]
    t = T.call("reshape", arr, [4])  # requireTensorOrConvertArray builds a host tensor
    assert t.dtype_code == T.TC_INT64
    assert t.numpy().tolist() == [1, 2, 3, 4]


def test_release_bookkeeping():
    T.release_all()
    a = host(np.zeros(4, np.float32))
    assert T.live_count() == 1
    a.release()
    assert T.live_count() == 0
    with pytest.raises(T.CamelError):
        a.handle = 12345
        a.release()


def test_failed_operator_releases_what_it_made():
    # concat(Array, Tensor) converts the array into a new host tensor
    # (requireTensorOrConvertArray), then the shape check throws: the
    # converted tensor never reaches the caller, so the layer releases it.
    x = host(np.zeros((2, 3), np.float32))
    arr = T.Array.from_list([[1.0, 2.0], [3.0, 4.0]])
    before = T.live_count()
    with pytest.raises(T.CamelError, match="concat requires equal non-axis dimensions"):
        T.call("concat", arr, x, 0)
    assert T.live_count() == before


def test_noalloc_sgemm_refuses_before_initialisation():
    # Initialisation allocates (stream, error flag), so the allocation-free
    # entry point will not do it: a fresh process that never initialised the
    # library gets an error and no device work.
    import subprocess
    import sys
    code = ("import ctypes as C; from camel_amd import _hip as H; L = H.load(); p = C.c_void_p(256); "
            "rc = L.camel_hip_sgemm_noalloc(p, p, p, 4, 4, 4, None, 0); "
            "print(rc, L.camel_hip_last_error().decode())")
    out = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr
    rc, msg = out.stdout.strip().split(" ", 1)
    assert int(rc) == H.ERR_ARG and "camel_hip_init" in msg


def test_transpose_is_a_view_made_contiguous_on_read():
    # Float32 transpose shares the payload (no copy at the call); reading it
    # back makes it contiguous once, here on the host (the source never went
    # to the device), and the values are the reference's transpose.
    x = np.arange(12, dtype=np.float32).reshape(3, 4) * np.float32(0.5) - np.float32(2.0)
    t = host(x)
    tt = T.call("transpose", t)
    assert tt.shape == (4, 3)
    assert tt.residency() == (True, False)
    np.testing.assert_array_equal(tt.numpy(), x.T)
    # the transpose of a transposed view is the original layout again
    np.testing.assert_array_equal(T.call("transpose", T.call("transpose", t)).numpy(), x)
    # a reshape of a transposed view reads the transposed element order
    r = T.call("reshape", T.call("transpose", t), [12])
    np.testing.assert_array_equal(r.numpy(), x.T.reshape(12))
    # indexing reads the logical layout
    assert T.call("idx2d", T.call("transpose", t), 3, 1) == float(x[1, 3])


def test_clone_is_a_deep_copy_with_its_own_handle():
    x = np.arange(6, dtype=np.float32).reshape(2, 3)
    t = host(x)
    c = t.clone()
    assert c.handle != t.handle and c.equals(t)
    t.release()
    np.testing.assert_array_equal(c.numpy(), x)
    with pytest.raises(T.CamelError):
        T.Tensor(12345).clone()


def test_release_since_bounds_a_loop_to_its_live_values():
    # A train loop (test/run/nn/mnist.cml:44-58) makes temporaries every
    # iteration; the reference frees none.  With one mark before the loop and
    # release_since keeping only the new weights at each iteration's end, the
    # previous weights and every temporary go, and the live count stays flat.
    T.release_all()
    w = host(np.arange(12, dtype=np.float32).reshape(3, 4))
    counts = []
    m = T.mark()
    for it in range(4):
        live0 = T.live_count()
        tt = T.call("transpose", w)                       # a view of w
        r = T.call("reshape", tt, [12])                   # another view (and a shape Array)
        arr = T.Array.from_list([[1.0, 2.0], [3.0, 4.0]])  # array temporaries
        w_next = T.call("reshape", r, [4, 3]).clone()      # the "updated weights"
        assert arr.to_list() == [[1.0, 2.0], [3.0, 4.0]]
        made_tensors = T.live_count() - live0              # tt, r, reshape(r), w_next
        assert made_tensors == 4
        released = T.release_since(m, keep=[w_next])
        # the three tensor temporaries and every array (the nested list, the
        # shape arguments)
        assert released >= 3 + 3
        # w_next stays; the previous weights go too (made after the mark)
        # except the loop's initial ones
        assert T.live_count() == (live0 + 1 if it == 0 else live0)
        with pytest.raises(T.CamelError):
            tt.numpy()
        w = w_next
        counts.append(T.live_count())
    assert counts[1:] == counts[:-1], counts                # no growth per iteration
    assert w.shape == (4, 3)
    x = np.arange(12, dtype=np.float32).reshape(3, 4)
    want = x
    for _ in range(4):
        want = want.T.reshape(4, 3)
    np.testing.assert_array_equal(w.numpy(), want)
    # a kept view keeps its payload when its source is released
    src = host(x)
    m = T.mark()
    view = T.call("transpose", src)
    src.release()
    assert T.release_since(m, keep=[view]) == 0
    np.testing.assert_array_equal(view.numpy(), x.T)
    # objects made before the mark are never touched
    before = T.live_count()
    assert T.release_since(T.mark()) == 0 and T.live_count() == before
    with pytest.raises(T.CamelError, match="bad arguments"):
        load = T.load()
        import ctypes as C
        T._check(load.camel_tensor_release_since(0, -1, None, None))
