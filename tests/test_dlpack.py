"""DLPack exchange of the operator layer's tensors
(tensorToDLPackCopy / tensorFromDLPackCopy, modules/tensor/runtime.cpp:1079-1124).

The reference exchanges host copies only; this layer adds a zero-copy export
of the device payload (kDLROCM) and a copying import from device memory.
Host-side cases run on the CPU (they never touch the GPU); device cases are
marked gpu, and one of them exchanges tensors with PyTorch-ROCm.
"""
import ctypes as C
import os
import subprocess
import sys

import numpy as np
import pytest

from camel_amd import _hip as H
from camel_amd import tensor as T

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(autouse=True)
def _release():
    yield
    T.release_all()


class HostExport:
    """Wraps a tensor so numpy consumes its host-copy export."""

    def __init__(self, t):
        self.t = t

    def __dlpack__(self, stream=None, max_version=None, dl_device=None, copy=None):
        return self.t.to_dlpack(on_device=False)

    def __dlpack_device__(self):
        return (T.KDL_CPU, 0)


@pytest.mark.parametrize("arr", [
    np.arange(12, dtype=np.float32).reshape(3, 4) - 5.5,
    np.arange(-6, 6, dtype=np.int64).reshape(2, 3, 2),
    np.array([[True, False, True]]),
    np.zeros((0, 3), np.float32),
])
def test_host_round_trip(arr):
    t = T.Tensor.from_numpy(arr)
    back = np.from_dlpack(HostExport(t))
    assert back.dtype == arr.dtype  # kDLBool reads back as bool
    assert back.shape == arr.shape
    assert np.array_equal(back, arr)
    # import: a copy, independent of the source
    src = arr.copy()
    u = T.Tensor.from_dlpack(src)
    assert u.shape == arr.shape
    got = u.numpy()
    if src.size:
        src.reshape(-1)[0] = 0
    assert np.array_equal(got.astype(arr.dtype), arr)


def test_host_export_keeps_reference_dtype_codes():
    # runtime.cpp:221-232: Float32 -> (kDLFloat, 32), Int64 -> (kDLInt, 64), Bool -> (kDLBool, 8)
    for arr, code, bits in [(np.ones(2, np.float32), 2, 32), (np.ones(2, np.int64), 0, 64),
                            (np.ones(2, np.bool_), 6, 8)]:
        t = T.Tensor.from_numpy(arr)
        cap = t.to_dlpack(on_device=False)
        dl = _managed(cap).contents.dl_tensor
        assert (dl.dtype.code, dl.dtype.bits, dl.dtype.lanes) == (code, bits, 1)
        assert dl.device.device_type == T.KDL_CPU and dl.ndim == 1 and not dl.strides
        del cap  # the capsule's destructor runs the deleter


@pytest.mark.parametrize("arr,msg", [
    (np.arange(12, dtype=np.float32).reshape(3, 4).T, "Only contiguous DLPack tensors are supported"),
    (np.ones(4, np.float16), "Unsupported DLPack dtype"),
    (np.ones(4, np.int32), "Unsupported DLPack dtype"),
    (np.ones(4, np.float64), "Unsupported DLPack dtype"),
])
def test_import_errors_use_reference_text(arr, msg):
    with pytest.raises(T.CamelError, match=msg):
        T.Tensor.from_dlpack(arr)


def test_import_accepts_compact_strides():
    # numpy (like PyTorch) may export explicit strides; compact ones are row-major.
    a = np.arange(24, dtype=np.float32).reshape(2, 3, 4)[:, :, :]
    assert np.array_equal(T.Tensor.from_dlpack(a).numpy(), a)
    b = np.arange(6, dtype=np.int64).reshape(6, 1)
    assert np.array_equal(T.Tensor.from_dlpack(b).numpy(), b)


# ---- device exchange ---------------------------------------------------------------


def _managed(cap):
    return C.cast(T._capsule_get(cap, b"dltensor"), C.POINTER(T.DLManagedTensor))


@pytest.mark.gpu
def test_device_export_is_zero_copy_and_outlives_the_handle():
    x = np.random.default_rng(1).standard_normal((64, 33)).astype(np.float32)
    t = T.call("relu", T.Tensor.from_numpy(x))  # a device-born operator output
    assert t.residency() == (False, True)
    ptr, want = t.device_ptr(), t.numpy()
    cap = t.to_dlpack(on_device=True)
    dl = _managed(cap).contents.dl_tensor
    assert dl.device.device_type == T.KDL_ROCM and dl.device.device_id == 0
    assert dl.data == ptr, "a kDLROCM export is the payload itself"
    assert (dl.ndim, dl.shape[0], dl.shape[1]) == (2, 64, 33) and not dl.strides
    t.release()
    T.release_all()
    # The export holds the payload: new tensors must not reuse its block.
    junk = [T.call("zeros", [64, 33]) for _ in range(4)]
    assert all(j.device_ptr() != ptr for j in junk)
    back = T.Tensor.from_dlpack(cap)  # consumes the capsule, runs the deleter
    assert back.residency() == (False, True) and back.device_ptr() != ptr
    assert np.array_equal(back.numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,code,bits", [(np.float32, 2, 32), (np.int64, 0, 64),
                                             (np.bool_, 6, 8)])
def test_device_import_from_a_foreign_buffer(dtype, code, bits):
    # A producer's device buffer described by a hand-built DLManagedTensor
    # with explicit compact strides (what PyTorch exports).
    src = (np.random.default_rng(2).standard_normal((37, 50)) * 10)
    src = src.astype(dtype) if dtype != np.bool_ else src > 0
    buf = H.to_device(src.view(np.uint8) if dtype == np.bool_ else src)
    shape, strides = (C.c_int64 * 2)(37, 50), (C.c_int64 * 2)(50, 1)
    m = T.DLManagedTensor()
    m.dl_tensor.data = buf.ptr
    m.dl_tensor.device = T.DLDevice(T.KDL_ROCM, 0)
    m.dl_tensor.ndim = 2
    m.dl_tensor.dtype = T.DLDataType(code, bits, 1)
    m.dl_tensor.shape = shape
    m.dl_tensor.strides = strides
    h = C.c_uint64()
    T._check(T.load().camel_tensor_from_dlpack(C.byref(m), C.byref(h)))
    t = T.Tensor(h.value)
    assert t.residency() == (False, True) and t.device_ptr() != buf.ptr
    buf.free()  # the import is a finished copy
    assert np.array_equal(t.numpy().astype(src.dtype), src)
    m.dl_tensor.device = T.DLDevice(T.KDL_ROCM, 5)
    with pytest.raises(T.CamelError, match="DLPack tensor is on another device"):
        T._check(T.load().camel_tensor_from_dlpack(C.byref(m), C.byref(h)))


PYTORCH_CHILD = r"""
import sys
import numpy as np
import torch  # first: a ROCm wheel of PyTorch brings its own HIP runtime, and
              # the process must hold one, so it is initialised before libcamel
torch.ones(1, device="cuda").sum().item()
from camel_amd import tensor as T

a = np.random.default_rng(3).uniform(-1, 1, (128, 96)).astype(np.float32)
b = np.random.default_rng(4).uniform(-1, 1, (96, 64)).astype(np.float32)
c = T.call("matmul", T.Tensor.from_numpy(a), T.Tensor.from_numpy(b))
ptr = c.device_ptr()
tc = torch.from_dlpack(c)                      # zero-copy device export
assert tc.device.type == "cuda" and tc.data_ptr() == ptr, (tc.device, tc.data_ptr(), ptr)
assert np.array_equal(tc.cpu().numpy(), c.numpy())
c.release()
T.release_all()
assert np.array_equal(tc.cpu().numpy() @ np.eye(64, dtype=np.float32), tc.cpu().numpy())
for dt in (torch.float32, torch.int64, torch.bool):
    src = (torch.randn(37, 50, device="cuda") * 10)
    src = src > 0 if dt == torch.bool else src.to(dt)
    torch.cuda.synchronize()                    # the producer's writes are complete
    t = T.Tensor.from_dlpack(src)               # device import (a copy)
    want = src.cpu().numpy()
    del src
    torch.cuda.empty_cache()
    assert t.residency() == (False, True)
    assert np.array_equal(t.numpy().astype(want.dtype), want), dt
td = (tc * 2.0).contiguous()
torch.cuda.synchronize()
d = T.Tensor.from_dlpack(td)
assert np.array_equal(d.numpy(), tc.cpu().numpy() * np.float32(2.0))
try:
    T.Tensor.from_dlpack(tc.t())
    raise SystemExit("transposed view accepted")
except T.CamelError as e:
    assert "Only contiguous DLPack tensors are supported" in str(e)
print("pytorch interop ok")
"""


@pytest.mark.gpu
def test_pytorch_rocm_interop_in_a_fresh_process():
    # PyTorch's ROCm wheel bundles a HIP runtime of its own; one process can
    # hold one, so the exchange runs in a child that initialises torch first.
    pytest.importorskip("torch")
    env = dict(os.environ, PYTHONPATH=ROOT)
    r = subprocess.run([sys.executable, "-c", PYTORCH_CHILD], cwd=ROOT, env=env,
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "pytorch interop ok" in r.stdout
