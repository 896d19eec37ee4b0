"""Helpers for the GPU tests: device buffers in, numpy out, through the C-ABI."""
from __future__ import annotations

import ctypes as C

import numpy as np

from camel_amd import _hip as H

P = C.c_void_p


def dev(a: np.ndarray) -> H.DeviceBuffer:
    return H.to_device(np.ascontiguousarray(a))


def empty(nbytes: int) -> H.DeviceBuffer:
    return H.DeviceBuffer(max(int(nbytes), 4))


def host(buf: H.DeviceBuffer, dtype, shape) -> np.ndarray:
    n = int(np.prod(shape)) if len(shape) else 1
    return buf.download(dtype, n).reshape(shape)


def sgemm(a: np.ndarray, b: np.ndarray, bias=None, flags: int = 0) -> np.ndarray:
    M, K = a.shape
    N = b.shape[1]
    da, db = dev(a), dev(b)
    dc = empty(M * N * 4)
    dbias = dev(bias) if bias is not None else None
    H.call("camel_hip_sgemm", P(da.ptr), P(db.ptr), P(dc.ptr), M, N, K,
           P(dbias.ptr) if dbias is not None else None, flags)
    return host(dc, np.float32, (M, N))


def gemm_tol_ok(c_gpu: np.ndarray, c_ref: np.ndarray, a: np.ndarray, b: np.ndarray):
    """Per-element |dC| <= 1e-5 * sqrt(K) * sum_k |A_ik||B_kj| (the GEMM tolerance)."""
    K = a.shape[1]
    bound = 1e-5 * np.sqrt(max(K, 1)) * (np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64)))
    err = np.abs(c_gpu.astype(np.float64) - c_ref.astype(np.float64))
    bad = err > bound
    return not bad.any(), float((err / np.maximum(bound, 1e-300)).max(initial=0.0))
