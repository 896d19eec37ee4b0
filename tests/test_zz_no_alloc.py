"""camel_hip_sgemm_noalloc: the allocation-free sgemm (split-K partials in the
library's static scratch) gives camel_hip_sgemm's results bit for bit, on two
calls in a row with the second one smaller, over every path that uses
partials; a shape whose partials would not fit is refused before launch."""
import ctypes as C

import numpy as np
import pytest

from camel_amd import _hip as H
from camel_amd import datagen as D
from tests import hipkit as K

pytestmark = pytest.mark.gpu

P = C.c_void_p
F = np.float32
SCRATCH = 64 << 20


def _run(entry, a, b, bias, flags):
    M, Kd = a.shape
    N = b.shape[1]
    da, db = K.dev(a), K.dev(b)
    dbias = K.dev(bias) if bias is not None else None
    dc = K.empty(M * N * 4)
    H.call(entry, P(da.ptr), P(db.ptr), P(dc.ptr), M, N, Kd, P(dbias.ptr) if dbias else None, flags)
    return K.host(dc, F, (M, N))


# Pairs of (first, second smaller) shapes per scratch-using path.
PAIRS = [
    ((16, 4096, 4096), (16, 1024, 2048)),      # skinny streaming kernel, k partials
    ((32, 4096, 8192), (8, 512, 4096)),        # skinny, two 16-row groups, then M < 16
    ((512, 128, 9216), (200, 72, 1000)),       # 64x64 split-K, then 32x32 split-K
    ((4352, 4352, 512), (1024, 1024, 1024)),   # 256x256 round + split tail (57.75 MiB), then unsplit
    ((256, 256, 256), (64, 64, 64)),           # 32x32 tiles with splits
    ((16, 4094, 1000), (16, 100, 300)),        # 32x128 tiles (N % 4 != 0), split
    ((1024, 10, 1024), (300, 3, 50)),          # thin kernel: no scratch
]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_sgemm_matches_sgemm_on_two_calls(first, second):
    H.call("camel_hip_init", 0)
    for i, (M, N, Kd) in enumerate((first, second)):
        print(f"sgemm_noalloc {M}x{N}x{Kd} (call {i + 1})", flush=True)
        a = D.uniform(0x9000 + M + Kd, (M, Kd), -1.0, 1.0)
        b = D.uniform(0x9100 + N + Kd, (Kd, N), -1.0, 1.0)
        bias = D.uniform(0x9200 + N, (N,), -1.0, 1.0)
        for flags in (H.EPI_BIAS | H.EPI_RELU, 0):
            bb = bias if flags else None
            want = _run("camel_hip_sgemm", a, b, bb, flags)
            got = _run("camel_hip_sgemm_noalloc", a, b, bb, flags)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (M, N, Kd, flags)


def test_noalloc_sgemm_allocates_nothing():
    # The pool's counters do not move: no block is taken or returned.
    H.call("camel_hip_init", 0)
    a = D.uniform(0x9300, (512, 9216), -1.0, 1.0)
    b = D.uniform(0x9301, (9216, 128), -1.0, 1.0)
    da, db, dc = K.dev(a), K.dev(b), K.empty(512 * 128 * 4)
    H.call("camel_hip_sync")
    in_use, cached = C.c_size_t(), C.c_size_t()
    H.call("camel_hip_pool_stats", C.byref(in_use), C.byref(cached))
    before = (in_use.value, cached.value)
    for _ in range(3):
        H.call("camel_hip_sgemm_noalloc", P(da.ptr), P(db.ptr), P(dc.ptr), 512, 128, 9216, None, 0)
    H.call("camel_hip_sync")
    H.call("camel_hip_pool_stats", C.byref(in_use), C.byref(cached))
    assert (in_use.value, cached.value) == before


def test_noalloc_sgemm_refuses_partials_beyond_the_scratch():
    # 32 x 65536 x 16384 streams B in 16 k groups: 16 * 32 * 65536 * 4 bytes
    # = 128 MiB of partials.  The buffers are real and whole, and the call is
    # refused on the host before any launch; the same shape with K = 8192
    # (64 MiB of partials) fits and runs.
    H.call("camel_hip_init", 0)
    M, N = 32, 65536
    db = K.empty(16384 * N * 4)
    da, dc = K.empty(M * 16384 * 4), K.empty(M * N * 4)
    lib = H.load()
    rc = lib.camel_hip_sgemm_noalloc(P(da.ptr), P(db.ptr), P(dc.ptr), M, N, 16384, None, 0)
    assert rc == H.ERR_SHAPE
    assert b"static scratch" in lib.camel_hip_last_error()
    a = D.uniform(0x9400, (M, 8192), -1.0, 1.0)
    b = D.uniform(0x9401, (8192, 4096), -1.0, 1.0)
    bw = np.zeros((8192, N), F)
    bw[:, :4096] = b
    want = _run("camel_hip_sgemm", a, bw, None, 0)
    got = _run("camel_hip_sgemm_noalloc", a, bw, None, 0)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
