"""The bandwidth kernels at the sizes bench.py times, against the oracle over
every element: add / mul / relu at n = 2**28 (bit-exact, tensorBinary and
the x*(x>0) idiom, runtime.cpp:775-793 and test/run/nn/svm.cml:31) and the
row softmax at [262144, 1024] (rel-err <= 1e-6, the mnist.cml:13-25
composition).  Inputs are seeded numpy draws with special values planted
(signed zeros, infinities, NaN, subnormals), so the vector and tail paths of
each kernel see them."""
import ctypes as C

import numpy as np
import pytest

from camel_amd import _hip as H
from oracle import ffi as O
from tests import hipkit as K

pytestmark = pytest.mark.gpu

P = C.c_void_p
F = np.float32
N_ELT = 1 << 28
SPECIALS = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 3.4028235e38, -2.5], F)


def _plant(x, seed):
    rng = np.random.default_rng(seed)
    idx = rng.choice(x.size, size=4096, replace=False)
    x.reshape(-1)[idx] = np.resize(SPECIALS, idx.size)
    x.reshape(-1)[-len(SPECIALS):] = SPECIALS  # the tail of the last vector
    return x


def _uniform(seed, n):
    return np.random.default_rng(seed).random(n, dtype=F) * F(2.0) - F(1.0)


def _same_bits(got, want):
    nan = np.isnan(got) & np.isnan(want)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    bad = np.flatnonzero(got.view(np.uint32)[~nan] != want.view(np.uint32)[~nan])
    assert bad.size == 0, f"{bad.size} elements differ"


@pytest.mark.parametrize("op", [H.OP_ADD, H.OP_MUL])
def test_binary_at_bench_size_is_bit_exact(op):
    print(f"binary op {op} at n = 2^28", flush=True)
    a, b = _plant(_uniform(0x8000 + op, N_ELT), 1), _plant(_uniform(0x8100 + op, N_ELT), 2)
    da, db = K.dev(a), K.dev(b)
    dc = K.empty(a.nbytes)
    H.call("camel_hip_binary", op, H.DT_F32, P(da.ptr), H.DT_F32, P(db.ptr), H.DT_F32, P(dc.ptr),
           N_ELT)
    del da, db
    got = K.host(dc, F, a.shape)
    _same_bits(got, O.binary(op, a, b))


def test_relu_at_bench_size_is_bit_exact():
    print("relu at n = 2^28", flush=True)
    x = _plant(np.random.default_rng(0x8200).standard_normal(N_ELT, dtype=F), 3)
    dx, dy = K.dev(x), K.empty(x.nbytes)
    H.call("camel_hip_relu", P(dx.ptr), P(dy.ptr), N_ELT)
    _same_bits(K.host(dy, F, x.shape), O.relu(x))


def test_softmax_at_bench_size_matches_the_composition():
    print("softmax at [262144, 1024]", flush=True)
    rows, cols = 262144, 1024
    x = np.random.default_rng(0x8300).standard_normal((rows, cols), dtype=F)
    x[7, 3] = -np.inf                       # exp(-inf) = 0 in the sum
    x[11, :] = 0.0                          # a uniform row: 1/1024 everywhere
    x[13, 5] = 80.0                         # a dominant element
    dx, dy = K.dev(x), K.empty(x.nbytes)
    H.call("camel_hip_softmax_rows", P(dx.ptr), P(dy.ptr), rows, cols)
    del dx
    got = K.host(dy, F, x.shape)
    ref = O.softmax_rows(x)
    rel = np.abs(got.astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-38)
    assert rel.max() <= 1e-6, f"max rel err {rel.max()} at {np.unravel_index(rel.argmax(), rel.shape)}"
    assert np.all(got[11] == F(1.0 / 1024))
