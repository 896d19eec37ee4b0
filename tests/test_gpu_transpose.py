"""transpose(X) @ E without a copy of X (test/run/nn/mnist.cml:39,
test/run/nn/lr.cml:28): the GEMM's transposed-A loaders (CAMEL_GEMM_A_T)
bit-exact on small-integer operands over every tile path, the Float32
transpose operator as a view, and the mnist.cml `update` training step run
on the device against the oracle composition, step by step."""
import ctypes as C

import numpy as np
import pytest

from camel_amd import _hip as H
from camel_amd import datagen as D
from camel_amd import tensor as T
from oracle import ffi as O
from tests import hipkit as K
from tests.test_gpu_exact import assert_bits, exact_dense, ints, wide, wide_pair

pytestmark = pytest.mark.gpu

P = C.c_void_p
F = np.float32


def sgemm_at(at, b, bias=None, flags=0):
    """C = At^T . B through camel_hip_sgemm with CAMEL_GEMM_A_T (At is [K, M])."""
    Kd, M = at.shape
    N = b.shape[1]
    da, db = K.dev(at), K.dev(b)
    dc = K.empty(M * N * 4)
    dbias = K.dev(bias) if bias is not None else None
    H.call("camel_hip_sgemm", P(da.ptr), P(db.ptr), P(dc.ptr), M, N, Kd,
           P(dbias.ptr) if dbias is not None else None, flags | H.GEMM_A_T)
    return K.host(dc, F, (M, N))


TN_SHAPES = [
    # M, N, K, epilogue, path
    (784, 10, 1024, 0, "MNIST-scale gradient: 64x64 or 32x32 tiles with K splits"),
    (33, 10, 100, 0, "mnist.cml's own shape (M % 4 != 0: scalar transposed loads)"),
    (1024, 1024, 1024, 3, "64x64 tiles, one per CU"),
    (2048, 2048, 512, 0, "128x128 tiles"),
    (4096, 4096, 1024, 0, "8-wave 256x256 tiles"),
    (4352, 4352, 256, 3, "256x256 round + split tail"),
    (512, 33024, 128, 0, "256x256 round + column band"),
    (16, 4096, 2048, 3, "M <= 32: 32x128 tiles"),
    (1001, 130, 777, 3, "ragged M, N, K with scalar loads"),
]


@pytest.mark.parametrize("M,N,Kd,epi,path", TN_SHAPES, ids=[s[4].split(":")[0] for s in TN_SHAPES])
def test_transposed_a_gemm_is_exact(M, N, Kd, epi, path):
    print(f"TN sgemm {M}x{N}x{Kd} ({path})", flush=True)
    seed = 0xA000 + M + N + Kd
    a, b = ints(seed, (M, Kd)), ints(seed + 1, (Kd, N))
    bias = ints(seed + 2, (N,)) if epi & H.EPI_BIAS else None
    want = exact_dense(a, b, bias, bool(epi & H.EPI_RELU))
    got = sgemm_at(np.ascontiguousarray(a.T), b, bias, epi)
    assert_bits(got, want, path)


@pytest.mark.parametrize("wide_side", ["A", "B"])
@pytest.mark.parametrize("M,N,Kd,epi,path", TN_SHAPES, ids=[s[4].split(":")[0] for s in TN_SHAPES])
def test_transposed_a_gemm_wide_operands_stay_fp32(M, N, Kd, epi, path, wide_side):
    # One operand wide (12-bit integers), the other ternary: the transposed
    # loaders must hand the MFMA fp32 operands (see tests/test_gpu_exact.py).
    print(f"wide TN sgemm {M}x{N}x{Kd} wide {wide_side} ({path})", flush=True)
    seed = 0xE000 + M + N + Kd
    a, b = wide_pair(seed, (M, Kd), (Kd, N), wide_side)
    bias = wide(seed + 2, (N,)) if epi & H.EPI_BIAS else None
    want = exact_dense(a, b, bias, bool(epi & H.EPI_RELU))
    got = sgemm_at(np.ascontiguousarray(a.T), b, bias, epi)
    assert_bits(got, want, f"{path}, wide {wide_side}")


def test_transposed_a_gemm_matches_the_oracle_on_real_values():
    # U(-1, 1) operands: the GEMM bar against the oracle's ijk matmul of the
    # materialised transpose.
    x = D.uniform(0xA100, (1024, 784), -1.0, 1.0)
    e = D.uniform(0xA101, (1024, 10), -1.0, 1.0)
    got = sgemm_at(x, e)
    ref = O.matmul(np.ascontiguousarray(x.T), e)
    ok, worst = K.gemm_tol_ok(got, ref, np.ascontiguousarray(x.T), e)
    assert ok, f"worst error / bound = {worst}"


def test_sgemm_rejects_unknown_flags():
    d = K.empty(64)
    lib = H.load()
    assert lib.camel_hip_sgemm(P(d.ptr), P(d.ptr), P(d.ptr), 2, 2, 2, None, 0x40) == H.ERR_ARG


# ---------------------------------------------------------- operator layer

@pytest.fixture(autouse=True)
def _release():
    yield
    T.release_all()


def t(a):
    return T.Tensor.from_numpy(np.asarray(a))


def test_transpose_operator_feeds_the_gemm_without_a_copy():
    x = ints(0xA200, (300, 130), -2, 2)
    e = ints(0xA201, (300, 12), -2, 2)
    xt = t(x)
    xt.numpy()  # host copy only
    tr = T.call("transpose", xt)
    g = T.call("matmul", tr, t(e))
    assert_bits(g.numpy(), exact_dense(np.ascontiguousarray(x.T), e), "transpose(X) @ E")
    # the view was read in place: it still shares X's payload, now on the device
    assert tr.residency() == (True, True)
    # other readers see the contiguous transpose
    np.testing.assert_array_equal(T.call("exp", tr).numpy(), O.exp(np.ascontiguousarray(x.T)))
    # dense reads a transposed input in place too (bias in the epilogue)
    w, b = np.ascontiguousarray(e[:, :7]), ints(0xA202, (7,), -2, 2)
    d = T.call("dense_relu", T.call("transpose", xt), with_=(t(w), t(b)))
    assert_bits(d.numpy(), exact_dense(np.ascontiguousarray(x.T), w, b, True), "dense(transpose(X))")


def _oracle_softmax_mnist(logits):
    return O.softmax_rows(logits)


def test_mnist_update_step_on_the_device_matches_the_oracle():
    # mnist.cml:35-41:
    #   logits = X @ W; probs = softmax(logits) (mnist.cml:13-25, as tensor ops)
    #   grad = transpose(X) @ (probs - y_onehot)
    #   W' = W - lr * (1.0 / float(m)) * grad
    # Every device step is checked against the oracle applied to the device's
    # own inputs for that step, at that step's bar: the GEMMs under the GEMM
    # bound, the softmax composition within 1e-6, the element-wise ops bit
    # for bit.  Shapes: mnist.cml's 100 x 33 (features + bias column) and an
    # MNIST-scale 1024 x 785.
    for n, d in ((100, 33), (1024, 785)):
        X = D.uniform(0xA300 + n, (n, d), 0.0, 1.0)
        X[:, -1] = 1.0                                   # the concat'ed bias column
        Y = np.zeros((n, 10), F)
        Y[np.arange(n), np.arange(n) % 10] = 1.0         # build_one_hot: i % 10
        W = D.normal(0xA301 + n, (d, 10), std=0.1)
        lr = 0.1
        Xt, Yt, Wt = t(X), t(Y), t(W)
        logits = T.call("matmul", Xt, Wt)
        ok, worst = K.gemm_tol_ok(logits.numpy(), O.matmul(X, W), X, W)
        assert ok, f"logits: {worst}"
        # softmax exactly as mnist.cml spells it, one tensor operator per line
        k = 10
        row_max = T.call("max_axis", logits, 1)
        row_max_b = T.call("matmul", T.call("reshape", row_max, [n, 1]), T.call("ones", [1, k]))
        stable = T.call("subtract", logits, row_max_b)
        exp_logits = T.call("exp", stable)
        row_sums = T.call("sum_axis", exp_logits, 1)
        row_sums_b = T.call("matmul", T.call("reshape", row_sums, [n, 1]), T.call("ones", [1, k]))
        probs = T.call("divide", exp_logits, row_sums_b)
        p_ref = _oracle_softmax_mnist(logits.numpy())
        assert np.max(np.abs(probs.numpy() - p_ref) / np.maximum(p_ref, 1e-30)) <= 1e-6
        err = T.call("subtract", probs, Yt)
        assert_bits(err.numpy(), O.binary(O.SUB, probs.numpy(), Y), "probs - y")
        grad = T.call("matmul", T.call("transpose", Xt), err)
        xT = np.ascontiguousarray(X.T)
        ok, worst = K.gemm_tol_ok(grad.numpy(), O.matmul(xT, err.numpy()), xT, err.numpy())
        assert ok, f"grad: {worst}"
        scale = lr * (1.0 / float(n))                   # scalar arithmetic in double
        step = T.call("multiply", scale, grad)
        assert_bits(step.numpy(), O.binary_scalar(O.MUL, grad.numpy(), scale, O.F32, side=1),
                    "lr/m * grad")
        W1 = T.call("subtract", Wt, step)
        assert_bits(W1.numpy(), O.binary(O.SUB, W, step.numpy()), "W - step")
        # and the whole step against the oracle's own composition
        g_ref = O.matmul(xT, O.binary(O.SUB, O.softmax_rows(O.matmul(X, W)), Y))
        w_ref = O.binary(O.SUB, W, O.binary_scalar(O.MUL, g_ref, scale, O.F32, side=1))
        assert np.max(np.abs(W1.numpy() - w_ref)) <= 1e-5 * scale * n
