"""GPU parity of the non-GEMM kernels against the CPU oracle, through the C-ABI.

Bars: bit-exact for add/sub/mul/div, compares, relu, maxpool, transpose,
concat, argmax, max (NaN payloads aside), axis-0 sums (same order as the
reference); fp64-order-dependent results (axis-1 sums, whole sums, softmax)
within rel-err 1e-6; libm calls (exp/log/pow) within rel-err 1e-6 and
otherwise expected bit-equal (ocml vs glibc differ below fp32 rounding);
softmax uses the fp32 device expf (within 1 ulp of fl32(exp(double))), so
most but not all of its outputs are bit-equal, all within rel-err 1e-6;
conv2d under the GEMM bound 1e-5*sqrt(K)*sum|x||w|.
"""
import ctypes as C

import numpy as np
import pytest

from camel_amd import _hip as H
from camel_amd import datagen as D
from oracle import ffi as O
from tests import hipkit as K

pytestmark = pytest.mark.gpu

P = C.c_void_p
F = np.float32
DT = {np.dtype(F): H.DT_F32, np.dtype(np.int64): H.DT_I64, np.dtype(np.uint8): H.DT_BOOL}


def bits_equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == F:
        nan = np.isnan(a) & np.isnan(b)
        return np.array_equal(np.isnan(a), np.isnan(b)) and \
            np.array_equal(a.view(np.uint32)[~nan], b.view(np.uint32)[~nan])
    return np.array_equal(a, b)


def gpu_binary(op, l, r, odt):
    dl, dr = K.dev(l), K.dev(r)
    do = K.empty(l.size * 8)
    H.call("camel_hip_binary", op, DT[l.dtype], P(dl.ptr), DT[r.dtype], P(dr.ptr), odt, P(do.ptr),
           l.size)
    return K.host(do, H.NP_DTYPE[odt], l.shape)


SPECIALS = np.array([0.0, -0.0, 1.0, -1.0, 1.5, -2.75, np.inf, -np.inf, np.nan, 1e-45, -1e-45,
                     1.17549435e-38, 3.4028235e38, -3.4028235e38, 0.1, 3.0, 7e-39, 1e30], F)


def _special_pairs():
    return np.repeat(SPECIALS, SPECIALS.size), np.tile(SPECIALS, SPECIALS.size)


@pytest.mark.parametrize("op", [H.OP_ADD, H.OP_SUB, H.OP_MUL])
@pytest.mark.parametrize("n", [0, 1, 3, 4, 1023, 4096 + 5, 1 << 20])
def test_binary_f32_bit_exact(op, n):
    l = D.normal(100 + n, (n,))
    r = D.normal(200 + n, (n,))
    assert bits_equal(gpu_binary(op, l, r, H.DT_F32), O.binary(op, l, r))


@pytest.mark.parametrize("op", [H.OP_ADD, H.OP_SUB, H.OP_MUL, H.OP_DIV])
def test_binary_special_values_bit_exact(op):
    a, b = _special_pairs()
    if op == H.OP_DIV:
        keep = b != 0
        a, b = a[keep], b[keep]
    assert bits_equal(gpu_binary(op, a, b, H.DT_F32), O.binary(op, a, b))


def test_divide_by_zero_raises():
    l = np.ones(1000, F)
    r = np.ones(1000, F)
    r[777] = 0.0
    with pytest.raises(H.CamelHipError, match="Division by zero"):
        gpu_binary(H.OP_DIV, l, r, H.DT_F32)
    r[777] = -0.0
    with pytest.raises(H.CamelHipError, match="Division by zero"):
        gpu_binary(H.OP_DIV, l, r, H.DT_F32)
    # and the flag is cleared for the next call
    r[777] = 2.0
    assert bits_equal(gpu_binary(H.OP_DIV, l, r, H.DT_F32), O.binary(O.DIV, l, r))


@pytest.mark.parametrize("ldt,rdt", [(np.int64, np.int64), (np.int64, F), (np.uint8, np.uint8),
                                     (np.uint8, F), (np.int64, np.uint8)])
@pytest.mark.parametrize("op", [H.OP_ADD, H.OP_SUB, H.OP_MUL, H.OP_DIV, H.OP_POW])
def test_binary_mixed_dtypes(ldt, rdt, op):
    rng = np.random.default_rng(3)
    def mk(dt):
        if dt == np.uint8:
            return rng.integers(0, 2, 500).astype(np.uint8)
        if dt == np.int64:
            return np.concatenate([rng.integers(-50, 50, 496), [2 ** 53 + 1, -(2 ** 62), 7, 9]]).astype(np.int64)
        return rng.uniform(-3, 3, 500).astype(F)
    l, r = mk(ldt), mk(rdt)
    if op == H.OP_DIV:
        r = np.where(r == 0, 1, r).astype(r.dtype)
    if op == H.OP_POW:
        l = np.abs(l).astype(l.dtype)
        r = (np.abs(r) % 3).astype(r.dtype)
    ref = O.binary(op, l, r)
    got = gpu_binary(op, l, r, O.binary_out_dtype(op, O.dt_of(l), O.dt_of(r)))
    if op == H.OP_POW:
        np.testing.assert_allclose(got, ref, rtol=1e-6)
    else:
        assert bits_equal(got, ref)


def test_int64_out_of_range_matches_x86_conversion():
    l = np.array([2 ** 62, -(2 ** 62), 2 ** 62], np.int64)
    r = np.array([2 ** 62, -(2 ** 62) - 2, 1], np.int64)
    got = gpu_binary(H.OP_ADD, l, r, H.DT_I64)
    assert bits_equal(got, O.binary(O.ADD, l, r))
    assert got[0] == np.iinfo(np.int64).min  # 2^63 does not fit: cvttsd2si gives INT64_MIN


@pytest.mark.parametrize("side", [0, 1])
@pytest.mark.parametrize("op", [H.OP_ADD, H.OP_SUB, H.OP_MUL, H.OP_DIV, H.OP_POW])
@pytest.mark.parametrize("s", [0.1, -2.0, 3.0])
def test_binary_scalar_f32(side, op, s):
    t = D.uniform(300, (4099,), 0.25, 4.0)
    dt, do = K.dev(t), K.empty(t.nbytes)
    H.call("camel_hip_binary_scalar", op, side, H.DT_F32, P(dt.ptr), s, H.DT_F32, P(do.ptr), t.size)
    got = K.host(do, F, t.shape)
    ref = O.binary_scalar(op, t, s, O.F32, side)
    if op == H.OP_POW:
        np.testing.assert_allclose(got, ref, rtol=1e-6)
    else:
        assert bits_equal(got, ref)


def test_binary_scalar_int_and_errors():
    t = np.arange(-5, 5, dtype=np.int64)
    dt, do = K.dev(t), K.empty(t.size * 8)
    H.call("camel_hip_binary_scalar", H.OP_MUL, 0, H.DT_I64, P(dt.ptr), 3.0, H.DT_I64, P(do.ptr), t.size)
    assert bits_equal(K.host(do, np.int64, t.shape), O.binary_scalar(O.MUL, t, 3.0, O.I64))
    with pytest.raises(H.CamelHipError, match="Division by zero"):
        H.call("camel_hip_binary_scalar", H.OP_DIV, 0, H.DT_I64, P(dt.ptr), 0.0, H.DT_F32, P(do.ptr), t.size)
    with pytest.raises(H.CamelHipError, match="Division by zero"):  # 1 / t with t containing 0
        H.call("camel_hip_binary_scalar", H.OP_DIV, 1, H.DT_I64, P(dt.ptr), 1.0, H.DT_F32, P(do.ptr), t.size)


@pytest.mark.parametrize("op", [H.CMP_LT, H.CMP_LE, H.CMP_GT, H.CMP_GE, H.CMP_EQ])
def test_compare_bit_exact(op):
    a, b = _special_pairs()
    da, db, do = K.dev(a), K.dev(b), K.empty(a.size)
    H.call("camel_hip_compare", op, H.DT_F32, P(da.ptr), H.DT_F32, P(db.ptr), P(do.ptr), a.size)
    assert np.array_equal(K.host(do, np.uint8, a.shape), O.compare(op, a, b))
    for side in (0, 1):
        H.call("camel_hip_compare_scalar", op, side, H.DT_F32, P(da.ptr), 1.5, P(do.ptr), a.size)
        assert np.array_equal(K.host(do, np.uint8, a.shape), O.compare_scalar(op, a, 1.5, side))


@pytest.mark.parametrize("n", [0, 5, 1 << 16, (1 << 20) + 3])
def test_relu_bit_exact(n):
    x = D.normal(400 + n, (n,))
    if n >= 8:
        x[:8] = np.array([-3.0, -0.0, 0.0, np.nan, -np.inf, np.inf, -1e-45, 2.0], F)
    dx, dy = K.dev(x), K.empty(x.nbytes)
    H.call("camel_hip_relu", P(dx.ptr), P(dy.ptr), n)
    assert bits_equal(K.host(dy, F, x.shape), O.relu(x))


def test_relu_idiom_via_compare_and_multiply():
    # the reference composition multiply(x, x > 0) run as two GPU ops (svm.cml:31)
    x = D.normal(401, (3001,))
    dx, dm, dy = K.dev(x), K.empty(x.size), K.empty(x.nbytes)
    H.call("camel_hip_compare_scalar", H.CMP_GT, 0, H.DT_F32, P(dx.ptr), 0.0, P(dm.ptr), x.size)
    H.call("camel_hip_binary", H.OP_MUL, H.DT_F32, P(dx.ptr), H.DT_BOOL, P(dm.ptr), H.DT_F32,
           P(dy.ptr), x.size)
    assert bits_equal(K.host(dy, F, x.shape), O.relu(x))


def test_exp_log():
    x = D.uniform(500, (100003,), -30.0, 30.0)
    dx, dy = K.dev(x), K.empty(x.nbytes)
    H.call("camel_hip_exp", P(dx.ptr), P(dy.ptr), x.size)
    got, ref = K.host(dy, F, x.shape), O.exp(x)
    np.testing.assert_allclose(got, ref, rtol=1e-6)
    assert np.mean(got == ref) > 0.9999
    p = np.abs(x) + F(1e-3)
    dp = K.dev(p)
    H.call("camel_hip_log", P(dp.ptr), P(dy.ptr), p.size)
    np.testing.assert_allclose(K.host(dy, F, p.shape), O.log(p), rtol=1e-6, atol=1e-7)
    p[12345] = 0.0
    dp = K.dev(p)
    with pytest.raises(H.CamelHipError, match="log: input must be positive"):
        H.call("camel_hip_log", P(dp.ptr), P(dy.ptr), p.size)


# ---------------------------------------------------------------- softmax

@pytest.mark.parametrize("rows,cols", [(1024, 10), (512, 10), (7, 1), (33, 255), (64, 256),
                                       (100, 1000), (40, 1024), (9, 2047), (5, 3000), (3, 9000)])
def test_softmax_matches_composition(rows, cols):
    x = D.normal(600 + cols, (rows, cols)) * F(4.0)
    dx, dy = K.dev(x), K.empty(x.nbytes)
    H.call("camel_hip_softmax_rows", P(dx.ptr), P(dy.ptr), rows, cols)
    got, ref = K.host(dy, F, x.shape), O.softmax_rows(x)
    # north-star softmax tolerance: rel-err <= 1e-6 per element
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-38)) <= 1e-6
    assert np.mean(got == ref) > 0.75
    np.testing.assert_allclose(got.sum(axis=1, dtype=np.float64), 1.0, rtol=2e-6)


def test_softmax_nan_and_ties():
    x = np.array([[np.nan, 1.0, 2.0, 3.0], [1.0, np.nan, 2.0, 3.0], [-0.0, 0.0, -1.0, -2.0],
                  [5.0, 5.0, 5.0, 5.0]], F)
    dx, dy = K.dev(x), K.empty(x.nbytes)
    H.call("camel_hip_softmax_rows", P(dx.ptr), P(dy.ptr), 4, 4)
    got, ref = K.host(dy, F, x.shape), O.softmax_rows(x)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.isnan(got[:2]).all()  # a NaN anywhere in a row poisons the fp64 row sum
    np.testing.assert_allclose(got[2:], ref[2:], rtol=1e-6)
    assert bits_equal(got[3], ref[3])  # ties: exp(0) = 1 exactly, 1/4 exactly


# ----------------------------------------------------------- reductions

@pytest.mark.parametrize("rows,cols", [(1, 1), (5, 7), (1024, 10), (64, 4096), (3000, 3)])
@pytest.mark.parametrize("axis", [0, 1, -1, -2])
def test_axis_reductions(rows, cols, axis):
    x = D.normal(700 + rows, (rows, cols))
    x.flat[::97] = x.flat[::97].round()  # plant ties
    out_n = cols if axis in (0, -2) else rows
    dx, dout = K.dev(x), K.empty(out_n * 8)
    H.call("camel_hip_sum_axis", H.DT_F32, P(dx.ptr), rows, cols, axis, P(dout.ptr))
    s = K.host(dout, F, (out_n,))
    ref = O.sum_axis(x, axis)
    if axis in (0, -2):
        assert bits_equal(s, ref)  # same order as the reference
    else:
        np.testing.assert_allclose(s, ref, rtol=1e-6, atol=1e-6)
    H.call("camel_hip_max_axis", H.DT_F32, P(dx.ptr), rows, cols, axis, P(dout.ptr))
    assert bits_equal(K.host(dout, F, (out_n,)), O.max_axis(x, axis))
    H.call("camel_hip_argmax_axis", H.DT_F32, P(dx.ptr), rows, cols, axis, P(dout.ptr))
    assert np.array_equal(K.host(dout, np.int64, (out_n,)), O.argmax_axis(x, axis))


def test_axis_reduction_nan_and_signed_zero_rules():
    x = np.array([[1.0, 3.0, 3.0, 2.0], [np.nan, 5.0, 1.0, 9.0], [1.0, np.nan, 2.0, 0.5],
                  [-0.0, 0.0, -1.0, -0.0], [0.0, -0.0, -1.0, -2.0]], F)
    for axis, xx in ((1, x), (0, x.T.copy())):
        dx, dout = K.dev(xx), K.empty(64)
        H.call("camel_hip_max_axis", H.DT_F32, P(dx.ptr), xx.shape[0], xx.shape[1], axis, P(dout.ptr))
        assert bits_equal(K.host(dout, F, (5,)), O.max_axis(xx, axis))
        H.call("camel_hip_argmax_axis", H.DT_F32, P(dx.ptr), xx.shape[0], xx.shape[1], axis, P(dout.ptr))
        assert np.array_equal(K.host(dout, np.int64, (5,)), O.argmax_axis(xx, axis))


def test_reductions_int64_bool_and_bad_axis():
    x = (np.arange(60, dtype=np.int64).reshape(6, 10) * 7919) % 101
    dx, dout = K.dev(x), K.empty(128)
    H.call("camel_hip_argmax_axis", H.DT_I64, P(dx.ptr), 6, 10, 1, P(dout.ptr))
    assert np.array_equal(K.host(dout, np.int64, (6,)), O.argmax_axis(x, 1))
    H.call("camel_hip_max_axis", H.DT_I64, P(dx.ptr), 6, 10, 0, P(dout.ptr))
    assert bits_equal(K.host(dout, F, (10,)), O.max_axis(x, 0))
    with pytest.raises(H.CamelHipError, match="axis must be 0 or 1"):
        H.call("camel_hip_sum_axis", H.DT_I64, P(dx.ptr), 6, 10, 2, P(dout.ptr))


@pytest.mark.parametrize("n", [0, 1, 1000, (1 << 22) + 17])
def test_sum_all(n):
    x = D.normal(800 + n, (n,))
    dx = K.dev(x) if n else K.empty(4)
    r = C.c_double()
    H.call("camel_hip_sum", H.DT_F32, P(dx.ptr), n, C.byref(r))
    ref = O.sum_all(x)
    assert abs(r.value - ref) <= 1e-9 * max(1.0, np.abs(x.astype(np.float64)).sum())


# -------------------------------------------------------- conv2d / pooling

def conv_bound_ok(got, ref, x, w, stride, pad):
    # |dy| <= 1e-5*sqrt(K)*sum|x||w| via a conv of |x| with |w| (oracle, fp64 accumulate)
    K_ = w.shape[1] * w.shape[2] * w.shape[3]
    mag = O.conv2d(np.abs(x), np.abs(w), None, False, stride, pad).astype(np.float64)
    return np.all(np.abs(got.astype(np.float64) - ref.astype(np.float64)) <= 1e-5 * np.sqrt(K_) * mag + 1e-30)


@pytest.mark.parametrize("N,Cin,H_,W_,Co,k,stride,pad", [
    (2, 3, 9, 7, 5, 3, 1, 1), (1, 1, 28, 28, 32, 3, 1, 0), (2, 32, 26, 26, 64, 3, 1, 0),
    (1, 64, 56, 56, 128, 3, 1, 1), (3, 8, 11, 13, 70, 3, 2, 1), (2, 16, 10, 10, 130, 1, 1, 0)])
def test_conv2d_matches_oracle(N, Cin, H_, W_, Co, k, stride, pad):
    x = D.normal(900 + Cin, (N, Cin, H_, W_))
    w = D.normal(901 + Co, (Co, Cin, k, k)) * F(np.sqrt(2.0 / (k * k * Cin)))
    b = D.uniform(902, (Co,), -0.1, 0.1)
    ref = O.conv2d(x, w, b, True, stride, pad)
    dx, dw, db, dy = K.dev(x), K.dev(w), K.dev(b), K.empty(ref.nbytes)
    H.call("camel_hip_conv2d", P(dx.ptr), P(dw.ptr), P(db.ptr), P(dy.ptr), N, Cin, H_, W_, Co, k, k,
           stride, pad, H.EPI_BIAS | H.EPI_RELU)
    got = K.host(dy, F, ref.shape)
    assert conv_bound_ok(got, ref, x, w, stride, pad)


@pytest.mark.parametrize("N,Cin,H_,W_,Co,kh,kw,stride,pad", [
    (2, 64, 17, 15, 96, 3, 3, 2, 1),    # implicit GEMM (channel-plane loads), 128-row tile, stride 2
    (3, 32, 12, 10, 40, 3, 5, 1, 2),    # implicit GEMM, 64-row tile, KH != KW, wide pad
    (1, 64, 9, 9, 200, 1, 1, 1, 0),     # implicit GEMM, 1x1 kernel, two row tiles
    (2, 48, 7, 7, 150, 3, 3, 1, 1),     # implicit GEMM with C = 48 (3 stages per (kh, kw))
    (2, 12, 8, 8, 24, 3, 3, 1, 1),      # gather path: C % 16 != 0, K = 108
    (4, 2, 10, 10, 33, 4, 4, 2, 1),     # direct path, K = 32, Co not a multiple of 8
    (2, 3, 16, 16, 16, 3, 3, 1, 1),     # direct, K = 27, 2 pixels per thread
    (2, 3, 32, 32, 16, 3, 3, 2, 1),     # direct, K = 27, stride 2, 2 pixels per thread
    (3, 1, 12, 12, 8, 5, 5, 1, 2),      # direct, K = 25, 2 pixels per thread
    (2, 1, 13, 13, 7, 5, 5, 2, 0),      # direct, K = 25, P = 25: one pixel per thread
])
def test_conv2d_paths_rect_kernels(N, Cin, H_, W_, Co, kh, kw, stride, pad):
    x = D.normal(910 + Cin, (N, Cin, H_, W_))
    w = D.normal(911 + Co, (Co, Cin, kh, kw)) * F(np.sqrt(2.0 / (kh * kw * Cin)))
    b = D.uniform(912, (Co,), -0.1, 0.1)
    for flags, relu in ((H.EPI_BIAS | H.EPI_RELU, True), (0, False)):
        ref = O.conv2d(x, w, b if flags else None, relu, stride, pad)
        dx, dw, db, dy = K.dev(x), K.dev(w), K.dev(b), K.empty(ref.nbytes)
        H.call("camel_hip_conv2d", P(dx.ptr), P(dw.ptr), P(db.ptr) if flags else None, P(dy.ptr), N,
               Cin, H_, W_, Co, kh, kw, stride, pad, flags)
        got = K.host(dy, F, ref.shape)
        assert conv_bound_ok(got, ref, x, w, stride, pad)


def test_conv2d_full_config_slab():
    # The 64x64x56x56 -> 128 3x3 benchmark conv at full size; the oracle checks images 0 and 63
    x = D.normal(D.SEED_CONV_X, (64, 64, 56, 56))
    w = D.normal(D.SEED_CONV_W, (128, 64, 3, 3)) * F(np.sqrt(2.0 / (9 * 64)))
    b = np.zeros(128, F)
    dx, dw, db = K.dev(x), K.dev(w), K.dev(b)
    dy = K.empty(64 * 128 * 56 * 56 * 4)
    H.call("camel_hip_conv2d", P(dx.ptr), P(dw.ptr), P(db.ptr), P(dy.ptr), 64, 64, 56, 56, 128, 3, 3,
           1, 1, H.EPI_BIAS | H.EPI_RELU)
    got = K.host(dy, F, (64, 128, 56, 56))
    for n in (0, 63):
        ref = O.conv2d_images(x, w, b, True, n, n + 1, 1, 1)
        assert conv_bound_ok(got[n:n + 1], ref, x[n:n + 1], w, 1, 1)


@pytest.mark.parametrize("shape,k,stride", [((512, 64, 24, 24), 2, 2), ((2, 3, 7, 9), 2, 2),
                                            ((1, 2, 6, 6), 3, 1), ((2, 2, 5, 8), 2, 1)])
def test_maxpool_bit_exact(shape, k, stride):
    x = D.normal(1000 + shape[0], shape)
    x.flat[::13] = 0.0
    x.flat[::17] = -0.0
    ref = O.maxpool2d(x, k, stride)
    dx, dy = K.dev(x), K.empty(ref.nbytes)
    H.call("camel_hip_maxpool2d", P(dx.ptr), P(dy.ptr), *shape, k, k, stride)
    assert bits_equal(K.host(dy, F, ref.shape), ref)


# ---------------------------------------------------------------- layout

@pytest.mark.parametrize("dtype", [F, np.int64, np.uint8])
@pytest.mark.parametrize("rows,cols", [(1, 1), (5, 7), (33, 65), (1024, 300)])
def test_transpose(dtype, rows, cols):
    x = (D.uniform(1100, (rows, cols), -100, 100)).astype(dtype)
    if dtype == np.int64 and rows * cols > 2:
        x.flat[1] = 2 ** 53 + 1
    dx, dy = K.dev(x), K.empty(x.nbytes)
    H.call("camel_hip_transpose2d", DT[x.dtype], P(dx.ptr), P(dy.ptr), rows, cols)
    assert bits_equal(K.host(dy, dtype, (cols, rows)), O.transpose2d(x))


@pytest.mark.parametrize("axis", [0, 1, 2])
def test_concat(axis):
    a = np.arange(2 * 3 * 4, dtype=np.int64).reshape(2, 3, 4)
    bshape = list(a.shape)
    bshape[axis] = 5
    b = np.arange(int(np.prod(bshape)), dtype=np.int64).reshape(bshape) + 1000
    ref = O.concat(a, b, axis)
    outer = int(np.prod(a.shape[:axis])) if axis else 1
    inner = int(np.prod(a.shape[axis + 1:])) if axis < 2 else 1
    da, db, do = K.dev(a), K.dev(b), K.empty(ref.nbytes)
    H.call("camel_hip_concat", H.DT_I64, P(da.ptr), P(db.ptr), P(do.ptr), outer, a.shape[axis],
           b.shape[axis], inner)
    assert np.array_equal(K.host(do, np.int64, ref.shape), ref)


def test_fill_eye_arange():
    do = K.empty(64 * 8)
    H.call("camel_hip_fill", H.DT_F32, P(do.ptr), 37, 1.0)
    assert np.all(K.host(do, F, (37,)) == 1.0)
    H.call("camel_hip_fill", H.DT_I64, P(do.ptr), 5, -2.7)
    assert list(K.host(do, np.int64, (5,))) == [-2] * 5  # (int64)-2.7 truncates
    H.call("camel_hip_fill", H.DT_BOOL, P(do.ptr), 9, 0.5)
    assert list(K.host(do, np.uint8, (9,))) == [1] * 9
    H.call("camel_hip_eye", P(do.ptr), 7)
    assert np.array_equal(K.host(do, F, (7, 7)), np.eye(7, dtype=F))
    H.call("camel_hip_arange", P(do.ptr), 10, -3, 4)
    assert list(K.host(do, np.int64, (4,))) == [10, 7, 4, 1]


def test_pool_does_not_leak():
    in_use0 = C.c_size_t()
    H.call("camel_hip_pool_stats", C.byref(in_use0), None)
    for _ in range(5):
        b = K.empty(1 << 20)
        b.free()
    in_use1 = C.c_size_t()
    H.call("camel_hip_pool_stats", C.byref(in_use1), None)
    assert in_use1.value == in_use0.value


@pytest.mark.parametrize("nbytes", [(2 << 20) - 1, 2 << 20, (8 << 20) - 1, 8 << 20, (8 << 20) + 1,
                                    (24 << 20) + 5, 67108864 + 8 * 4096 + 3])
def test_boundary_copies_through_the_staging_ring(nbytes):
    # camel_hip_h2d / camel_hip_d2h at and around the staging slots' edges
    # (copies >= 2 MiB go through 8 MiB pinned slots), from and into host
    # buffers at every offset mod 8 that the tests reach (the reference's
    # payload is 8-byte aligned only, runtime.cpp:482-485).  Each direction
    # is checked against the direct path on its own: the staged upload is
    # read back in 1 MiB pieces (below the staging threshold), and the staged
    # download reads a buffer uploaded in 1 MiB pieces.
    piece = 1 << 20
    rng = np.random.default_rng(nbytes)

    def direct(name, dev, host_ptr):
        for o in range(0, nbytes, piece):
            m = min(piece, nbytes - o)
            a, b = (C.c_void_p(dev + o), C.c_void_p(host_ptr + o)) if name == "camel_hip_h2d" \
                else (C.c_void_p(host_ptr + o), C.c_void_p(dev + o))
            H.call(name, a, b, C.c_size_t(m))

    for off_in, off_out in ((0, 0), (1, 5), (3, 8), (8, 1)):
        raw = rng.integers(0, 256, size=nbytes + 16, dtype=np.uint8)
        src = raw.ctypes.data + off_in
        want = raw[off_in:off_in + nbytes]
        d = H.DeviceBuffer(nbytes)
        H.call("camel_hip_h2d", C.c_void_p(d.ptr), C.c_void_p(src), C.c_size_t(nbytes))
        back = np.full(nbytes + 16, 0xA5, dtype=np.uint8)
        direct("camel_hip_d2h", d.ptr, back.ctypes.data + off_out)
        assert np.array_equal(back[off_out:off_out + nbytes], want), "staged upload"
        e = H.DeviceBuffer(nbytes)
        direct("camel_hip_h2d", e.ptr, src)
        back[:] = 0xA5
        H.call("camel_hip_d2h", C.c_void_p(back.ctypes.data + off_out), C.c_void_p(e.ptr),
               C.c_size_t(nbytes))
        assert np.array_equal(back[off_out:off_out + nbytes], want), "staged download"
        assert np.all(back[:off_out] == 0xA5) and np.all(back[off_out + nbytes:] == 0xA5)
