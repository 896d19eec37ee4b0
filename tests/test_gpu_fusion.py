"""Fused layer kernels (graph-level fusion of composed layers) against the
unfused device chain and the CPU oracle.

* dense..softmax (README.md:43 `dense<w3, b3>..softmax`): camel_hip_dense_softmax
  equals camel_hip_sgemm then camel_hip_softmax_rows bit for bit where the
  fused path serves (N <= 32, one value per lane), and the softmax of the
  device GEMM result per the oracle.
* dense..relu..dense..softmax: camel_hip_dense_head equals camel_hip_sgemm
  then camel_hip_dense_softmax (or camel_hip_sgemm) bit for bit, whether
  layer 2 rebuilds layer 1's rows from its split-K partials or the two
  layers run as two calls.
* conv2d layouts: CAMEL_CONV_X_NHWC / CAMEL_CONV_Y_NHWC and
  CAMEL_CONV_X_NCHW4 / CAMEL_CONV_Y_NCHW4 change addressing only, so results
  equal the NCHW conv bit for bit.
* conv2d..maxpool2d: camel_hip_conv2d_pool2 equals camel_hip_conv2d then
  camel_hip_maxpool2d(2, 2, 2) bit for bit when both run one launch of the
  same tile (every output then sums in the same order); the oracle bounds the
  rest.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from camel_amd import _hip as H
from camel_amd import datagen as D
from oracle import ffi as O
from tests import hipkit as K
from tests.test_gpu_exact import ints

pytestmark = pytest.mark.gpu
P = C.c_void_p
F = np.float32


@pytest.fixture(autouse=True, scope="module")
def _init():
    H.call("camel_hip_init", 0)


def _dense_softmax(x, w, b, flags):
    M, Kd = x.shape
    N = w.shape[1]
    dx, dw, dy = K.dev(x), K.dev(w), K.empty(M * N * 4)
    db = K.dev(b) if b is not None else None
    H.call("camel_hip_dense_softmax", P(dx.ptr), P(dw.ptr), P(db.ptr) if db else None, P(dy.ptr),
           M, N, Kd, flags)
    return K.host(dy, F, (M, N))


def _dense_then_softmax(x, w, b, flags):
    M, Kd = x.shape
    N = w.shape[1]
    dx, dw, dh, dy = K.dev(x), K.dev(w), K.empty(M * N * 4), K.empty(M * N * 4)
    db = K.dev(b) if b is not None else None
    H.call("camel_hip_sgemm", P(dx.ptr), P(dw.ptr), P(dh.ptr), M, N, Kd, P(db.ptr) if db else None,
           flags)
    H.call("camel_hip_softmax_rows", P(dh.ptr), P(dy.ptr), M, N)
    return K.host(dh, F, (M, N)), K.host(dy, F, (M, N))


@pytest.mark.parametrize("M,N,Kd,flags", [
    (1024, 10, 1024, H.EPI_BIAS),               # the benchmark MLP's classifier
    (512, 10, 128, H.EPI_BIAS),                 # the benchmark CNN's classifier
    (300, 7, 50, H.EPI_BIAS | H.EPI_RELU),      # relu before the softmax
    (257, 32, 512, 0),                          # widest fused row, longest K for it
    (200, 3, 1, H.EPI_BIAS),                    # K = 1
])
def test_dense_softmax_equals_unfused_chain(M, N, Kd, flags):
    x = D.uniform(0x5100 + M, (M, Kd), -1.0, 1.0)
    w = D.normal(0x5101 + N, (Kd, N), std=float(np.sqrt(1.0 / Kd)))
    b = D.uniform(0x5102, (N,), -0.5, 0.5)
    got = _dense_softmax(x, w, b, flags)
    h, ref = _dense_then_softmax(x, w, b, flags)
    np.testing.assert_array_equal(got, ref)
    # and the softmax of the device dense result per the oracle (1e-6 relative)
    p = O.softmax_rows(h)
    assert np.max(np.abs(got - p) / np.maximum(p, 1e-30)) <= 1e-6
    np.testing.assert_allclose(got.sum(axis=1, dtype=np.float64), 1.0, rtol=0, atol=1e-5)


def test_dense_softmax_special_values_follow_the_softmax_rules():
    # bias NaN in column 0: every row NaN (NaN wins only as element 0); +inf
    # in another column: inf - inf = NaN there, the rest 0 -- the unfused
    # kernel's rules, bit for bit.
    x = D.uniform(0x5200, (96, 40), -1.0, 1.0)
    w = D.normal(0x5201, (40, 9), std=0.2)
    for col, val in ((0, np.nan), (4, np.inf), (2, -np.inf), (5, np.nan)):
        b = D.uniform(0x5202, (9,), -0.5, 0.5)
        b[col] = val
        got = _dense_softmax(x, w, b, H.EPI_BIAS)
        _, ref = _dense_then_softmax(x, w, b, H.EPI_BIAS)
        np.testing.assert_array_equal(got, ref)


def test_dense_softmax_wide_rows_take_the_unfused_path():
    # N > 32: GEMM then the softmax kernel in place
    x = D.uniform(0x5300, (64, 100), -1.0, 1.0)
    w = D.normal(0x5301, (100, 70), std=0.1)
    b = D.uniform(0x5302, (70,), -0.5, 0.5)
    got = _dense_softmax(x, w, b, H.EPI_BIAS)
    _, ref = _dense_then_softmax(x, w, b, H.EPI_BIAS)
    np.testing.assert_array_equal(got, ref)


def test_dense_softmax_argument_errors():
    lib = H.load()
    assert lib.camel_hip_dense_softmax(None, None, None, None, -1, 2, 2, 0) == H.ERR_SHAPE
    assert lib.camel_hip_dense_softmax(None, None, None, None, 2, 2, 2, H.EPI_BIAS) == H.ERR_ARG
    assert lib.camel_hip_dense_softmax(None, None, None, None, 0, 2, 2, 0) == 0


# ------------------------------------------------------------------ dense head

def _dense_head(x, w1, b1, w2, b2, flags1, flags2, softmax):
    M, K1 = x.shape
    N1, N2 = w1.shape[1], w2.shape[1]
    dx, dw1, dw2, dy = K.dev(x), K.dev(w1), K.dev(w2), K.empty(M * N2 * 4)
    db1, db2 = K.dev(b1), K.dev(b2)
    H.call("camel_hip_dense_head", P(dx.ptr), P(dw1.ptr), P(db1.ptr), P(dw2.ptr), P(db2.ptr),
           P(dy.ptr), M, K1, N1, N2, flags1, flags2, int(softmax))
    return K.host(dy, F, (M, N2))


def _head_in_two_calls(x, w1, b1, w2, b2, flags1, flags2, softmax):
    h = K.sgemm(x, w1, b1, flags1)
    if softmax:
        return h, _dense_softmax(h, w2, b2, flags2)
    return h, K.sgemm(h, w2, b2, flags2)


@pytest.mark.parametrize("M,K1,N1,N2,flags2,softmax", [
    (512, 9216, 128, 10, H.EPI_BIAS, True),             # the benchmark CNN's head (16 K splits)
    (512, 9216, 128, 10, H.EPI_BIAS | H.EPI_RELU, False),
    (300, 2000, 200, 16, H.EPI_BIAS, True),             # ragged tiles, N2 = 16
    (130, 700, 72, 5, 0, True),                         # 32x32 tiles with K splits
    (1000, 1024, 1024, 10, H.EPI_BIAS, True),           # unsplit, M % 64 != 0: two calls
    (257, 300, 24, 9, H.EPI_BIAS, True),                # layer 1 on the thin-N kernel, two calls
])
def test_dense_head_equals_two_calls(M, K1, N1, N2, flags2, softmax):
    x = D.uniform(0x5400 + M, (M, K1), 0.0, 1.0)
    w1 = D.normal(0x5401 + N1, (K1, N1), std=float(np.sqrt(2.0 / K1)))
    b1 = D.uniform(0x5402, (N1,), -0.1, 0.1)
    w2 = D.normal(0x5403 + N2, (N1, N2), std=float(np.sqrt(2.0 / N1)))
    b2 = D.uniform(0x5404, (N2,), -0.1, 0.1)
    flags1 = H.EPI_BIAS | H.EPI_RELU
    got = _dense_head(x, w1, b1, w2, b2, flags1, flags2, softmax)
    h, ref = _head_in_two_calls(x, w1, b1, w2, b2, flags1, flags2, softmax)
    np.testing.assert_array_equal(got, ref)
    # and layer 1 itself against the oracle's dense (the GEMM tolerance)
    rows = slice(0, 8)
    ok, worst = K.gemm_tol_ok(h[rows], O.dense(x[rows], w1, b1, True), x[rows], w1)
    assert ok, f"layer 1 worst error / bound = {worst}"


HEAD_EPILOGUE_SHAPES = [
    # layer 1 unsplit on 64 x 64 tiles that fill the chip: the head runs in
    # its epilogue and head_finish_kernel adds the 64-column shares
    (1024, 1024, 1024, 10),   # the benchmark MLP's head
    (2048, 512, 512, 16),     # N2 = 16, 8 column tiles
    (4096, 300, 256, 7),      # K % 64 != 0 (ragged first stage), 4 column tiles
]


@pytest.mark.parametrize("M,K1,N1,N2", HEAD_EPILOGUE_SHAPES)
def test_dense_head_in_the_gemm_epilogue(M, K1, N1, N2):
    # Small integers: the logits are exact whatever the order, so they equal
    # the two calls bit for bit.
    xi = ints(0x5500 + M, (M, K1), 0, 2)
    w1i, b1i = ints(0x5501, (K1, N1), -1, 1), ints(0x5502, (N1,), -1, 1)
    w2i, b2i = ints(0x5503, (N1, N2), -1, 1), ints(0x5504, (N2,), -2, 2)
    e1 = H.EPI_BIAS | H.EPI_RELU
    for flags2 in (H.EPI_BIAS, H.EPI_BIAS | H.EPI_RELU):
        got = _dense_head(xi, w1i, b1i, w2i, b2i, e1, flags2, False)
        _, ref = _head_in_two_calls(xi, w1i, b1i, w2i, b2i, e1, flags2, False)
        np.testing.assert_array_equal(got, ref)
    # Real values: the tiles' shares add in another order than the thin
    # kernel's, so the logits match the two calls within the GEMM bound of
    # layer 2, and the fused softmax is the softmax of the fused logits
    # within the softmax bar.
    x = D.uniform(0x5600 + M, (M, K1), 0.0, 1.0)
    w1 = D.normal(0x5601, (K1, N1), std=float(np.sqrt(2.0 / K1)))
    b1 = D.uniform(0x5602, (N1,), -0.1, 0.1)
    w2 = D.normal(0x5603, (N1, N2), std=float(np.sqrt(2.0 / N1)))
    b2 = D.uniform(0x5604, (N2,), -0.1, 0.1)
    logits = _dense_head(x, w1, b1, w2, b2, e1, H.EPI_BIAS, False)
    h, ref = _head_in_two_calls(x, w1, b1, w2, b2, e1, H.EPI_BIAS, False)
    ok, worst = K.gemm_tol_ok(logits, ref, h, w2)
    assert ok, f"logits worst error / bound = {worst}"
    p = _dense_head(x, w1, b1, w2, b2, e1, H.EPI_BIAS, True)
    q = O.softmax_rows(logits)
    assert np.max(np.abs(p.astype(np.float64) - q) / np.maximum(q, 1e-30)) <= 1e-6
    # and against the oracle's layers on a few rows
    rows = slice(M - 4, M)
    hr = O.dense(x[rows], w1, b1, True)
    ok, worst = K.gemm_tol_ok(logits[rows], O.dense(hr, w2, b2, False), hr, w2)
    assert ok, f"oracle logits worst error / bound = {worst}"


def test_dense_head_argument_errors():
    lib = H.load()
    z = (None,) * 6
    assert lib.camel_hip_dense_head(*z, -1, 2, 2, 2, 0, 0, 0) == H.ERR_SHAPE
    assert lib.camel_hip_dense_head(*z, 2, 2, 2, 2, H.EPI_BIAS, 0, 0) == H.ERR_ARG
    assert lib.camel_hip_dense_head(*z, 2, 2, 2, 2, 0, 0x100, 0) == H.ERR_ARG
    assert lib.camel_hip_dense_head(*z, 2, 2, 2, 2, 0, 0, 0) == H.ERR_ARG  # null operands
    assert lib.camel_hip_dense_head(*z, 0, 2, 2, 2, 0, 0, 1) == 0


# ------------------------------------------------------------------ conv2d layouts

def _conv(x, w, b, geom, flags, pooled=False):
    N, Cin, H_, W_, Co, kh, kw, stride, pad = geom
    OH, OW = (H_ + 2 * pad - kh) // stride + 1, (W_ + 2 * pad - kw) // stride + 1
    if pooled:
        OH, OW = OH // 2, OW // 2
    dx, dw = K.dev(x), K.dev(w)
    db = K.dev(b) if b is not None else None
    dy = K.empty(N * Co * OH * OW * 4)
    H.call("camel_hip_conv2d_pool2" if pooled else "camel_hip_conv2d", P(dx.ptr), P(dw.ptr),
           P(db.ptr) if db else None, P(dy.ptr), N, Cin, H_, W_, Co, kh, kw, stride, pad, flags)
    return dy, (N, Co, OH, OW)


GEOMS = [
    (4, 1, 28, 28, 32, 3, 3, 1, 0),     # direct, K = 9 (CNN conv1), NHWC out in place
    (2, 1, 13, 13, 6, 5, 5, 2, 0),      # direct, Co % 4 != 0: NHWC out through scratch
    (3, 32, 26, 26, 64, 3, 3, 1, 0),    # NHWC implicit GEMM (CNN conv2)
    (2, 16, 9, 11, 130, 3, 3, 2, 1),    # NHWC GEMM, 16-channel stages, Co > 128
    (2, 12, 8, 8, 24, 3, 3, 1, 1),      # gather path (C % 16 != 0)
]


@pytest.mark.parametrize("geom", GEOMS)
def test_conv2d_nhwc_layouts_change_addressing_only(geom):
    N, Cin, H_, W_, Co, kh, kw, stride, pad = geom
    x = D.normal(0x5400 + Cin, (N, Cin, H_, W_))
    w = D.normal(0x5401 + Co, (Co, Cin, kh, kw)) * F(np.sqrt(2.0 / (kh * kw * Cin)))
    b = D.uniform(0x5402, (Co,), -0.1, 0.1)
    epi = H.EPI_BIAS | H.EPI_RELU
    dref, shape = _conv(x, w, b, geom, epi)
    ref = K.host(dref, F, shape)
    x_nhwc = np.ascontiguousarray(x.transpose(0, 2, 3, 1))
    dy, _ = _conv(x_nhwc, w, b, geom, epi | H.CONV_X_NHWC)
    np.testing.assert_array_equal(K.host(dy, F, shape), ref)
    dy, _ = _conv(x, w, b, geom, epi | H.CONV_Y_NHWC)
    np.testing.assert_array_equal(K.host(dy, F, (shape[0], shape[2], shape[3], shape[1])),
                                  ref.transpose(0, 2, 3, 1))
    dy, _ = _conv(x_nhwc, w, b, geom, epi | H.CONV_X_NHWC | H.CONV_Y_NHWC)
    np.testing.assert_array_equal(K.host(dy, F, (shape[0], shape[2], shape[3], shape[1])),
                                  ref.transpose(0, 2, 3, 1))


def test_conv2d_chain_in_nhwc_equals_nchw_chain():
    # CNN conv1 (direct) writing NHWC straight into conv2 (NHWC GEMM) reading it
    x = D.uniform(0x5500, (6, 1, 28, 28), 0.0, 1.0)
    w1 = D.normal(0x5501, (32, 1, 3, 3), std=float(np.sqrt(2.0 / 9)))
    w2 = D.normal(0x5502, (64, 32, 3, 3), std=float(np.sqrt(2.0 / 288)))
    b1, b2 = np.zeros(32, F), D.uniform(0x5503, (64,), -0.1, 0.1)
    epi = H.EPI_BIAS | H.EPI_RELU
    h, _ = _conv(x, w1, b1, (6, 1, 28, 28, 32, 3, 3, 1, 0), epi)
    y_ref, shape = _conv(K.host(h, F, (6, 32, 26, 26)), w2, b2, (6, 32, 26, 26, 64, 3, 3, 1, 0), epi)
    h_nhwc, _ = _conv(x, w1, b1, (6, 1, 28, 28, 32, 3, 3, 1, 0), epi | H.CONV_Y_NHWC)
    y, _ = _conv(K.host(h_nhwc, F, (6, 26, 26, 32)), w2, b2, (6, 32, 26, 26, 64, 3, 3, 1, 0),
                 epi | H.CONV_X_NHWC)
    np.testing.assert_array_equal(K.host(y, F, shape), K.host(y_ref, F, shape))


def _nchw4(a):
    """[N, C, H, W] -> NCHW4 [N, C/4, H, W, 4]."""
    n, c, h, w = a.shape
    return np.ascontiguousarray(a.reshape(n, c // 4, 4, h, w).transpose(0, 1, 3, 4, 2))


def _from_nchw4(a):
    n, q, h, w, _ = a.shape
    return np.ascontiguousarray(a.transpose(0, 1, 4, 2, 3).reshape(n, 4 * q, h, w))


NCHW4_GEOMS = GEOMS + [
    (2, 3, 11, 11, 8, 3, 3, 1, 0),      # direct K = 27, odd P: one pixel per thread
    (3, 1, 12, 12, 16, 5, 5, 1, 0),     # direct K = 25, even P: pixel pairs
    (2, 1, 9, 9, 8, 4, 4, 1, 0),        # direct K = 16 (guarded k loop)
    (2, 2, 9, 9, 12, 4, 4, 1, 1),       # direct K = 32
    (2, 4, 10, 10, 20, 3, 3, 1, 1),     # NCHW4 input to the direct path (converted)
    (2, 16, 9, 11, 132, 3, 3, 2, 1),    # implicit GEMM, NCHW4 out from partial row tiles
]


@pytest.mark.parametrize("geom", NCHW4_GEOMS)
def test_conv2d_nchw4_layouts_change_addressing_only(geom):
    N, Cin, H_, W_, Co, kh, kw, stride, pad = geom
    x = D.normal(0x5480 + Cin, (N, Cin, H_, W_))
    w = D.normal(0x5481 + Co, (Co, Cin, kh, kw)) * F(np.sqrt(2.0 / (kh * kw * Cin)))
    b = D.uniform(0x5482, (Co,), -0.1, 0.1)
    for epi in (H.EPI_BIAS | H.EPI_RELU, 0):
        bb = b if epi else None
        dref, shape = _conv(x, w, bb, geom, epi)
        ref = K.host(dref, F, shape)
        q4 = (shape[0], shape[1] // 4, shape[2], shape[3], 4)
        if Cin % 4 == 0:
            dy, _ = _conv(_nchw4(x), w, bb, geom, epi | H.CONV_X_NCHW4)
            np.testing.assert_array_equal(K.host(dy, F, shape), ref)
        if Co % 4 == 0:
            dy, _ = _conv(x, w, bb, geom, epi | H.CONV_Y_NCHW4)
            np.testing.assert_array_equal(_from_nchw4(K.host(dy, F, q4)), ref)
        if Cin % 4 == 0 and Co % 4 == 0:
            dy, _ = _conv(_nchw4(x), w, bb, geom, epi | H.CONV_X_NCHW4 | H.CONV_Y_NCHW4)
            np.testing.assert_array_equal(_from_nchw4(K.host(dy, F, q4)), ref)
            # NCHW4 in, NHWC out and the reverse
            dy, _ = _conv(_nchw4(x), w, bb, geom, epi | H.CONV_X_NCHW4 | H.CONV_Y_NHWC)
            np.testing.assert_array_equal(K.host(dy, F, (shape[0], shape[2], shape[3], shape[1])),
                                          ref.transpose(0, 2, 3, 1))
            dy, _ = _conv(np.ascontiguousarray(x.transpose(0, 2, 3, 1)), w, bb, geom,
                          epi | H.CONV_X_NHWC | H.CONV_Y_NCHW4)
            np.testing.assert_array_equal(_from_nchw4(K.host(dy, F, q4)), ref)


def test_conv2d_nchw4_output_from_whole_rounds_and_split_tails():
    # enough tiles for whole rounds plus a K-split tail: the GEMM epilogue's
    # 16-byte NCHW4 stores and the split reduce's NCHW4 addressing
    geom = (32, 64, 56, 56, 128, 3, 3, 1, 1)
    N, Cin, H_, W_, Co, kh, kw, stride, pad = geom
    x = D.normal(0x5490, (N, Cin, H_, W_))
    w = D.normal(0x5491, (Co, Cin, kh, kw)) * F(np.sqrt(2.0 / (kh * kw * Cin)))
    b = D.uniform(0x5492, (Co,), -0.1, 0.1)
    epi = H.EPI_BIAS | H.EPI_RELU
    dref, shape = _conv(x, w, b, geom, epi)
    dy, _ = _conv(x, w, b, geom, epi | H.CONV_Y_NCHW4)
    got = K.host(dy, F, (shape[0], shape[1] // 4, shape[2], shape[3], 4))
    np.testing.assert_array_equal(_from_nchw4(got), K.host(dref, F, shape))


def test_conv2d_chain_in_nchw4_equals_nchw_chain():
    # CNN conv1 (direct) writing NCHW4 straight into conv2 (implicit GEMM)
    # reading it in place, with packed weights, plain and pooled
    x = D.uniform(0x5580, (6, 1, 28, 28), 0.0, 1.0)
    w1 = D.normal(0x5581, (32, 1, 3, 3), std=float(np.sqrt(2.0 / 9)))
    w2 = D.normal(0x5582, (64, 32, 3, 3), std=float(np.sqrt(2.0 / 288)))
    b1, b2 = D.uniform(0x5583, (32,), -0.1, 0.1), D.uniform(0x5584, (64,), -0.1, 0.1)
    epi = H.EPI_BIAS | H.EPI_RELU
    g1, g2 = (6, 1, 28, 28, 32, 3, 3, 1, 0), (6, 32, 26, 26, 64, 3, 3, 1, 0)
    h, _ = _conv(x, w1, b1, g1, epi)
    hn = K.host(h, F, (6, 32, 26, 26))
    y_ref, shape = _conv(hn, w2, b2, g2, epi)
    p_ref, pshape = _conv(hn, w2, b2, g2, epi, pooled=True)
    h4, _ = _conv(x, w1, b1, g1, epi | H.CONV_Y_NCHW4)
    h4n = K.host(h4, F, (6, 8, 26, 26, 4))
    np.testing.assert_array_equal(_from_nchw4(h4n), hn)
    dw2, dwp = K.dev(w2), K.empty(w2.nbytes)
    H.call("camel_hip_conv2d_pack_weights", P(dw2.ptr), P(dwp.ptr), 64, 32, 3, 3)
    wp = K.host(dwp, F, (64, 3, 3, 32))
    y, _ = _conv(h4n, wp, b2, g2, epi | H.CONV_X_NCHW4 | H.CONV_W_PACKED)
    np.testing.assert_array_equal(K.host(y, F, shape), K.host(y_ref, F, shape))
    py, _ = _conv(h4n, wp, b2, g2, epi | H.CONV_X_NCHW4 | H.CONV_W_PACKED, pooled=True)
    np.testing.assert_array_equal(K.host(py, F, pshape), K.host(p_ref, F, pshape))


def test_conv2d_nchw4_argument_errors():
    lib = H.load()
    d = K.empty(4 * 8 * 8 * 64)
    ok = P(d.ptr)
    off = P(d.ptr + 4)  # 4-byte aligned only
    conv = lib.camel_hip_conv2d
    # C % 4 != 0 / Co % 4 != 0
    assert conv(ok, ok, None, ok, 1, 6, 8, 8, 8, 3, 3, 1, 0, H.CONV_X_NCHW4) == H.ERR_ARG
    assert conv(ok, ok, None, ok, 1, 8, 8, 8, 6, 3, 3, 1, 0, H.CONV_Y_NCHW4) == H.ERR_ARG
    # misaligned NCHW4 operands
    assert conv(off, ok, None, ok, 1, 8, 8, 8, 8, 3, 3, 1, 0, H.CONV_X_NCHW4) == H.ERR_ARG
    assert conv(ok, ok, None, off, 1, 8, 8, 8, 8, 3, 3, 1, 0, H.CONV_Y_NCHW4) == H.ERR_ARG
    # two layouts for one operand
    assert conv(ok, ok, None, ok, 1, 8, 8, 8, 8, 3, 3, 1, 0,
                H.CONV_X_NCHW4 | H.CONV_X_NHWC) == H.ERR_ARG
    assert conv(ok, ok, None, ok, 1, 8, 8, 8, 8, 3, 3, 1, 0,
                H.CONV_Y_NCHW4 | H.CONV_Y_NHWC) == H.ERR_ARG
    # the pooled output is NCHW only
    assert lib.camel_hip_conv2d_pool2(ok, ok, None, ok, 1, 8, 8, 8, 8, 3, 3, 1, 0,
                                      H.CONV_Y_NCHW4) == H.ERR_ARG
    # nothing was launched on the error paths
    H.sync()


def test_conv2d_unknown_flags_rejected():
    lib = H.load()
    x = K.empty(4 * 16 * 16 * 4)
    rc = lib.camel_hip_conv2d(P(x.ptr), P(x.ptr), None, P(x.ptr), 1, 4, 4, 4, 4, 3, 3, 1, 0, 0x4000)
    assert rc == H.ERR_ARG


# ------------------------------------------------------------------ conv2d..maxpool2d

POOL_GEOMS = [
    (3, 32, 26, 26, 64, 3, 3, 1, 0),    # CNN conv2 + pool (24 -> 12)
    (2, 32, 27, 25, 64, 3, 3, 1, 0),    # odd conv output (25 x 23): last row / column dropped
    (2, 16, 12, 12, 130, 3, 3, 1, 1),   # 16-channel stages, Co > 128, pad 1
    (2, 64, 9, 9, 96, 3, 3, 2, 1),      # stride 2 (5 x 5 -> 2 x 2)
    (2, 1, 12, 12, 8, 3, 3, 1, 0),      # direct path: conv to scratch, then the pool kernel
    (2, 12, 10, 10, 24, 3, 3, 1, 1),    # gather path: conv to scratch, then the pool kernel
]


@pytest.mark.parametrize("geom", POOL_GEOMS)
def test_conv2d_pool2_equals_conv_then_maxpool(geom):
    N, Cin, H_, W_, Co, kh, kw, stride, pad = geom
    x = D.normal(0x5600 + Cin, (N, Cin, H_, W_))
    w = D.normal(0x5601 + Co, (Co, Cin, kh, kw)) * F(np.sqrt(2.0 / (kh * kw * Cin)))
    b = D.uniform(0x5602, (Co,), -0.1, 0.1)
    for flags in (H.EPI_BIAS | H.EPI_RELU, 0):
        bb = b if flags else None
        dfull, shape = _conv(x, w, bb, geom, flags)
        OH, OW = shape[2], shape[3]
        dref = K.empty(N * Co * (OH // 2) * (OW // 2) * 4)
        H.call("camel_hip_maxpool2d", P(dfull.ptr), P(dref.ptr), N, Co, OH, OW, 2, 2, 2)
        dy, pshape = _conv(x, w, bb, geom, flags, pooled=True)
        got = K.host(dy, F, pshape)
        np.testing.assert_array_equal(got, K.host(dref, F, pshape))
        # oracle: pool of the oracle conv, within the conv bound (max is 1-Lipschitz)
        ref = O.maxpool2d(O.conv2d(x, w, bb, bool(flags), stride, pad), 2, 2)
        K_ = Cin * kh * kw
        mag = O.maxpool2d(O.conv2d(np.abs(x), np.abs(w), None, False, stride, pad), 2, 2)
        assert np.all(np.abs(got.astype(np.float64) - ref) <= 1e-5 * np.sqrt(K_) * mag + 1e-30)


def test_conv2d_pool2_nan_windows_follow_the_pool_rule():
    # NaN inputs reach some window positions; the fused epilogue keeps
    # maxpool's order (first element, strict '>'), bit for bit.
    geom = (2, 32, 14, 14, 64, 3, 3, 1, 1)
    x = D.normal(0x5700, (2, 32, 14, 14))
    x[0, 3, 5, 6] = np.nan
    x[1, 0, 0, 0] = np.nan
    x[1, 7, 13, 2] = -np.inf
    w = D.normal(0x5701, (64, 32, 3, 3)) * F(0.08)
    b = D.uniform(0x5702, (64,), -0.1, 0.1)
    flags = H.EPI_BIAS | H.EPI_RELU
    dfull, shape = _conv(x, w, b, geom, flags)
    dref = K.empty(2 * 64 * 7 * 7 * 4)
    H.call("camel_hip_maxpool2d", P(dfull.ptr), P(dref.ptr), 2, 64, 14, 14, 2, 2, 2)
    dy, pshape = _conv(x, w, b, geom, flags, pooled=True)
    got, ref = K.host(dy, F, pshape), K.host(dref, F, pshape)
    assert np.isnan(ref).any()
    np.testing.assert_array_equal(got, ref)


def test_conv2d_pool2_nhwc_input_and_errors():
    geom = (3, 32, 26, 26, 64, 3, 3, 1, 0)
    x = D.normal(0x5800, (3, 32, 26, 26))
    w = D.normal(0x5801, (64, 32, 3, 3)) * F(0.08)
    b = D.uniform(0x5802, (64,), -0.1, 0.1)
    flags = H.EPI_BIAS | H.EPI_RELU
    dy, pshape = _conv(x, w, b, geom, flags, pooled=True)
    dy2, _ = _conv(np.ascontiguousarray(x.transpose(0, 2, 3, 1)), w, b, geom,
                   flags | H.CONV_X_NHWC, pooled=True)
    np.testing.assert_array_equal(K.host(dy2, F, pshape), K.host(dy, F, pshape))
    lib = H.load()
    d = K.empty(64)
    assert lib.camel_hip_conv2d_pool2(P(d.ptr), P(d.ptr), None, P(d.ptr), 1, 1, 3, 3, 1, 3, 3, 1, 0,
                                      0) == H.ERR_SHAPE
    assert lib.camel_hip_conv2d_pool2(P(d.ptr), P(d.ptr), None, P(d.ptr), 1, 1, 8, 8, 1, 3, 3, 1, 0,
                                      H.CONV_Y_NHWC) == H.ERR_ARG


def test_conv2d_pool2_large_schedules_match_conv_then_pool():
    # Enough tiles for whole rounds plus a partial round (column band or K
    # split tail); schedule-dependent rounding stays within the conv bound.
    for geom in ((64, 64, 56, 56, 128, 3, 3, 1, 1), (1, 16, 112, 130, 640, 3, 3, 1, 0)):
        N, Cin, H_, W_, Co, kh, kw, stride, pad = geom
        x = D.normal(0x5900 + Cin, (N, Cin, H_, W_))
        w = D.normal(0x5901 + Co, (Co, Cin, kh, kw)) * F(np.sqrt(2.0 / (kh * kw * Cin)))
        b = np.zeros(Co, F)
        flags = H.EPI_BIAS | H.EPI_RELU
        dfull, shape = _conv(x, w, b, geom, flags)
        OH, OW = shape[2], shape[3]
        dref = K.empty(N * Co * (OH // 2) * (OW // 2) * 4)
        H.call("camel_hip_maxpool2d", P(dfull.ptr), P(dref.ptr), N, Co, OH, OW, 2, 2, 2)
        dy, pshape = _conv(x, w, b, geom, flags, pooled=True)
        got, ref = K.host(dy, F, pshape), K.host(dref, F, pshape)
        mag = O.maxpool2d(O.conv2d_images(np.abs(x), np.abs(w), None, False, 0, 1, stride, pad), 2, 2)
        diff = np.abs(got[:1].astype(np.float64) - ref[:1])
        assert np.all(diff <= 2e-5 * np.sqrt(Cin * kh * kw) * mag + 1e-30)
        assert np.all(np.abs(got.astype(np.float64) - ref) <= 1e-3)


@pytest.mark.parametrize("geom", GEOMS + [(2, 64, 9, 9, 96, 3, 3, 2, 1)])
def test_conv2d_packed_weights_change_addressing_only(geom):
    # camel_hip_conv2d_pack_weights gives w as [Co, KH, KW, C]; a conv given
    # CAMEL_CONV_W_PACKED reads it directly on the NHWC GEMM path and unpacks
    # it on the others: the same values either way.
    N, Cin, H_, W_, Co, kh, kw, stride, pad = geom
    x = D.normal(0x5A00 + Cin, (N, Cin, H_, W_))
    w = D.normal(0x5A01 + Co, (Co, Cin, kh, kw)) * F(np.sqrt(2.0 / (kh * kw * Cin)))
    b = D.uniform(0x5A02, (Co,), -0.1, 0.1)
    dw, dwp = K.dev(w), K.empty(w.nbytes)
    H.call("camel_hip_conv2d_pack_weights", P(dw.ptr), P(dwp.ptr), Co, Cin, kh, kw)
    assert np.array_equal(K.host(dwp, F, (Co, kh, kw, Cin)), w.transpose(0, 2, 3, 1))
    epi = H.EPI_BIAS | H.EPI_RELU
    dref, shape = _conv(x, w, b, geom, epi)
    ref = K.host(dref, F, shape)
    wp = K.host(dwp, F, (Co, kh, kw, Cin))
    dy, _ = _conv(x, wp, b, geom, epi | H.CONV_W_PACKED)
    np.testing.assert_array_equal(K.host(dy, F, shape), ref)
    x_nhwc = np.ascontiguousarray(x.transpose(0, 2, 3, 1))
    dy, _ = _conv(x_nhwc, wp, b, geom, epi | H.CONV_W_PACKED | H.CONV_X_NHWC)
    np.testing.assert_array_equal(K.host(dy, F, shape), ref)
    if shape[2] >= 2 and shape[3] >= 2:
        dpool, pshape = _conv(x, w, b, geom, epi, pooled=True)
        dy, _ = _conv(x, wp, b, geom, epi | H.CONV_W_PACKED, pooled=True)
        np.testing.assert_array_equal(K.host(dy, F, pshape), K.host(dpool, F, pshape))


# ------------------------------------------- conv2d..conv2d..maxpool2d in one kernel

def _pair_unfused(x, w1, b1, w2, b2, f1, f2):
    N, _, H_, W_ = x.shape
    C1, Co2 = w1.shape[0], w2.shape[0]
    dx, dw1, dw2 = K.dev(x), K.dev(w1), K.dev(w2)
    db1 = K.dev(b1) if b1 is not None else None
    db2 = K.dev(b2) if b2 is not None else None
    h = K.empty(N * C1 * (H_ - 2) * (W_ - 2) * 4)
    H.call("camel_hip_conv2d", P(dx.ptr), P(dw1.ptr), P(db1.ptr) if db1 else None, P(h.ptr), N, 1,
           H_, W_, C1, 3, 3, 1, 0, f1 | H.CONV_Y_NCHW4)
    OH, OW = (H_ - 4) // 2, (W_ - 4) // 2
    y = K.empty(N * Co2 * OH * OW * 4)
    H.call("camel_hip_conv2d_pool2", P(h.ptr), P(dw2.ptr), P(db2.ptr) if db2 else None, P(y.ptr),
           N, C1, H_ - 2, W_ - 2, Co2, 3, 3, 1, 0, f2 | H.CONV_X_NCHW4)
    return K.host(y, F, (N, Co2, OH, OW))


def _pair_fused(x, w1, b1, w2, b2, f1, f2, packed=False):
    N, _, H_, W_ = x.shape
    C1, Co2 = w1.shape[0], w2.shape[0]
    w2x = np.ascontiguousarray(w2.transpose(0, 2, 3, 1)) if packed else w2
    dx, dw1, dw2 = K.dev(x), K.dev(w1), K.dev(w2x)
    db1 = K.dev(b1) if b1 is not None else None
    db2 = K.dev(b2) if b2 is not None else None
    OH, OW = (H_ - 4) // 2, (W_ - 4) // 2
    y = K.empty(N * Co2 * OH * OW * 4)
    H.call("camel_hip_conv2d_pair_pool2", P(dx.ptr), P(dw1.ptr), P(db1.ptr) if db1 else None,
           P(dw2.ptr), P(db2.ptr) if db2 else None, P(y.ptr), N, H_, W_, C1, Co2, f1,
           f2 | (H.CONV_W_PACKED if packed else 0))
    return K.host(y, F, (N, Co2, OH, OW))


@pytest.mark.parametrize("N,H_,Co2,f1,f2", [
    (512, 28, 64, H.EPI_BIAS | H.EPI_RELU, H.EPI_BIAS | H.EPI_RELU),
    (3, 28, 64, H.EPI_RELU, H.EPI_RELU),
    (7, 36, 128, H.EPI_BIAS | H.EPI_RELU, H.EPI_BIAS),                  # taller images, 2 M tiles
    (2, 12, 64, 0, 0),
])
def test_conv_pair_pool_equals_the_two_conv_calls(N, H_, Co2, f1, f2):
    x = D.uniform(0x5B00 + N, (N, 1, H_, 28), 0.0, 1.0)
    w1 = D.normal(0x5B01, (32, 1, 3, 3), std=float(np.sqrt(2.0 / 9)))
    w2 = D.normal(0x5B02 + Co2, (Co2, 32, 3, 3), std=float(np.sqrt(2.0 / 288)))
    b1 = D.uniform(0x5B03, (32,), -0.1, 0.1)
    b2 = D.uniform(0x5B04, (Co2,), -0.1, 0.1)
    bb1 = b1 if f1 & H.EPI_BIAS else None
    bb2 = b2 if f2 & H.EPI_BIAS else None
    want = _pair_unfused(x, w1, bb1, w2, bb2, f1, f2)
    for packed in (False, True):
        got = _pair_fused(x, w1, bb1, w2, bb2, f1, f2, packed)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"packed={packed}"
    # and the oracle on the first image
    h = O.conv2d_images(x, w1, bb1, bool(f1 & H.EPI_RELU), 0, 1)
    ref = O.maxpool2d(O.conv2d(h, w2, bb2, bool(f2 & H.EPI_RELU)), 2, 2)
    assert np.max(np.abs(got[:1] - ref)) <= 1e-4 * max(1.0, float(np.abs(ref).max()))
