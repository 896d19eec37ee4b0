"""Exact parity at the benchmark shapes: GEMM, dense and conv2d on small-integer
operands, compared bit for bit over the whole output.

Why this discriminates: with integer operands and biases, every product and
every partial sum of a dot product is an integer; when
``sum_k |A_ik| |B_kj| + |bias_j| < 2**24`` for an output (asserted for every
output before a comparison), all of them are exact in fp32, whatever the
summation order -- MFMA k-groups, LDS group sums, K splits, split reduces,
column bands, thin-kernel quarters.  The reference's loop
(modules/tensor/operators.cpp:757-766: fp64 accumulation in k order, then
one rounding to fp32) yields the same exact integer, and so does numpy's
float64 product, which these tests use as the reference at sizes the ijk
oracle cannot finish in seconds (a row slab of the oracle is checked
against it too).  A dropped, doubled or misplaced k term, tile, split or
band moves some output by at least 1, so it fails here, where the general
fp32 bound (1e-5 sqrt(K) sum |A||B|, about 0.66 per element at K = 4096)
could not see it.

Every kernel path of the GEMM and conv entry points is reached at its
benchmark shape (the path each shape takes is named beside it).

Operands in [-2, 2] are exact in bf16 as well, so they cannot tell an fp32
MFMA from one fed narrower operands.  The wide-operand tests therefore give
one operand integers with |x| <= 4095 (12 significant bits: exact in fp32,
rounded in bf16's 8 and in fp16's or tf32's 11) and the other {-1, 0, 1}
with at most 4000 nonzeros per dot product, so sum |a||b| + |bias| < 2**24
still holds for every output: every product is a wide value or 0, every
partial sum an exact integer, and rounding either operand to a narrower
type moves outputs (tests/test_exact_operands.py shows that on the CPU for
bf16, fp16 and tf32).  The reference widens every fp32 operand to double
exactly (modules/tensor/operators.cpp:757-766), so any narrower operand path
fails them.
"""
import ctypes as C

import numpy as np
import pytest

from camel_amd import _hip as H
from camel_amd import tensor as T
from oracle import ffi as O
from tests import hipkit as K

pytestmark = pytest.mark.gpu

P = C.c_void_p
F = np.float32
F64 = np.float64
EXACT = 2.0 ** 24


def ints(seed, shape, lo=-2, hi=2):
    """Integers in [lo, hi] as fp32 (seeded)."""
    return np.random.default_rng(seed).integers(lo, hi + 1, size=shape).astype(F)


WIDE = 4095


def wide(seed, shape, lo=-WIDE, hi=WIDE):
    """Integers with up to 12 significant bits as fp32 (seeded)."""
    return ints(seed, shape, lo, hi)


def ternary(seed, shape, k_axis, nnz=4000):
    """Signs +-1 at exactly min(nnz, K) positions of every k-vector along
    k_axis, 0 elsewhere (seeded).  With |a| <= 4095 on the other side and nnz
    <= 4095, every dot product keeps sum |a||b| + 4095 < 2**24."""
    rng = np.random.default_rng(seed)
    keys = rng.random(shape)
    K = shape[k_axis]
    take = min(nnz, K)
    if take == K:
        mask = np.ones(shape, bool)
    else:
        kth = np.partition(keys, take - 1, axis=k_axis).take([take - 1], axis=k_axis)
        mask = keys <= kth
    sign = rng.integers(0, 2, size=shape).astype(F) * 2 - 1
    return (sign * mask).astype(F)


def wide_pair(seed, a_shape, b_shape, wide_side, nnz=4000):
    """(A, B) for C = A.B with the wide operand on wide_side ("A" or "B")."""
    if wide_side == "A":
        return wide(seed, a_shape), ternary(seed + 1, b_shape, 0, nnz)
    return ternary(seed, a_shape, 1, nnz), wide(seed + 1, b_shape)


def relu32(y):
    # x * (x > 0) in fp32: negatives become -0.0, as the reference idiom does
    return y * (y > 0).astype(F)


def exact_dense(a, b, bias=None, relu=False):
    """A.B (+bias) (relu) in float64 (exact for these operands), rounded once."""
    mag = np.abs(a).astype(F64) @ np.abs(b).astype(F64)
    c = a.astype(F64) @ b.astype(F64)
    if bias is not None:
        mag += np.abs(bias).astype(F64)
        c += bias.astype(F64)
    assert mag.max(initial=0.0) < EXACT, "operands too large for exact fp32 partial sums"
    y = c.astype(F)
    return relu32(y) if relu else y


def exact_conv(x, w, bias=None, stride=1, pad=0, relu=False):
    """conv2d NCHW in float64, as a sum over (kh, kw) of channel contractions."""
    N, Cin, H_, W_ = x.shape
    Co, _, kh, kw = w.shape
    OH, OW = (H_ + 2 * pad - kh) // stride + 1, (W_ + 2 * pad - kw) // stride + 1
    xp = np.zeros((N, Cin, H_ + 2 * pad, W_ + 2 * pad), F64)
    xp[:, :, pad:pad + H_, pad:pad + W_] = x
    acc = np.zeros((Co, N, OH, OW), F64)
    mag = np.zeros((Co, N, OH, OW), F64)
    for i in range(kh):
        for j in range(kw):
            patch = xp[:, :, i:i + stride * (OH - 1) + 1:stride, j:j + stride * (OW - 1) + 1:stride]
            wij = w[:, :, i, j].astype(F64)
            acc += np.tensordot(wij, patch, axes=([1], [1]))
            mag += np.tensordot(np.abs(wij), np.abs(patch), axes=([1], [1]))
    acc = acc.transpose(1, 0, 2, 3)
    mag = mag.transpose(1, 0, 2, 3)
    if bias is not None:
        acc = acc + bias.astype(F64)[None, :, None, None]
        mag = mag + np.abs(bias).astype(F64)[None, :, None, None]
    assert mag.max(initial=0.0) < EXACT, "operands too large for exact fp32 partial sums"
    y = np.ascontiguousarray(acc).astype(F)
    return relu32(y) if relu else y


def pool2(y):
    # the oracle's 2x2 / stride 2 pool: the window's first element, replaced
    # only by a strictly greater one, so a -0.0 / +0.0 tie keeps the first
    return O.maxpool2d(y, 2, 2)


def assert_bits(got, want, what=""):
    assert got.shape == want.shape, (got.shape, want.shape)
    g, w = got.view(np.uint32), want.view(np.uint32)
    bad = np.flatnonzero(g.reshape(-1) != w.reshape(-1))
    assert bad.size == 0, (f"{what}: {bad.size} of {g.size} outputs differ; first at flat index "
                           f"{bad[0]}: got {got.reshape(-1)[bad[0]]} want {want.reshape(-1)[bad[0]]}")


def nchw4(a):
    n, c, h, w = a.shape
    return np.ascontiguousarray(a.reshape(n, c // 4, 4, h, w).transpose(0, 1, 3, 4, 2))


def from_nchw4(a):
    n, q, h, w, _ = a.shape
    return np.ascontiguousarray(a.transpose(0, 1, 4, 2, 3).reshape(n, 4 * q, h, w))


# --------------------------------------------------------------------- GEMM

GEMM_SHAPES = [
    # M, N, K, epilogue, path
    (256, 256, 256, 0, "config 1: 32x32 tiles, four k-groups, K splits"),
    (1024, 1024, 1024, 3, "64x64 tiles with two k-groups, one tile per CU"),
    (1024, 1024, 784, 3, "MLP layer 1: 64x64 tiles, ragged first K stage"),
    (2048, 2048, 2048, 0, "128x128 tiles, one round: 8 waves in two k-groups"),
    (2000, 2100, 1000, 3, "128x128 two-k-group tiles, ragged edges, K % 64 = 40"),
    (2048, 4096, 2048, 0, "128x128 tiles, two rounds: 4 waves"),
    (4096, 4096, 20, 3, "256x256 tiles, K < BK: one ragged stage, guarded loop"),
    (4096, 4096, 40, 0, "256x256 tiles, a ragged stage then a whole one read again"),
    (2048, 2048, 40, 3, "two-k-group 128x128 tiles, K < BK: one ragged stage"),
    (2048, 2048, 100, 0, "two-k-group 128x128 tiles, ragged stage + one whole stage"),
    (4096, 4096, 4096, 0, "headline: 8-wave 256x256 tiles, one round, XCD remap"),
    (8192, 8192, 8192, 0, "256x256 tiles, four rounds"),
    (4352, 4352, 512, 3, "256x256 whole round + K-split tail + ordered reduce"),
    (512, 33024, 256, 3, "256x256 whole round + column band of small tiles"),
    (512, 128, 9216, 3, "CNN dense1: 64x64 tiles, 16 K splits, XCD remap over splits"),
    (200, 72, 1000, 1, "32x32 tiles with K splits"),
    (2048, 2048, 1001, 0, "128x128 tiles, odd K: scalar A loads"),
    (1000, 1003, 777, 3, "ragged M, N and K, scalar B loads"),
    (16, 4096, 4096, 0, "skinny M = 16: streaming kernel, 4 chunks per work-group"),
    (32, 4096, 4096, 3, "skinny M = 32: two 16-row groups"),
    (8, 2048, 8192, 3, "skinny M < 16: rows past M read as zero"),
    (16, 4094, 1000, 3, "skinny with N % 4 != 0: 32x128 MFMA tiles"),
    (1024, 10, 1024, 3, "MLP layer 3: thin kernel, 16-wave rows, N <= 16"),
    (512, 10, 128, 1, "CNN dense2: thin kernel"),
    (2000, 32, 512, 3, "thin kernel, 16 < N <= 32"),
]


@pytest.mark.parametrize("M,N,Kd,epi,path", GEMM_SHAPES, ids=[s[4].split(":")[0] for s in GEMM_SHAPES])
def test_sgemm_integer_operands_are_exact_at_full_size(M, N, Kd, epi, path):
    print(f"exact sgemm {M}x{N}x{Kd} epi={epi} ({path})", flush=True)
    seed = M * 131 + N * 7 + Kd
    a, b = ints(seed, (M, Kd)), ints(seed + 1, (Kd, N))
    bias = ints(seed + 2, (N,)) if epi & H.EPI_BIAS else None
    want = exact_dense(a, b, bias, bool(epi & H.EPI_RELU))
    got = K.sgemm(a, b, bias, epi)
    assert_bits(got, want, path)
    r = min(M, 4)
    if r * N * Kd <= 3e8:
        # the ijk oracle itself, on its first rows
        ref = O.dense(a[:r], b, bias, bool(epi & H.EPI_RELU))
        assert_bits(ref, want[:r], "oracle slab")


@pytest.mark.parametrize("wide_side", ["A", "B"])
@pytest.mark.parametrize("M,N,Kd,epi,path", GEMM_SHAPES, ids=[s[4].split(":")[0] for s in GEMM_SHAPES])
def test_sgemm_wide_operands_stay_fp32(M, N, Kd, epi, path, wide_side):
    # One operand wide (12-bit integers), the other ternary: bit-exact only
    # if neither operand is narrowed on its way into the MFMA (or FMA).
    print(f"wide sgemm {M}x{N}x{Kd} epi={epi} wide {wide_side} ({path})", flush=True)
    seed = 0xB000 + M * 131 + N * 7 + Kd
    a, b = wide_pair(seed, (M, Kd), (Kd, N), wide_side)
    bias = wide(seed + 2, (N,)) if epi & H.EPI_BIAS else None
    want = exact_dense(a, b, bias, bool(epi & H.EPI_RELU))
    assert_bits(K.sgemm(a, b, bias, epi), want, f"{path}, wide {wide_side}")


def test_sgemm_exact_results_repeat_across_calls():
    # Split partial scratch reused by a second, smaller call (skinny and tiles).
    for M, N, Kd in ((16, 4096, 4096), (16, 1024, 8192), (512, 128, 9216), (200, 72, 1000)):
        a, b = ints(M + Kd, (M, Kd)), ints(N + Kd, (Kd, N))
        want = exact_dense(a, b)
        assert_bits(K.sgemm(a, b), want, f"{M}x{N}x{Kd}")


# ----------------------------------------------------------- fused dense paths

def _dense_head(x, w1, b1, w2, b2, flags1, flags2, softmax):
    M, K1 = x.shape
    N1, N2 = w1.shape[1], w2.shape[1]
    dx, dw1, db1, dw2, db2 = K.dev(x), K.dev(w1), K.dev(b1), K.dev(w2), K.dev(b2)
    dy = K.empty(M * N2 * 4)
    H.call("camel_hip_dense_head", P(dx.ptr), P(dw1.ptr), P(db1.ptr), P(dw2.ptr), P(db2.ptr),
           P(dy.ptr), M, K1, N1, N2, flags1, flags2, softmax)
    return K.host(dy, F, (M, N2))


def softmax_close(got, logits):
    p = O.softmax_rows(logits)
    assert np.max(np.abs(got.astype(F64) - p) / np.maximum(p, 1e-30)) <= 1e-6


def test_dense_head_on_split_partials_is_exact():
    # The CNN head 512x9216 -> 128 (relu) -> 10: layer 2's thin kernel adds
    # layer 1's 16 K-split partials itself.  The logits are exact; the fused
    # softmax is within the softmax bar of the oracle's softmax of them.
    x = ints(0x7000, (512, 9216), 0, 1)
    w1, b1 = ints(0x7001, (9216, 128), -1, 1), ints(0x7002, (128,), -1, 1)
    w2, b2 = ints(0x7003, (128, 10), -1, 1), ints(0x7004, (10,), -1, 1)
    epi = H.EPI_BIAS | H.EPI_RELU
    h = exact_dense(x, w1, b1, True)
    logits = exact_dense(h, w2, b2, False)
    assert_bits(_dense_head(x, w1, b1, w2, b2, epi, H.EPI_BIAS, 0), logits, "head logits")
    assert_bits(_dense_head(x, w1, b1, w2, b2, epi, epi, 0), relu32(logits), "head relu")
    softmax_close(_dense_head(x, w1, b1, w2, b2, epi, H.EPI_BIAS, 1), logits)


def test_dense_softmax_logits_are_exact_before_the_softmax():
    # MLP layer 3 + softmax fused (1024 x 1024 -> 10): against the oracle's
    # softmax of the exact logits.
    x, w, b = ints(0x7010, (1024, 1024), 0, 2), ints(0x7011, (1024, 10)), ints(0x7012, (10,))
    logits = exact_dense(x, w, b, False)
    dx, dw, db = K.dev(x), K.dev(w), K.dev(b)
    dy = K.empty(1024 * 10 * 4)
    H.call("camel_hip_dense_softmax", P(dx.ptr), P(dw.ptr), P(db.ptr), P(dy.ptr), 1024, 10, 1024,
           H.EPI_BIAS)
    softmax_close(K.host(dy, F, (1024, 10)), logits)


# ------------------------------------------------------------------- conv2d

def _conv(x, w, b, geom, flags, pooled=False, x_layout=None, y_nchw4=False):
    N, Cin, H_, W_, Co, kh, kw, stride, pad = geom
    OH, OW = (H_ + 2 * pad - kh) // stride + 1, (W_ + 2 * pad - kw) // stride + 1
    if pooled:
        OH, OW = OH // 2, OW // 2
    if x_layout == "nhwc":
        x = np.ascontiguousarray(x.transpose(0, 2, 3, 1))
    elif x_layout == "nchw4":
        x = nchw4(x)
    dx, dw = K.dev(x), K.dev(w)
    db = K.dev(b) if b is not None else None
    dy = K.empty(N * Co * OH * OW * 4)
    H.call("camel_hip_conv2d_pool2" if pooled else "camel_hip_conv2d", P(dx.ptr), P(dw.ptr),
           P(db.ptr) if db else None, P(dy.ptr), N, Cin, H_, W_, Co, kh, kw, stride, pad, flags)
    if y_nchw4:
        return from_nchw4(K.host(dy, F, (N, Co // 4, OH, OW, 4)))
    return K.host(dy, F, (N, Co, OH, OW))


CONV_CASES = [
    # geometry (N, C, H, W, Co, KH, KW, stride, pad), operand ranges, path
    ((64, 64, 56, 56, 128, 3, 3, 1, 1), (-2, 2), "config 4: NCHW planes loader, column band"),
    ((32, 64, 56, 56, 128, 3, 3, 1, 1), (-2, 2), "whole rounds + K-split tail"),
    ((512, 1, 28, 28, 32, 3, 3, 1, 0), (-2, 2), "CNN conv1: direct kernel, K = 9"),
    ((512, 32, 26, 26, 64, 3, 3, 1, 0), (-1, 1), "CNN conv2: planes loader, 64-row tiles"),
    ((8, 12, 30, 30, 40, 3, 3, 1, 1), (-2, 2), "NCHW gather loader (C % 16 != 0)"),
    ((16, 16, 33, 35, 130, 3, 3, 2, 1), (-2, 2), "16-channel stages, stride 2, Co > 128"),
    ((4, 3, 40, 40, 16, 5, 5, 1, 2), (-2, 2), "gather loader, 5x5 window, pad 2"),
    ((6, 2, 21, 19, 12, 4, 4, 1, 1), (-2, 2), "direct kernel, K = 32"),
]


@pytest.mark.parametrize("geom,rng_,path", CONV_CASES, ids=[c[2].split(":")[0] for c in CONV_CASES])
def test_conv2d_integer_operands_are_exact_at_full_size(geom, rng_, path):
    N, Cin, H_, W_, Co, kh, kw, stride, pad = geom
    print(f"exact conv2d {geom} ({path})", flush=True)
    seed = N * 1000 + Cin * 10 + Co
    x = ints(seed, (N, Cin, H_, W_), *rng_)
    w = ints(seed + 1, (Co, Cin, kh, kw), *rng_)
    b = ints(seed + 2, (Co,), *rng_)
    _conv_every_mode_is_exact(x, w, b, geom, path)


@pytest.mark.parametrize("wide_side", ["x", "w"])
@pytest.mark.parametrize("geom,rng_,path", CONV_CASES, ids=[c[2].split(":")[0] for c in CONV_CASES])
def test_conv2d_wide_operands_stay_fp32(geom, rng_, path, wide_side):
    # One of x and w wide (12-bit integers), the other in {-1, 0, 1}; the
    # GEMM views K = C*KH*KW <= 576, so sum |x||w| + |b| < 2**24.
    N, Cin, H_, W_, Co, kh, kw, stride, pad = geom
    print(f"wide conv2d {geom} wide {wide_side} ({path})", flush=True)
    seed = 0xC000 + N * 1000 + Cin * 10 + Co
    if wide_side == "x":
        x, w = wide(seed, (N, Cin, H_, W_)), ints(seed + 1, (Co, Cin, kh, kw), -1, 1)
    else:
        x, w = ints(seed, (N, Cin, H_, W_), -1, 1), wide(seed + 1, (Co, Cin, kh, kw))
    b = wide(seed + 2, (Co,))
    _conv_every_mode_is_exact(x, w, b, geom, f"{path}, wide {wide_side}")


def _conv_every_mode_is_exact(x, w, b, geom, path):
    N, Cin, H_, W_, Co, kh, kw, stride, pad = geom
    epi = H.EPI_BIAS | H.EPI_RELU
    want = exact_conv(x, w, b, stride, pad, relu=True)
    assert_bits(_conv(x, w, b, geom, epi), want, path)
    # the same values from the other addressing modes
    if Cin % 4 == 0:
        assert_bits(_conv(x, w, b, geom, epi | H.CONV_X_NHWC, x_layout="nhwc"), want, "x NHWC")
        assert_bits(_conv(x, w, b, geom, epi | H.CONV_X_NCHW4, x_layout="nchw4"), want, "x NCHW4")
    if Co % 4 == 0:
        assert_bits(_conv(x, w, b, geom, epi | H.CONV_Y_NCHW4, y_nchw4=True), want, "y NCHW4")
    wp = np.ascontiguousarray(w.transpose(0, 2, 3, 1))
    assert_bits(_conv(x, wp, b, geom, epi | H.CONV_W_PACKED), want, "packed weights")
    if want.shape[2] >= 2 and want.shape[3] >= 2:
        assert_bits(_conv(x, w, b, geom, epi, pooled=True), pool2(want), "pooled")
    if Co * want.shape[2] * want.shape[3] * Cin * kh * kw <= 3e8:
        # the oracle's direct loop on image 0
        ref = O.conv2d_images(x, w, b, True, 0, 1, stride, pad)
        assert_bits(ref, want[:1], "oracle image 0")


def test_cnn_pooled_conv2_from_nchw4_is_exact():
    # The benchmarked CNN group: conv2 reads conv1's NCHW4 output in place
    # with packed weights and stores only the 2x2 pooled values.
    geom = (512, 32, 26, 26, 64, 3, 3, 1, 0)
    x = ints(0x7100, (512, 32, 26, 26), 0, 2)
    w = ints(0x7101, (64, 32, 3, 3), -1, 1)
    b = ints(0x7102, (64,), -1, 1)
    want = pool2(exact_conv(x, w, b, 1, 0, relu=True))
    wp = np.ascontiguousarray(w.transpose(0, 2, 3, 1))
    flags = H.EPI_BIAS | H.EPI_RELU | H.CONV_X_NCHW4 | H.CONV_W_PACKED
    assert_bits(_conv(x, wp, b, geom, flags, pooled=True, x_layout="nchw4"), want, "pooled conv2")


def test_conv_pair_pool_kernel_is_exact():
    # camel_hip_conv2d_pair_pool2 at BASELINE config 5's shape: conv1 into LDS,
    # conv2 from it, the 2x2 pool, against the exact result.
    x = ints(0x7150, (512, 1, 28, 28), 0, 1)
    w1, b1 = ints(0x7151, (32, 1, 3, 3), -1, 1), ints(0x7152, (32,), -1, 1)
    w2, b2 = ints(0x7153, (64, 32, 3, 3), -1, 1), ints(0x7154, (64,), -1, 1)
    want = pool2(exact_conv(exact_conv(x, w1, b1, relu=True), w2, b2, relu=True))
    dx, dw1, db1, dw2, db2 = K.dev(x), K.dev(w1), K.dev(b1), K.dev(w2), K.dev(b2)
    dy = K.empty(want.nbytes)
    epi = H.EPI_BIAS | H.EPI_RELU
    H.call("camel_hip_conv2d_pair_pool2", P(dx.ptr), P(dw1.ptr), P(db1.ptr), P(dw2.ptr),
           P(db2.ptr), P(dy.ptr), 512, 28, 28, 32, 64, epi, epi)
    assert_bits(K.host(dy, F, want.shape), want, "conv pair + pool")


# ------------------------------------------------------------- layer chains

@pytest.fixture
def _release():
    yield
    T.release_all()


def t(a):
    return T.Tensor.from_numpy(np.asarray(a))


def test_mlp_chain_full_batch_is_exact(_release):
    # BASELINE config 2's shapes (1024 x 784 -> 1024 -> 1024 -> 10) through
    # the fused chain: the logits exactly, then the softmax within its bar
    # for every row.
    dims = [784, 1024, 1024, 10]
    x = ints(0x7200, (1024, 784), 0, 1)
    wn = [ints(0x7201 + i, (dims[i], dims[i + 1]), -1, 1) for i in range(3)]
    bn = [ints(0x7205 + i, (dims[i + 1],), -1, 1) for i in range(3)]
    h = exact_dense(x, wn[0], bn[0], True)
    h = exact_dense(h, wn[1], bn[1], True)
    logits = exact_dense(h, wn[2], bn[2], False)
    ws, bs = [t(w) for w in wn], [t(b) for b in bn]
    head = T.Chain(("dense_relu", ws[0], bs[0]), ("dense_relu", ws[1], bs[1]), ("dense", ws[2], bs[2]))
    assert_bits(head(t(x)).numpy(), logits, "MLP logits")
    full = T.Chain(("dense_relu", ws[0], bs[0]), ("dense_relu", ws[1], bs[1]),
                   ("dense", ws[2], bs[2]), "softmax")
    softmax_close(full(t(x)).numpy(), logits)
    head.release()
    full.release()


def test_cnn_chain_full_batch_is_exact(_release):
    # BASELINE config 5's shapes at batch 512 through the fused chain (conv1
    # into LDS -> conv2 -> pool in one kernel, dense head on split partials):
    # the logits exactly, then the softmax within its bar, for all 512 images.
    x = ints(0x7300, (512, 1, 28, 28), 0, 1)
    w1, b1 = ints(0x7301, (32, 1, 3, 3), -1, 1), ints(0x7302, (32,), -1, 1)
    w2, b2 = ints(0x7303, (64, 32, 3, 3), -1, 1), ints(0x7304, (64,), -1, 1)
    w3, b3 = ints(0x7305, (9216, 128), -1, 1), ints(0x7306, (128,), -1, 1)
    w4, b4 = ints(0x7307, (128, 10), -1, 1), ints(0x7308, (10,), -1, 1)
    h = exact_conv(x, w1, b1, relu=True)
    h = pool2(exact_conv(h, w2, b2, relu=True)).reshape(512, 9216)
    h = exact_dense(h, w3, b3, True)
    logits = exact_dense(h, w4, b4, False)
    tw = [t(a) for a in (w1, b1, w2, b2, w3, b3, w4, b4)]
    layers = [("conv2d_relu", tw[0], tw[1]), ("conv2d_relu", tw[2], tw[3]), ("maxpool2d", 2, 2),
              ("reshape", 512, 9216), ("dense_relu", tw[4], tw[5]), ("dense", tw[6], tw[7])]
    head = T.Chain(*layers)
    assert head.plan((512, 1, 28, 28))[:2] == ["conv2d_relu+conv2d_relu+maxpool2d(2,2)",
                                               "reshape"]
    assert_bits(head(t(x)).numpy(), logits, "CNN logits")
    full = T.Chain(*layers, "softmax")
    softmax_close(full(t(x)).numpy(), logits)
    head.release()
    full.release()


@pytest.mark.parametrize("M,N,Kd", [(16, 4096, 4096), (32, 4096, 8192), (8, 1000, 20000),
                                     (24, 64, 200)])
def test_skinny_split_sums_are_exact_on_every_call(M, N, Kd):
    # The streaming kernel's k partials and their ordered reduce: 40 calls in
    # a row into an output pre-filled with NaN, each bit-exact (a partial read
    # before its writer finished would show up here).
    a, b = ints(M * Kd, (M, Kd)), ints(N + Kd, (Kd, N))
    bias = ints(N, (N,))
    want = exact_dense(a, b, bias, True)
    da, db, dbias = K.dev(a), K.dev(b), K.dev(bias)
    dc = K.empty(M * N * 4)
    for i in range(40):
        H.call("camel_hip_fill", H.DT_F32, P(dc.ptr), M * N, float("nan"))
        H.call("camel_hip_sgemm", P(da.ptr), P(db.ptr), P(dc.ptr), M, N, Kd, P(dbias.ptr),
               H.EPI_BIAS | H.EPI_RELU)
        assert_bits(K.host(dc, F, (M, N)), want, f"call {i}")


# ----------------------------------------- fused paths with wide operands
# Each case makes one operand of one layer wide (12-bit integers, or the wide
# activations a wide layer produces) and keeps every other operand ternary
# and sparse enough that every layer's sum |a||b| + |bias| < 2**24
# (exact_dense / exact_conv assert it), so each layer's operands are pinned
# to fp32 in turn.

def _conv_w(seed, co, c, k, nnz):
    """Ternary conv weights with exactly min(nnz, c*k*k) nonzeros per output channel."""
    return ternary(seed, (co, c * k * k), 1, nnz).reshape(co, c, k, k)


HEAD_WIDE = {
    # x, w1, w2 generators for the CNN head 512x9216 -> 128 (relu) -> 10
    "x": lambda s: (wide(s, (512, 9216)), ternary(s + 1, (9216, 128), 0, 4),
                    ternary(s + 3, (128, 10), 0, 128)),
    "w1": lambda s: (ternary(s, (512, 9216), 1, 40), wide(s + 1, (9216, 128)),
                     ternary(s + 3, (128, 10), 0, 64)),
    "w2": lambda s: (ternary(s, (512, 9216), 1, 4), ternary(s + 1, (9216, 128), 0, 4000),
                     wide(s + 3, (128, 10))),
}


@pytest.mark.parametrize("which", sorted(HEAD_WIDE))
def test_dense_head_wide_operands_stay_fp32(which):
    # camel_hip_dense_head on 16 split partials: layer 1's A or B wide, or
    # layer 2's B wide (layer 2's A, the split sums, is wide in the first two).
    s = 0xD000 + len(which)
    x, w1, w2 = HEAD_WIDE[which](s)
    b1 = ints(s + 2, (128,), -1, 1)
    b2 = wide(s + 4, (10,))
    epi = H.EPI_BIAS | H.EPI_RELU
    h = exact_dense(x, w1, b1, True)
    logits = exact_dense(h, w2, b2, False)
    assert_bits(_dense_head(x, w1, b1, w2, b2, epi, H.EPI_BIAS, 0), logits, f"head, wide {which}")


@pytest.mark.parametrize("wide_side", ["A", "B"])
def test_dense_softmax_wide_operands_stay_fp32(wide_side):
    # MLP layer 3 + softmax fused (1024 x 1024 -> 10): the softmax of the
    # exact logits within the softmax bar.  The logits of wide operands are
    # large, so most rows are near one-hot; the bar still holds per element.
    x, w = wide_pair(0xD100, (1024, 1024), (1024, 10), wide_side)
    b = wide(0xD102, (10,))
    logits = exact_dense(x, w, b, False)
    dx, dw, db = K.dev(x), K.dev(w), K.dev(b)
    dy = K.empty(1024 * 10 * 4)
    H.call("camel_hip_dense_softmax", P(dx.ptr), P(dw.ptr), P(db.ptr), P(dy.ptr), 1024, 10, 1024,
           H.EPI_BIAS)
    softmax_close(K.host(dy, F, (1024, 10)), logits)
    # the logits alone through the thin kernel, bit for bit
    assert_bits(K.sgemm(x, w, b, H.EPI_BIAS), logits, f"classifier, wide {wide_side}")


CONV2_WIDE = {
    # x (conv2's input, NCHW4), w: conv2 of the CNN, 512x32x26x26 -> 64, pooled
    "x": lambda s: (wide(s, (512, 32, 26, 26), 0, WIDE), _conv_w(s + 1, 64, 32, 3, 288)),
    "w": lambda s: (ints(s, (512, 32, 26, 26), 0, 1), wide(s + 1, (64, 32, 3, 3))),
}


@pytest.mark.parametrize("which", sorted(CONV2_WIDE))
def test_cnn_pooled_conv2_wide_operands_stay_fp32(which):
    geom = (512, 32, 26, 26, 64, 3, 3, 1, 0)
    x, w = CONV2_WIDE[which](0xD200 + len(which))
    b = wide(0xD202, (64,))
    want = pool2(exact_conv(x, w, b, 1, 0, relu=True))
    wp = np.ascontiguousarray(w.transpose(0, 2, 3, 1))
    flags = H.EPI_BIAS | H.EPI_RELU | H.CONV_X_NCHW4 | H.CONV_W_PACKED
    assert_bits(_conv(x, wp, b, geom, flags, pooled=True, x_layout="nchw4"), want,
                f"pooled conv2, wide {which}")


PAIR_WIDE = {
    # x, w1, w2 of the fused conv pair (512x1x28x28 -> 32 -> 64, pooled):
    # wide pixels make conv1's output (conv2's B operand) wide; wide w2 is
    # conv2's A operand.
    "x": lambda s: (wide(s, (512, 1, 28, 28)), ints(s + 1, (32, 1, 3, 3), -1, 1),
                    ints(s + 3, (64, 32, 3, 3), -1, 1)),
    "w2": lambda s: (ints(s, (512, 1, 28, 28), 0, 1), ints(s + 1, (32, 1, 3, 3), -1, 1),
                     wide(s + 3, (64, 32, 3, 3))),
}


@pytest.mark.parametrize("which", sorted(PAIR_WIDE))
def test_conv_pair_pool_wide_operands_stay_fp32(which):
    s = 0xD300 + len(which)
    x, w1, w2 = PAIR_WIDE[which](s)
    b1, b2 = ints(s + 2, (32,), -1, 1), wide(s + 4, (64,))
    want = pool2(exact_conv(exact_conv(x, w1, b1, relu=True), w2, b2, relu=True))
    dx, dw1, db1, dw2, db2 = K.dev(x), K.dev(w1), K.dev(b1), K.dev(w2), K.dev(b2)
    dy = K.empty(want.nbytes)
    epi = H.EPI_BIAS | H.EPI_RELU
    H.call("camel_hip_conv2d_pair_pool2", P(dx.ptr), P(dw1.ptr), P(db1.ptr), P(dw2.ptr),
           P(db2.ptr), P(dy.ptr), 512, 28, 28, 32, 64, epi, epi)
    assert_bits(K.host(dy, F, want.shape), want, f"conv pair, wide {which}")


MLP_WIDE = {
    # x, W1, W2, W3 for 1024 x 784 -> 1024 -> 1024 -> 10 (relu, relu, logits)
    # wide activations all the way (layer 1's A, then layers 2 and 3 see
    # 15- and 24-bit activations)
    "x": lambda s: (wide(s, (1024, 784)), ternary(s + 1, (784, 1024), 0, 4),
                    ternary(s + 2, (1024, 1024), 0, 512), ternary(s + 3, (1024, 10), 0, 1)),
    # layer 1's weights wide
    "w1": lambda s: (ints(s, (1024, 784), 0, 1) * ternary(s + 9, (1024, 784), 1, 4) ** 2,
                     wide(s + 1, (784, 1024)), ternary(s + 2, (1024, 1024), 0, 512),
                     ternary(s + 3, (1024, 10), 0, 1)),
    # layer 2's weights wide (its input has entries in {0, 1, 2})
    "w2": lambda s: (ints(s, (1024, 784), 0, 1) * ternary(s + 9, (1024, 784), 1, 2) ** 2,
                     ternary(s + 1, (784, 1024), 0, 784), wide(s + 2, (1024, 1024)),
                     ternary(s + 3, (1024, 10), 0, 1)),
}


@pytest.mark.parametrize("which", sorted(MLP_WIDE))
def test_mlp_chain_wide_operands_stay_fp32(which, _release):
    # BASELINE config 2's shapes through the fused chain, the logits bit for
    # bit, with one layer's operands wide in turn.
    s = 0xD400 + 16 * len(which)
    x, *wn = MLP_WIDE[which](s)
    bn = [ints(s + 5, (1024,), -1, 1), ints(s + 6, (1024,), -1, 1), wide(s + 7, (10,))]
    h = exact_dense(x, wn[0], bn[0], True)
    h = exact_dense(h, wn[1], bn[1], True)
    logits = exact_dense(h, wn[2], bn[2], False)
    ws, bs = [t(w) for w in wn], [t(b) for b in bn]
    head = T.Chain(("dense_relu", ws[0], bs[0]), ("dense_relu", ws[1], bs[1]), ("dense", ws[2], bs[2]))
    assert_bits(head(t(x)).numpy(), logits, f"MLP logits, wide {which}")
    head.release()


CNN_WIDE = {
    # x, w1, w2, w3, w4: wide pixels (conv2's B and dense1's A wide), or wide
    # conv2 weights (conv2's A wide, dense1's A wide)
    "x": lambda s: (wide(s, (512, 1, 28, 28)), ints(s + 1, (32, 1, 3, 3), -1, 1),
                    ints(s + 2, (64, 32, 3, 3), -1, 1), ternary(s + 3, (9216, 128), 0, 1),
                    ternary(s + 4, (128, 10), 0, 1)),
    "w2": lambda s: (ints(s, (512, 1, 28, 28), 0, 1), ints(s + 1, (32, 1, 3, 3), -1, 1),
                     wide(s + 2, (64, 32, 3, 3)), ternary(s + 3, (9216, 128), 0, 1),
                     ternary(s + 4, (128, 10), 0, 1)),
}


@pytest.mark.parametrize("which", sorted(CNN_WIDE))
def test_cnn_chain_wide_operands_stay_fp32(which, _release):
    s = 0xD500 + 16 * len(which)
    x, w1, w2, w3, w4 = CNN_WIDE[which](s)
    b1, b2 = ints(s + 5, (32,), -1, 1), ints(s + 6, (64,), -1, 1)
    b3, b4 = ints(s + 7, (128,), -1, 1), wide(s + 8, (10,))
    h = exact_conv(x, w1, b1, relu=True)
    h = pool2(exact_conv(h, w2, b2, relu=True)).reshape(512, 9216)
    h = exact_dense(h, w3, b3, True)
    logits = exact_dense(h, w4, b4, False)
    tw = [t(a) for a in (w1, b1, w2, b2, w3, b3, w4, b4)]
    head = T.Chain(("conv2d_relu", tw[0], tw[1]), ("conv2d_relu", tw[2], tw[3]), ("maxpool2d", 2, 2),
                   ("reshape", 512, 9216), ("dense_relu", tw[4], tw[5]), ("dense", tw[6], tw[7]))
    assert_bits(head(t(x)).numpy(), logits, f"CNN logits, wide {which}")
    head.release()
