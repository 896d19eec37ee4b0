"""Composed layer chains on the GPU: x -> chain equals the layer-by-layer
operator calls (tensor:dense_relu, tensor:conv2d_relu, tensor:maxpool2d, ...)
that the chain stands for.  The fused groups compute the same values, so
the comparison is bit for bit (the pooled convolution included: at these
sizes it runs as one launch of one tile shape, so every output sums in the
same order).  The layer-by-layer results are pinned against the oracle by
tests/test_gpu_operators.py and tests/test_gpu_fusion.py."""
import numpy as np
import pytest

from camel_amd import datagen as D
from camel_amd import tensor as T
from oracle import ffi as O

pytestmark = pytest.mark.gpu

F = np.float32


@pytest.fixture(autouse=True)
def _release():
    yield
    T.release_all()


def t(a):
    return T.Tensor.from_numpy(np.asarray(a))


def test_mlp_chain_equals_layer_calls():
    # README.md:40-46: the benchmark MLP at batch 256
    dims = [784, 1024, 1024, 10]
    x = D.uniform(0x6000, (256, 784), 0.0, 1.0)
    ws = [t(D.normal(0x6001 + i, (dims[i], dims[i + 1]), std=float(np.sqrt(1.0 / dims[i]))))
          for i in range(3)]
    bs = [t(D.uniform(0x6005 + i, (dims[i + 1],), -0.1, 0.1)) for i in range(3)]
    chain = T.Chain(("dense", ws[0], bs[0]), "relu", ("dense", ws[1], bs[1]), "relu",
                    ("dense", ws[2], bs[2]), "softmax")
    assert chain.plan((256, 784)) == ["dense_relu", "dense_relu+dense+softmax"]
    xt = t(x)
    got = chain(xt)
    h = T.call("dense_relu", xt, with_=(ws[0], bs[0]))
    h = T.call("dense_relu", h, with_=(ws[1], bs[1]))
    h = T.call("dense", h, with_=(ws[2], bs[2]))
    ref = T.call("softmax", h)
    assert got.shape == (256, 10)
    # the chain's output is a device tensor like any operator result
    assert got.residency() == (False, True)
    np.testing.assert_array_equal(got.numpy(), ref.numpy())
    p = O.softmax_rows(h.numpy())
    assert np.max(np.abs(got.numpy() - p) / np.maximum(p, 1e-30)) <= 1e-6
    chain.release()


def test_mlp_chain_full_batch_against_the_oracle():
    # BASELINE config 2 at its full batch (1024): every row a probability
    # vector, and rows from the first, a middle and the last tile row within
    # 1e-4 of the oracle's dense layers and softmax (device and oracle logits
    # differ by the GEMM bound, about 1e-6 here, and a softmax output moves by
    # no more than its largest input change).
    dims = [784, 1024, 1024, 10]
    x = D.uniform(D.SEED_MLP, (1024, 784), 0.0, 1.0)
    wn = [D.normal(D.SEED_MLP + 1 + i, (dims[i], dims[i + 1]), std=float(np.sqrt(1.0 / dims[i])))
          for i in range(3)]
    bn = [D.uniform(0x6800 + i, (dims[i + 1],), -0.05, 0.05) for i in range(3)]
    ws, bs = [t(w) for w in wn], [t(b) for b in bn]
    chain = T.Chain(("dense_relu", ws[0], bs[0]), ("dense_relu", ws[1], bs[1]),
                    ("dense", ws[2], bs[2]), "softmax")
    got = chain(t(x)).numpy()
    np.testing.assert_allclose(got.sum(axis=1, dtype=np.float64), 1.0, rtol=0, atol=1e-5)
    for r0, r1 in ((0, 4), (510, 514), (1020, 1024)):
        h = x[r0:r1]
        for i in range(2):
            h = O.dense(h, wn[i], bn[i], True)
        logits = O.dense(h, wn[2], bn[2], False)
        p = O.softmax_rows(logits)
        assert np.max(np.abs(got[r0:r1] - p)) <= 1e-4
    chain.release()


def test_cnn_chain_equals_layer_calls():
    # The benchmark small CNN at batch 16: both convs and the pool in one
    # kernel (conv1's output in LDS), the dense head (at 16 rows layer 1 is
    # the skinny kernel: the head runs as two calls); the layer-by-layer
    # calls take the direct conv, the implicit GEMM and the pool kernel
    B = 16
    x = D.uniform(0x6100, (B, 1, 28, 28), 0.0, 1.0)
    w1 = t(D.normal(0x6101, (32, 1, 3, 3), std=float(np.sqrt(2.0 / 9))))
    w2 = t(D.normal(0x6102, (64, 32, 3, 3), std=float(np.sqrt(2.0 / 288))))
    w3 = t(D.normal(0x6103, (9216, 128), std=float(np.sqrt(2.0 / 9216))))
    w4 = t(D.normal(0x6104, (128, 10), std=float(np.sqrt(2.0 / 128))))
    b1, b2 = t(D.uniform(0x6105, (32,), -0.1, 0.1)), t(D.uniform(0x6106, (64,), -0.1, 0.1))
    b3, b4 = t(D.uniform(0x6107, (128,), -0.1, 0.1)), t(D.uniform(0x6108, (10,), -0.1, 0.1))
    chain = T.Chain(("conv2d_relu", w1, b1), ("conv2d_relu", w2, b2), ("maxpool2d", 2, 2),
                    ("reshape", B, 9216), ("dense_relu", w3, b3), ("dense", w4, b4), "softmax")
    assert chain.plan((B, 1, 28, 28)) == [
        "conv2d_relu+conv2d_relu+maxpool2d(2,2)", "reshape", "dense_relu+dense+softmax"]
    xt = t(x)
    got = chain(xt)
    h = T.call("conv2d_relu", xt, with_=(w1, b1))
    h = T.call("conv2d_relu", h, with_=(w2, b2))
    h = T.call("maxpool2d", h, with_=(2, 2))
    h = T.call("reshape", h, [B, 9216])
    h = T.call("dense_relu", h, with_=(w3, b3))
    h = T.call("dense", h, with_=(w4, b4))
    ref = T.call("softmax", h)
    np.testing.assert_array_equal(got.numpy(), ref.numpy())
    chain.release()


def test_cnn_chain_full_batch_against_the_oracle():
    # BASELINE config 5 at its full batch (512), the benchmarked path: NCHW4
    # between the convs, pooled conv2, and the dense head whose second layer
    # adds dense1's 16 K splits.  Every row a probability vector; images 0,
    # 255 and 511 within 1e-4 of the oracle's layers (conv, pool, dense,
    # softmax).
    B = 512
    x = D.uniform(D.SEED_CNN, (B, 1, 28, 28), 0.0, 1.0)
    wn = [D.normal(D.SEED_CNN + 1, (32, 1, 3, 3), std=float(np.sqrt(2.0 / 9))),
          D.normal(D.SEED_CNN + 2, (64, 32, 3, 3), std=float(np.sqrt(2.0 / 288))),
          D.normal(D.SEED_CNN + 3, (9216, 128), std=float(np.sqrt(2.0 / 9216))),
          D.normal(D.SEED_CNN + 4, (128, 10), std=float(np.sqrt(2.0 / 128)))]
    bn = [D.uniform(0x6900 + i, (n,), -0.05, 0.05) for i, n in enumerate((32, 64, 128, 10))]
    w, b = [t(a) for a in wn], [t(a) for a in bn]
    chain = T.Chain(("conv2d_relu", w[0], b[0]), ("conv2d_relu", w[1], b[1]), ("maxpool2d", 2, 2),
                    ("reshape", B, 9216), ("dense_relu", w[2], b[2]), ("dense", w[3], b[3]),
                    "softmax")
    got = chain(t(x)).numpy()
    np.testing.assert_allclose(got.sum(axis=1, dtype=np.float64), 1.0, rtol=0, atol=1e-5)
    for n in (0, 255, 511):
        h = O.conv2d_images(x, wn[0], bn[0], True, n, n + 1)
        h = O.conv2d(h, wn[1], bn[1], True)
        h = O.maxpool2d(h, 2, 2).reshape(1, 9216)
        h = O.dense(h, wn[2], bn[2], True)
        p = O.softmax_rows(O.dense(h, wn[3], bn[3], False))
        assert np.max(np.abs(got[n:n + 1] - p)) <= 1e-4, f"image {n}"
    chain.release()


@pytest.mark.parametrize("M,softmax", [(96, True), (200, False)])
def test_dense_head_chain_from_split_partials_equals_layer_calls(M, softmax):
    # The CNN's classifier head at 96 / 200 rows (ragged 64x64 tiles, 36 / 32
    # K splits): layer 2's kernel rebuilds layer 1's rows from the partials.
    x = t(D.uniform(0x6600 + M, (M, 9216), 0.0, 1.0))
    w1 = t(D.normal(0x6601, (9216, 128), std=float(np.sqrt(2.0 / 9216))))
    w2 = t(D.normal(0x6602, (128, 10), std=float(np.sqrt(2.0 / 128))))
    b1, b2 = t(D.uniform(0x6603, (128,), -0.1, 0.1)), t(D.uniform(0x6604, (10,), -0.1, 0.1))
    layers = [("dense_relu", w1, b1), ("dense", w2, b2)] + (["softmax"] if softmax else ["relu"])
    chain = T.Chain(*layers)
    assert chain.plan((M, 9216)) == ["dense_relu+dense+softmax" if softmax else "dense_relu+dense_relu"]
    got = chain(x)
    h = T.call("dense_relu", x, with_=(w1, b1))
    h = T.call("dense", h, with_=(w2, b2))
    ref = T.call("softmax" if softmax else "relu", h)
    np.testing.assert_array_equal(got.numpy(), ref.numpy())
    chain.release()


def test_dense_head_chain_errors_match_the_failing_layer():
    x = t(D.uniform(0x6700, (40, 8), -1.0, 1.0))
    w1 = t(D.normal(0x6701, (8, 6), std=0.3))
    bad_w2 = t(np.zeros((7, 3), F))
    chain = T.Chain(("dense_relu", w1), ("dense", bad_w2), "softmax")
    assert chain.plan((40, 8)) == ["dense_relu+dense+softmax"]
    with pytest.raises(T.CamelError, match="dense dimension mismatch"):
        chain(x)
    w2 = t(np.zeros((6, 3), F))
    bad_b2 = t(np.zeros((4,), F))
    chain2 = T.Chain(("dense_relu", w1), ("dense", w2, bad_b2))
    with pytest.raises(T.CamelError, match=r"dense bias must have shape \[N\] or \[1, N\]"):
        chain2(x)
    with pytest.raises(T.CamelError, match="dense dimension mismatch"):
        chain2(t(np.zeros((40, 5), F)))  # layer 1's error comes first
    for c in (chain, chain2):
        c.release()


def test_dense_head_chain_int64_follows_the_composition():
    x = t((np.arange(20).reshape(5, 4) - 7).astype(np.int64))
    w1 = t((np.arange(12).reshape(4, 3) % 4 - 1).astype(np.int64))
    w2 = t((np.arange(6).reshape(3, 2) % 3).astype(np.int64))
    chain = T.Chain(("dense_relu", w1), ("dense", w2), "softmax")
    assert chain.plan((5, 4)) == ["dense_relu+dense+softmax"]
    got = chain(x)
    ref = T.call("softmax", T.call("dense", T.call("dense_relu", x, with_=(w1,)), with_=(w2,)))
    assert got.dtype_code == ref.dtype_code
    np.testing.assert_array_equal(got.numpy(), ref.numpy())
    chain.release()


def test_conv_chain_with_padding_stride_and_three_convs():
    # conv -> conv -> conv through two NCHW4 intermediates, then a 3x3 pool
    x = D.normal(0x6200, (3, 3, 20, 18))
    ws = [t(D.normal(0x6201, (32, 3, 3, 3)) * F(0.2)), t(D.normal(0x6202, (48, 32, 3, 3)) * F(0.06)),
          t(D.normal(0x6203, (16, 48, 1, 1)) * F(0.15))]
    bs = [t(D.uniform(0x6204 + i, (n,), -0.1, 0.1)) for i, n in enumerate((32, 48, 16))]
    chain = T.Chain(("conv2d_relu", ws[0], bs[0], 1, 1), ("conv2d", ws[1], bs[1], 2, 1), "relu",
                    ("conv2d_relu", ws[2], bs[2]), ("maxpool2d", 3, 2))
    assert chain.plan((3, 3, 20, 18)) == [
        "conv2d_relu y=nchw4", "conv2d_relu x=nchw4 y=nchw4", "conv2d_relu x=nchw4", "maxpool2d(3,2)"]
    xt = t(x)
    got = chain(xt)
    h = T.call("conv2d_relu", xt, with_=(ws[0], bs[0], 1, 1))
    h = T.call("conv2d", h, with_=(ws[1], bs[1], 2, 1))
    h = T.call("relu", h)
    h = T.call("conv2d_relu", h, with_=(ws[2], bs[2]))
    ref = T.call("maxpool2d", h, with_=(3, 2))
    assert got.shape == ref.shape
    np.testing.assert_array_equal(got.numpy(), ref.numpy())
    chain.release()


def test_chain_errors_match_the_failing_layer():
    x = t(D.uniform(0x6300, (4, 8), -1.0, 1.0))
    chain = T.Chain(("dense", t(np.zeros((9, 3), F))), "softmax")
    with pytest.raises(T.CamelError, match="dense dimension mismatch"):
        chain(x)
    conv = T.Chain(("conv2d", t(np.zeros((4, 2, 3, 3), F))), ("maxpool2d", 2, 2))
    with pytest.raises(T.CamelError, match="conv2d channel mismatch"):
        conv(t(np.zeros((1, 3, 8, 8), F)))
    with pytest.raises(T.CamelError, match="maxpool2d window larger than input"):
        conv(t(np.zeros((1, 2, 4, 3), F)))
    w = t(np.zeros((8, 3), F))
    dangling = T.Chain(("dense", w))
    w.release()
    with pytest.raises(T.CamelError, match="chain layer weights were released"):
        dangling(x)
    for c in (chain, conv, dangling):
        c.release()


def test_empty_and_single_layer_chains():
    x = t(D.uniform(0x6400, (5, 7), -1.0, 1.0))
    same = T.Chain()(x)
    np.testing.assert_array_equal(same.numpy(), x.numpy())
    r = T.Chain("relu")(x)
    np.testing.assert_array_equal(r.numpy(), T.call("relu", x).numpy())


def test_chain_int64_dense_and_softmax_follow_the_composition():
    # non-Float32 operands: dense runs matmul + add through the device
    # composition, then the softmax composition, as the layer calls do
    x = t((np.arange(12).reshape(4, 3) - 5).astype(np.int64))
    w = t((np.arange(6).reshape(3, 2) % 3).astype(np.int64))
    chain = T.Chain(("dense", w), "softmax")
    assert chain.plan((4, 3)) == ["dense+softmax"]
    got = chain(x)
    ref = T.call("softmax", T.call("dense", x, with_=(w,)))
    assert got.dtype_code == ref.dtype_code
    np.testing.assert_array_equal(got.numpy(), ref.numpy())
    chain.release()


def test_conv_chain_without_nchw4_consumer_and_empty_batch():
    # second conv has C % 16 != 0: NCHW between them; and a batch of 0
    w1 = t(D.normal(0x6500, (12, 3, 3, 3)) * F(0.2))
    w2 = t(D.normal(0x6501, (8, 12, 3, 3)) * F(0.1))
    chain = T.Chain(("conv2d_relu", w1), ("conv2d", w2, None, 1, 1), ("maxpool2d", 2, 2))
    assert chain.plan((2, 3, 10, 10)) == ["conv2d_relu", "conv2d+maxpool2d(2,2)"]
    x = t(D.normal(0x6502, (2, 3, 10, 10)))
    got = chain(x)
    h = T.call("conv2d_relu", x, with_=(w1,))
    h = T.call("conv2d", h, with_=(w2, None, 1, 1))
    ref = T.call("maxpool2d", h, with_=(2, 2))
    np.testing.assert_array_equal(got.numpy(), ref.numpy())
    empty = chain(t(np.zeros((0, 3, 10, 10), F)))
    assert empty.shape == (0, 8, 4, 4)
    chain.release()
