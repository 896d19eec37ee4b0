"""Composed layer chains (the object a compose `..` over tensor layers builds;
the reference's compose is a stub, src/builtin/operators/macro.cpp:30): the
fusion plan and the argument checks, on the CPU.  Planning reads only shapes,
so no device is needed; tests/test_gpu_chain.py runs the chains."""
import numpy as np
import pytest

from camel_amd import tensor as T

F = np.float32


@pytest.fixture(autouse=True)
def _release():
    yield
    T.release_all()


def z(*shape):
    return T.Tensor.from_numpy(np.zeros(shape, F))


def cnn_chain(c1=1, c2=32, c3=64):
    return T.Chain(("conv2d", z(c2, c1, 3, 3), z(c2)), "relu",
                   ("conv2d_relu", z(c3, c2, 3, 3), z(c3)), ("maxpool2d", 2, 2),
                   ("reshape", 512, c3 * 144), ("dense_relu", z(c3 * 144, 128), z(128)),
                   ("dense", z(128, 10), z(10)), "softmax")


def test_cnn_chain_plan_fuses_every_pair():
    # The benchmark small CNN as a chain: both convs, their relus and the pool
    # are one kernel (conv1's output stays in LDS), and the two dense layers
    # with the softmax one head.
    assert cnn_chain().plan((512, 1, 28, 28)) == [
        "conv2d_relu+conv2d_relu+maxpool2d(2,2)", "reshape", "dense_relu+dense+softmax"]
    # Shapes the fused pair does not serve keep the NCHW4 hand-off: a 32-wide
    # image, 16 conv1 channels, or 96 conv2 channels.
    assert T.Chain(("conv2d", z(32, 1, 3, 3), z(32)), "relu",
                   ("conv2d_relu", z(64, 32, 3, 3), z(64)), ("maxpool2d", 2, 2)).plan(
        (8, 1, 28, 32)) == ["conv2d_relu y=nchw4", "conv2d_relu+maxpool2d(2,2) x=nchw4"]
    assert cnn_chain(c2=16, c3=64).plan((8, 1, 28, 28))[:2] == [
        "conv2d_relu y=nchw4", "conv2d_relu+maxpool2d(2,2) x=nchw4"]
    assert T.Chain(("conv2d_relu", z(32, 1, 3, 3)), ("conv2d_relu", z(96, 32, 3, 3)),
                   ("maxpool2d", 2, 2)).plan((8, 1, 28, 28)) == [
        "conv2d_relu y=nchw4", "conv2d_relu+maxpool2d(2,2) x=nchw4"]
    # without the pool the pair is not fused either
    assert T.Chain(("conv2d_relu", z(32, 1, 3, 3)), ("conv2d_relu", z(64, 32, 3, 3))).plan(
        (8, 1, 28, 28)) == ["conv2d_relu y=nchw4", "conv2d_relu x=nchw4"]


def test_mlp_chain_plan():
    # README.md:40-46: dense<w1, b1>..relu.., dense<w3, b3>..softmax
    c = T.Chain(("dense", z(784, 1024), z(1024)), "relu", ("dense", z(1024, 1024), z(1024)),
                "relu", ("dense", z(1024, 10), z(10)), "softmax")
    assert c.plan((1024, 784)) == ["dense_relu", "dense_relu+dense+softmax"]
    c = T.Chain(("dense_relu", z(8, 4)), "softmax")
    assert c.plan((2, 8)) == ["dense_relu+softmax"]
    # a head needs a second dense of at most 16 columns; its relu and the
    # softmax are optional
    c = T.Chain(("dense", z(8, 6)), ("dense", z(6, 17)), "softmax")
    assert c.plan((2, 8)) == ["dense", "dense+softmax"]
    c = T.Chain(("dense", z(8, 6)), ("dense", z(6, 16)), "relu")
    assert c.plan((2, 8)) == ["dense+dense_relu"]
    c = T.Chain(("dense_relu", z(8, 6)), ("dense_relu", z(6, 3)), "softmax", "relu")
    assert c.plan((2, 8)) == ["dense_relu+dense_relu+softmax", "relu"]


W = "w"  # a weight tensor of the given shape, made inside the test


@pytest.mark.parametrize("layers,shape,plan", [
    # consumer with C % 16 != 0 takes the NCHW gather path: no NCHW4 intermediate
    ([("conv2d", (W, 12, 3, 3, 3)), ("conv2d", (W, 8, 12, 3, 3))], (2, 3, 9, 9),
     ["conv2d", "conv2d"]),
    # consumer 1x1 over 16 channels is a direct conv (K = 16 <= 32): NCHW
    ([("conv2d", (W, 16, 1, 3, 3)), ("conv2d", (W, 8, 16, 1, 1))], (2, 1, 9, 9),
     ["conv2d", "conv2d"]),
    # a relu between two convs joins the first; three convs chain NCHW4 twice
    ([("conv2d", (W, 32, 1, 3, 3)), "relu", ("conv2d", (W, 32, 32, 3, 3)),
      ("conv2d", (W, 16, 32, 3, 3))],
     (2, 1, 12, 12), ["conv2d_relu y=nchw4", "conv2d x=nchw4 y=nchw4", "conv2d x=nchw4"]),
    # an NCHW4 intermediate needs the producer's Co % 4 == 0 (here 18: the
    # consumer then fails on its channel count, as the layer call would)
    ([("conv2d", (W, 18, 1, 3, 3)), ("conv2d", (W, 8, 16, 3, 3))], (2, 1, 9, 9),
     ["conv2d", "conv2d"]),
    # a pool that is not 2x2 stride 2 stays its own kernel
    ([("conv2d_relu", (W, 16, 16, 3, 3)), ("maxpool2d", 3, 2)], (1, 16, 9, 9),
     ["conv2d_relu", "maxpool2d(3,2)"]),
    ([("conv2d_relu", (W, 16, 16, 3, 3)), ("maxpool2d", 2)], (1, 16, 9, 9),
     ["conv2d_relu+maxpool2d(2,2)"]),
    # a pooled conv writes NCHW (the pool output is the chain's tensor)
    ([("conv2d", (W, 32, 1, 3, 3)), ("maxpool2d", 2, 2), ("conv2d", (W, 8, 32, 3, 3))],
     (2, 1, 14, 14), ["conv2d+maxpool2d(2,2)", "conv2d"]),
    # standalone relu / softmax / pool / reshape
    (["relu", "softmax"], (3, 4), ["relu", "softmax"]),
    ([("maxpool2d", 2, 2), ("reshape", 2, 8)], (2, 2, 4, 4), ["maxpool2d(2,2)", "reshape"]),
])
def test_chain_plans(layers, shape, plan):
    def build(layer):
        if isinstance(layer, str):
            return layer
        return (layer[0],) + tuple(z(*a[1:]) if isinstance(a, tuple) and a[0] == W else a
                                   for a in layer[1:])
    c = T.Chain(*[build(layer) for layer in layers])
    assert c.plan(shape) == plan


def test_chain_append_errors_use_layer_texts():
    with pytest.raises(T.CamelError, match="Unrecognized layer operator: tensor:matmul"):
        T.Chain(("tensor:matmul",))
    with pytest.raises(T.CamelError, match="dense requires weights"):
        T.Chain(("dense",))
    with pytest.raises(T.CamelError, match="conv2d requires weights"):
        T.Chain(("conv2d_relu",))
    with pytest.raises(T.CamelError, match="conv2d requires rank-4"):
        T.Chain(("conv2d", z(3, 3)))
    with pytest.raises(T.CamelError, match="Expected integer argument"):
        T.Chain(("maxpool2d", 2.5))


def test_chain_handles():
    c = T.Chain("relu")
    c.release()
    lib = T.load()
    assert lib.camel_chain_release(c.handle or 12345) == T.ERR_ARG
    out = T.C.c_uint64()
    assert lib.camel_chain_apply(777, 0, T.C.byref(out)) == T.ERR_ARG


def test_plan_follows_the_input_dtype():
    # The fused conv pair serves Float32 inputs only: for an Int64 input plan()
    # lists the per-layer groups that apply() runs, and apply() stops at the
    # first conv with the layer's own error, before any device work.
    c = cnn_chain()
    assert c.plan((512, 1, 28, 28), T.TC_INT64)[:2] == [
        "conv2d_relu y=nchw4", "conv2d_relu+maxpool2d(2,2) x=nchw4"]
    assert c.plan((512, 1, 28, 28), T.TC_BOOL) == c.plan((512, 1, 28, 28), T.TC_INT64)
    # Float64 and Int32 are normalised as tensor creation does (runtime.cpp:553-566)
    assert c.plan((512, 1, 28, 28), T.TC_FLOAT64) == c.plan((512, 1, 28, 28))
    x = T.Tensor.from_numpy(np.zeros((2, 1, 28, 28), np.int64))
    with pytest.raises(T.CamelError, match="conv2d requires Float32 tensors"):
        c(x)
    with pytest.raises(T.CamelError, match="not a tensor dtype"):
        c.plan((512, 1, 28, 28), T.TC_VOID)
