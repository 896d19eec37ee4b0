"""GPU tests of the operator layer: the tensor:* operators run end to end on
the MI355X through libcamel_tensor.so -> libcamel_hip.so and match the CPU
oracle (a restatement of the reference kernels) on the same seeded inputs.

They read like the reference's own NN programs: test/run/nn/tensor_smoke.cml
(closed forms), mnist.cml (the composed softmax), svm.cml (the relu idiom)
and the benchmark MLP / CNN chains built from the layer operators.  They also
check the residency contract: operator outputs stay on the device, and a
chain of operators never copies through the host.
"""
import numpy as np
import pytest

from camel_amd import datagen as D
from camel_amd import tensor as T
from oracle import ffi as O
from tests import hipkit as K

pytestmark = pytest.mark.gpu

F = np.float32


@pytest.fixture(autouse=True)
def _release():
    yield
    T.release_all()


def t(a):
    return T.Tensor.from_numpy(np.asarray(a))


def gemm_ok(got, ref, a, b):
    ok, worst = K.gemm_tol_ok(got, ref, a, b)
    assert ok, f"GEMM tolerance exceeded (worst err/bound {worst:.3g})"


def test_tensor_smoke_closed_forms():
    # test/run/nn/tensor_smoke.cml:8-32
    ones = T.call("ones", [2, 2])
    eye = T.call("eye", 2)
    prod = T.call("matmul", ones, eye)
    assert np.array_equal(prod.numpy(), np.ones((2, 2), F))
    plus = T.call("add", prod, 2.0)
    assert np.array_equal(plus.numpy(), np.full((2, 2), 3.0, F))
    assert T.call("sum", plus) == 12.0
    tr = T.call("transpose", T.call("zeros", [2, 3]))
    assert T.call("shape", tr) == [3, 2]
    r = T.call("reshape", T.call("range", 6), [2, 3])
    assert r.dtype_code == T.TC_INT64 and r.numpy().tolist() == [[0, 1, 2], [3, 4, 5]]
    assert T.call("range", 5, 0, -2).numpy().tolist() == [5, 3, 1]
    assert T.call("full", [2], T.Int32(7)).numpy().tolist() == [7, 7]


def test_matmul_config1_matches_oracle():
    # The 256^3 plumbing case: U(-1,1), seeds 0x5EED0001 / 0x5EED0002.
    a = D.uniform(D.SEED_MATMUL_A, (256, 256), -1.0, 1.0)
    b = D.uniform(D.SEED_MATMUL_B, (256, 256), -1.0, 1.0)
    c = T.call("tensor:matmul", t(a), t(b))
    assert c.residency() == (False, True)
    gemm_ok(c.numpy(), O.matmul(a, b), a, b)


def test_matmul_promotes_and_int_path_is_exact():
    a = np.arange(12, dtype=np.int64).reshape(3, 4) - 5
    b = (np.arange(8, dtype=np.int64).reshape(4, 2) % 3).astype(np.uint8)
    c = T.call("matmul", t(a), t(b))
    assert c.dtype_code == T.TC_INT64
    # a Bool tensor reads as 0/1 (getAsDouble, runtime.cpp:298-310), so 2 counts as 1
    assert np.array_equal(c.numpy(), a @ (b != 0).astype(np.int64))


def test_elementwise_operators_bit_exact_and_errors():
    x = D.uniform(11, (64, 33), -2.0, 2.0)
    y = D.uniform(12, (64, 33), -2.0, 2.0)
    for uri, op in [("add", O.ADD), ("subtract", O.SUB), ("multiply", O.MUL), ("divide", O.DIV)]:
        got = T.call(uri, t(x), t(y)).numpy()
        assert np.array_equal(got.view(np.uint32), O.binary(op, x, y).view(np.uint32)), uri
    # tensor (op) scalar, both sides, one rounding from double
    got = T.call("subtract", 0.1, t(x)).numpy()
    assert np.array_equal(got, O.binary_scalar(O.SUB, x, 0.1, O.F32, side=1))
    z = y.copy()
    z[3, 7] = 0.0
    with pytest.raises(T.CamelError, match="Division by zero"):
        T.call("divide", t(x), t(z))
    with pytest.raises(T.CamelError, match="log: input must be positive"):
        T.call("log", t(z))


def test_relu_operator_equals_reference_idiom():
    # test/run/nn/svm.cml:31: relu(x) = x * (x > 0)
    x = D.normal(21, (1000,))
    x[:6] = [0.0, -0.0, -3.0, np.inf, -np.inf, np.nan]
    xt = t(x)
    fused = T.call("relu", xt).numpy()
    idiom = T.call("multiply", xt, T.call("gt", xt, 0.0)).numpy()
    assert np.array_equal(fused.view(np.uint32)[6:], idiom.view(np.uint32)[6:])
    assert np.array_equal(np.isnan(fused), np.isnan(idiom))
    assert np.array_equal(fused[~np.isnan(fused)].view(np.uint32),
                          O.relu(x)[~np.isnan(fused)].view(np.uint32))


def composed_softmax(logits):
    """test/run/nn/mnist.cml:13-25, operator for operator."""
    n, k = T.call("shape", logits)
    row_max = T.call("max_axis", logits, 1)
    row_max_b = T.call("matmul", T.call("reshape", row_max, [n, 1]), T.call("ones", [1, k]))
    exp_logits = T.call("exp", T.call("subtract", logits, row_max_b))
    row_sums = T.call("sum_axis", exp_logits, 1)
    row_sums_b = T.call("matmul", T.call("reshape", row_sums, [n, 1]), T.call("ones", [1, k]))
    return T.call("divide", exp_logits, row_sums_b)


@pytest.mark.parametrize("rows,cols", [(1024, 10), (512, 10), (37, 300)])
def test_softmax_operator_matches_the_mnist_composition(rows, cols):
    x = D.normal(31 + cols, (rows, cols)) * F(3.0)
    xt = t(x)
    fused = T.call("softmax", xt).numpy()
    composed = composed_softmax(xt).numpy()
    ref = O.softmax_rows(x)
    # The composition on the device is the reference's op sequence (fp64 exp):
    assert np.max(np.abs(composed - ref) / ref) <= 1e-6
    assert np.mean(composed == ref) > 0.999
    # The fused kernel meets the softmax bar.
    assert np.max(np.abs(fused - ref) / ref) <= 1e-6


def test_mlp_config2_chain_stays_on_device():
    # The benchmark MLP: dense<w,b>..relu chain 784 -> 1024 -> 1024 -> 10, softmax.
    B, dims = 1024, [784, 1024, 1024, 10]
    x = D.uniform(D.SEED_MLP, (B, dims[0]), 0.0, 1.0)
    ws = [D.normal(D.SEED_MLP + 1 + i, (dims[i], dims[i + 1]), std=float(np.sqrt(1.0 / dims[i])))
          for i in range(3)]
    bs = [np.zeros(dims[i + 1], F) for i in range(3)]
    h = t(x)
    acts = []
    for i in range(3):
        uri = "dense_relu" if i < 2 else "dense"
        h = T.call(uri, h, with_=(t(ws[i]), t(bs[i])))
        assert h.residency() == (False, True), "layer output must stay on the device"
        acts.append(h)
    p = T.call("softmax", h)
    assert p.residency() == (False, True)
    # Oracle: the same chain on the CPU, each layer from the GPU's own input
    # so the per-layer GEMM bound applies to one GEMM at a time.
    prev = x
    for i in range(3):
        got = acts[i].numpy()
        ref = O.dense(prev, ws[i], bs[i], i < 2)
        gemm_ok(got, ref, prev, ws[i])
        prev = got
    got_p = p.numpy()
    ref_p = O.softmax_rows(prev)
    assert np.max(np.abs(got_p - ref_p) / ref_p) <= 1e-6


def test_dense_bias_operand_forms_agree():
    x = D.uniform(41, (70, 50), -1.0, 1.0)
    w = D.uniform(42, (50, 30), -1.0, 1.0)
    b = D.uniform(43, (30,), -1.0, 1.0)
    bound = t(x), t(w), t(b)
    a1 = T.call("dense_relu", bound[0], with_=(bound[1], bound[2])).numpy()
    a2 = T.call("dense_relu", bound[0], bound[1], t(b.reshape(1, 30))).numpy()
    assert np.array_equal(a1, a2)
    gemm_ok(a1, O.dense(x, w, b, True), x, w)
    no_bias = T.call("dense", bound[0], with_=(bound[1],)).numpy()
    gemm_ok(no_bias, O.matmul(x, w), x, w)


def test_conv_pool_cnn_slice_matches_oracle():
    # The benchmark small-CNN layers (28x28 -> 26 -> 24 -> pool 12) at batch 4.
    x = D.uniform(D.SEED_CNN, (4, 1, 28, 28), 0.0, 1.0)
    w1 = D.normal(D.SEED_CNN + 1, (32, 1, 3, 3), std=float(np.sqrt(2.0 / 9)))
    w2 = D.normal(D.SEED_CNN + 2, (64, 32, 3, 3), std=float(np.sqrt(2.0 / 288)))
    b1, b2 = np.zeros(32, F), np.zeros(64, F)
    h1 = T.call("conv2d_relu", t(x), with_=(t(w1), t(b1), 1, 0))
    h2 = T.call("conv2d_relu", h1, with_=(t(w2), t(b2)))
    p = T.call("maxpool2d", h2, with_=(2,))
    assert p.shape == (4, 64, 12, 12)
    g1, g2, gp = h1.numpy(), h2.numpy(), p.numpy()
    r1 = O.conv2d(x, w1, b1, True, 1, 0)
    assert np.allclose(g1, r1, rtol=0, atol=1e-5 * 3 * np.abs(r1).max())
    r2 = O.conv2d(g1, w2, b2, True, 1, 0)
    assert np.allclose(g2, r2, rtol=0, atol=1e-5 * np.sqrt(288) * np.abs(r2).max())
    assert np.array_equal(gp, O.maxpool2d(g2, 2, 2))


def test_reductions_and_indexing_match_oracle():
    x = D.normal(51, (300, 77))
    xt = t(x)
    assert np.array_equal(T.call("sum_axis", xt, 0).numpy(), O.sum_axis(x, 0))
    assert np.array_equal(T.call("max_axis", xt, -1).numpy(), O.max_axis(x, 1))
    assert np.array_equal(T.call("argmax_axis", xt, 0).numpy(), O.argmax_axis(x, 0))
    s = T.call("sum", xt)
    assert abs(s - O.sum_all(x)) <= 1e-12 * np.abs(x.astype(np.float64)).sum()
    y = T.call("exp", xt)  # device-only output
    assert y.residency() == (False, True)
    assert T.call("idx2d", y, 5, 6) == float(O.exp(x)[5, 6])
    assert y.residency() == (False, True), "indexing copies one element, not the tensor"


def test_concat_transpose_eq_with_arrays():
    a = np.arange(6, dtype=np.int64).reshape(2, 3)
    c = T.call("concat", t(a), [[6, 7, 8]], 0)
    assert c.numpy().tolist() == [[0, 1, 2], [3, 4, 5], [6, 7, 8]]
    tr = T.call("transpose", c)
    assert np.array_equal(tr.numpy(), c.numpy().T)
    eq = T.call("eq", tr, T.call("transpose", c))
    assert eq.numpy().all()


def test_random_range_and_show(capfd):
    r = T.call("random", [1000], 2.0, -1.0)
    v = r.numpy()
    assert v.shape == (1000,) and v.min() >= -1.0 and v.max() <= 2.0
    assert T.call("show", T.call("eye", 2)) is None
    out = capfd.readouterr().out
    assert out == "tensor([[      1.,       0.],\n        [      0.,       1.]], dtype=float32)\n"


def test_operator_results_have_the_resolved_dtype():
    # Each operator's result dtype at run time is the element type its group
    # resolves (Tensor<bool> for compares, Tensor<i64> for range / argmax,
    # Float32 otherwise; modules/tensor/operators.cpp:41-43, 137, 382, 458).
    a = t(np.arange(6, dtype=np.float32).reshape(2, 3))
    cases = [
        ("__lt__", (a, 2.0), (T.TC_TENSOR, T.TC_FLOAT64)),
        ("__eq__", (3.0, a), (T.TC_FLOAT64, T.TC_TENSOR)),
        ("range", (5,), (T.TC_INT64,)),
        ("argmax", (a, 1), (T.TC_TENSOR, T.TC_INT64)),
        ("__add__", (a, a), (T.TC_TENSOR, T.TC_TENSOR)),
        ("exp", (a,), (T.TC_TENSOR,)),
    ]
    for group, args, codes in cases:
        uri, code, elem = T.resolve_type(group, list(codes))
        out = T.call(uri, *args)
        assert code == T.TC_TENSOR and out.dtype_code == elem, group


def test_division_by_zero_releases_the_abandoned_output():
    # The output is created on the device before the kernel's zero flag is
    # read back; when the operator throws "Division by zero" that output is
    # released, so a loop that catches the error does not grow memory.
    a = t(np.ones((64, 64), np.float32))
    z = t(np.zeros((64, 64), np.float32))
    T.call("divide", a, a)  # uploads the operand
    before = T.live_count()
    for _ in range(3):
        with pytest.raises(T.CamelError, match="Division by zero"):
            T.call("divide", a, z)
    assert T.live_count() == before


def test_empty_operands_follow_the_reference():
    # Zero-size operands through the operators (runtime.cpp's loops simply
    # do not run): empty results keep their shapes, a K = 0 matmul is the
    # zero-initialised output (operators.cpp:757-766 never adds a term), and
    # the sum of nothing is 0.
    e03, e34 = np.zeros((0, 3), F), D.uniform(0x7E00, (3, 4), -1.0, 1.0)
    got = T.call("matmul", t(e03), t(e34)).numpy()
    assert got.shape == (0, 4)
    k0 = T.call("matmul", t(np.zeros((2, 0), F)), t(np.zeros((0, 4), F))).numpy()
    np.testing.assert_array_equal(k0, O.matmul(np.zeros((2, 0), F), np.zeros((0, 4), F)))
    assert not np.signbit(k0).any()
    e05 = np.zeros((0, 5), F)
    assert T.call("add", t(e05), t(e05)).numpy().shape == (0, 5)
    assert T.call("multiply", t(e05), 2.0).numpy().shape == (0, 5)
    assert T.call("relu", t(e05)).numpy().shape == (0, 5)
    assert T.call("exp", t(e05)).numpy().shape == (0, 5)
    assert T.call("softmax", t(np.zeros((0, 10), F))).numpy().shape == (0, 10)
    assert T.call("transpose", t(e05)).numpy().shape == (5, 0)
    assert T.call("sum", t(e05)) == O.sum_all(e05) == 0.0
    w, b = D.uniform(0x7E01, (5, 7), -1.0, 1.0), np.zeros(7, F)
    assert T.call("dense_relu", t(e05), with_=(t(w), t(b))).numpy().shape == (0, 7)
