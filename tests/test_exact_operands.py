"""The wide-operand exact tests (tests/test_gpu_exact.py) on the CPU: that
their operands stay inside the exact-fp32 bound, and that they discriminate.

For each case the exact result is recomputed with one operand rounded to a
narrower type a matrix core could be fed instead of fp32 -- bf16 (8
significant bits), fp16 and tf32 (11) -- and a large share of the outputs
must change, so a GPU path that narrowed that operand would fail the
bit-exact comparison.  The mistake is planted here, in numpy, never on the
device."""
import numpy as np
import pytest

from tests.test_gpu_exact import (CNN_WIDE, CONV2_WIDE, HEAD_WIDE, MLP_WIDE, PAIR_WIDE, EXACT,
                                  exact_conv, exact_dense, ints, pool2, ternary, wide, wide_pair)

F = np.float32


def bf16(a):
    u = np.ascontiguousarray(a, F).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(F)


def tf32(a):
    u = np.ascontiguousarray(a, F).view(np.uint32).astype(np.uint64)
    u = (u + 0xFFF + ((u >> 13) & 1)) & 0xFFFFE000
    return u.astype(np.uint32).view(F)


def fp16(a):
    return np.asarray(a, F).astype(np.float16).astype(F)


NARROW = {"bf16": bf16, "tf32": tf32, "fp16": fp16}


def changed(got, want):
    return float(np.mean(got.view(np.uint32) != want.view(np.uint32)))


def test_generators_are_what_the_bound_assumes():
    w = wide(1, (64, 4096))
    assert np.abs(w).max() <= 4095 and np.all(w == np.round(w))
    # 12 significant bits are used: odd values above 2048 are common
    assert np.mean((np.abs(w) > 2048) & (w % 2 == 1)) > 0.2
    t = ternary(2, (4096, 96), 0, 4000)
    assert set(np.unique(t)) <= {-1.0, 0.0, 1.0}
    assert np.all((t != 0).sum(axis=0) == 4000)
    t = ternary(3, (96, 300), 1, 4000)
    assert np.all((t != 0).sum(axis=1) == 300)
    # the worst case the bound allows: 4000 products of 4095 plus a bias
    assert 4000 * 4095 + 4095 < EXACT


@pytest.mark.parametrize("wide_side", ["A", "B"])
@pytest.mark.parametrize("M,N,Kd", [(64, 96, 4096), (16, 256, 9216), (32, 48, 20)])
def test_gemm_wide_operand_rounded_narrower_changes_outputs(M, N, Kd, wide_side):
    a, b = wide_pair(7 + Kd, (M, Kd), (Kd, N), wide_side)
    want = exact_dense(a, b)
    for name, narrow in NARROW.items():
        a2, b2 = (narrow(a), b) if wide_side == "A" else (a, narrow(b))
        assert changed(exact_dense(a2, b2), want) > 0.5, name


@pytest.mark.parametrize("which", sorted(HEAD_WIDE))
def test_head_cases_discriminate(which):
    s = 0xD000 + len(which)
    x, w1, w2 = HEAD_WIDE[which](s)
    b1, b2 = ints(s + 2, (128,), -1, 1), wide(s + 4, (10,))
    h = exact_dense(x, w1, b1, True)
    want = exact_dense(h, w2, b2)
    for name, narrow in (("bf16", bf16), ("tf32", tf32)):
        if which == "x":
            got = exact_dense(exact_dense(narrow(x), w1, b1, True), w2, b2)
        elif which == "w1":
            got = exact_dense(exact_dense(x, narrow(w1), b1, True), w2, b2)
        else:
            got = exact_dense(h, narrow(w2), b2)
        assert changed(got, want) > 0.5, name
        if which != "w2":
            # layer 2's A operand (the split sums) is wide as well
            assert changed(exact_dense(narrow(h), w2, b2), want) > 0.5, name


@pytest.mark.parametrize("which", sorted(MLP_WIDE))
def test_mlp_cases_discriminate(which):
    s = 0xD400 + 16 * len(which)
    x, *wn = MLP_WIDE[which](s)
    bn = [ints(s + 5, (1024,), -1, 1), ints(s + 6, (1024,), -1, 1), wide(s + 7, (10,))]

    def run(narrow_at=None, narrow=None):
        h = x
        for i in range(3):
            a, w = h, wn[i]
            if narrow_at == ("a", i):
                a = narrow(a)
            if narrow_at == ("w", i):
                w = narrow(w)
            h = exact_dense(a, w, bn[i], i < 2)
        return h

    want = run()
    # the operands each case makes wide
    wide_ops = {"x": [("a", 0), ("a", 1), ("a", 2)], "w1": [("w", 0), ("a", 1), ("a", 2)],
                "w2": [("w", 1), ("a", 2)]}[which]
    for at in wide_ops:
        assert changed(run(at, bf16), want) > 0.25, at
        assert changed(run(at, tf32), want) > 0.1, at


def test_conv_cases_discriminate():
    # CONV_CASES' wide x / wide w form at a reduced batch of the config-4 shape
    x, w = wide(1, (2, 64, 20, 20)), ints(2, (128, 64, 3, 3), -1, 1)
    b = wide(3, (128,))
    want = exact_conv(x, w, b, 1, 1, relu=True)
    assert changed(exact_conv(bf16(x), w, b, 1, 1, relu=True), want) > 0.25
    assert changed(exact_conv(tf32(x), w, b, 1, 1, relu=True), want) > 0.1
    x, w = ints(1, (2, 64, 20, 20), -1, 1), wide(2, (128, 64, 3, 3))
    want = exact_conv(x, w, b, 1, 1, relu=True)
    assert changed(exact_conv(x, bf16(w), b, 1, 1, relu=True), want) > 0.25
    assert changed(exact_conv(x, fp16(w), b, 1, 1, relu=True), want) > 0.1


@pytest.mark.parametrize("which", sorted(CONV2_WIDE))
def test_conv2_cases_discriminate(which):
    x, w = CONV2_WIDE[which](0xD200 + len(which))
    x = x[:8]
    b = wide(0xD202, (64,))
    want = pool2(exact_conv(x, w, b, 1, 0, relu=True))
    x2, w2 = (bf16(x), w) if which == "x" else (x, bf16(w))
    assert changed(pool2(exact_conv(x2, w2, b, 1, 0, relu=True)), want) > 0.25


@pytest.mark.parametrize("which", sorted(PAIR_WIDE))
def test_pair_cases_discriminate(which):
    s = 0xD300 + len(which)
    x, w1, w2 = PAIR_WIDE[which](s)
    x = x[:8]
    b1, b2 = ints(s + 2, (32,), -1, 1), wide(s + 4, (64,))
    h = exact_conv(x, w1, b1, relu=True)
    want = pool2(exact_conv(h, w2, b2, relu=True))
    h2, w22 = (bf16(h), w2) if which == "x" else (h, bf16(w2))
    assert changed(pool2(exact_conv(h2, w22, b2, relu=True)), want) > 0.25


@pytest.mark.parametrize("which", sorted(CNN_WIDE))
def test_cnn_cases_discriminate(which):
    s = 0xD500 + 16 * len(which)
    x, w1, w2, w3, w4 = CNN_WIDE[which](s)
    x = x[:16]
    b1, b2 = ints(s + 5, (32,), -1, 1), ints(s + 6, (64,), -1, 1)
    b3, b4 = ints(s + 7, (128,), -1, 1), wide(s + 8, (10,))
    n = x.shape[0]

    def run(narrow_conv2=None, narrow_dense1=False):
        h = exact_conv(x, w1, b1, relu=True)
        a, w = h, w2
        if narrow_conv2 == "a":
            a = bf16(a)
        if narrow_conv2 == "w":
            w = bf16(w)
        h = pool2(exact_conv(a, w, b2, relu=True)).reshape(n, 9216)
        h = exact_dense(bf16(h) if narrow_dense1 else h, w3, b3, True)
        return exact_dense(h, w4, b4)

    want = run()
    assert changed(run(narrow_conv2="a" if which == "x" else "w"), want) > 0.25
    assert changed(run(narrow_dense1=True), want) > 0.25
