"""GPU parity of the MFMA fp32 GEMM (tensor:matmul / dense) against the CPU oracle.

Tolerance (the north star's GEMM bar, stated per element): |C_gpu - C_ref| <=
1e-5 * sqrt(K) * sum_k |A_ik| |B_kj|; the oracle accumulates in fp64 in k
order exactly as operators.cpp:757-766.  Full-size shapes are checked on a
row slab computed by the oracle plus size-independent identities.
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


def _ab(M, N, Kd, seed):
    a = D.uniform(seed, (M, Kd), -1.0, 1.0)
    b = D.uniform(seed + 1, (Kd, N), -1.0, 1.0)
    return a, b


@pytest.mark.parametrize("M,N,Kd", [
    (256, 256, 256),            # config 1
    (1, 1, 1), (33, 17, 65), (7, 300, 5), (64, 64, 64), (100, 36, 1000),
    (130, 258, 190),            # ragged edges on every tile shape
    (1024, 10, 1024),           # MLP last layer (N=10, unaligned rows)
    (512, 10, 128), (16, 512, 777), (31, 40, 12),
])
def test_sgemm_matches_oracle(M, N, Kd):
    a, b = _ab(M, N, Kd, 0x1000 + M * 7 + N * 13 + Kd)
    ref = O.matmul(a, b)
    got = K.sgemm(a, b)
    ok, worst = K.gemm_tol_ok(got, ref, a, b)
    assert ok, f"worst error / bound = {worst}"


@pytest.mark.parametrize("M,N,Kd", [
    (1024, 1024, 784),   # 64x64 tiles (the MLP's first layer), ragged first stage
    (512, 128, 9216),    # 64x64 tiles with 16 K splits (the CNN's dense1)
    (1024, 1024, 1024),  # 64x64 tiles, whole stages
    (2048, 2048, 1000),  # one-round 128x128 tiles with k-groups, ragged first stage
])
def test_lds_dma_path_equals_register_path(M, N, Kd):
    # Row-major operands with 16-byte rows and M, N multiples of the tile take
    # the LDS DMA stage loop (global_load_lds straight into LDS); one row less
    # (M - 1, the same tile grid and K splits) takes the register-staged
    # loaders of the same tile.  Both feed the MFMAs the same values in the
    # same order, so the rows they share are bit-identical on random floats
    # (bias and relu too).
    a, b = _ab(M, N, Kd, 0x1700 + M + N + Kd)
    bias = D.uniform(0x1701 + N, (N,), -1.0, 1.0)
    flags = H.EPI_BIAS | H.EPI_RELU
    dma = K.sgemm(a, b, bias, flags)
    staged = K.sgemm(a[:M - 1], b, bias, flags)
    assert np.array_equal(dma[:M - 1].view(np.uint32), staged.view(np.uint32))
    # and the DMA path's first rows against the oracle (no bias or relu)
    plain = K.sgemm(a, b)[:64]
    ok, worst = K.gemm_tol_ok(plain, O.matmul(a[:64], b), a[:64], b)
    assert ok, f"worst error / bound = {worst}"


@pytest.mark.parametrize("M,N,Kd", [
    (512, 256, 2000),    # 64x64 tiles, 7 K splits, K % 64 = 16
    (1024, 2048, 1000),  # 64x64 tiles, no split, K % 64 = 40
    (2048, 2048, 1001),  # 128x128 tiles, odd K (scalar A loads), K % 32 = 9
    (2000, 2100, 1000),  # 128x128 tiles in two k-groups (one round), K % 64 = 40
    (2048, 2048, 1000),  # the same tiles staged by LDS DMA (M, N multiples of 128)
    (4096, 4096, 1000),  # 256x256 tiles, K % 32 = 8
    (200, 72, 1000),     # 32x32 tiles, K splits, K % 64 = 40
])
def test_ragged_k_first_stage(M, N, Kd):
    # When BK does not divide K the first stage of split 0 starts below k = 0
    # and is loaded with guards; every later stage is whole.  Rows from the
    # first, a middle and the last tile row, against the oracle's fp64 k-order
    # loop.
    a, b = _ab(M, N, Kd, 0x1500 + M + N + Kd)
    bias = D.uniform(0x1600 + N, (N,), -1.0, 1.0)
    got = K.sgemm(a, b, bias, H.EPI_BIAS)
    for r0, r1 in ((0, 8), (M // 2 - 3, M // 2 + 3), (M - 8, M)):
        ref = O.dense(a[r0:r1], b, bias, False)
        ok, worst = K.gemm_tol_ok(got[r0:r1], ref, a[r0:r1], b)
        assert ok, f"rows {r0}-{r1}: worst error / bound = {worst}"


def test_sgemm_zero_k_gives_zeros():
    a = np.zeros((5, 0), np.float32)
    b = np.zeros((0, 7), np.float32)
    da, db = K.empty(4), K.empty(4)
    dc = K.dev(np.full((5, 7), 3.0, np.float32))
    H.call("camel_hip_sgemm", P(da.ptr), P(db.ptr), P(dc.ptr), 5, 7, 0, None, 0)
    out = K.host(dc, np.float32, (5, 7))
    assert np.array_equal(out, O.matmul(a, b))


@pytest.mark.parametrize("M,N,Kd", [(1024, 10, 1024), (300, 3, 50), (257, 31, 200), (100, 4, 0),
                                    (4096, 1, 1000), (2000, 32, 512), (600, 20, 300)])
def test_thin_n_dense_matches_oracle(M, N, Kd):
    # N <= 32 with B small enough for LDS: the thin (non-MFMA) kernel.
    a, w = _ab(M, N, Kd, 0x3000 + M + N + Kd)
    b = D.uniform(0x3100 + N, (N,), -1.0, 1.0)
    got = K.sgemm(a, w, b, H.EPI_BIAS | H.EPI_RELU)
    ref = O.dense(a, w, b, True)
    ok, worst = K.gemm_tol_ok(got, ref, a, w)
    assert ok, f"worst error / bound = {worst}"
    neg = (ref < 0) | ((ref == 0) & np.signbit(ref))
    assert np.all(np.signbit(got[(got == 0) & neg]))


@pytest.mark.parametrize("M,N,Kd", [(1024, 1024, 784), (1024, 1024, 1024), (512, 128, 9216)])
def test_dense_bias_relu_matches_oracle(M, N, Kd):
    a, w = _ab(M, N, Kd, 0x2000 + Kd)
    bias = D.uniform(0x2100 + N, (N,), -0.5, 0.5)
    ref = O.dense(a, w, bias, True)
    got = K.sgemm(a, w, bias, H.EPI_BIAS | H.EPI_RELU)
    ok, worst = K.gemm_tol_ok(got, ref, a, w)
    assert ok, f"worst error / bound = {worst}"
    # relu keeps the sign of zero: negatives become -0.0, never +0.0
    neg = (ref < 0) | ((ref == 0) & np.signbit(ref))
    assert np.all(np.signbit(got[(got == 0) & neg]))


def test_gemm_8192_row_sums_and_slab():
    # The largest square config at full size: every row's sum checked through
    # C 1 = A (B 1) in fp64 (size-independent: a dropped or repeated k term,
    # tile or split shows up in its row), plus 4 rows against the oracle.
    n = 8192
    a, b = _ab(n, n, n, D.SEED_GEMM + n)
    got = K.sgemm(a, b)
    bv = b.astype(np.float64).sum(axis=1)
    ref_sums = a.astype(np.float64) @ bv
    # bound: the per-element GEMM bound summed over the row
    mag = np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64)).sum(axis=1)
    err = np.abs(got.astype(np.float64).sum(axis=1) - ref_sums)
    assert np.all(err <= 1e-5 * np.sqrt(n) * mag + n * 1e-30)
    for r0 in (0, n - 4):
        ref = O.matmul_rows(a, b, r0, r0 + 4)
        ok, worst = K.gemm_tol_ok(got[r0:r0 + 4], ref, a[r0:r0 + 4], b)
        assert ok, f"rows {r0}+4: worst error / bound = {worst}"


@pytest.mark.parametrize("n", [1024, 2048, 4096])
def test_square_gemm_row_slab(n):
    a, b = _ab(n, n, n, D.SEED_GEMM + n)
    got = K.sgemm(a, b)
    rows = 32 if n <= 2048 else 16
    ref = O.matmul_rows(a, b, 0, rows)
    ok, worst = K.gemm_tol_ok(got[:rows], ref, a[:rows], b)
    assert ok, f"worst error / bound = {worst}"
    # last rows too (different tile, different XCD)
    ref_tail = O.matmul_rows(a, b, n - 8, n)
    ok, worst = K.gemm_tol_ok(got[n - 8:], ref_tail, a[n - 8:], b)
    assert ok, f"tail worst error / bound = {worst}"


def test_partial_round_is_split_along_k():
    # 4352^2 in 256x256 tiles = 289 tiles on 256 resident work-groups: one
    # whole round, then 33 tiles split along K and folded by the reduce kernel.
    # The last tile-row and the right column band are such tail tiles.
    n, k = 4352, 512
    a, b = _ab(n, n, k, D.SEED_GEMM + 7)
    bias = D.uniform(D.SEED_GEMM + 8, (n,), -1.0, 1.0)
    got = K.sgemm(a, b, bias, H.EPI_BIAS | H.EPI_RELU)
    for r0, r1 in ((0, 8), (3100, 3106), (n - 12, n)):
        ref = O.dense(a[r0:r1], b, bias, True)
        ok, worst = K.gemm_tol_ok(got[r0:r1], ref, a[r0:r1], b)
        assert ok, f"rows {r0}-{r1}: worst error / bound = {worst}"


def test_partial_round_column_band():
    # M = 512 in 256x256 tiles: 2 tile rows in one group, so the 2 tiles left
    # after a whole round (N = 33024 -> 129 tile columns) are the last tile
    # column, run as a band of 64x32 tiles over all of K.
    m, n, k = 512, 33024, 256
    a, b = _ab(m, n, k, D.SEED_GEMM + 9)
    bias = D.uniform(D.SEED_GEMM + 10, (n,), -1.0, 1.0)
    got = K.sgemm(a, b, bias, H.EPI_BIAS | H.EPI_RELU)
    for r0, r1 in ((0, 6), (250, 262), (m - 6, m)):
        ref = O.dense(a[r0:r1], b, bias, True)
        ok, worst = K.gemm_tol_ok(got[r0:r1], ref, a[r0:r1], b)
        assert ok, f"rows {r0}-{r1}: worst error / bound = {worst}"


def test_skinny_gemm_matches_oracle():
    a, b = _ab(16, 4096, 4096, D.SEED_GEMM + 16)
    got = K.sgemm(a, b)
    ref = O.matmul(a, b)
    ok, worst = K.gemm_tol_ok(got, ref, a, b)
    assert ok, f"worst error / bound = {worst}"


@pytest.mark.parametrize("M,N,Kd", [
    (16, 4096, 1000),   # K tail inside one wave's range
    (32, 4100, 3000),   # two 16-row groups, last strip partial, short k ranges
    (17, 64, 5000),     # one strip, many k work-groups
    (3, 8, 7),          # one work-group, no partials
    (16, 256, 65536),   # 64 k work-groups per strip
    (16, 4096, 2048),   # two chunks per work-group, every work-group guard-free
    (32, 4096, 4096),   # two 16-row groups, four chunks per work-group
    (16, 1024, 4099),   # K % 4 != 0: every work-group takes the guarded loads
    (8, 2048, 8192),    # M < 16: rows past M read as zero
    (20, 64, 100),      # two 16-row groups, one work-group, no partials
    (32, 128, 256),     # two full 16-row groups, one k group per strip
    (17, 4096, 4096),   # one row past a 16-row group, four k groups per strip
])
def test_skinny_streaming_kernel_matches_oracle(M, N, Kd):
    # M <= 32, N % 4 == 0: the streaming kernel (16x16x4 MFMA), k partials
    # summed in order by the reduce kernel, which applies bias + relu.
    a, b = _ab(M, N, Kd, 0x4000 + M + N + Kd)
    bias = D.uniform(0x4100 + N, (N,), -1.0, 1.0)
    ref = O.dense(a, b, bias, True)
    for _ in range(2):  # a second call reuses the partial scratch
        got = K.sgemm(a, b, bias, H.EPI_BIAS | H.EPI_RELU)
        ok, worst = K.gemm_tol_ok(got, ref, a, b)
        assert ok, f"worst error / bound = {worst}"
    neg = (ref < 0) | ((ref == 0) & np.signbit(ref))
    assert np.all(np.signbit(got[(got == 0) & neg]))


def test_skinny_results_do_not_depend_on_scheduling():
    # The k work-groups of a strip finish in any order; the sum order is fixed.
    a, b = _ab(16, 1024, 8192, 0x4200)
    first = K.sgemm(a, b)
    for _ in range(3):
        assert np.array_equal(K.sgemm(a, b).view(np.uint32), first.view(np.uint32))


def test_identity_and_ones_closed_forms():
    # A @ I = A exactly; ones @ ones = K exactly (tensor_smoke.cml:9-11 pattern)
    a = D.uniform(7, (300, 260), -1, 1)
    eye = np.eye(260, dtype=np.float32)
    assert np.array_equal(K.sgemm(a, eye), a)
    ones_a = np.ones((70, 333), np.float32)
    ones_b = np.ones((333, 90), np.float32)
    assert np.all(K.sgemm(ones_a, ones_b) == 333.0)


def test_generic_matmul_int64_bool_is_exact():
    a = (np.arange(6 * 5).reshape(6, 5) - 11).astype(np.int64)
    b = (np.arange(5 * 4).reshape(5, 4) % 2).astype(np.uint8)
    ref = O.matmul(a, b)
    da, db = K.dev(a), K.dev(b)
    dc = K.empty(ref.nbytes)
    H.call("camel_hip_matmul_generic", H.DT_I64, P(da.ptr), H.DT_BOOL, P(db.ptr), H.DT_I64,
           P(dc.ptr), 6, 4, 5)
    assert np.array_equal(K.host(dc, np.int64, (6, 4)), ref)


@pytest.mark.parametrize("M,N,Kd", [
    (130, 96, 200),    # MFMA tiles with ragged edges
    (300, 7, 64),      # thin-N kernel
    (16, 512, 300),    # skinny streaming kernel
    (1024, 1024, 64),  # guard-free interior tiles
])
def test_sgemm_special_values_propagate_like_the_reference(M, N, Kd):
    # inf / NaN in the operands: inf*0 = NaN, inf + (-inf) = NaN, NaN absorbs
    # -- the same IEEE rules in the fp32 MFMA as in the reference's fp64 loop,
    # so the non-finite outputs match exactly and the finite ones stay within
    # the GEMM bar.  (Finite operands whose products or partial sums pass the
    # fp32 range are the one known difference: the fp64 accumulator of the
    # reference does not overflow there; see the design notes.)
    rng = np.random.default_rng(M * 31 + N)
    a, b = _ab(M, N, Kd, 0x4300 + M + N + Kd)
    for arr in (a, b):
        flat = arr.reshape(-1)
        idx = rng.choice(flat.size, size=6, replace=False)
        flat[idx[:2]] = np.inf
        flat[idx[2:4]] = -np.inf
        flat[idx[4:]] = np.nan
    a[3, :] = 0.0
    a[3, 5] = np.inf                      # row 3: inf * B[5, j] -> +-inf or NaN (B zero -> NaN)
    b[5, :8] = 0.0
    ref = O.matmul(a, b)
    got = K.sgemm(a, b)
    fin = np.isfinite(ref)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isposinf(got), np.isposinf(ref))
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    # finite entries: the GEMM bar over the finite terms of each dot product
    af = np.where(np.isfinite(a), a, 0).astype(np.float64)
    bf = np.where(np.isfinite(b), b, 0).astype(np.float64)
    bound = 1e-5 * np.sqrt(Kd) * (np.abs(af) @ np.abs(bf))
    err = np.abs(got.astype(np.float64)[fin] - ref.astype(np.float64)[fin])
    assert np.all(err <= bound[fin] + 1e-30)
