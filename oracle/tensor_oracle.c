/*
 * tensor_oracle.c -- CPU restatement of the Camel `tensor` module kernels.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the timed CPU
 * baseline.  The product never links or calls this file.
 *
 * Loop-for-loop restatement of modules/tensor/runtime.cpp and
 * modules/tensor/operators.cpp (OpenCML/Camel 0.1.19): every element is read
 * through an out-of-line dtype switch and widened to double, each reference
 * operation rounds once to the output dtype, reductions run in the reference's
 * loop order with a double accumulator.  Parity status of each function is
 * recorded next to it ("pinned by" = the checks in tests/test_oracle.py).
 */
#include "tensor_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* TensorObject::getAsDouble, runtime.cpp:298-310.  Kept out of line, as the
 * reference's accessor lives in another translation unit from its callers. */
__attribute__((noinline)) double ot_get(int dt, const void *p, uint64_t i) {
    switch (dt) {
    case OT_F32:
        return (double)((const float *)p)[i];
    case OT_I64:
        return (double)((const int64_t *)p)[i];
    case OT_BOOL:
        return ((const uint8_t *)p)[i] != 0 ? 1.0 : 0.0;
    default:
        abort();
    }
}

/* TensorObject::setFromDouble, runtime.cpp:340-355.  The double->int64 cast
 * is the x86-64 cvttsd2si conversion (INT64_MIN for NaN / out of range). */
__attribute__((noinline)) void ot_set(int dt, void *p, uint64_t i, double v) {
    switch (dt) {
    case OT_F32:
        ((float *)p)[i] = (float)v;
        break;
    case OT_I64:
        ((int64_t *)p)[i] = (int64_t)v;
        break;
    case OT_BOOL:
        ((uint8_t *)p)[i] = v != 0.0 ? 1 : 0;
        break;
    default:
        abort();
    }
}

/* promoteTensorTypes, runtime.cpp:570-580.  Pinned by: dtype table test. */
int ot_promote(int lhs, int rhs) {
    if (lhs == OT_F32 || rhs == OT_F32) return OT_F32;
    if (lhs == OT_I64 || rhs == OT_I64) return OT_I64;
    return OT_BOOL;
}

/* applyBinary, runtime.cpp:113-130.  Pinned by: IEEE special-value KATs
 * (double-then-round equals the correctly rounded fp32 op). */
double ot_apply_binary(int op, double l, double r, int *err) {
    switch (op) {
    case OT_ADD:
        return l + r;
    case OT_SUB:
        return l - r;
    case OT_MUL:
        return l * r;
    case OT_DIV:
        if (r == 0.0) {
            *err = OT_ERR_DIV_ZERO;
            return 0.0;
        }
        return l / r;
    case OT_POW:
        return pow(l, r);
    }
    return 0.0;
}

/* applyCompare, runtime.cpp:132-146. */
static int apply_compare(int op, double l, double r) {
    switch (op) {
    case OT_LT:
        return l < r;
    case OT_LE:
        return l <= r;
    case OT_GT:
        return l > r;
    case OT_GE:
        return l >= r;
    case OT_EQ:
        return l == r;
    }
    return 0;
}

/* tensorBinary, runtime.cpp:775-793 (shape check is the caller's). */
int ot_binary(int op, int ldt, const void *l, int rdt, const void *r, int odt, void *out,
              uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) {
        int err = OT_OK;
        double v = ot_apply_binary(op, ot_get(ldt, l, i), ot_get(rdt, r, i), &err);
        if (err) return err;
        ot_set(odt, out, i, v);
    }
    return OT_OK;
}

/* tensorBinaryScalarRight, runtime.cpp:795-812. */
int ot_binary_scalar_right(int op, int ldt, const void *l, double s, int odt, void *out,
                           uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) {
        int err = OT_OK;
        double v = ot_apply_binary(op, ot_get(ldt, l, i), s, &err);
        if (err) return err;
        ot_set(odt, out, i, v);
    }
    return OT_OK;
}

/* tensorBinaryScalarLeft, runtime.cpp:814-831. */
int ot_binary_scalar_left(int op, double s, int rdt, const void *r, int odt, void *out,
                          uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) {
        int err = OT_OK;
        double v = ot_apply_binary(op, s, ot_get(rdt, r, i), &err);
        if (err) return err;
        ot_set(odt, out, i, v);
    }
    return OT_OK;
}

/* tensorCompare, runtime.cpp:863-877. */
void ot_compare(int op, int ldt, const void *l, int rdt, const void *r, uint8_t *out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i)
        out[i] = (uint8_t)apply_compare(op, ot_get(ldt, l, i), ot_get(rdt, r, i));
}

/* tensorCompareScalarRight, runtime.cpp:833-846. */
void ot_compare_scalar_right(int op, int ldt, const void *l, double s, uint8_t *out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = (uint8_t)apply_compare(op, ot_get(ldt, l, i), s);
}

/* tensorCompareScalarLeft, runtime.cpp:848-861. */
void ot_compare_scalar_left(int op, double s, int rdt, const void *r, uint8_t *out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = (uint8_t)apply_compare(op, s, ot_get(rdt, r, i));
}

/* __tensor_matmul__ hot loop, operators.cpp:757-766: i, j, then k ascending
 * with a double accumulator starting at 0.0; one rounding per output.
 * Pinned by: A*I = A, ones*ones = K, the k-order KAT [2^24, 1, -2^24], brute
 * force in exact rationals on tiny shapes. */
static void matmul_rows(int adt, const void *A, int bdt, const void *B, int odt, void *C,
                        int64_t K, int64_t N, int64_t r0, int64_t r1) {
    for (int64_t i = r0; i < r1; ++i) {
        for (int64_t j = 0; j < N; ++j) {
            double acc = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                acc += ot_get(adt, A, (uint64_t)(i * K + k)) * ot_get(bdt, B, (uint64_t)(k * N + j));
            }
            ot_set(odt, C, (uint64_t)(i * N + j), acc);
        }
    }
}

int ot_matmul(int adt, const void *A, int bdt, const void *B, int odt, void *C, int64_t M,
              int64_t K, int64_t N) {
    matmul_rows(adt, A, bdt, B, odt, C, K, N, 0, M);
    return OT_OK;
}

/* Rows [row_begin, row_end) of an fp32 matmul: the timed slab of the CPU
 * baseline (the cost per row of the ijk loop is constant). */
int64_t ot_matmul_rows(const float *A, const float *B, float *C, int64_t M, int64_t K, int64_t N,
                       int64_t row_begin, int64_t row_end) {
    if (row_end > M) row_end = M;
    matmul_rows(OT_F32, A, OT_F32, B, OT_F32, C, K, N, row_begin, row_end);
    return row_end - row_begin;
}

/* tensorSum, runtime.cpp:879-885 (double result, not rounded). */
double ot_sum(int dt, const void *x, uint64_t n) {
    double value = 0.0;
    for (uint64_t i = 0; i < n; ++i) value += ot_get(dt, x, i);
    return value;
}

static int normalize_axis(int64_t *axis) {
    if (*axis < 0) *axis += 2;
    return (*axis == 0 || *axis == 1) ? OT_OK : OT_ERR_SHAPE;
}

/* tensorSumAxis, runtime.cpp:887-922: double accumulation in index order,
 * Float32 output. */
int ot_sum_axis(int dt, const void *x, int64_t rows, int64_t cols, int64_t axis, float *out) {
    if (normalize_axis(&axis)) return OT_ERR_SHAPE;
    if (axis == 0) {
        for (int64_t j = 0; j < cols; ++j) {
            double acc = 0.0;
            for (int64_t i = 0; i < rows; ++i) acc += ot_get(dt, x, (uint64_t)(i * cols + j));
            out[j] = (float)acc;
        }
    } else {
        for (int64_t i = 0; i < rows; ++i) {
            double acc = 0.0;
            for (int64_t j = 0; j < cols; ++j) acc += ot_get(dt, x, (uint64_t)(i * cols + j));
            out[i] = (float)acc;
        }
    }
    return OT_OK;
}

/* tensorMaxAxis, runtime.cpp:924-963: first element, then strict '>'.  An
 * empty reduced axis reads element 0 of the next slice in the reference
 * (out of range); this restatement requires a non-empty axis. */
int ot_max_axis(int dt, const void *x, int64_t rows, int64_t cols, int64_t axis, float *out) {
    if (normalize_axis(&axis)) return OT_ERR_SHAPE;
    if (axis == 0) {
        for (int64_t j = 0; j < cols; ++j) {
            double best = ot_get(dt, x, (uint64_t)j);
            for (int64_t i = 1; i < rows; ++i) {
                double v = ot_get(dt, x, (uint64_t)(i * cols + j));
                if (v > best) best = v;
            }
            out[j] = (float)best;
        }
    } else {
        for (int64_t i = 0; i < rows; ++i) {
            double best = ot_get(dt, x, (uint64_t)(i * cols));
            for (int64_t j = 1; j < cols; ++j) {
                double v = ot_get(dt, x, (uint64_t)(i * cols + j));
                if (v > best) best = v;
            }
            out[i] = (float)best;
        }
    }
    return OT_OK;
}

/* tensorArgmaxAxis, runtime.cpp:965-1011. */
int ot_argmax_axis(int dt, const void *x, int64_t rows, int64_t cols, int64_t axis, int64_t *out) {
    if (normalize_axis(&axis)) return OT_ERR_SHAPE;
    if (axis == 0) {
        for (int64_t j = 0; j < cols; ++j) {
            int64_t best_idx = 0;
            double best = ot_get(dt, x, (uint64_t)j);
            for (int64_t i = 1; i < rows; ++i) {
                double v = ot_get(dt, x, (uint64_t)(i * cols + j));
                if (v > best) {
                    best = v;
                    best_idx = i;
                }
            }
            out[j] = best_idx;
        }
    } else {
        for (int64_t i = 0; i < rows; ++i) {
            int64_t best_idx = 0;
            double best = ot_get(dt, x, (uint64_t)(i * cols));
            for (int64_t j = 1; j < cols; ++j) {
                double v = ot_get(dt, x, (uint64_t)(i * cols + j));
                if (v > best) {
                    best = v;
                    best_idx = j;
                }
            }
            out[i] = best_idx;
        }
    }
    return OT_OK;
}

/* tensorExp, runtime.cpp:1013-1026.  glibc exp() is the third-party routine
 * at the libm boundary; the tests pin it element for element against Python's
 * math.exp (the same glibc) and against closed forms. */
int ot_exp(int dt, const void *x, float *out, uint64_t n) {
    if (dt != OT_F32) return OT_ERR_DTYPE;
    for (uint64_t i = 0; i < n; ++i) out[i] = (float)exp(ot_get(dt, x, i));
    return OT_OK;
}

/* tensorLog, runtime.cpp:1028-1045: throws on v <= 0.0 (NaN passes). */
int ot_log(int dt, const void *x, float *out, uint64_t n) {
    if (dt != OT_F32) return OT_ERR_DTYPE;
    for (uint64_t i = 0; i < n; ++i) {
        double v = ot_get(dt, x, i);
        if (v <= 0.0) return OT_ERR_LOG_DOMAIN;
        out[i] = (float)log(v);
    }
    return OT_OK;
}

/* tensorTranspose2D, runtime.cpp:704-720: element copy through double. */
void ot_transpose2d(int dt, const void *x, void *out, int64_t rows, int64_t cols) {
    for (int64_t i = 0; i < rows; ++i)
        for (int64_t j = 0; j < cols; ++j)
            ot_set(dt, out, (uint64_t)(j * rows + i), ot_get(dt, x, (uint64_t)(i * cols + j)));
}

/* tensorConcat, runtime.cpp:722-773: per outer index, the lhs slab then the
 * rhs slab (l_axis, r_axis are the two axis extents). */
void ot_concat(int dt, const void *l, const void *r, void *out, uint64_t outer, uint64_t l_axis,
               uint64_t r_axis, uint64_t inner) {
    size_t item = dt == OT_F32 ? 4 : (dt == OT_I64 ? 8 : 1);
    for (uint64_t o = 0; o < outer; ++o) {
        uint64_t lo = o * l_axis * inner, ro = o * r_axis * inner;
        uint64_t oo = o * (l_axis + r_axis) * inner;
        memcpy((char *)out + oo * item, (const char *)l + lo * item, l_axis * inner * item);
        memcpy((char *)out + (oo + l_axis * inner) * item, (const char *)r + ro * item,
               r_axis * inner * item);
    }
}

/* ReLU, defined as the reference idiom multiply(x, x > 0) (test/run/nn/svm.cml:31):
 * tensorCompareScalarRight(Greater, 0) then tensorBinary(Multiply) with a
 * Bool rhs promoted to Float32.  Pinned by: sign-of-zero / NaN / inf KATs. */
void ot_relu(const float *x, float *out, uint64_t n) {
    uint8_t *mask = (uint8_t *)malloc(n ? n : 1);
    ot_compare_scalar_right(OT_GT, OT_F32, x, 0.0, mask, n);
    int rc = ot_binary(OT_MUL, OT_F32, x, OT_BOOL, mask, OT_F32, out, n);
    (void)rc;
    free(mask);
}

/* Row softmax, the composition of test/run/nn/mnist.cml:13-25, op for op:
 *   row_max = max(logits, 1); broadcast = reshape(row_max,[n,1]) @ ones([1,k])
 *   stable = logits - broadcast; e = exp(stable); s = sum(e, 1)
 *   out = e / (reshape(s,[n,1]) @ ones([1,k]))     (throws if a divisor is 0)
 * Pinned by: rows sum to 1, shift invariance, one-hot limit, uniform rows,
 * fp64 closed form on small rows. */
int ot_softmax_rows(const float *x, float *out, int64_t n, int64_t k) {
    uint64_t nk = (uint64_t)n * (uint64_t)k;
    float *row_max = (float *)malloc(sizeof(float) * (size_t)(n ? n : 1));
    float *ones = (float *)malloc(sizeof(float) * (size_t)(k ? k : 1));
    float *bcast = (float *)malloc(sizeof(float) * (nk ? nk : 1));
    float *stable = (float *)malloc(sizeof(float) * (nk ? nk : 1));
    float *e = (float *)malloc(sizeof(float) * (nk ? nk : 1));
    int rc = OT_OK;
    for (int64_t j = 0; j < k; ++j) ones[j] = 1.0f;
    if (n > 0 && k > 0) {
        ot_max_axis(OT_F32, x, n, k, 1, row_max);
        ot_matmul(OT_F32, row_max, OT_F32, ones, OT_F32, bcast, n, 1, k);
        ot_binary(OT_SUB, OT_F32, x, OT_F32, bcast, OT_F32, stable, nk);
        ot_exp(OT_F32, stable, e, nk);
        ot_sum_axis(OT_F32, e, n, k, 1, row_max); /* row_max now holds the row sums */
        ot_matmul(OT_F32, row_max, OT_F32, ones, OT_F32, bcast, n, 1, k);
        rc = ot_binary(OT_DIV, OT_F32, e, OT_F32, bcast, OT_F32, out, nk);
    }
    free(row_max);
    free(ones);
    free(bcast);
    free(stable);
    free(e);
    return rc;
}

/* Dense layer y = x @ W (+ b) (relu): matmul (operators.cpp:757-766), the bias
 * broadcast idiom ones([M,1]) @ reshape(b,[1,N]) (mnist.cml:18) and add
 * (runtime.cpp:775-793), then the relu idiom above. */
int ot_dense(const float *x, const float *W, const float *b, int relu, float *out, int64_t M,
             int64_t K, int64_t N) {
    ot_matmul(OT_F32, x, OT_F32, W, OT_F32, out, M, K, N);
    if (b) {
        for (int64_t i = 0; i < M; ++i) {
            for (int64_t j = 0; j < N; ++j) {
                double bias = 0.0;
                bias += 1.0 * (double)b[j]; /* the [M,1] @ [1,N] broadcast matmul */
                float bj = (float)bias;
                uint64_t idx = (uint64_t)(i * N + j);
                out[idx] = (float)((double)out[idx] + (double)bj);
            }
        }
    }
    if (relu) ot_relu(out, out, (uint64_t)(M * N));
    return OT_OK;
}

/* conv2d NCHW, no reference op: defined as im2col(x) @ W^T with the matmul
 * semantics of operators.cpp:757-766 -- one double accumulator per output,
 * k = (c, kh, kw) ascending, zero padding contributes its 0.0 * w terms --
 * then the bias add and relu idioms as in ot_dense.  The reference has no
 * conv op to compare with; the tests pin this one by equivalence with
 * ot_matmul on an explicit im2col and by integer brute force on tiny shapes. */
int64_t ot_conv2d_images(const float *x, const float *w, const float *b, int relu, float *y,
                         int64_t n_begin, int64_t n_end, int64_t C, int64_t H, int64_t W,
                         int64_t Co, int64_t KH, int64_t KW, int64_t stride, int64_t pad) {
    int64_t OH = (H + 2 * pad - KH) / stride + 1;
    int64_t OW = (W + 2 * pad - KW) / stride + 1;
    int64_t K = C * KH * KW;
    for (int64_t n = n_begin; n < n_end; ++n) {
        for (int64_t co = 0; co < Co; ++co) {
            for (int64_t oh = 0; oh < OH; ++oh) {
                for (int64_t ow = 0; ow < OW; ++ow) {
                    double acc = 0.0;
                    for (int64_t k = 0; k < K; ++k) {
                        int64_t c = k / (KH * KW), r = k % (KH * KW);
                        int64_t ih = oh * stride + r / KW - pad, iw = ow * stride + r % KW - pad;
                        double xv = 0.0;
                        if (ih >= 0 && ih < H && iw >= 0 && iw < W)
                            xv = ot_get(OT_F32, x, (uint64_t)(((n * C + c) * H + ih) * W + iw));
                        acc += xv * ot_get(OT_F32, w, (uint64_t)(co * K + k));
                    }
                    float v = (float)acc;
                    if (b) {
                        double bias = 0.0;
                        bias += 1.0 * (double)b[co];
                        v = (float)((double)v + (double)(float)bias);
                    }
                    if (relu) v = (float)((double)v * ((double)v > 0.0 ? 1.0 : 0.0));
                    y[((n * Co + co) * OH + oh) * OW + ow] = v;
                }
            }
        }
    }
    return n_end - n_begin;
}

int ot_conv2d(const float *x, const float *w, const float *b, int relu, float *y, int64_t N,
              int64_t C, int64_t H, int64_t W, int64_t Co, int64_t KH, int64_t KW, int64_t stride,
              int64_t pad) {
    if (stride <= 0 || pad < 0 || H + 2 * pad < KH || W + 2 * pad < KW) return OT_ERR_SHAPE;
    ot_conv2d_images(x, w, b, relu, y, 0, N, C, H, W, Co, KH, KW, stride, pad);
    return OT_OK;
}

/* maxpool2d NCHW, no reference op: window scanned (kh, kw) ascending with the
 * first-element-then-strict-'>' rule of tensorMaxAxis (runtime.cpp:953-958).
 * Pinned by brute force. */
int ot_maxpool2d(const float *x, float *y, int64_t N, int64_t C, int64_t H, int64_t W, int64_t KH,
                 int64_t KW, int64_t stride) {
    if (stride <= 0 || H < KH || W < KW) return OT_ERR_SHAPE;
    int64_t OH = (H - KH) / stride + 1, OW = (W - KW) / stride + 1;
    for (int64_t p = 0; p < N * C; ++p) {
        const float *src = x + p * H * W;
        for (int64_t oh = 0; oh < OH; ++oh) {
            for (int64_t ow = 0; ow < OW; ++ow) {
                double best = (double)src[(oh * stride) * W + ow * stride];
                for (int64_t kh = 0; kh < KH; ++kh) {
                    for (int64_t kw = 0; kw < KW; ++kw) {
                        if (kh == 0 && kw == 0) continue;
                        double v = (double)src[(oh * stride + kh) * W + ow * stride + kw];
                        if (v > best) best = v;
                    }
                }
                y[(p * OH + oh) * OW + ow] = (float)best;
            }
        }
    }
    return OT_OK;
}

/* SplitMix64 output function on a counter (Vigna, public domain). */
uint64_t ot_splitmix64(uint64_t seed, uint64_t index) {
    uint64_t z = seed + (index + 1) * 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

/* U[lo, hi) from the top 24 bits: u = (x >> 40) * 2^-24 is exact in fp32. */
void ot_fill_uniform(float *out, uint64_t n, uint64_t seed, float lo, float hi) {
    for (uint64_t i = 0; i < n; ++i) {
        float u = (float)(ot_splitmix64(seed, i) >> 40) * (1.0f / 16777216.0f);
        out[i] = lo + (hi - lo) * u;
    }
}
