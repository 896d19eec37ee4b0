// Tensor kernels of the operator layer on the gfx950 device.  Each function
// keeps the checks and error texts of the reference function it replaces
// (modules/tensor/runtime.cpp, cited per function) and launches the matching
// libcamel_hip entry point on the library's stream.  Outputs are born on the
// device; nothing is copied back to the host unless a host value is asked for.
#include "runtime.h"

#include "camel_hip.h"

#include <array>
#include <random>

namespace camel_amd::tensor {

namespace {

TensorObject *deviceTensor(TypeCode dtype, std::span<const int64_t> shape) {
    return TensorObject::create(dtype, shape, Residence::Device);
}

std::span<const int64_t> shapeOf(const TensorObject *t) { return {t->shape(), t->rank()}; }

int hipBinary(BinaryOp op) {
    switch (op) {
    case BinaryOp::Add:
        return CAMEL_OP_ADD;
    case BinaryOp::Subtract:
        return CAMEL_OP_SUB;
    case BinaryOp::Multiply:
        return CAMEL_OP_MUL;
    case BinaryOp::Divide:
        return CAMEL_OP_DIV;
    default:
        return CAMEL_OP_POW;
    }
}

int hipCompare(CompareOp op) {
    switch (op) {
    case CompareOp::Less:
        return CAMEL_CMP_LT;
    case CompareOp::LessEqual:
        return CAMEL_CMP_LE;
    case CompareOp::Greater:
        return CAMEL_CMP_GT;
    case CompareOp::GreaterEqual:
        return CAMEL_CMP_GE;
    default:
        return CAMEL_CMP_EQ;
    }
}

// The shim reports value-dependent failures with the reference's own texts
// ("Division by zero", "log: input must be positive"); checkHip rethrows them.
void fill(TensorObject *t, double value) {
    if (t->numel() == 0) return;
    checkHip(camel_hip_fill(hipDType(t->dtype()), t->deviceOutput(), (int64_t)t->numel(), value));
}

void requireRank2(const TensorObject *t, const char *what) {
    if (t->rank() != 2)
        throw std::invalid_argument(std::string(what) + " currently only supports rank-2 tensors");
}

int64_t normaliseAxis(int64_t axis, const char *what) {
    if (axis < 0) axis += 2;
    if (axis != 0 && axis != 1)
        throw std::invalid_argument(std::string(what) + "(axis): axis must be 0 or 1 for rank-2 tensors");
    return axis;
}

} // namespace

// tensorEmpty / tensorZeros (runtime.cpp:614-624): zero-initialised.
TensorObject *tensorEmpty(TypeCode dtype, std::span<const int64_t> shape) {
    return TensorObject::create(dtype, shape, Residence::Device, true);
}
TensorObject *tensorZeros(TypeCode dtype, std::span<const int64_t> shape) {
    return TensorObject::create(dtype, shape, Residence::Device, true);
}

// tensorOnes / tensorFull (runtime.cpp:626-640): value through setFromDouble.
TensorObject *tensorOnes(TypeCode dtype, std::span<const int64_t> shape) {
    return tensorFull(dtype, shape, 1.0);
}
TensorObject *tensorFull(TypeCode dtype, std::span<const int64_t> shape, double value) {
    TensorObject *t = deviceTensor(dtype, shape);
    fill(t, value);
    return t;
}

// tensorRandom (runtime.cpp:642-654): the reference seeds mt19937 from
// std::random_device, so the stream cannot be reproduced; the same generator
// and distribution run on the host and the payload is uploaded at first use.
TensorObject *tensorRandom(std::span<const int64_t> shape, double low, double high) {
    if (low > high) std::swap(low, high);
    TensorObject *t = TensorObject::create(TypeCode::Float32, shape, Residence::Host);
    std::mt19937 rng(std::random_device{}());
    std::uniform_real_distribution<float> dist(static_cast<float>(low), static_cast<float>(high));
    float *p = static_cast<float *>(t->hostOutput());
    for (uint64_t i = 0; i < t->numel(); ++i) p[i] = dist(rng);
    return t;
}

// tensorArange (runtime.cpp:656-677): values start, start+step, ... while
// < stop (step > 0) or > stop (step < 0).
TensorObject *tensorArange(int64_t start, int64_t stop, int64_t step) {
    if (step == 0) throw std::invalid_argument("range step cannot be zero");
    __int128 span = step > 0 ? (__int128)stop - start : (__int128)start - stop;
    const __int128 mag = step > 0 ? (__int128)step : -(__int128)step;
    const int64_t count = span <= 0 ? 0 : (int64_t)((span + mag - 1) / mag);
    int64_t shape[] = {count};
    TensorObject *t = deviceTensor(TypeCode::Int64, shape);
    if (count > 0)
        checkHip(camel_hip_arange(static_cast<int64_t *>(t->deviceOutput()), start, step, count));
    return t;
}

// tensorEye (runtime.cpp:679-690).
TensorObject *tensorEye(int64_t size) {
    if (size < 0) throw std::invalid_argument("eye size cannot be negative");
    int64_t shape[] = {size, size};
    TensorObject *t = deviceTensor(TypeCode::Float32, shape);
    if (size > 0) checkHip(camel_hip_eye(static_cast<float *>(t->deviceOutput()), size));
    return t;
}

// tensorReshape (runtime.cpp:692-702): same element count; a view here.
TensorObject *tensorReshape(const TensorObject *tensor, std::span<const int64_t> shape) {
    return TensorObject::view(tensor, shape);
}

// tensorTranspose2D (runtime.cpp:704-720).  Float32: a view, read in place
// by matmul / dense (the GEMM's transposed-A loaders) and made contiguous by
// any other reader; the reference's element copy through double is exact
// for Float32.  Int64 and Bool are copied through double (int64 values past
// 2^53 round, bools normalise to 0/1) as the reference does.
TensorObject *tensorTranspose2D(const TensorObject *tensor) {
    if (tensor->rank() != 2)
        throw std::invalid_argument("transpose currently only supports rank-2 tensors");
    if (tensor->dtype() == TypeCode::Float32) return TensorObject::transposedView(tensor);
    int64_t shape[] = {tensor->dim(1), tensor->dim(0)};
    TensorObject *out = deviceTensor(tensor->dtype(), shape);
    if (tensor->numel() > 0)
        checkHip(camel_hip_transpose2d(hipDType(tensor->dtype()), tensor->deviceData(),
                                       out->deviceOutput(), tensor->dim(0), tensor->dim(1)));
    return out;
}

// tensorConcat (runtime.cpp:722-773).
TensorObject *tensorConcat(const TensorObject *lhs, const TensorObject *rhs, int64_t axis) {
    if (lhs->rank() != rhs->rank())
        throw std::invalid_argument("concat requires tensors with the same rank");
    if (axis < 0 || axis >= static_cast<int64_t>(lhs->rank()))
        throw std::invalid_argument("concat axis out of range");
    if (lhs->dtype() != rhs->dtype())
        throw std::invalid_argument("concat currently requires matching dtypes");
    std::vector<int64_t> shape(lhs->shape(), lhs->shape() + lhs->rank());
    for (size_t i = 0; i < lhs->rank(); ++i) {
        if (static_cast<int64_t>(i) == axis) continue;
        if (lhs->dim(i) != rhs->dim(i))
            throw std::invalid_argument("concat requires equal non-axis dimensions");
    }
    shape[static_cast<size_t>(axis)] += rhs->dim(static_cast<size_t>(axis));
    TensorObject *out = deviceTensor(lhs->dtype(), shape);
    int64_t inner = 1, outer = 1;
    for (size_t i = static_cast<size_t>(axis) + 1; i < lhs->rank(); ++i) inner *= lhs->dim(i);
    for (size_t i = 0; i < static_cast<size_t>(axis); ++i) outer *= lhs->dim(i);
    if (out->numel() > 0)
        checkHip(camel_hip_concat(hipDType(lhs->dtype()), lhs->deviceData(), rhs->deviceData(),
                                  out->deviceOutput(), outer, lhs->dim(axis), rhs->dim(axis), inner));
    return out;
}

// tensorBinary (runtime.cpp:775-793): matching shapes only; divide and pow
// produce Float32.
TensorObject *tensorBinary(const TensorObject *lhs, const TensorObject *rhs, BinaryOp op) {
    if (!lhs->sameShape(rhs))
        throw std::invalid_argument("Tensor binary operation requires matching shapes");
    TypeCode outType = promoteTensorTypes(lhs->dtype(), rhs->dtype());
    if (op == BinaryOp::Divide || op == BinaryOp::Power) outType = TypeCode::Float32;
    TensorObject *out = deviceTensor(outType, shapeOf(lhs));
    if (lhs->numel() > 0)
        checkHip(camel_hip_binary(hipBinary(op), hipDType(lhs->dtype()), lhs->deviceData(),
                                  hipDType(rhs->dtype()), rhs->deviceData(), hipDType(outType),
                                  out->deviceOutput(), (int64_t)lhs->numel()));
    return out;
}

// tensorBinaryScalarRight / Left (runtime.cpp:795-831).
TensorObject *tensorBinaryScalarRight(const TensorObject *lhs, TypeCode rhsType, slot_t rhs,
                                      BinaryOp op) {
    TypeCode outType = promoteTensorTypes(lhs->dtype(), tensorDTypeFromValueType(rhsType));
    if (op == BinaryOp::Divide || op == BinaryOp::Power) outType = TypeCode::Float32;
    const double value = scalarToDouble(rhsType, rhs);
    TensorObject *out = deviceTensor(outType, shapeOf(lhs));
    if (lhs->numel() > 0)
        checkHip(camel_hip_binary_scalar(hipBinary(op), 0, hipDType(lhs->dtype()), lhs->deviceData(),
                                         value, hipDType(outType), out->deviceOutput(),
                                         (int64_t)lhs->numel()));
    return out;
}

TensorObject *tensorBinaryScalarLeft(TypeCode lhsType, slot_t lhs, const TensorObject *rhs,
                                     BinaryOp op) {
    TypeCode outType = promoteTensorTypes(tensorDTypeFromValueType(lhsType), rhs->dtype());
    if (op == BinaryOp::Divide || op == BinaryOp::Power) outType = TypeCode::Float32;
    const double value = scalarToDouble(lhsType, lhs);
    TensorObject *out = deviceTensor(outType, shapeOf(rhs));
    if (rhs->numel() > 0)
        checkHip(camel_hip_binary_scalar(hipBinary(op), 1, hipDType(rhs->dtype()), rhs->deviceData(),
                                         value, hipDType(outType), out->deviceOutput(),
                                         (int64_t)rhs->numel()));
    return out;
}

// tensorCompareScalarRight / Left / tensorCompare (runtime.cpp:833-877).
TensorObject *tensorCompareScalarRight(const TensorObject *lhs, TypeCode rhsType, slot_t rhs,
                                       CompareOp op) {
    const double value = scalarToDouble(rhsType, rhs);
    TensorObject *out = deviceTensor(TypeCode::Bool, shapeOf(lhs));
    if (lhs->numel() > 0)
        checkHip(camel_hip_compare_scalar(hipCompare(op), 0, hipDType(lhs->dtype()), lhs->deviceData(),
                                          value, static_cast<uint8_t *>(out->deviceOutput()),
                                          (int64_t)lhs->numel()));
    return out;
}

TensorObject *tensorCompareScalarLeft(TypeCode lhsType, slot_t lhs, const TensorObject *rhs,
                                      CompareOp op) {
    const double value = scalarToDouble(lhsType, lhs);
    TensorObject *out = deviceTensor(TypeCode::Bool, shapeOf(rhs));
    if (rhs->numel() > 0)
        checkHip(camel_hip_compare_scalar(hipCompare(op), 1, hipDType(rhs->dtype()), rhs->deviceData(),
                                          value, static_cast<uint8_t *>(out->deviceOutput()),
                                          (int64_t)rhs->numel()));
    return out;
}

TensorObject *tensorCompare(const TensorObject *lhs, const TensorObject *rhs, CompareOp op) {
    if (!lhs->sameShape(rhs))
        throw std::invalid_argument("Tensor comparison requires matching shapes");
    TensorObject *out = deviceTensor(TypeCode::Bool, shapeOf(lhs));
    if (lhs->numel() > 0)
        checkHip(camel_hip_compare(hipCompare(op), hipDType(lhs->dtype()), lhs->deviceData(),
                                   hipDType(rhs->dtype()), rhs->deviceData(),
                                   static_cast<uint8_t *>(out->deviceOutput()), (int64_t)lhs->numel()));
    return out;
}

// __tensor_matmul__ (operators.cpp:740-769): rank-2 operands, inner
// dimensions equal, output dtype promoteTensorTypes.  fp32 x fp32 runs on the
// MFMA GEMM; other dtypes take the exact fp64-accumulating kernel.
TensorObject *tensorMatmul(const TensorObject *lhs, const TensorObject *rhs) {
    if (lhs->rank() != 2 || rhs->rank() != 2)
        throw std::invalid_argument("matmul currently only supports rank-2 tensors");
    if (lhs->dim(1) != rhs->dim(0)) throw std::invalid_argument("matmul dimension mismatch");
    const int64_t M = lhs->dim(0), K = lhs->dim(1), N = rhs->dim(1);
    int64_t shape[] = {M, N};
    const TypeCode outType = promoteTensorTypes(lhs->dtype(), rhs->dtype());
    TensorObject *out = deviceTensor(outType, shape);
    if (M == 0 || N == 0) return out;
    if (K == 0) {
        fill(out, 0.0);
        return out;
    }
    if (lhs->dtype() == TypeCode::Float32 && rhs->dtype() == TypeCode::Float32) {
        // A transposed lhs (transpose(X) @ E) is read in place.
        std::shared_ptr<Storage> keep;
        bool lhsT = false;
        const void *a = lhs->storedDeviceData(keep, lhsT);
        checkHip(camel_hip_sgemm(static_cast<const float *>(a),
                                 static_cast<const float *>(rhs->deviceData()),
                                 static_cast<float *>(out->deviceOutput()), M, N, K, nullptr,
                                 lhsT ? CAMEL_GEMM_A_T : CAMEL_EPI_NONE));
    } else {
        checkHip(camel_hip_matmul_generic(hipDType(lhs->dtype()), lhs->deviceData(),
                                          hipDType(rhs->dtype()), rhs->deviceData(),
                                          hipDType(outType), out->deviceOutput(), M, N, K));
    }
    return out;
}

// tensorSum (runtime.cpp:879-885): fp64 sum of all elements.
double tensorSum(const TensorObject *tensor) {
    double result = 0.0;
    if (tensor->numel() > 0)
        checkHip(camel_hip_sum(hipDType(tensor->dtype()), tensor->deviceData(),
                               (int64_t)tensor->numel(), &result));
    return result;
}

// tensorSumAxis / MaxAxis / ArgmaxAxis (runtime.cpp:887-1011).
TensorObject *tensorSumAxis(const TensorObject *tensor, int64_t axis) {
    if (tensor->rank() != 2)
        throw std::invalid_argument("sum(axis) currently only supports rank-2 tensors");
    axis = normaliseAxis(axis, "sum");
    int64_t shape[] = {axis == 0 ? tensor->dim(1) : tensor->dim(0)};
    TensorObject *out = TensorObject::create(TypeCode::Float32, shape, Residence::Device, true);
    if (shape[0] > 0 && tensor->numel() > 0)
        checkHip(camel_hip_sum_axis(hipDType(tensor->dtype()), tensor->deviceData(), tensor->dim(0),
                                    tensor->dim(1), axis, static_cast<float *>(out->deviceOutput())));
    return out;
}

TensorObject *tensorMaxAxis(const TensorObject *tensor, int64_t axis) {
    if (tensor->rank() != 2)
        throw std::invalid_argument("max(axis) currently only supports rank-2 tensors");
    axis = normaliseAxis(axis, "max");
    int64_t shape[] = {axis == 0 ? tensor->dim(1) : tensor->dim(0)};
    TensorObject *out = deviceTensor(TypeCode::Float32, shape);
    if (shape[0] > 0) {
        if (tensor->numel() == 0) throw std::invalid_argument("Tensor flat index out of range");
        checkHip(camel_hip_max_axis(hipDType(tensor->dtype()), tensor->deviceData(), tensor->dim(0),
                                    tensor->dim(1), axis, static_cast<float *>(out->deviceOutput())));
    }
    return out;
}

TensorObject *tensorArgmaxAxis(const TensorObject *tensor, int64_t axis) {
    if (tensor->rank() != 2)
        throw std::invalid_argument("argmax(axis) currently only supports rank-2 tensors");
    axis = normaliseAxis(axis, "argmax");
    int64_t shape[] = {axis == 0 ? tensor->dim(1) : tensor->dim(0)};
    TensorObject *out = deviceTensor(TypeCode::Int64, shape);
    if (shape[0] > 0) {
        if (tensor->numel() == 0) throw std::invalid_argument("Tensor flat index out of range");
        checkHip(camel_hip_argmax_axis(hipDType(tensor->dtype()), tensor->deviceData(),
                                       tensor->dim(0), tensor->dim(1), axis,
                                       static_cast<int64_t *>(out->deviceOutput())));
    }
    return out;
}

// tensorExp / tensorLog (runtime.cpp:1013-1045).
TensorObject *tensorExp(const TensorObject *tensor) {
    if (!isFloatingTensorType(tensor->dtype()))
        throw std::invalid_argument("exp requires floating-point tensor");
    TensorObject *out = deviceTensor(TypeCode::Float32, shapeOf(tensor));
    if (tensor->numel() > 0)
        checkHip(camel_hip_exp(static_cast<const float *>(tensor->deviceData()),
                               static_cast<float *>(out->deviceOutput()), (int64_t)tensor->numel()));
    return out;
}

TensorObject *tensorLog(const TensorObject *tensor) {
    if (!isFloatingTensorType(tensor->dtype()))
        throw std::invalid_argument("log requires floating-point tensor");
    TensorObject *out = deviceTensor(TypeCode::Float32, shapeOf(tensor));
    if (tensor->numel() > 0)
        checkHip(camel_hip_log(static_cast<const float *>(tensor->deviceData()),
                               static_cast<float *>(out->deviceOutput()), (int64_t)tensor->numel()));
    return out;
}

// tensorIndex1D / 2D (runtime.cpp:1047-1065): one element crosses to the host.
double tensorIndex1D(const TensorObject *tensor, int64_t index) {
    if (tensor->rank() != 1)
        throw std::invalid_argument("Single-index tensor access requires rank-1 tensor");
    if (index < 0 || index >= tensor->dim(0)) throw std::invalid_argument("Tensor index out of bounds");
    return tensor->getAsDouble(static_cast<uint64_t>(index));
}

double tensorIndex2D(const TensorObject *tensor, int64_t row, int64_t col) {
    if (tensor->rank() != 2)
        throw std::invalid_argument("Two-index tensor access requires rank-2 tensor");
    if (row < 0 || row >= tensor->dim(0) || col < 0 || col >= tensor->dim(1))
        throw std::invalid_argument("Tensor index out of bounds");
    return tensor->getAsDouble(static_cast<uint64_t>(row * tensor->dim(1) + col));
}

// ---- layers ----------------------------------------------------------------------

// relu(x) = multiply(x, gt(x, 0)) (test/run/nn/svm.cml:31): Float32 in one
// pass; other dtypes through the two reference ops on the device.
TensorObject *tensorRelu(const TensorObject *tensor) {
    if (tensor->dtype() == TypeCode::Float32) {
        TensorObject *out = deviceTensor(TypeCode::Float32, shapeOf(tensor));
        if (tensor->numel() > 0)
            checkHip(camel_hip_relu(static_cast<const float *>(tensor->deviceData()),
                                    static_cast<float *>(out->deviceOutput()), (int64_t)tensor->numel()));
        return out;
    }
    TensorObject *mask = tensorCompareScalarRight(tensor, TypeCode::Int64, toSlot<int64_t>(0),
                                                  CompareOp::Greater);
    TensorObject *out = tensorBinary(tensor, mask, BinaryOp::Multiply);
    releaseTensor(mask);
    return out;
}

// softmax(logits) of test/run/nn/mnist.cml:13-25, rows of a rank-2 tensor.
// Float32 runs the fused one-pass kernel; other dtypes run the nine-operator
// composition itself on the device (subtract promotes them to Float32).
TensorObject *tensorSoftmax(const TensorObject *tensor) {
    requireRank2(tensor, "softmax");
    const int64_t n = tensor->dim(0), k = tensor->dim(1);
    if (tensor->dtype() == TypeCode::Float32) {
        TensorObject *out = deviceTensor(TypeCode::Float32, shapeOf(tensor));
        if (tensor->numel() > 0)
            checkHip(camel_hip_softmax_rows(static_cast<const float *>(tensor->deviceData()),
                                            static_cast<float *>(out->deviceOutput()), n, k));
        return out;
    }
    std::vector<TensorObject *> tmp;
    auto keep = [&](TensorObject *t) {
        tmp.push_back(t);
        return t;
    };
    int64_t col[] = {n, 1}, row[] = {1, k};
    TensorObject *ones = keep(tensorOnes(TypeCode::Float32, row));
    TensorObject *mb = keep(tensorMatmul(keep(tensorReshape(keep(tensorMaxAxis(tensor, 1)), col)), ones));
    TensorObject *e = keep(tensorExp(keep(tensorBinary(tensor, mb, BinaryOp::Subtract))));
    TensorObject *sb = keep(tensorMatmul(keep(tensorReshape(keep(tensorSumAxis(e, 1)), col)), ones));
    TensorObject *out = tensorBinary(e, sb, BinaryOp::Divide);
    for (TensorObject *t : tmp) releaseTensor(t);
    return out;
}

// dense: y = x @ W (+ b) (relu).  x [M, K], W [K, N], b [N] or [1, N].  The
// bias add and relu run in the GEMM epilogue (one rounding each, as the
// reference's separate add and multiply ops round).
TensorObject *tensorDense(const TensorObject *x, const TensorObject *w, const TensorObject *bias,
                          bool relu) {
    if (x->rank() != 2 || w->rank() != 2)
        throw std::invalid_argument("dense currently only supports rank-2 tensors");
    if (x->dim(1) != w->dim(0)) throw std::invalid_argument("dense dimension mismatch");
    const int64_t M = x->dim(0), K = x->dim(1), N = w->dim(1);
    if (bias && !(bias->numel() == static_cast<uint64_t>(N) &&
                  (bias->rank() == 1 || (bias->rank() == 2 && bias->dim(0) == 1))))
        throw std::invalid_argument("dense bias must have shape [N] or [1, N]");
    const bool fp32 = x->dtype() == TypeCode::Float32 && w->dtype() == TypeCode::Float32 &&
                      (!bias || bias->dtype() == TypeCode::Float32);
    if (!fp32 || K == 0) {
        // Composition on the device: matmul, then add (bias broadcast), then relu.
        TensorObject *y = tensorMatmul(x, w);
        if (bias) {
            int64_t ones_shape[] = {M, 1}, b_shape[] = {1, N};
            TensorObject *ones = tensorOnes(TypeCode::Float32, ones_shape);
            TensorObject *b2 = tensorReshape(bias, b_shape);
            TensorObject *bb = tensorMatmul(ones, b2);
            TensorObject *sum = tensorBinary(y, bb, BinaryOp::Add);
            for (TensorObject *t : {ones, b2, bb, y}) releaseTensor(t);
            y = sum;
        }
        if (relu) {
            TensorObject *r = tensorRelu(y);
            releaseTensor(y);
            y = r;
        }
        return y;
    }
    int64_t shape[] = {M, N};
    TensorObject *out = deviceTensor(TypeCode::Float32, shape);
    if (M == 0 || N == 0) return out;
    std::shared_ptr<Storage> keep;
    bool xT = false;
    const void *a = x->storedDeviceData(keep, xT);
    const int flags = (bias ? CAMEL_EPI_BIAS : 0) | (relu ? CAMEL_EPI_RELU : 0) |
                      (xT ? CAMEL_GEMM_A_T : 0);
    checkHip(camel_hip_sgemm(static_cast<const float *>(a),
                             static_cast<const float *>(w->deviceData()),
                             static_cast<float *>(out->deviceOutput()), M, N, K,
                             bias ? static_cast<const float *>(bias->deviceData()) : nullptr, flags));
    return out;
}

// dense (relu) then row softmax, the classifier head of README.md:43.  Float32
// runs camel_hip_dense_softmax (one fused kernel for N <= 32, otherwise the
// GEMM then the softmax kernel: the values of tensorDense then
// tensorSoftmax); other dtypes run those two functions.
TensorObject *tensorDenseSoftmax(const TensorObject *x, const TensorObject *w,
                                 const TensorObject *bias, bool relu) {
    if (x->rank() != 2 || w->rank() != 2)
        throw std::invalid_argument("dense currently only supports rank-2 tensors");
    if (x->dim(1) != w->dim(0)) throw std::invalid_argument("dense dimension mismatch");
    const int64_t M = x->dim(0), K = x->dim(1), N = w->dim(1);
    if (bias && !(bias->numel() == static_cast<uint64_t>(N) &&
                  (bias->rank() == 1 || (bias->rank() == 2 && bias->dim(0) == 1))))
        throw std::invalid_argument("dense bias must have shape [N] or [1, N]");
    const bool fp32 = x->dtype() == TypeCode::Float32 && w->dtype() == TypeCode::Float32 &&
                      (!bias || bias->dtype() == TypeCode::Float32);
    if (!fp32 || K == 0) {
        TensorObject *y = tensorDense(x, w, bias, relu);
        TensorObject *p = tensorSoftmax(y);
        releaseTensor(y);
        return p;
    }
    int64_t shape[] = {M, N};
    TensorObject *out = deviceTensor(TypeCode::Float32, shape);
    if (M == 0 || N == 0) return out;
    const int flags = (bias ? CAMEL_EPI_BIAS : 0) | (relu ? CAMEL_EPI_RELU : 0);
    checkHip(camel_hip_dense_softmax(static_cast<const float *>(x->deviceData()),
                                     static_cast<const float *>(w->deviceData()),
                                     bias ? static_cast<const float *>(bias->deviceData()) : nullptr,
                                     static_cast<float *>(out->deviceOutput()), M, N, K, flags));
    return out;
}

// dense (relu) then dense (relu) (then softmax): a classifier head of
// README.md:40-46.  Float32 runs camel_hip_dense_head (layer 2's kernel adds
// layer 1's split-K partials itself where layer 1 splits K; the values of
// the two layers' functions either way); other dtypes and empty inner
// dimensions run tensorDense then tensorDense / tensorDenseSoftmax.
TensorObject *tensorDenseHead(const TensorObject *x, const TensorObject *w1,
                              const TensorObject *b1, bool relu1, const TensorObject *w2,
                              const TensorObject *b2, bool relu2, bool softmax) {
    auto check = [](const TensorObject *a, const TensorObject *w, const TensorObject *b) {
        if (a->rank() != 2 || w->rank() != 2)
            throw std::invalid_argument("dense currently only supports rank-2 tensors");
        if (a->dim(1) != w->dim(0)) throw std::invalid_argument("dense dimension mismatch");
        if (b && !(b->numel() == static_cast<uint64_t>(w->dim(1)) &&
                   (b->rank() == 1 || (b->rank() == 2 && b->dim(0) == 1))))
            throw std::invalid_argument("dense bias must have shape [N] or [1, N]");
    };
    check(x, w1, b1);
    const int64_t M = x->dim(0), K1 = x->dim(1), N1 = w1->dim(1);
    if (w2->rank() != 2) throw std::invalid_argument("dense currently only supports rank-2 tensors");
    if (N1 != w2->dim(0)) throw std::invalid_argument("dense dimension mismatch");
    if (b2 && !(b2->numel() == static_cast<uint64_t>(w2->dim(1)) &&
                (b2->rank() == 1 || (b2->rank() == 2 && b2->dim(0) == 1))))
        throw std::invalid_argument("dense bias must have shape [N] or [1, N]");
    const int64_t N2 = w2->dim(1);
    auto f32 = [](const TensorObject *t) { return !t || t->dtype() == TypeCode::Float32; };
    const bool fp32 = x->dtype() == TypeCode::Float32 && f32(w1) && f32(b1) && f32(w2) && f32(b2);
    if (!fp32 || K1 == 0 || N1 == 0) {
        TensorObject *h = tensorDense(x, w1, b1, relu1);
        TensorObject *y = nullptr;
        try {
            y = softmax ? tensorDenseSoftmax(h, w2, b2, relu2) : tensorDense(h, w2, b2, relu2);
        } catch (...) {
            releaseTensor(h);
            throw;
        }
        releaseTensor(h);
        return y;
    }
    int64_t shape[] = {M, N2};
    TensorObject *out = deviceTensor(TypeCode::Float32, shape);
    if (M == 0 || N2 == 0) return out;
    auto dev = [](const TensorObject *t) {
        return t ? static_cast<const float *>(t->deviceData()) : nullptr;
    };
    checkHip(camel_hip_dense_head(dev(x), dev(w1), dev(b1), dev(w2), dev(b2),
                                  static_cast<float *>(out->deviceOutput()), M, K1, N1, N2,
                                  (b1 ? CAMEL_EPI_BIAS : 0) | (relu1 ? CAMEL_EPI_RELU : 0),
                                  (b2 ? CAMEL_EPI_BIAS : 0) | (relu2 ? CAMEL_EPI_RELU : 0),
                                  softmax ? 1 : 0));
    return out;
}

// conv2d: x [N, C, H, W], w [Co, C, KH, KW], bias [Co] -> y [N, Co, OH, OW],
// OH = (H + 2 pad - KH) / stride + 1.  Float32 only.
std::array<int64_t, 4> conv2dOutputShape(std::span<const int64_t> xs, TypeCode xdtype,
                                         const TensorObject *w, const TensorObject *bias,
                                         int64_t stride, int64_t pad) {
    if (xs.size() != 4 || w->rank() != 4)
        throw std::invalid_argument("conv2d requires rank-4 NCHW input and rank-4 weights");
    if (xdtype != TypeCode::Float32 || w->dtype() != TypeCode::Float32 ||
        (bias && bias->dtype() != TypeCode::Float32))
        throw std::invalid_argument("conv2d requires Float32 tensors");
    if (xs[1] != w->dim(1)) throw std::invalid_argument("conv2d channel mismatch");
    if (stride <= 0 || pad < 0) throw std::invalid_argument("conv2d stride must be positive and pad non-negative");
    const int64_t H = xs[2], W = xs[3];
    const int64_t Co = w->dim(0), KH = w->dim(2), KW = w->dim(3);
    if (bias && bias->numel() != static_cast<uint64_t>(Co))
        throw std::invalid_argument("conv2d bias must have one value per output channel");
    if (H + 2 * pad < KH || W + 2 * pad < KW)
        throw std::invalid_argument("conv2d kernel larger than padded input");
    return {xs[0], Co, (H + 2 * pad - KH) / stride + 1, (W + 2 * pad - KW) / stride + 1};
}

void conv2dLaunch(const void *x, std::span<const int64_t> xs, const TensorObject *w,
                  const TensorObject *bias, int64_t stride, int64_t pad, bool relu, bool pool,
                  int layout, void *y, const void *w_packed) {
    const int64_t C = xs[1], KH = w->dim(2), KW = w->dim(3);
    if (C == 0 || KH == 0 || KW == 0) throw std::invalid_argument("conv2d requires a non-empty kernel");
    const int flags = (bias ? CAMEL_EPI_BIAS : 0) | (relu ? CAMEL_EPI_RELU : 0) | layout |
                      (w_packed ? CAMEL_CONV_W_PACKED : 0);
    const float *b = bias ? static_cast<const float *>(bias->deviceData()) : nullptr;
    const void *wd = w_packed ? w_packed : w->deviceData();
    auto *fn = pool ? camel_hip_conv2d_pool2 : camel_hip_conv2d;
    checkHip(fn(static_cast<const float *>(x), static_cast<const float *>(wd), b,
                static_cast<float *>(y), xs[0], C, xs[2], xs[3], w->dim(0), KH, KW, stride, pad,
                flags));
}

TensorObject *tensorConv2d(const TensorObject *x, const TensorObject *w, const TensorObject *bias,
                           int64_t stride, int64_t pad, bool relu) {
    const auto shape = conv2dOutputShape(shapeOf(x), x->dtype(), w, bias, stride, pad);
    TensorObject *out = deviceTensor(TypeCode::Float32, shape);
    if (out->numel() == 0) return out;
    conv2dLaunch(x->deviceData(), shapeOf(x), w, bias, stride, pad, relu, false, 0,
                 out->deviceOutput());
    return out;
}

// conv2d (+bias)(relu) then maxpool2d(2, 2): one fused kernel when the
// convolution runs as the NHWC implicit GEMM (the pool max is taken in its
// epilogue), else the convolution into scratch and the pool kernel.
TensorObject *tensorConv2dPool2(const TensorObject *x, const TensorObject *w,
                                const TensorObject *bias, int64_t stride, int64_t pad, bool relu) {
    const auto cs = conv2dOutputShape(shapeOf(x), x->dtype(), w, bias, stride, pad);
    if (cs[2] < 2 || cs[3] < 2) throw std::invalid_argument("maxpool2d window larger than input");
    int64_t shape[] = {cs[0], cs[1], cs[2] / 2, cs[3] / 2};
    TensorObject *out = deviceTensor(TypeCode::Float32, shape);
    if (out->numel() == 0) return out;
    conv2dLaunch(x->deviceData(), shapeOf(x), w, bias, stride, pad, relu, true, 0,
                 out->deviceOutput());
    return out;
}

// maxpool2d: x [N, C, H, W] -> [N, C, (H-k)/s+1, (W-k)/s+1].
TensorObject *tensorMaxPool2d(const TensorObject *x, int64_t kernel, int64_t stride) {
    if (x->rank() != 4) throw std::invalid_argument("maxpool2d requires a rank-4 NCHW tensor");
    if (x->dtype() != TypeCode::Float32) throw std::invalid_argument("maxpool2d requires a Float32 tensor");
    if (kernel <= 0 || stride <= 0) throw std::invalid_argument("maxpool2d kernel and stride must be positive");
    const int64_t N = x->dim(0), C = x->dim(1), H = x->dim(2), W = x->dim(3);
    if (H < kernel || W < kernel) throw std::invalid_argument("maxpool2d window larger than input");
    int64_t shape[] = {N, C, (H - kernel) / stride + 1, (W - kernel) / stride + 1};
    TensorObject *out = deviceTensor(TypeCode::Float32, shape);
    if (out->numel() == 0) return out;
    checkHip(camel_hip_maxpool2d(static_cast<const float *>(x->deviceData()),
                                 static_cast<float *>(out->deviceOutput()), N, C, H, W, kernel, kernel,
                                 stride));
    return out;
}

} // namespace camel_amd::tensor
