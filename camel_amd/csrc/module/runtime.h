// Tensor kernels of the operator layer: the functions of the reference's
// modules/tensor/runtime.h:116-165, same names and checks, running on the
// gfx950 device through libcamel_hip (include/camel_hip.h), plus the layers
// the reference composes in Camel source (relu, softmax, dense, conv2d,
// maxpool2d).
#pragma once

#include "tensor_object.h"

#include <array>

namespace camel_amd::tensor {

TensorObject *tensorEmpty(TypeCode dtype, std::span<const int64_t> shape);
TensorObject *tensorZeros(TypeCode dtype, std::span<const int64_t> shape);
TensorObject *tensorOnes(TypeCode dtype, std::span<const int64_t> shape);
TensorObject *tensorFull(TypeCode dtype, std::span<const int64_t> shape, double value);
TensorObject *tensorRandom(std::span<const int64_t> shape, double low, double high);
TensorObject *tensorArange(int64_t start, int64_t stop, int64_t step);
TensorObject *tensorEye(int64_t size);
TensorObject *tensorReshape(const TensorObject *tensor, std::span<const int64_t> shape);
TensorObject *tensorTranspose2D(const TensorObject *tensor);
TensorObject *tensorConcat(const TensorObject *lhs, const TensorObject *rhs, int64_t axis);
TensorObject *tensorBinary(const TensorObject *lhs, const TensorObject *rhs, BinaryOp op);
TensorObject *tensorBinaryScalarRight(const TensorObject *lhs, TypeCode rhsType, slot_t rhs,
                                      BinaryOp op);
TensorObject *tensorBinaryScalarLeft(TypeCode lhsType, slot_t lhs, const TensorObject *rhs,
                                     BinaryOp op);
TensorObject *tensorCompareScalarRight(const TensorObject *lhs, TypeCode rhsType, slot_t rhs,
                                       CompareOp op);
TensorObject *tensorCompareScalarLeft(TypeCode lhsType, slot_t lhs, const TensorObject *rhs,
                                      CompareOp op);
TensorObject *tensorCompare(const TensorObject *lhs, const TensorObject *rhs, CompareOp op);
TensorObject *tensorMatmul(const TensorObject *lhs, const TensorObject *rhs);

double tensorSum(const TensorObject *tensor);
TensorObject *tensorSumAxis(const TensorObject *tensor, int64_t axis);
TensorObject *tensorMaxAxis(const TensorObject *tensor, int64_t axis);
TensorObject *tensorArgmaxAxis(const TensorObject *tensor, int64_t axis);
TensorObject *tensorExp(const TensorObject *tensor);
TensorObject *tensorLog(const TensorObject *tensor);
double tensorIndex1D(const TensorObject *tensor, int64_t index);
double tensorIndex2D(const TensorObject *tensor, int64_t row, int64_t col);

// Layers with no reference operator, defined by the reference compositions:
// relu(x) = x * (x > 0) (test/run/nn/svm.cml:31); softmax = the row softmax of
// test/run/nn/mnist.cml:13-25; dense = x @ W (+ ones @ b) (mnist.cml:18,
// README.md:40-46), optionally followed by relu; conv2d = direct NCHW
// convolution with matmul semantics, optional bias and relu; maxpool2d =
// window max with tensorMaxAxis's first-strict-'>' rule.
TensorObject *tensorRelu(const TensorObject *tensor);
TensorObject *tensorSoftmax(const TensorObject *tensor);
TensorObject *tensorDense(const TensorObject *x, const TensorObject *w, const TensorObject *bias,
                          bool relu);
TensorObject *tensorConv2d(const TensorObject *x, const TensorObject *w, const TensorObject *bias,
                           int64_t stride, int64_t pad, bool relu);
TensorObject *tensorMaxPool2d(const TensorObject *x, int64_t kernel, int64_t stride);

// Fused layer pairs for composed chains (the reference's compose `..` is a
// stub, src/builtin/operators/macro.cpp:30): dense (relu) then softmax,
// dense (relu) then a narrow dense (relu, softmax), and conv2d (relu) then
// maxpool2d(2, 2).  Same checks and error texts as the layers they fuse.
TensorObject *tensorDenseSoftmax(const TensorObject *x, const TensorObject *w,
                                 const TensorObject *bias, bool relu);
TensorObject *tensorConv2dPool2(const TensorObject *x, const TensorObject *w,
                                const TensorObject *bias, int64_t stride, int64_t pad, bool relu);
// dense (relu) then dense (relu) (then softmax), the two layers of a
// classifier head; the values of the two layers' functions.
TensorObject *tensorDenseHead(const TensorObject *x, const TensorObject *w1,
                              const TensorObject *b1, bool relu1, const TensorObject *w2,
                              const TensorObject *b2, bool relu2, bool softmax);
// The conv2d checks (error texts of tensorConv2d) on an input of shape xs and
// dtype xdtype; returns the NCHW output shape.
std::array<int64_t, 4> conv2dOutputShape(std::span<const int64_t> xs, TypeCode xdtype,
                                         const TensorObject *w, const TensorObject *bias,
                                         int64_t stride, int64_t pad);
// Runs a checked conv2d on device memory: x and y are NCHW unless `layout`
// carries CAMEL_CONV_X_NHWC / CAMEL_CONV_Y_NHWC; pool adds maxpool2d(2, 2)
// (y is then the pooled NCHW result); w_packed, if given, is w already
// packed by camel_hip_conv2d_pack_weights.
void conv2dLaunch(const void *x, std::span<const int64_t> xs, const TensorObject *w,
                  const TensorObject *bias, int64_t stride, int64_t pad, bool relu, bool pool,
                  int layout, void *y, const void *w_packed = nullptr);

} // namespace camel_amd::tensor
