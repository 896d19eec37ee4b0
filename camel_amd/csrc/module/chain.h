// Composed layer chains: what `dense<w1, b1>..relu..dense<w2, b2>..softmax`
// denotes (README.md:40-46).  The reference's compose operator `..` is a
// stub (src/builtin/operators/macro.cpp:30); a LayerChain is the object a
// compose over tensor layer operators builds, and apply(x) is `x->chain`.
//
// apply runs the layers in order and replaces adjacent layers by one fused
// kernel where that computes the same values:
//   dense + relu, conv2d + relu       -> the GEMM epilogue (as dense_relu,
//                                        conv2d_relu)
//   dense (+relu) + softmax           -> camel_hip_dense_softmax
//   conv2d (+relu) + maxpool2d(2, 2)  -> camel_hip_conv2d_pool2
//   conv2d -> conv2d that reads NHWC  -> the first writes NHWC and the second
//                                        reads it in place (no transpose)
// Every group's values equal the layer-by-layer operators' bit for bit,
// except conv2d + maxpool2d where the partial last round of a large
// convolution may sum a pixel in another tile shape (within the conv2d
// tolerance).
#pragma once

#include "tensor_object.h"

#include <string>
#include <vector>

namespace camel_amd::tensor {

enum class LayerKind { Dense, Relu, Softmax, Conv2d, MaxPool2d, Reshape };

struct LayerStep {
    LayerKind kind;
    bool relu = false;                  // dense_relu / conv2d_relu
    const TensorObject *w = nullptr;    // weights (dense, conv2d)
    const TensorObject *bias = nullptr; // optional bias
    std::vector<int64_t> ints;          // conv2d: stride, pad; maxpool2d: kernel, stride;
                                        // reshape: the target shape
};

class LayerChain {
public:
    // Appends the layer operator `name` ("dense", "dense_relu", "relu",
    // "softmax", "conv2d", "conv2d_relu", "maxpool2d", "reshape"; a
    // "tensor:" prefix is accepted) with its bind arguments: leading tensors
    // (weights, then an optional bias, null for none), then integers.
    void append(const std::string &name, std::vector<const TensorObject *> tensors,
                std::vector<int64_t> ints);
    // x -> chain: a new device tensor.  Throws with the failing layer's error
    // text.
    TensorObject *apply(const TensorObject *x) const;
    // The kernel groups apply would run for an input of this shape, one per
    // line (e.g. "conv2d_relu+maxpool2d(2,2) x=nhwc").
    std::string plan(std::span<const int64_t> shape) const;
    size_t size() const { return steps_.size(); }

private:
    struct Group {
        enum Kind { Dense, DenseSoftmax, Conv, Relu, Softmax, MaxPool, Reshape } kind;
        const LayerStep *step; // first layer of the group
        bool relu = false;
        bool pool = false;     // conv + maxpool2d(2, 2)
        bool x_nhwc = false;   // conv input comes NHWC from the previous conv
        bool y_nhwc = false;   // conv output goes NHWC to the next conv
    };
    std::vector<Group> schedule(std::span<const int64_t> shape) const;
    std::vector<LayerStep> steps_;
};

} // namespace camel_amd::tensor
