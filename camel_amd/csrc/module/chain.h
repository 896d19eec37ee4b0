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
//   dense (+relu) + dense with N <= 16 (+relu) (+softmax)
//                                     -> camel_hip_dense_head (the second
//                                        layer's kernel adds the first
//                                        one's split-K partials)
//   conv2d (+relu) + maxpool2d(2, 2)  -> camel_hip_conv2d_pool2
//   conv2d 1->32 3x3 (+relu) + conv2d 32->Co 3x3 (+relu) + maxpool2d(2, 2)
//     on 28-wide images               -> camel_hip_conv2d_pair_pool2 (the
//                                        first conv's output stays in LDS)
//   conv2d -> conv2d that reads NCHW4 -> the first writes NCHW4
//                                        ([N][C/4][H][W][4]) and the second
//                                        reads it in place (no transpose)
// A conv2d that runs as the implicit GEMM gets its weights packed once
// per chain (camel_hip_conv2d_pack_weights) instead of once per call.
// Every group's values equal the layer-by-layer operators' bit for bit,
// except conv2d + maxpool2d where the partial last round of a large
// convolution may sum a pixel in another tile shape (within the conv2d
// tolerance).
#pragma once

#include "tensor_object.h"

#include <memory>
#include <mutex>
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
    // payload blocks of w and bias when appended: a handle released and
    // reused for another tensor is caught at apply
    std::shared_ptr<Storage> w_storage, bias_storage;
};

class LayerChain {
public:
    LayerChain() = default;
    LayerChain(const LayerChain &) = delete;
    LayerChain &operator=(const LayerChain &) = delete;
    ~LayerChain();

    // Appends the layer operator `name` ("dense", "dense_relu", "relu",
    // "softmax", "conv2d", "conv2d_relu", "maxpool2d", "reshape"; a
    // "tensor:" prefix is accepted) with its bind arguments: leading tensors
    // (weights, then an optional bias, null for none), then integers.
    void append(const std::string &name, std::vector<const TensorObject *> tensors,
                std::vector<int64_t> ints);
    // x -> chain: a new device tensor.  Throws with the failing layer's error
    // text.
    TensorObject *apply(const TensorObject *x) const;
    // The kernel groups apply would run for an input of this shape and
    // dtype, one per line (e.g. "conv2d_relu+maxpool2d(2,2) x=nchw4").
    std::string plan(std::span<const int64_t> shape, TypeCode dtype = TypeCode::Float32) const;
    size_t size() const { return steps_.size(); }

private:
    struct Group {
        enum Kind { Dense, DenseSoftmax, DenseHead, Conv, ConvPair, Relu, Softmax, MaxPool, Reshape } kind;
        const LayerStep *step; // first layer of the group
        const LayerStep *step2 = nullptr; // DenseHead / ConvPair: the second dense / conv
        bool relu = false;
        bool relu2 = false;    // DenseHead / ConvPair: relu after the second layer
        bool softmax = false;  // DenseHead: row softmax at the end
        bool pool = false;     // conv + maxpool2d(2, 2)
        bool x_nchw4 = false;  // conv input comes NCHW4 from the previous conv
        bool y_nchw4 = false;  // conv output goes NCHW4 to the next conv
        bool w_packed = false; // conv runs as the implicit GEMM: weights packed once
    };
    std::vector<Group> schedule(std::span<const int64_t> shape,
                                TypeCode dtype = TypeCode::Float32) const;
    // The packed form of step i's conv weights (made on first use; tensors
    // never change once made, so it stays valid while the chain lives).
    const void *packedWeights(size_t i) const;
    std::vector<LayerStep> steps_;
    mutable std::mutex pack_mutex_;
    mutable std::vector<void *> packed_;
};

} // namespace camel_amd::tensor
