// LayerChain: composed tensor layers applied in order, with adjacent layers
// run as one fused kernel where that computes the same values (chain.h).
#include "chain.h"

#include "camel_hip.h"
#include "runtime.h"

#include <sstream>
#include <stdexcept>

namespace camel_amd::tensor {

namespace {

std::string stripPrefix(const std::string &name) {
    return name.rfind("tensor:", 0) == 0 ? name.substr(7) : name;
}

// The implicit GEMM of libcamel_hip reads an NCHW4 input in place when
// C % 16 == 0 and C*KH*KW exceeds the direct kernel's 32 (for an NCHW input
// its transpose runs one image per grid z, so the batch stays below 65535).
// Only then is an NCHW4 intermediate worth writing.
bool readsInPlace(const LayerStep &conv, int64_t batch) {
    const int64_t C = conv.w->dim(1), KH = conv.w->dim(2), KW = conv.w->dim(3);
    return C % 16 == 0 && C * KH * KW > 32 && batch < 65535;
}

int64_t intOr(const LayerStep &s, size_t i, int64_t fallback) {
    return i < s.ints.size() ? s.ints[i] : fallback;
}

bool isF32(const TensorObject *t) { return !t || t->dtype() == TypeCode::Float32; }

// The shapes camel_hip_conv2d_pair_pool2 serves: x [N, 1, H, 28] Float32,
// conv1 32 x 1 x 3 x 3 and conv2 Co x 32 x 3 x 3 (Co % 64 == 0), both
// stride 1, unpadded, with [Co] biases, and (H - 4) % 8 == 0.
bool pairServes(std::span<const int64_t> xs, TypeCode xdt, const LayerStep &c1,
                const LayerStep &c2) {
    auto conv3 = [](const LayerStep &c, int64_t cin) {
        return c.w->rank() == 4 && c.w->dim(1) == cin && c.w->dim(2) == 3 && c.w->dim(3) == 3 &&
               intOr(c, 0, 1) == 1 && intOr(c, 1, 0) == 0 && isF32(c.w) && isF32(c.bias) &&
               (!c.bias || (c.bias->rank() == 1 && c.bias->dim(0) == c.w->dim(0)));
    };
    return xs.size() == 4 && xdt == TypeCode::Float32 && xs[1] == 1 && xs[3] == 28 && xs[2] >= 6 &&
           (xs[2] - 4) % 8 == 0 && conv3(c1, 1) && c1.w->dim(0) == 32 && conv3(c2, 32) &&
           c2.w->dim(0) % 64 == 0;
}

// A device activation between two groups: a tensor, or an NCHW4 buffer
// ([N][C/4][H][W][4]) of the logical NCHW shape `shape` that only a conv
// reads.
struct Activation {
    const TensorObject *tensor = nullptr;
    bool owned = false;
    void *nchw4 = nullptr;
    std::vector<int64_t> shape;

    Activation() = default;
    Activation(const Activation &) = delete;
    Activation &operator=(const Activation &) = delete;
    Activation(Activation &&o) noexcept { *this = std::move(o); }
    Activation &operator=(Activation &&o) noexcept {
        if (this != &o) {
            reset();
            tensor = o.tensor;
            owned = o.owned;
            nchw4 = o.nchw4;
            shape = std::move(o.shape);
            o.tensor = nullptr;
            o.owned = false;
            o.nchw4 = nullptr;
        }
        return *this;
    }
    ~Activation() { reset(); }
    void reset() {
        if (owned && tensor) releaseTensor(const_cast<TensorObject *>(tensor));
        if (nchw4) camel_hip_free(nchw4);
        tensor = nullptr;
        owned = false;
        nchw4 = nullptr;
    }
    static Activation of(TensorObject *t) {
        Activation a;
        a.tensor = t;
        a.owned = true;
        a.shape.assign(t->shape(), t->shape() + t->rank());
        return a;
    }
};

void requireLive(const TensorObject *t, const std::shared_ptr<Storage> &storage) {
    if (t && (!isLiveTensor(t) || t->storage() != storage))
        throw std::invalid_argument("chain layer weights were released");
}

} // namespace

void LayerChain::append(const std::string &name, std::vector<const TensorObject *> tensors,
                        std::vector<int64_t> ints) {
    const std::string op = stripPrefix(name);
    LayerStep s{};
    auto tensor = [&](size_t i) { return i < tensors.size() ? tensors[i] : nullptr; };
    if (op == "dense" || op == "dense_relu") {
        s.kind = LayerKind::Dense;
        s.relu = op == "dense_relu";
        if (!tensor(0)) throw std::invalid_argument("dense requires weights");
    } else if (op == "conv2d" || op == "conv2d_relu") {
        s.kind = LayerKind::Conv2d;
        s.relu = op == "conv2d_relu";
        if (!tensor(0)) throw std::invalid_argument("conv2d requires weights");
        if (tensor(0)->rank() != 4)
            throw std::invalid_argument("conv2d requires rank-4 NCHW input and rank-4 weights");
    } else if (op == "relu") {
        s.kind = LayerKind::Relu;
    } else if (op == "softmax") {
        s.kind = LayerKind::Softmax;
    } else if (op == "maxpool2d") {
        s.kind = LayerKind::MaxPool2d;
    } else if (op == "reshape") {
        s.kind = LayerKind::Reshape;
    } else {
        throw std::invalid_argument("Unrecognized layer operator: " + name);
    }
    s.w = tensor(0);
    s.bias = tensor(1);
    if (s.w) s.w_storage = s.w->storage();
    if (s.bias) s.bias_storage = s.bias->storage();
    s.ints = std::move(ints);
    steps_.push_back(std::move(s));
    std::lock_guard<std::mutex> lock(pack_mutex_);
    packed_.push_back(nullptr);
}

LayerChain::~LayerChain() {
    for (void *p : packed_)
        if (p) camel_hip_free(p);
}

const void *LayerChain::packedWeights(size_t i) const {
    std::lock_guard<std::mutex> lock(pack_mutex_);
    if (!packed_[i]) {
        const TensorObject *w = steps_[i].w;
        void *p = nullptr;
        checkHip(camel_hip_malloc(&p, w->byteSize()));
        const int rc = camel_hip_conv2d_pack_weights(static_cast<const float *>(w->deviceData()),
                                                     static_cast<float *>(p), w->dim(0), w->dim(1),
                                                     w->dim(2), w->dim(3));
        if (rc != CAMEL_HIP_OK) {
            camel_hip_free(p);
            checkHip(rc);
        }
        packed_[i] = p;
    }
    return packed_[i];
}

std::vector<LayerChain::Group> LayerChain::schedule(std::span<const int64_t> shape,
                                                    TypeCode dtype) const {
    std::vector<Group> groups;
    // Batch of the current activation where it is known (rank-4 shapes are
    // propagated through conv / pool / relu; anything else stops NCHW4
    // pairing, which only changes speed, never values).
    int64_t batch = shape.size() == 4 ? shape[0] : -1;
    const size_t n = steps_.size();
    for (size_t i = 0; i < n;) {
        const LayerStep &s = steps_[i];
        Group g{};
        g.step = &s;
        size_t j = i + 1;
        switch (s.kind) {
        case LayerKind::Dense:
            g.relu = s.relu;
            if (!g.relu && j < n && steps_[j].kind == LayerKind::Relu) {
                g.relu = true;
                ++j;
            }
            g.kind = Group::Dense;
            if (j < n && steps_[j].kind == LayerKind::Softmax) {
                g.kind = Group::DenseSoftmax;
                ++j;
            } else if (j < n && steps_[j].kind == LayerKind::Dense && steps_[j].w->rank() == 2 &&
                       steps_[j].w->dim(1) <= 16) {
                // a narrow second dense: the pair runs as one head
                g.kind = Group::DenseHead;
                g.step2 = &steps_[j];
                g.relu2 = steps_[j].relu;
                ++j;
                if (!g.relu2 && j < n && steps_[j].kind == LayerKind::Relu) {
                    g.relu2 = true;
                    ++j;
                }
                if (j < n && steps_[j].kind == LayerKind::Softmax) {
                    g.softmax = true;
                    ++j;
                }
            }
            batch = -1;
            break;
        case LayerKind::Conv2d:
            g.kind = Group::Conv;
            g.relu = s.relu;
            if (!g.relu && j < n && steps_[j].kind == LayerKind::Relu) {
                g.relu = true;
                ++j;
            }
            if (groups.empty() && j < n && steps_[j].kind == LayerKind::Conv2d &&
                pairServes(shape, dtype, s, steps_[j])) {
                // conv2d (relu) conv2d (relu) maxpool2d(2, 2) at the chain's
                // start: one kernel, the first conv's output kept in LDS
                size_t k = j + 1;
                bool relu2 = steps_[j].relu;
                if (!relu2 && k < n && steps_[k].kind == LayerKind::Relu) {
                    relu2 = true;
                    ++k;
                }
                if (k < n && steps_[k].kind == LayerKind::MaxPool2d && intOr(steps_[k], 0, 2) == 2 &&
                    intOr(steps_[k], 1, intOr(steps_[k], 0, 2)) == 2) {
                    g.kind = Group::ConvPair;
                    g.step2 = &steps_[j];
                    g.relu2 = relu2;
                    g.pool = true;
                    groups.push_back(g);
                    i = k + 1;
                    continue;
                }
            }
            if (j < n && steps_[j].kind == LayerKind::MaxPool2d && intOr(steps_[j], 0, 2) == 2 &&
                intOr(steps_[j], 1, intOr(steps_[j], 0, 2)) == 2) {
                g.pool = true;
                ++j;
            }
            g.x_nchw4 = !groups.empty() && groups.back().kind == Group::Conv && groups.back().y_nchw4;
            g.w_packed = batch >= 0 && readsInPlace(s, batch);
            g.y_nchw4 = !g.pool && s.w->dim(0) % 4 == 0 && j < n &&
                        steps_[j].kind == LayerKind::Conv2d && batch >= 0 &&
                        readsInPlace(steps_[j], batch);
            break;
        case LayerKind::Relu:
            g.kind = Group::Relu;
            break;
        case LayerKind::Softmax:
            g.kind = Group::Softmax;
            batch = -1;
            break;
        case LayerKind::MaxPool2d:
            g.kind = Group::MaxPool;
            break;
        case LayerKind::Reshape:
            g.kind = Group::Reshape;
            batch = s.ints.size() == 4 ? s.ints[0] : -1;
            break;
        }
        groups.push_back(g);
        i = j;
    }
    return groups;
}

std::string LayerChain::plan(std::span<const int64_t> shape, TypeCode dtype) const {
    std::ostringstream out;
    for (const Group &g : schedule(shape, dtype)) {
        const LayerStep &s = *g.step;
        switch (g.kind) {
        case Group::Dense:
            out << (g.relu ? "dense_relu" : "dense");
            break;
        case Group::DenseSoftmax:
            out << (g.relu ? "dense_relu+softmax" : "dense+softmax");
            break;
        case Group::DenseHead:
            out << (g.relu ? "dense_relu+" : "dense+") << (g.relu2 ? "dense_relu" : "dense");
            if (g.softmax) out << "+softmax";
            break;
        case Group::ConvPair:
            out << (g.relu ? "conv2d_relu+" : "conv2d+") << (g.relu2 ? "conv2d_relu" : "conv2d")
                << "+maxpool2d(2,2)";
            break;
        case Group::Conv:
            out << (g.relu ? "conv2d_relu" : "conv2d");
            if (g.pool) out << "+maxpool2d(2,2)";
            if (g.x_nchw4) out << " x=nchw4";
            if (g.y_nchw4) out << " y=nchw4";
            break;
        case Group::Relu:
            out << "relu";
            break;
        case Group::Softmax:
            out << "softmax";
            break;
        case Group::MaxPool: {
            const int64_t k = intOr(s, 0, 2);
            out << "maxpool2d(" << k << "," << intOr(s, 1, k) << ")";
            break;
        }
        case Group::Reshape:
            out << "reshape";
            break;
        }
        out << "\n";
    }
    return out.str();
}

TensorObject *LayerChain::apply(const TensorObject *x) const {
    for (const LayerStep &s : steps_) {
        requireLive(s.w, s.w_storage);
        requireLive(s.bias, s.bias_storage);
    }
    Activation cur;
    cur.tensor = x;
    cur.shape.assign(x->shape(), x->shape() + x->rank());
    for (const Group &g : schedule(cur.shape, cur.tensor->dtype())) {
        const LayerStep &s = *g.step;
        Activation next;
        switch (g.kind) {
        case Group::ConvPair: {
            // schedule() checked every shape and dtype this kernel needs
            const LayerStep &s2 = *g.step2;
            const int64_t N = cur.shape[0], H = cur.shape[2], W = cur.shape[3];
            const int64_t Co2 = s2.w->dim(0);
            const int64_t os[4] = {N, Co2, (H - 4) / 2, (W - 4) / 2};
            next = Activation::of(TensorObject::create(TypeCode::Float32, os, Residence::Device));
            if (N > 0) {
                const int f1 = (s.bias ? CAMEL_EPI_BIAS : 0) | (g.relu ? CAMEL_EPI_RELU : 0);
                const int f2 = (s2.bias ? CAMEL_EPI_BIAS : 0) | (g.relu2 ? CAMEL_EPI_RELU : 0) |
                               CAMEL_CONV_W_PACKED;
                const void *w2p = packedWeights((size_t)(&s2 - steps_.data()));
                checkHip(camel_hip_conv2d_pair_pool2(
                    static_cast<const float *>(cur.tensor->deviceData()),
                    static_cast<const float *>(s.w->deviceData()),
                    s.bias ? static_cast<const float *>(s.bias->deviceData()) : nullptr,
                    static_cast<const float *>(w2p),
                    s2.bias ? static_cast<const float *>(s2.bias->deviceData()) : nullptr,
                    static_cast<float *>(const_cast<TensorObject *>(next.tensor)->deviceOutput()),
                    N, H, W, 32, Co2, f1, f2));
            }
            break;
        }
        case Group::Dense:
            next = Activation::of(tensorDense(cur.tensor, s.w, s.bias, g.relu));
            break;
        case Group::DenseSoftmax:
            next = Activation::of(tensorDenseSoftmax(cur.tensor, s.w, s.bias, g.relu));
            break;
        case Group::DenseHead:
            next = Activation::of(tensorDenseHead(cur.tensor, s.w, s.bias, g.relu, g.step2->w,
                                                  g.step2->bias, g.relu2, g.softmax));
            break;
        case Group::Relu:
            next = Activation::of(tensorRelu(cur.tensor));
            break;
        case Group::Softmax:
            next = Activation::of(tensorSoftmax(cur.tensor));
            break;
        case Group::MaxPool: {
            const int64_t k = intOr(s, 0, 2);
            next = Activation::of(tensorMaxPool2d(cur.tensor, k, intOr(s, 1, k)));
            break;
        }
        case Group::Reshape:
            next = Activation::of(tensorReshape(cur.tensor, s.ints));
            break;
        case Group::Conv: {
            const int64_t stride = intOr(s, 0, 1), pad = intOr(s, 1, 0);
            const TypeCode xdt = cur.nchw4 ? TypeCode::Float32 : cur.tensor->dtype();
            auto os = conv2dOutputShape(cur.shape, xdt, s.w, s.bias, stride, pad);
            if (g.pool) {
                if (os[2] < 2 || os[3] < 2)
                    throw std::invalid_argument("maxpool2d window larger than input");
                os[2] /= 2;
                os[3] /= 2;
            }
            const int64_t numel = os[0] * os[1] * os[2] * os[3];
            void *y;
            if (g.y_nchw4) {
                next.shape.assign(os.begin(), os.end());
                checkHip(camel_hip_malloc(&next.nchw4, (size_t)std::max<int64_t>(numel, 1) * 4));
                y = next.nchw4;
            } else {
                next = Activation::of(TensorObject::create(TypeCode::Float32, os, Residence::Device));
                y = numel > 0 ? const_cast<TensorObject *>(next.tensor)->deviceOutput() : nullptr;
            }
            if (numel > 0) {
                const void *xin = cur.nchw4 ? cur.nchw4 : cur.tensor->deviceData();
                const int layout =
                    (g.x_nchw4 ? CAMEL_CONV_X_NCHW4 : 0) | (g.y_nchw4 ? CAMEL_CONV_Y_NCHW4 : 0);
                const void *wp = g.w_packed ? packedWeights((size_t)(&s - steps_.data())) : nullptr;
                conv2dLaunch(xin, cur.shape, s.w, s.bias, stride, pad, g.relu, g.pool, layout, y, wp);
            }
            break;
        }
        }
        cur = std::move(next);
    }
    if (cur.nchw4) throw std::logic_error("chain ended on an NCHW4 intermediate");
    if (!cur.owned) {
        // an empty chain: x -> x is a new tensor with the same payload
        return tensorReshape(cur.tensor, cur.shape);
    }
    cur.owned = false;
    return const_cast<TensorObject *>(cur.tensor);
}

} // namespace camel_amd::tensor
