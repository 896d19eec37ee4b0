// TensorObject: header, device/host residency and the reference's element
// semantics (modules/tensor/runtime.cpp:252-612).
#include "tensor_object.h"

#include "camel_hip.h"

#include <cmath>
#include <exception>
#include <cstdio>
#include <iomanip>
#include <iostream>
#include <sstream>
#include <unordered_map>
#include <unordered_set>

namespace camel_amd::tensor {

void checkHip(int status) {
    if (status == CAMEL_HIP_OK) return;
    const char *msg = camel_hip_last_error();
    throwRuntimeFault(msg && *msg ? std::string(msg) : "HIP backend error " + std::to_string(status));
}

Storage::~Storage() {
    if (!dev) return;
    // A shared block's last reader may be a consumer's stream: the shim holds
    // it back until a device-wide wait, without waiting here (this may run in
    // a consumer's garbage collector).
    if (shared)
        camel_hip_free_shared(dev);
    else
        camel_hip_free(dev);
}

namespace {

uint64_t product(std::span<const int64_t> shape) {
    uint64_t value = 1;
    for (int64_t dim : shape) {
        if (dim < 0) throw std::invalid_argument("Tensor shape cannot contain negative dimensions");
        value *= static_cast<uint64_t>(dim);
    }
    return value;
}

// Allocates the device block of a storage (caller holds the storage mutex).
void ensureDevBlock(Storage &s) {
    if (s.dev || s.bytes == 0) return;
    checkHip(camel_hip_malloc(&s.dev, s.bytes));
}

void ensureHostBlock(Storage &s) {
    if (!s.host) s.host.reset(new std::byte[s.bytes > 0 ? s.bytes : 1]);
}

} // namespace

TensorObject *TensorObject::create(TypeCode dtype, std::span<const int64_t> shape, Residence where,
                                   bool zeroInit) {
    dtype = normalizeTensorDType(dtype);
    const uint64_t numel = product(shape);
    const size_t bytes = static_cast<size_t>(numel * elementSize(dtype));
    auto storage = std::make_shared<Storage>(bytes);
    auto *t = new TensorObject(dtype, std::vector<int64_t>(shape.begin(), shape.end()), numel,
                               bytes, storage);
    registerObject(t);
    if (where == Residence::Device) {
        ensureDevBlock(*storage);
        storage->devValid = true;
        if (zeroInit && bytes > 0)
            checkHip(camel_hip_fill(hipDType(dtype), storage->dev, (int64_t)numel, 0.0));
    } else {
        ensureHostBlock(*storage);
        storage->hostValid = true;
        if (zeroInit && bytes > 0) std::memset(storage->host.get(), 0, bytes);
    }
    return t;
}

TensorObject *TensorObject::view(const TensorObject *src, std::span<const int64_t> shape) {
    const uint64_t numel = product(shape);
    if (numel != src->numel_) throw std::invalid_argument("reshape changes tensor element count");
    auto *t = new TensorObject(src->dtype_, std::vector<int64_t>(shape.begin(), shape.end()), numel,
                               src->byteSize_, src->storage());
    registerObject(t);
    return t;
}

TensorObject *TensorObject::transposedView(const TensorObject *src) {
    if (src->rank() != 2 || src->dtype_ != TypeCode::Float32)
        throw std::invalid_argument("transposed view needs a rank-2 Float32 tensor");
    std::shared_ptr<Storage> block;
    bool srcTransposed = false;
    {
        std::lock_guard<std::mutex> lock(src->layoutMutex_);
        block = src->storage_;
        srcTransposed = src->transposed_.load(std::memory_order_relaxed);
    }
    // The transpose of a transposed view is its source's layout again.
    auto *t = new TensorObject(src->dtype_, {src->shape_[1], src->shape_[0]}, src->numel_,
                               src->byteSize_, std::move(block));
    t->transposed_.store(!srcTransposed, std::memory_order_release);
    registerObject(t);
    return t;
}

void TensorObject::makeContiguous() const {
    if (!transposed_.load(std::memory_order_acquire)) return;
    std::lock_guard<std::mutex> lock(layoutMutex_);
    if (!transposed_.load(std::memory_order_relaxed)) return;
    // Stored as [dim1, dim0] row-major; the contiguous payload is its
    // transpose, [dim0, dim1].
    const int64_t storedRows = shape_[1], storedCols = shape_[0];
    auto fresh = std::make_shared<Storage>(byteSize_);
    {
        Storage &src = *storage_;
        std::lock_guard<std::mutex> slock(src.mutex);
        if (src.devValid || !src.hostValid) {
            ensureDevBlock(src);
            ensureDevBlock(*fresh);
            if (byteSize_ > 0)
                checkHip(camel_hip_transpose2d(hipDType(dtype_), src.dev, fresh->dev, storedRows,
                                               storedCols));
            fresh->devValid = true;
        } else {
            ensureHostBlock(*fresh);
            const auto *in = reinterpret_cast<const float *>(src.host.get());
            auto *out = reinterpret_cast<float *>(fresh->host.get());
            for (int64_t r = 0; r < storedRows; ++r)
                for (int64_t c = 0; c < storedCols; ++c) out[c * storedRows + r] = in[r * storedCols + c];
            fresh->hostValid = true;
        }
    }
    storage_ = std::move(fresh);
    transposed_.store(false, std::memory_order_release);
}

const std::shared_ptr<Storage> &TensorObject::storage() const {
    makeContiguous();
    return storage_;
}

const void *TensorObject::storedDeviceData(std::shared_ptr<Storage> &keep, bool &transposed) const {
    {
        std::lock_guard<std::mutex> lock(layoutMutex_);
        keep = storage_;
        transposed = transposed_.load(std::memory_order_relaxed);
    }
    Storage &s = *keep;
    std::lock_guard<std::mutex> lock(s.mutex);
    if (!s.devValid) {
        ensureDevBlock(s);
        if (s.bytes > 0) checkHip(camel_hip_h2d(s.dev, s.host.get(), s.bytes));
        s.devValid = true;
    }
    return s.dev;
}

int64_t TensorObject::dim(size_t index) const {
    if (index >= shape_.size()) throw std::invalid_argument("Tensor dimension out of range");
    return shape_[index];
}

bool TensorObject::sameShape(const TensorObject *other) const {
    return other && shape_ == other->shape_;
}

const void *TensorObject::deviceData() const {
    makeContiguous();
    Storage &s = *storage_;
    std::lock_guard<std::mutex> lock(s.mutex);
    if (!s.devValid) {
        ensureDevBlock(s);
        if (s.bytes > 0) checkHip(camel_hip_h2d(s.dev, s.host.get(), s.bytes));
        s.devValid = true;
    }
    return s.dev;
}

void *TensorObject::deviceOutput() {
    makeContiguous();
    Storage &s = *storage_;
    std::lock_guard<std::mutex> lock(s.mutex);
    ensureDevBlock(s);
    s.devValid = true;
    s.hostValid = false;
    return s.dev;
}

const void *TensorObject::hostData() const {
    makeContiguous();
    Storage &s = *storage_;
    std::lock_guard<std::mutex> lock(s.mutex);
    if (!s.hostValid) {
        ensureHostBlock(s);
        if (s.bytes > 0) checkHip(camel_hip_d2h(s.host.get(), s.dev, s.bytes));
        s.hostValid = true;
    }
    return s.host.get();
}

void *TensorObject::hostOutput() {
    makeContiguous();
    Storage &s = *storage_;
    std::lock_guard<std::mutex> lock(s.mutex);
    ensureHostBlock(s);
    s.hostValid = true;
    s.devValid = false;
    return s.host.get();
}

// Residency of the payload as stored (a transposed view is not made
// contiguous by asking).
bool TensorObject::hostValid() const {
    std::shared_ptr<Storage> block;
    {
        std::lock_guard<std::mutex> lock(layoutMutex_);
        block = storage_;
    }
    std::lock_guard<std::mutex> lock(block->mutex);
    return block->hostValid;
}

bool TensorObject::deviceValid() const {
    std::shared_ptr<Storage> block;
    {
        std::lock_guard<std::mutex> lock(layoutMutex_);
        block = storage_;
    }
    std::lock_guard<std::mutex> lock(block->mutex);
    return block->devValid;
}

void TensorObject::readElement(uint64_t flatIndex, void *dst) const {
    if (flatIndex >= numel_) throw std::invalid_argument("Tensor flat index out of range");
    const size_t es = elementSize(dtype_);
    makeContiguous();
    Storage &s = *storage_;
    std::lock_guard<std::mutex> lock(s.mutex);
    if (s.hostValid) {
        std::memcpy(dst, s.host.get() + flatIndex * es, es);
        return;
    }
    checkHip(camel_hip_d2h(dst, static_cast<const std::byte *>(s.dev) + flatIndex * es, es));
}

double TensorObject::getAsDouble(uint64_t flatIndex) const {
    switch (dtype_) {
    case TypeCode::Float32: {
        float v;
        readElement(flatIndex, &v);
        return static_cast<double>(v);
    }
    case TypeCode::Int64: {
        int64_t v;
        readElement(flatIndex, &v);
        return static_cast<double>(v);
    }
    case TypeCode::Bool: {
        uint8_t v;
        readElement(flatIndex, &v);
        return v != 0 ? 1.0 : 0.0;
    }
    default:
        throw std::invalid_argument("Unsupported Tensor dtype");
    }
}

int64_t TensorObject::getAsInt64(uint64_t flatIndex) const {
    switch (dtype_) {
    case TypeCode::Float32: {
        float v;
        readElement(flatIndex, &v);
        return static_cast<int64_t>(v);
    }
    case TypeCode::Int64: {
        int64_t v;
        readElement(flatIndex, &v);
        return v;
    }
    case TypeCode::Bool: {
        uint8_t v;
        readElement(flatIndex, &v);
        return v != 0 ? 1 : 0;
    }
    default:
        throw std::invalid_argument("Unsupported Tensor dtype");
    }
}

bool TensorObject::getAsBool(uint64_t flatIndex) const {
    switch (dtype_) {
    case TypeCode::Float32: {
        float v;
        readElement(flatIndex, &v);
        return v != 0.0f;
    }
    case TypeCode::Int64: {
        int64_t v;
        readElement(flatIndex, &v);
        return v != 0;
    }
    case TypeCode::Bool: {
        uint8_t v;
        readElement(flatIndex, &v);
        return v != 0;
    }
    default:
        throw std::invalid_argument("Unsupported Tensor dtype");
    }
}

// TensorObject::equals (runtime.cpp:391-405): same dtype, shape and bytes.
bool TensorObject::equals(const TensorObject *other) const {
    if (this == other) return true;
    if (!other) return false;
    if (dtype_ != other->dtype_ || shape_ != other->shape_ || numel_ != other->numel_) return false;
    if (byteSize_ == 0 || storage() == other->storage()) return true;
    return std::memcmp(hostData(), other->hostData(), byteSize_) == 0;
}

// TensorObject::clone (runtime.cpp:407-417): a deep copy, made on the device
// when the source has a device copy.
TensorObject *TensorObject::clone() const {
    if (deviceValid()) {
        TensorObject *copy = create(dtype_, shape_, Residence::Device);
        if (byteSize_ > 0) {
            checkHip(camel_hip_d2d(copy->deviceOutput(), deviceData(), byteSize_));
        }
        return copy;
    }
    TensorObject *copy = create(dtype_, shape_, Residence::Host);
    if (byteSize_ > 0) std::memcpy(copy->hostOutput(), hostData(), byteSize_);
    return copy;
}

// formatElementToString (runtime.cpp:422-450).
std::string TensorObject::formatElement(const std::byte *data, uint64_t flatIndex) const {
    char buf[32];
    std::ostringstream oss;
    switch (dtype_) {
    case TypeCode::Float32: {
        float f;
        std::memcpy(&f, data + flatIndex * 4, 4);
        const double v = f;
        if (v == std::floor(v) && std::abs(v) < 1e10)
            (void)std::snprintf(buf, sizeof(buf), "% 7.0f.", v);
        else
            (void)std::snprintf(buf, sizeof(buf), "% 7.4g", v);
        oss << buf;
        break;
    }
    case TypeCode::Int64: {
        int64_t v;
        std::memcpy(&v, data + flatIndex * 8, 8);
        oss << std::setw(7) << v;
        break;
    }
    case TypeCode::Bool:
        oss << (data[flatIndex] != std::byte{0} ? "  true" : " false");
        break;
    default:
        oss << "?";
        break;
    }
    return oss.str();
}

// printRecursive (runtime.cpp:487-528): PyTorch-style nesting, innermost rows
// wrapped at 100 columns with an 8-space indent step.
void TensorObject::printRecursive(std::ostream &os, size_t dimIndex, uint64_t &flatIndex,
                                  const std::string &indent, const std::byte *data) const {
    constexpr int indentStep = 8;
    constexpr size_t maxLineWidth = 100;
    const std::string innerIndent = indent + std::string(indentStep, ' ');
    if (shape_.empty()) {
        os << formatElement(data, 0);
        return;
    }
    if (dimIndex + 1 == shape_.size()) {
        os << "[";
        size_t width = indent.size() + indentStep;
        for (int64_t i = 0; i < shape_[dimIndex]; ++i) {
            std::string element = formatElement(data, flatIndex++);
            if (i > 0) {
                if (width + 2 + element.size() > maxLineWidth) {
                    os << ",\n" << innerIndent;
                    width = innerIndent.size();
                } else {
                    os << ", ";
                    width += 2;
                }
            }
            os << element;
            width += element.size();
        }
        os << "]";
        return;
    }
    os << "[";
    for (int64_t i = 0; i < shape_[dimIndex]; ++i) {
        if (i > 0) os << ",\n" << innerIndent;
        printRecursive(os, dimIndex + 1, flatIndex, innerIndent, data);
    }
    os << "]";
}

// TensorObject::print (runtime.cpp:452-474).
void TensorObject::print(std::ostream &os) const {
    const std::byte *data = byteSize_ > 0 ? static_cast<const std::byte *>(hostData()) : nullptr;
    os << "tensor(";
    uint64_t flatIndex = 0;
    printRecursive(os, 0, flatIndex, "", data);
    os << ", dtype=";
    switch (dtype_) {
    case TypeCode::Float32:
        os << "float32";
        break;
    case TypeCode::Int64:
        os << "int64";
        break;
    case TypeCode::Bool:
        os << "bool";
        break;
    default:
        os << "unknown";
        break;
    }
    os << ")";
}

// ---- dtype rules (runtime.cpp:530-580) -----------------------------------------

size_t elementSize(TypeCode dtype) {
    switch (dtype) {
    case TypeCode::Float32:
        return 4;
    case TypeCode::Int64:
        return 8;
    case TypeCode::Bool:
        return 1;
    default:
        throw std::invalid_argument("Unsupported Tensor dtype");
    }
}

bool isSupportedTensorScalar(TypeCode code) {
    return code == TypeCode::Int32 || code == TypeCode::Int64 || code == TypeCode::Float32 ||
           code == TypeCode::Float64 || code == TypeCode::Bool;
}

bool isFloatingTensorType(TypeCode code) {
    return code == TypeCode::Float32 || code == TypeCode::Float64;
}

TypeCode normalizeTensorDType(TypeCode code) {
    switch (code) {
    case TypeCode::Float32:
    case TypeCode::Float64:
        return TypeCode::Float32;
    case TypeCode::Int32:
    case TypeCode::Int64:
        return TypeCode::Int64;
    case TypeCode::Bool:
        return TypeCode::Bool;
    default:
        throw std::invalid_argument("Unsupported Tensor dtype");
    }
}

TypeCode tensorDTypeFromValueType(TypeCode code) { return normalizeTensorDType(code); }

TypeCode promoteTensorTypes(TypeCode lhs, TypeCode rhs) {
    lhs = normalizeTensorDType(lhs);
    rhs = normalizeTensorDType(rhs);
    if (lhs == TypeCode::Float32 || rhs == TypeCode::Float32) return TypeCode::Float32;
    if (lhs == TypeCode::Int64 || rhs == TypeCode::Int64) return TypeCode::Int64;
    return TypeCode::Bool;
}

int hipDType(TypeCode dtype) {
    switch (dtype) {
    case TypeCode::Float32:
        return CAMEL_DT_F32;
    case TypeCode::Int64:
        return CAMEL_DT_I64;
    case TypeCode::Bool:
        return CAMEL_DT_BOOL;
    default:
        throw std::invalid_argument("Unsupported Tensor dtype");
    }
}

// scalarToDouble (runtime.cpp:62-77).
double scalarToDouble(TypeCode code, slot_t value) {
    switch (code) {
    case TypeCode::Int32:
        return static_cast<double>(fromSlot<int32_t>(value));
    case TypeCode::Int64:
        return static_cast<double>(fromSlot<int64_t>(value));
    case TypeCode::Float32:
        return static_cast<double>(fromSlot<float>(value));
    case TypeCode::Float64:
        return fromSlot<double>(value);
    case TypeCode::Bool:
        return fromSlot<bool>(value) ? 1.0 : 0.0;
    default:
        throw std::invalid_argument("Unsupported scalar type for Tensor operation");
    }
}

namespace {

int64_t scalarToInt64(TypeCode code, slot_t value) {
    switch (code) {
    case TypeCode::Int32:
        return static_cast<int64_t>(fromSlot<int32_t>(value));
    case TypeCode::Int64:
        return fromSlot<int64_t>(value);
    case TypeCode::Float32:
        return static_cast<int64_t>(fromSlot<float>(value));
    case TypeCode::Float64:
        return static_cast<int64_t>(fromSlot<double>(value));
    case TypeCode::Bool:
        return fromSlot<bool>(value) ? 1 : 0;
    default:
        throw std::invalid_argument("Unsupported scalar type for Tensor operation");
    }
}

bool scalarToBool(TypeCode code, slot_t value) {
    switch (code) {
    case TypeCode::Bool:
        return fromSlot<bool>(value);
    case TypeCode::Int32:
        return fromSlot<int32_t>(value) != 0;
    case TypeCode::Int64:
        return fromSlot<int64_t>(value) != 0;
    case TypeCode::Float32:
        return fromSlot<float>(value) != 0.0f;
    case TypeCode::Float64:
        return fromSlot<double>(value) != 0.0;
    default:
        throw std::invalid_argument("Unsupported scalar type for Tensor operation");
    }
}

struct ArrayInference {
    TypeCode dtype;
    std::vector<int64_t> shape;
};

// inferArrayType (runtime.cpp:152-189).  An Array value's element type is
// carried by the ArrayObject itself.
ArrayInference inferArrayType(slot_t slot, TypeCode valueCode) {
    if (valueCode == TypeCode::Array) {
        const auto *array = fromSlot<const ArrayObject *>(slot);
        const int64_t size = array ? static_cast<int64_t>(array->size()) : 0;
        const TypeCode elem = array ? array->elem : TypeCode::Float32;
        ArrayInference inferred{elem == TypeCode::Array ? TypeCode::Float32
                                                        : normalizeTensorDType(elem),
                                {size}};
        if (!array || size == 0) return inferred;
        if (elem == TypeCode::Array) {
            ArrayInference child = inferArrayType(array->items[0], elem);
            inferred.dtype = child.dtype;
            inferred.shape.insert(inferred.shape.end(), child.shape.begin(), child.shape.end());
            for (size_t i = 1; i < array->size(); ++i) {
                ArrayInference another = inferArrayType(array->items[i], elem);
                if (another.shape != child.shape || another.dtype != child.dtype)
                    throw std::invalid_argument("Nested array shape or dtype mismatch");
            }
        }
        return inferred;
    }
    if (!isSupportedTensorScalar(valueCode))
        throw std::invalid_argument("Only numeric arrays can be converted to Tensor");
    return ArrayInference{normalizeTensorDType(valueCode), {}};
}

// flattenArray (runtime.cpp:191-220), writing the host payload.
void flattenArray(const ArrayObject *array, TypeCode dtype, std::byte *out, uint64_t &offset) {
    for (slot_t value : array->items) {
        if (array->elem == TypeCode::Array) {
            flattenArray(fromSlot<const ArrayObject *>(value), dtype, out, offset);
            continue;
        }
        switch (dtype) {
        case TypeCode::Float32: {
            const float f = static_cast<float>(scalarToDouble(array->elem, value));
            std::memcpy(out + 4 * offset++, &f, 4);
            break;
        }
        case TypeCode::Int64: {
            const int64_t v = scalarToInt64(array->elem, value);
            std::memcpy(out + 8 * offset++, &v, 8);
            break;
        }
        case TypeCode::Bool:
            out[offset++] = std::byte{static_cast<uint8_t>(scalarToBool(array->elem, value) ? 1 : 0)};
            break;
        default:
            throw std::invalid_argument("Unsupported Tensor dtype");
        }
    }
}

} // namespace

// parseShapeArray (runtime.cpp:582-605).
std::vector<int64_t> parseShapeArray(const ArrayObject *shapeArray, TypeCode shapeCode) {
    if (!shapeArray || shapeCode != TypeCode::Array)
        throw std::invalid_argument("Shape must be an integer array");
    if (shapeArray->elem != TypeCode::Int32 && shapeArray->elem != TypeCode::Int64)
        throw std::invalid_argument("Shape array must contain integers");
    std::vector<int64_t> shape;
    shape.reserve(shapeArray->size());
    for (slot_t item : shapeArray->items) {
        const int64_t value = shapeArray->elem == TypeCode::Int32
                                  ? static_cast<int64_t>(fromSlot<int32_t>(item))
                                  : fromSlot<int64_t>(item);
        if (value < 0) throw std::invalid_argument("Shape cannot contain negative values");
        shape.push_back(value);
    }
    return shape;
}

// makeShapeArray (runtime.cpp:607-613).
ArrayObject *makeShapeArray(const TensorObject *tensor) {
    auto *shape = new ArrayObject{TypeCode::Int64, {}};
    for (size_t i = 0; i < tensor->rank(); ++i) shape->items.push_back(toSlot<int64_t>(tensor->dim(i)));
    registerObject(shape);
    return shape;
}

// tensorFromArray (runtime.cpp:1067-1077): built on the host, uploaded at the
// first device use.
TensorObject *tensorFromArray(slot_t slot, TypeCode valueCode) {
    if (valueCode != TypeCode::Array)
        throw std::invalid_argument("Only array values can be converted to Tensor");
    ArrayInference inferred = inferArrayType(slot, valueCode);
    TensorObject *tensor = TensorObject::create(inferred.dtype, inferred.shape, Residence::Host);
    const auto *array = fromSlot<const ArrayObject *>(slot);
    uint64_t offset = 0;
    if (array && tensor->byteSize() > 0)
        flattenArray(array, tensor->dtype(), static_cast<std::byte *>(tensor->hostOutput()), offset);
    return tensor;
}

// ---- lifetime registry ----------------------------------------------------------

namespace {
// Each registered object carries a serial number, so a record of an object
// that was released (and whose address a new object may have taken since)
// never matches the new one.
struct Registry {
    std::mutex mutex;
    uint64_t next = 1;
    std::unordered_map<TensorObject *, uint64_t> tensors;
    std::unordered_map<ArrayObject *, uint64_t> arrays;
};
Registry &registry() {
    static Registry *r = new Registry(); // never destroyed: tensors may outlive static teardown
    return *r;
}

template <class Obj>
bool eraseIf(std::unordered_map<Obj *, uint64_t> &live, Obj *obj, uint64_t serial) {
    auto it = live.find(obj);
    if (it == live.end() || (serial != 0 && it->second != serial)) return false;
    live.erase(it);
    return true;
}
} // namespace

void registerObject(TensorObject *t) {
    uint64_t serial;
    {
        std::lock_guard<std::mutex> lock(registry().mutex);
        serial = registry().next++;
        registry().tensors[t] = serial;
    }
    CreationScope::record(t, serial);
}

void registerObject(ArrayObject *a) {
    uint64_t serial;
    {
        std::lock_guard<std::mutex> lock(registry().mutex);
        serial = registry().next++;
        registry().arrays[a] = serial;
    }
    CreationScope::record(a, serial);
}

namespace {
thread_local CreationScope *t_scope = nullptr;

bool releaseTensorSerial(TensorObject *t, uint64_t serial) {
    {
        std::lock_guard<std::mutex> lock(registry().mutex);
        if (!eraseIf(registry().tensors, t, serial)) return false;
    }
    delete t;
    return true;
}

bool releaseArraySerial(ArrayObject *a, uint64_t serial) {
    {
        std::lock_guard<std::mutex> lock(registry().mutex);
        if (!eraseIf(registry().arrays, a, serial)) return false;
    }
    delete a;
    return true;
}
} // namespace

CreationScope::CreationScope() : parent_(t_scope), uncaught_(std::uncaught_exceptions()) {
    t_scope = this;
}

CreationScope::~CreationScope() {
    t_scope = parent_;
    if (std::uncaught_exceptions() > uncaught_) {
        // Objects released meanwhile (an operator's freed temporaries) fail
        // the serial check, also when another thread's new object now has
        // the same address.
        for (const auto &[t, serial] : tensors_) releaseTensorSerial(t, serial);
        for (const auto &[a, serial] : arrays_) releaseArraySerial(a, serial);
    } else if (parent_) {
        parent_->tensors_.insert(parent_->tensors_.end(), tensors_.begin(), tensors_.end());
        parent_->arrays_.insert(parent_->arrays_.end(), arrays_.begin(), arrays_.end());
    }
}

void CreationScope::record(TensorObject *t, uint64_t serial) {
    if (t_scope) t_scope->tensors_.emplace_back(t, serial);
}

void CreationScope::record(ArrayObject *a, uint64_t serial) {
    if (t_scope) t_scope->arrays_.emplace_back(a, serial);
}

bool releaseTensor(TensorObject *t) { return releaseTensorSerial(t, 0); }

bool releaseArray(ArrayObject *a) { return releaseArraySerial(a, 0); }

bool isLiveTensor(const TensorObject *t) {
    std::lock_guard<std::mutex> lock(registry().mutex);
    return registry().tensors.count(const_cast<TensorObject *>(t)) != 0;
}

bool isLiveArray(const ArrayObject *a) {
    std::lock_guard<std::mutex> lock(registry().mutex);
    return registry().arrays.count(const_cast<ArrayObject *>(a)) != 0;
}

size_t liveTensorCount() {
    std::lock_guard<std::mutex> lock(registry().mutex);
    return registry().tensors.size();
}

uint64_t registryMark() {
    std::lock_guard<std::mutex> lock(registry().mutex);
    return registry().next - 1;
}

size_t releaseSince(uint64_t mark, std::span<const void *const> keep) {
    std::unordered_set<const void *> kept(keep.begin(), keep.end());
    std::vector<TensorObject *> tensors;
    std::vector<ArrayObject *> arrays;
    {
        std::lock_guard<std::mutex> lock(registry().mutex);
        auto take = [&](auto &live, auto &out) {
            for (auto it = live.begin(); it != live.end();) {
                if (it->second > mark && !kept.count(it->first)) {
                    out.push_back(it->first);
                    it = live.erase(it);
                } else {
                    ++it;
                }
            }
        };
        take(registry().tensors, tensors);
        take(registry().arrays, arrays);
    }
    // a view keeps its payload alive through the shared Storage, so the
    // objects can go in any order
    for (TensorObject *t : tensors) delete t;
    for (ArrayObject *a : arrays) delete a;
    return tensors.size() + arrays.size();
}

size_t releaseAll() {
    std::unordered_map<TensorObject *, uint64_t> tensors;
    std::unordered_map<ArrayObject *, uint64_t> arrays;
    {
        std::lock_guard<std::mutex> lock(registry().mutex);
        tensors.swap(registry().tensors);
        arrays.swap(registry().arrays);
    }
    for (const auto &entry : tensors) delete entry.first;
    for (const auto &entry : arrays) delete entry.first;
    return tensors.size() + arrays.size();
}

} // namespace camel_amd::tensor
