// TensorType: the tensor value's compile-time type (modules/tensor/type.cpp).
#include "tensor_type.h"

namespace camel_amd {

std::string primitiveTypeName(TypeCode code) {
    switch (code) {
    case TypeCode::Int32:
        return "i32";
    case TypeCode::Int64:
        return "i64";
    case TypeCode::Float32:
        return "f32";
    case TypeCode::Float64:
        return "f64";
    case TypeCode::Bool:
        return "bool";
    case TypeCode::Byte:
        return "byte";
    case TypeCode::Void:
        return "void";
    case TypeCode::String:
        return "string";
    case TypeCode::Array:
        return "array";
    case TypeCode::Tensor:
        return "Tensor";
    default:
        return "unknown";
    }
}

std::string primitiveTypeMangle(TypeCode code) {
    switch (code) {
    case TypeCode::Int32:
        return "i32";
    case TypeCode::Int64:
        return "i";
    case TypeCode::Float32:
        return "f32";
    case TypeCode::Float64:
        return "f";
    case TypeCode::Bool:
        return "b";
    case TypeCode::Byte:
        return "c";
    case TypeCode::Void:
        return "v";
    case TypeCode::String:
        return "s";
    default:
        throwRuntimeFault("Type::mangle: no mangled name for type code " +
                          std::to_string(static_cast<uint32_t>(code)));
    }
}

std::string TensorType::toString() const {
    const bool f32 = dtype_ == TypeCode::Float32;
    if (shape_.empty()) return f32 ? "Tensor" : "Tensor<" + primitiveTypeName(dtype_) + ">";
    std::string out = "Tensor<[";
    for (size_t i = 0; i < shape_.size(); ++i) {
        if (i) out += ", ";
        out += std::to_string(shape_[i]);
    }
    out += "]";
    if (!f32) out += ", " + primitiveTypeName(dtype_);
    return out + ">";
}

std::string TensorType::mangle() const {
    std::string out = "T";
    if (shape_.empty()) out += "_";
    for (size_t i = 0; i < shape_.size(); ++i) {
        if (i) out += ",";
        out += std::to_string(shape_[i]);
    }
    return out + ";" + primitiveTypeMangle(dtype_);
}

bool TensorType::equals(const TensorType &other) const {
    return shape_ == other.shape_ && dtype_ == other.dtype_;
}

bool TensorType::assignableFrom(const TensorType &source) const {
    const bool dtypeOk = dtype_ == TypeCode::Float32 || dtype_ == source.dtype_;
    const bool shapeOk = shape_.empty() || source.shape_.empty() || shape_ == source.shape_;
    return dtypeOk && shapeOk;
}

} // namespace camel_amd
