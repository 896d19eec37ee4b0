// The compile-time type of a tensor value (modules/tensor/type.h:32-59,
// type.cpp:21-145): an element dtype and a static shape, where an empty shape
// means "dynamic" (any shape).  The operator groups resolve their results to
// these types, so a compiler that binds this module sees the same result
// types as with the reference: Tensor (Float32, dynamic) by default,
// Tensor<bool> from comparisons, Tensor<i64> from range and argmax.
#pragma once

#include "camel_core.h"

#include <cstddef>
#include <string>
#include <vector>

namespace camel_amd {

class TensorType {
  public:
    // TensorType(shape, elementType) (type.cpp:31-33): the element type
    // defaults to Float32.
    explicit TensorType(std::vector<size_t> shape = {}, TypeCode dtype = TypeCode::Float32)
        : shape_(std::move(shape)), dtype_(dtype) {}

    // TensorType::Dynamic / Default (type.cpp:50-58): no static shape.
    static TensorType Dynamic(TypeCode dtype = TypeCode::Float32) { return TensorType({}, dtype); }
    static TensorType Default() { return Dynamic(TypeCode::Float32); }

    const std::vector<size_t> &shape() const { return shape_; }
    TypeCode dType() const { return dtype_; }

    // "Tensor", "Tensor<bool>", "Tensor<[2, 3]>", "Tensor<[2, 3], i64>"
    // (type.cpp:64-81): the dtype is named only when it is not Float32.
    std::string toString() const;
    // "T_;f32", "T2,3;i" (type.cpp:83-98): '_' for a dynamic shape, then the
    // dtype's mangled name.
    std::string mangle() const;
    // Same shape and dtype (type.cpp:105-114).
    bool equals(const TensorType &other) const;
    // A value of type `source` may be assigned to this type (type.cpp:122-131):
    // a Float32 target takes any dtype, otherwise the dtypes must be equal;
    // an empty (dynamic) shape on either side matches any shape.
    bool assignableFrom(const TensorType &source) const;

  private:
    std::vector<size_t> shape_;
    TypeCode dtype_;
};

// typeCodeToString (src/core/type/base.cpp:49-83) for the primitive codes a
// tensor dtype can carry; other codes are "unknown".
std::string primitiveTypeName(TypeCode code);
// Type::mangle (src/core/type/base.cpp:92-122) for primitive codes; throws
// RuntimeFault for codes it does not cover (the reference asserts).
std::string primitiveTypeMangle(TypeCode code);

} // namespace camel_amd
