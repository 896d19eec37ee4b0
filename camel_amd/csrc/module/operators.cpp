// Operator bodies of the tensor module on the MI355X backend.  Argument
// handling, dispatch between tensor/scalar overloads and error texts follow
// modules/tensor/operators.cpp (cited per operator); the arithmetic runs in
// runtime.cpp on the device.
#include "operators.h"

#include "runtime.h"

#include <iostream>

namespace camel_amd {

using namespace camel_amd::tensor;

namespace {

bool isTensor(TypeCode code) { return code == TypeCode::Tensor; }
bool isNumericScalar(TypeCode code) { return isSupportedTensorScalar(code); }
bool isIntCode(TypeCode code) { return code == TypeCode::Int32 || code == TypeCode::Int64; }

// requireTensor (operators.cpp:73-82).
TensorObject *requireTensor(ArgsView &args, size_t index) {
    if (index >= args.size() || !isTensor(args.code(index)))
        throwRuntimeFault("Expected Tensor argument");
    auto *tensor = args.get<TensorObject *>(index);
    if (!tensor) throwRuntimeFault("Tensor argument cannot be null");
    return tensor;
}

// requireTensorOrConvertArray (operators.cpp:84-99).
TensorObject *requireTensorOrConvertArray(ArgsView &args, size_t index) {
    if (isTensor(args.code(index))) return requireTensor(args, index);
    if (args.code(index) == TypeCode::Array) {
        try {
            return tensorFromArray(args.slot(index), args.code(index));
        } catch (const std::exception &e) {
            throwRuntimeFault(e.what());
        }
    }
    throwRuntimeFault("Expected Tensor or numeric array");
}

// An Int32 or Int64 argument as int64 (operators.cpp:1042-1045 etc.).
int64_t intArg(ArgsView &args, size_t index) {
    return args.code(index) == TypeCode::Int32 ? static_cast<int64_t>(args.get<int32_t>(index))
                                               : args.get<int64_t>(index);
}

// scalarAsDouble (operators.cpp:56-71).
double scalarAsDouble(TypeCode code, ArgsView &args, size_t index) {
    switch (code) {
    case TypeCode::Int32:
        return static_cast<double>(args.get<int32_t>(index));
    case TypeCode::Int64:
        return static_cast<double>(args.get<int64_t>(index));
    case TypeCode::Float32:
        return static_cast<double>(args.get<float>(index));
    case TypeCode::Float64:
        return args.get<double>(index);
    case TypeCode::Bool:
        return args.get<bool>(index) ? 1.0 : 0.0;
    default:
        throwRuntimeFault("Expected numeric scalar");
    }
}

slot_t wrap(TensorObject *t) { return toSlot(t); }

// withTensorErrors (operators.cpp:103-109): any std::exception becomes a
// RuntimeFault with the same text.  Tensors the failed call made (its output,
// temporaries of a composition) are released on the way out.
template <typename Fn> slot_t withTensorErrors(Fn &&fn) {
    try {
        CreationScope scope;
        return fn();
    } catch (const RuntimeFault &) {
        throw;
    } catch (const std::exception &e) {
        throwRuntimeFault(e.what());
    }
}

// The tensor/tensor, tensor/scalar and scalar/tensor forms shared by add,
// subtract, multiply and divide (operators.cpp:585-715).
slot_t binaryOperator(ArgsView &norm, BinaryOp op) {
    return withTensorErrors([&]() -> slot_t {
        const bool lhsTensor = isTensor(norm.code(0));
        const bool rhsTensor = isTensor(norm.code(1));
        if (lhsTensor && rhsTensor)
            return wrap(tensorBinary(requireTensor(norm, 0), requireTensor(norm, 1), op));
        if (lhsTensor)
            return wrap(tensorBinaryScalarRight(requireTensor(norm, 0), norm.code(1), norm.slot(1), op));
        return wrap(tensorBinaryScalarLeft(norm.code(0), norm.slot(0), requireTensor(norm, 1), op));
    });
}

// The comparison operators (operators.cpp:791-921); eq also accepts arrays.
slot_t compareOperator(ArgsView &norm, CompareOp op, bool arrays) {
    return withTensorErrors([&]() -> slot_t {
        auto operand = [&](size_t i) {
            return arrays ? requireTensorOrConvertArray(norm, i) : requireTensor(norm, i);
        };
        auto tensorLike = [&](size_t i) {
            return isTensor(norm.code(i)) || (arrays && norm.code(i) == TypeCode::Array);
        };
        const bool lhs = tensorLike(0), rhs = tensorLike(1);
        if (lhs && rhs) return wrap(tensorCompare(operand(0), operand(1), op));
        if (lhs) return wrap(tensorCompareScalarRight(operand(0), norm.code(1), norm.slot(1), op));
        return wrap(tensorCompareScalarLeft(norm.code(0), norm.slot(0), operand(1), op));
    });
}

// Operands of a layer operator: bound in `with` (dense<W, b>(x)) or appended
// to norm after the input x.  Leading operands are tensors (weights, then an
// optional bias; a Void operand stands for "no bias"), the rest integers.
struct LayerOperands {
    std::vector<TensorObject *> tensors;
    std::vector<int64_t> ints;

    LayerOperands(ArgsView &with, ArgsView &norm) {
        ArgsView &view = with.size() > 0 ? with : norm;
        size_t i = with.size() > 0 ? 0 : 1;
        for (; i < view.size() && (isTensor(view.code(i)) || view.code(i) == TypeCode::Void); ++i)
            tensors.push_back(view.code(i) == TypeCode::Void ? nullptr : requireTensor(view, i));
        for (; i < view.size(); ++i) {
            if (!isIntCode(view.code(i))) throwRuntimeFault("Expected integer argument");
            ints.push_back(intArg(view, i));
        }
    }
    TensorObject *tensor(size_t i) const { return i < tensors.size() ? tensors[i] : nullptr; }
    int64_t integer(size_t i, int64_t fallback) const { return i < ints.size() ? ints[i] : fallback; }
};

slot_t denseOperator(ArgsView &with, ArgsView &norm, bool relu) {
    return withTensorErrors([&]() -> slot_t {
        TensorObject *x = requireTensor(norm, 0);
        LayerOperands a(with, norm);
        if (!a.tensor(0)) throwRuntimeFault("dense requires weights");
        return wrap(tensorDense(x, a.tensor(0), a.tensor(1), relu));
    });
}

slot_t conv2dOperator(ArgsView &with, ArgsView &norm, bool relu) {
    return withTensorErrors([&]() -> slot_t {
        TensorObject *x = requireTensor(norm, 0);
        LayerOperands a(with, norm);
        if (!a.tensor(0)) throwRuntimeFault("conv2d requires weights");
        return wrap(tensorConv2d(x, a.tensor(0), a.tensor(1), a.integer(0, 1), a.integer(1, 0), relu));
    });
}

} // namespace

slot_t __tensor_add__(ArgsView &, ArgsView &norm, Context &) { return binaryOperator(norm, BinaryOp::Add); }
slot_t __tensor_subtract__(ArgsView &, ArgsView &norm, Context &) {
    return binaryOperator(norm, BinaryOp::Subtract);
}
slot_t __tensor_multiply__(ArgsView &, ArgsView &norm, Context &) {
    return binaryOperator(norm, BinaryOp::Multiply);
}
slot_t __tensor_divide__(ArgsView &, ArgsView &norm, Context &) {
    return binaryOperator(norm, BinaryOp::Divide);
}

// __tensor_pow__ (operators.cpp:717-738): tensor base; tensor or scalar exponent.
slot_t __tensor_pow__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t {
        if (isTensor(norm.code(1)))
            return wrap(tensorBinary(requireTensor(norm, 0), requireTensor(norm, 1), BinaryOp::Power));
        return wrap(tensorBinaryScalarRight(requireTensor(norm, 0), norm.code(1), norm.slot(1),
                                            BinaryOp::Power));
    });
}

// __tensor_matmul__ (operators.cpp:740-769).
slot_t __tensor_matmul__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors(
        [&]() -> slot_t { return wrap(tensorMatmul(requireTensor(norm, 0), requireTensor(norm, 1))); });
}

// __tensor_idx__ / __tensor_idx2d__ (operators.cpp:771-789): Float64 results.
slot_t __tensor_idx__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t {
        return toSlot(tensorIndex1D(requireTensor(norm, 0), norm.get<int64_t>(1)));
    });
}
slot_t __tensor_idx2d__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t {
        return toSlot(tensorIndex2D(requireTensor(norm, 0), norm.get<int64_t>(1), norm.get<int64_t>(2)));
    });
}

slot_t __tensor_lt__(ArgsView &, ArgsView &norm, Context &) {
    return compareOperator(norm, CompareOp::Less, false);
}
slot_t __tensor_le__(ArgsView &, ArgsView &norm, Context &) {
    return compareOperator(norm, CompareOp::LessEqual, false);
}
slot_t __tensor_gt__(ArgsView &, ArgsView &norm, Context &) {
    return compareOperator(norm, CompareOp::Greater, false);
}
slot_t __tensor_ge__(ArgsView &, ArgsView &norm, Context &) {
    return compareOperator(norm, CompareOp::GreaterEqual, false);
}
slot_t __tensor_eq__(ArgsView &, ArgsView &norm, Context &) {
    return compareOperator(norm, CompareOp::Equal, true);
}

// Creation operators (operators.cpp:923-1011): Float32 except full (dtype of
// the value) and range (Int64).
slot_t __tensor_empty__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t {
        auto shape = parseShapeArray(norm.get<const ArrayObject *>(0), norm.code(0));
        return wrap(tensorEmpty(TypeCode::Float32, shape));
    });
}
slot_t __tensor_zeros__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t {
        auto shape = parseShapeArray(norm.get<const ArrayObject *>(0), norm.code(0));
        return wrap(tensorZeros(TypeCode::Float32, shape));
    });
}
slot_t __tensor_ones__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t {
        auto shape = parseShapeArray(norm.get<const ArrayObject *>(0), norm.code(0));
        return wrap(tensorOnes(TypeCode::Float32, shape));
    });
}
slot_t __tensor_full__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t {
        auto shape = parseShapeArray(norm.get<const ArrayObject *>(0), norm.code(0));
        return wrap(tensorFull(tensorDTypeFromValueType(norm.code(1)), shape,
                               scalarAsDouble(norm.code(1), norm, 1)));
    });
}
slot_t __tensor_random__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t {
        auto shape = parseShapeArray(norm.get<const ArrayObject *>(0), norm.code(0));
        return wrap(tensorRandom(shape, scalarAsDouble(norm.code(1), norm, 1),
                                 scalarAsDouble(norm.code(2), norm, 2)));
    });
}

// __tensor_range__ (operators.cpp:977-1003): range(stop), range(start, stop[, step]).
slot_t __tensor_range__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t {
        int64_t start = 0, stop = 0, step = 1;
        if (norm.size() == 1) {
            stop = intArg(norm, 0);
        } else {
            start = intArg(norm, 0);
            stop = intArg(norm, 1);
            if (norm.size() == 3) step = intArg(norm, 2);
        }
        return wrap(tensorArange(start, stop, step));
    });
}

slot_t __tensor_eye__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t { return wrap(tensorEye(intArg(norm, 0))); });
}

slot_t __tensor_shape__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t { return toSlot(makeShapeArray(requireTensor(norm, 0))); });
}

slot_t __tensor_sum__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t { return toSlot(tensorSum(requireTensor(norm, 0))); });
}
slot_t __tensor_sum_axis__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors(
        [&]() -> slot_t { return wrap(tensorSumAxis(requireTensor(norm, 0), intArg(norm, 1))); });
}
slot_t __tensor_max_axis__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors(
        [&]() -> slot_t { return wrap(tensorMaxAxis(requireTensor(norm, 0), intArg(norm, 1))); });
}
slot_t __tensor_argmax_axis__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors(
        [&]() -> slot_t { return wrap(tensorArgmaxAxis(requireTensor(norm, 0), intArg(norm, 1))); });
}
slot_t __tensor_exp__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t { return wrap(tensorExp(requireTensor(norm, 0))); });
}
slot_t __tensor_log__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t { return wrap(tensorLog(requireTensor(norm, 0))); });
}
slot_t __tensor_transpose__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t { return wrap(tensorTranspose2D(requireTensor(norm, 0))); });
}

// __tensor_concat__ (operators.cpp:1125-1134): tensors or arrays, Int64 axis.
slot_t __tensor_concat__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t {
        TensorObject *lhs = requireTensorOrConvertArray(norm, 0);
        TensorObject *rhs = requireTensorOrConvertArray(norm, 1);
        return wrap(tensorConcat(lhs, rhs, norm.get<int64_t>(2)));
    });
}

// __tensor_reshape__ (operators.cpp:1136-1146).
slot_t __tensor_reshape__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t {
        auto shape = parseShapeArray(norm.get<const ArrayObject *>(1), norm.code(1));
        return wrap(tensorReshape(requireTensorOrConvertArray(norm, 0), shape));
    });
}

// __tensor_show__ (operators.cpp:1148-1169): prints to stdout, returns null.
slot_t __tensor_show__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t {
        TensorObject *tensor = requireTensorOrConvertArray(norm, 0);
        tensor->print(std::cout);
        std::cout << std::endl;
        return NullSlot;
    });
}

slot_t __tensor_relu__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t { return wrap(tensorRelu(requireTensor(norm, 0))); });
}
slot_t __tensor_softmax__(ArgsView &, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t { return wrap(tensorSoftmax(requireTensor(norm, 0))); });
}
slot_t __tensor_dense__(ArgsView &with, ArgsView &norm, Context &) {
    return denseOperator(with, norm, false);
}
slot_t __tensor_dense_relu__(ArgsView &with, ArgsView &norm, Context &) {
    return denseOperator(with, norm, true);
}
slot_t __tensor_conv2d__(ArgsView &with, ArgsView &norm, Context &) {
    return conv2dOperator(with, norm, false);
}
slot_t __tensor_conv2d_relu__(ArgsView &with, ArgsView &norm, Context &) {
    return conv2dOperator(with, norm, true);
}
slot_t __tensor_maxpool2d__(ArgsView &with, ArgsView &norm, Context &) {
    return withTensorErrors([&]() -> slot_t {
        TensorObject *x = requireTensor(norm, 0);
        LayerOperands a(with, norm);
        const int64_t kernel = a.integer(0, 2);
        return wrap(tensorMaxPool2d(x, kernel, a.integer(1, kernel)));
    });
}

// getTensorOpsMap (operators.cpp:160-194) plus the layer operators.
std::unordered_map<std::string, operator_t> getTensorOpsMap() {
    return {
        {"add", __tensor_add__},
        {"subtract", __tensor_subtract__},
        {"multiply", __tensor_multiply__},
        {"divide", __tensor_divide__},
        {"pow", __tensor_pow__},
        {"matmul", __tensor_matmul__},
        {"idx", __tensor_idx__},
        {"idx2d", __tensor_idx2d__},
        {"lt", __tensor_lt__},
        {"le", __tensor_le__},
        {"gt", __tensor_gt__},
        {"ge", __tensor_ge__},
        {"eq", __tensor_eq__},
        {"empty", __tensor_empty__},
        {"zeros", __tensor_zeros__},
        {"ones", __tensor_ones__},
        {"full", __tensor_full__},
        {"random", __tensor_random__},
        {"range", __tensor_range__},
        {"eye", __tensor_eye__},
        {"shape", __tensor_shape__},
        {"sum", __tensor_sum__},
        {"sum_axis", __tensor_sum_axis__},
        {"max_axis", __tensor_max_axis__},
        {"argmax_axis", __tensor_argmax_axis__},
        {"exp", __tensor_exp__},
        {"log", __tensor_log__},
        {"transpose", __tensor_transpose__},
        {"concat", __tensor_concat__},
        {"reshape", __tensor_reshape__},
        {"show", __tensor_show__},
        {"relu", __tensor_relu__},
        {"softmax", __tensor_softmax__},
        {"dense", __tensor_dense__},
        {"dense_relu", __tensor_dense_relu__},
        {"conv2d", __tensor_conv2d__},
        {"conv2d_relu", __tensor_conv2d_relu__},
        {"maxpool2d", __tensor_maxpool2d__},
    };
}

namespace {

using Codes = std::vector<TypeCode>;
using Result = std::optional<ResultType>;
// tensorType() (operators.cpp:41-43): Float32 unless an element type is given.
const ResultType kTensor = tensorResult();

// resolveTensorBinaryNamed (operators.cpp:111-124).
Result binaryNamed(const Codes &, const Codes &n) {
    if (n.size() != 2) return std::nullopt;
    const bool l = isTensor(n[0]), r = isTensor(n[1]);
    if ((l && r) || (l && isNumericScalar(n[1])) || (r && isNumericScalar(n[0]))) return kTensor;
    return std::nullopt;
}

// resolveTensorCompare (operators.cpp:126-140).
Result compare(const Codes &, const Codes &n) {
    if (n.size() != 2) return std::nullopt;
    const bool l = isTensor(n[0]), r = isTensor(n[1]);
    const bool la = n[0] == TypeCode::Array, ra = n[1] == TypeCode::Array;
    if ((l && r) || (l && isNumericScalar(n[1])) || (r && isNumericScalar(n[0])) ||
        (la && isNumericScalar(n[1])) || (isNumericScalar(n[0]) && ra))
        return tensorResult(TypeCode::Bool); // tensorType(Type::Bool()), operators.cpp:137
    return std::nullopt;
}

Result shapeCtor(const Codes &, const Codes &n) {
    return n.size() == 1 && n[0] == TypeCode::Array ? Result(kTensor) : std::nullopt;
}

Result power(const Codes &, const Codes &n) {
    if (n.size() != 2 || !isTensor(n[0])) return std::nullopt;
    return isTensor(n[1]) || isNumericScalar(n[1]) ? Result(kTensor) : std::nullopt;
}

Result matmul(const Codes &w, const Codes &n) {
    return w.empty() && n.size() == 2 && isTensor(n[0]) && isTensor(n[1]) ? Result(kTensor)
                                                                         : std::nullopt;
}

Result unaryTensor(const Codes &, const Codes &n) {
    return n.size() == 1 && isTensor(n[0]) ? Result(kTensor) : std::nullopt;
}

Result tensorAxis(const Codes &, const Codes &n) {
    return n.size() == 2 && isTensor(n[0]) && isIntCode(n[1]) ? Result(kTensor) : std::nullopt;
}

// Layer operators: the input in norm, operands bound in `with` or appended
// to norm; tensors for weights/bias, integers for geometry.
Result layer(const Codes &w, const Codes &n, size_t minTensors, size_t maxTensors, size_t maxInts) {
    if (n.empty() || !isTensor(n[0])) return std::nullopt;
    Codes ops = w.empty() ? Codes(n.begin() + 1, n.end()) : w;
    if (!w.empty() && n.size() != 1) return std::nullopt;
    size_t i = 0, tensors = 0, ints = 0;
    while (i < ops.size() && tensors < maxTensors && (isTensor(ops[i]) || ops[i] == TypeCode::Void)) {
        ++tensors;
        ++i;
    }
    while (i < ops.size() && isIntCode(ops[i]) && ints < maxInts) {
        ++ints;
        ++i;
    }
    if (i != ops.size() || tensors < minTensors) return std::nullopt;
    return kTensor;
}

OperatorGroup group(std::string name, std::vector<std::pair<std::string, resolver_t>> overloads) {
    return OperatorGroup{std::move(name), std::move(overloads)};
}

} // namespace

// getTensorOperatorGroups (operators.cpp:196-583): the same group names,
// URIs and acceptance rules, plus the layer groups.
const std::vector<OperatorGroup> &getTensorOperatorGroups() {
    static const std::vector<OperatorGroup> groups = [] {
        std::vector<OperatorGroup> g;
        for (auto [name, uri] : std::vector<std::pair<std::string, std::string>>{
                 {"__add__", "tensor:add"}, {"__sub__", "tensor:subtract"},
                 {"__mul__", "tensor:multiply"}, {"__div__", "tensor:divide"},
                 {"add", "tensor:add"}, {"subtract", "tensor:subtract"},
                 {"multiply", "tensor:multiply"}, {"divide", "tensor:divide"}})
            g.push_back(group(name, {{uri, binaryNamed}}));
        g.push_back(group("__pow__", {{"tensor:pow", power}}));
        g.push_back(group("pow", {{"tensor:pow", power}}));
        g.push_back(group("__mat__", {{"tensor:matmul", matmul}}));
        g.push_back(group("matmul", {{"tensor:matmul", matmul}}));
        g.push_back(group(
            "__idx__",
            {{"tensor:idx",
              [](const Codes &, const Codes &n) -> Result {
                  return n.size() == 2 && isTensor(n[0]) && n[1] == TypeCode::Int64
                             ? Result(scalarResult(TypeCode::Float64))
                             : std::nullopt;
              }},
             {"tensor:idx2d", [](const Codes &, const Codes &n) -> Result {
                  return n.size() == 3 && isTensor(n[0]) && n[1] == TypeCode::Int64 &&
                                 n[2] == TypeCode::Int64
                             ? Result(scalarResult(TypeCode::Float64))
                             : std::nullopt;
              }}}));
        for (auto [name, uri] : std::vector<std::pair<std::string, std::string>>{
                 {"__lt__", "tensor:lt"}, {"__le__", "tensor:le"}, {"__gt__", "tensor:gt"},
                 {"__ge__", "tensor:ge"}, {"__eq__", "tensor:eq"}})
            g.push_back(group(name, {{uri, compare}}));
        for (auto [name, uri] : std::vector<std::pair<std::string, std::string>>{
                 {"empty", "tensor:empty"}, {"zeros", "tensor:zeros"}, {"ones", "tensor:ones"}})
            g.push_back(group(name, {{uri, shapeCtor}}));
        g.push_back(group("full", {{"tensor:full", [](const Codes &, const Codes &n) -> Result {
                                        return n.size() == 2 && n[0] == TypeCode::Array &&
                                                       isNumericScalar(n[1])
                                                   ? Result(kTensor)
                                                   : std::nullopt;
                                    }}}));
        g.push_back(group("random", {{"tensor:random", [](const Codes &, const Codes &n) -> Result {
                                          return n.size() == 3 && n[0] == TypeCode::Array &&
                                                         isNumericScalar(n[1]) && isNumericScalar(n[2])
                                                     ? Result(kTensor)
                                                     : std::nullopt;
                                      }}}));
        g.push_back(group("range", {{"tensor:range", [](const Codes &, const Codes &n) -> Result {
                                         if (n.empty() || n.size() > 3) return std::nullopt;
                                         for (TypeCode c : n)
                                             if (!isIntCode(c)) return std::nullopt;
                                         // tensorType(Type::Int64()), operators.cpp:382
                                         return tensorResult(TypeCode::Int64);
                                     }}}));
        g.push_back(group("eye", {{"tensor:eye", [](const Codes &, const Codes &n) -> Result {
                                       return n.size() == 1 && isIntCode(n[0]) ? Result(kTensor)
                                                                               : std::nullopt;
                                   }}}));
        g.push_back(group("shape", {{"tensor:shape", [](const Codes &, const Codes &n) -> Result {
                                         // intArrayType(), operators.cpp:45-48
                                         return n.size() == 1 && isTensor(n[0])
                                                    ? Result(arrayResult(TypeCode::Int64))
                                                    : std::nullopt;
                                     }}}));
        g.push_back(group("sum", {{"tensor:sum",
                                   [](const Codes &, const Codes &n) -> Result {
                                       return n.size() == 1 && isTensor(n[0])
                                                  ? Result(scalarResult(TypeCode::Float64))
                                                  : std::nullopt;
                                   }},
                                  {"tensor:sum_axis", tensorAxis}}));
        g.push_back(group("max", {{"tensor:max_axis", tensorAxis}}));
        // tensorType(Type::Int64()), operators.cpp:458
        g.push_back(group("argmax", {{"tensor:argmax_axis", [](const Codes &w, const Codes &n) -> Result {
                                          return tensorAxis(w, n) ? Result(tensorResult(TypeCode::Int64))
                                                                  : std::nullopt;
                                      }}}));
        for (auto [name, uri] : std::vector<std::pair<std::string, std::string>>{
                 {"exp", "tensor:exp"}, {"log", "tensor:log"}, {"transpose", "tensor:transpose"},
                 {"relu", "tensor:relu"}, {"softmax", "tensor:softmax"}})
            g.push_back(group(name, {{uri, unaryTensor}}));
        g.push_back(group("concat", {{"tensor:concat", [](const Codes &, const Codes &n) -> Result {
                                          if (n.size() != 3 || n[2] != TypeCode::Int64)
                                              return std::nullopt;
                                          const bool l = isTensor(n[0]) || n[0] == TypeCode::Array;
                                          const bool r = isTensor(n[1]) || n[1] == TypeCode::Array;
                                          return l && r ? Result(kTensor) : std::nullopt;
                                      }}}));
        g.push_back(group("reshape", {{"tensor:reshape", [](const Codes &, const Codes &n) -> Result {
                                           return n.size() == 2 &&
                                                          (isTensor(n[0]) || n[0] == TypeCode::Array) &&
                                                          n[1] == TypeCode::Array
                                                      ? Result(kTensor)
                                                      : std::nullopt;
                                       }}}));
        g.push_back(group("show", {{"tensor:show", [](const Codes &, const Codes &n) -> Result {
                                        return n.size() == 1 &&
                                                       (isTensor(n[0]) || n[0] == TypeCode::Array)
                                                   ? Result(scalarResult(TypeCode::Void))
                                                   : std::nullopt;
                                    }}}));
        g.push_back(group("dense", {{"tensor:dense", [](const Codes &w, const Codes &n) {
                                         return layer(w, n, 1, 2, 0);
                                     }}}));
        g.push_back(group("dense_relu", {{"tensor:dense_relu", [](const Codes &w, const Codes &n) {
                                              return layer(w, n, 1, 2, 0);
                                          }}}));
        g.push_back(group("conv2d", {{"tensor:conv2d", [](const Codes &w, const Codes &n) {
                                          return layer(w, n, 1, 2, 2);
                                      }}}));
        g.push_back(group("conv2d_relu", {{"tensor:conv2d_relu", [](const Codes &w, const Codes &n) {
                                               return layer(w, n, 1, 2, 2);
                                           }}}));
        g.push_back(group("maxpool2d", {{"tensor:maxpool2d", [](const Codes &w, const Codes &n) {
                                             return layer(w, n, 0, 0, 2);
                                         }}}));
        return g;
    }();
    return groups;
}

} // namespace camel_amd
