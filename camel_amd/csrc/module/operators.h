// The tensor module's operator API: the 31 operators of the reference
// (modules/tensor/operators.h:30-60, same names and signature), the layer
// operators this backend adds (relu, softmax, dense, conv2d, maxpool2d), the
// URI-suffix map the executor registers (operators.cpp:160-194) and the
// operator groups the compiler resolves overloads through (196-583).
#pragma once

#include "camel_core.h"

#include <string>
#include <unordered_map>
#include <vector>

namespace camel_amd {

slot_t __tensor_add__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_subtract__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_multiply__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_divide__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_pow__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_matmul__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_idx__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_idx2d__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_lt__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_le__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_gt__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_ge__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_eq__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_empty__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_zeros__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_ones__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_full__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_random__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_range__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_eye__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_shape__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_sum__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_sum_axis__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_max_axis__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_argmax_axis__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_exp__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_log__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_transpose__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_concat__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_reshape__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_show__(ArgsView &with, ArgsView &norm, Context &ctx);

// Layer operators (no reference counterpart; each equals a reference
// composition, see runtime.h).  Bind arguments travel in `with`, as in
// `dense<w, b>` (README.md:40-46): dense<W[, b]>(x), conv2d<w[, b[, stride[,
// pad]]]>(x), maxpool2d<[kernel[, stride]]>(x); every operand may also be
// passed in `norm` after x.
slot_t __tensor_relu__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_softmax__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_dense__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_dense_relu__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_conv2d__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_conv2d_relu__(ArgsView &with, ArgsView &norm, Context &ctx);
slot_t __tensor_maxpool2d__(ArgsView &with, ArgsView &norm, Context &ctx);

std::unordered_map<std::string, operator_t> getTensorOpsMap();
const std::vector<OperatorGroup> &getTensorOperatorGroups();

} // namespace camel_amd
