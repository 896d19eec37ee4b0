/*
 * camel_tensor.h -- C-ABI of libcamel_tensor.so, the operator layer of the
 * Camel `tensor` module on the MI355X backend.
 *
 * The layer keeps the reference's operator API: every operator of
 * modules/tensor/operators.cpp:160-194 is registered under the same URI
 * suffix ("matmul", "add", ...) with the same argument conventions, result
 * types and error texts, and the layer operators relu / softmax / dense /
 * dense_relu / conv2d / conv2d_relu / maxpool2d are added under "tensor:".
 * This header is the host harness that drives those operators without the
 * Camel runtime, the role FrameArgsView plays in the reference
 * (include/camel/core/context/frame.h:459-492): values are {type code, slot}
 * pairs with the reference's type codes (include/camel/core/type/base.h:69-86)
 * and slot layout (include/camel/core/rtdata/base.h:87-127).
 *
 * Tensors are opaque handles.  Their payload lives on the GPU from the first
 * device operator until a host read (to_host, idx, show, equals) brings a
 * copy back; operators never copy through the host between each other.
 * Handles are released explicitly (the reference never frees tensors).
 * Status codes: 0 OK, otherwise an error whose text (the reference's
 * RuntimeFault message, e.g. "matmul dimension mismatch") is returned by
 * camel_tensor_last_error().
 */
#ifndef CAMEL_TENSOR_H
#define CAMEL_TENSOR_H

#include <stddef.h>
#include <stdint.h>

#include "camel_dlpack.h"

#ifdef __cplusplus
extern "C" {
#endif

enum camel_tensor_status {
    CAMEL_TENSOR_OK = 0,
    CAMEL_TENSOR_ERR_RUNTIME = 1, /* RuntimeFault raised by an operator         */
    CAMEL_TENSOR_ERR_URI = 2,     /* no operator / group with that name         */
    CAMEL_TENSOR_ERR_ARG = 3,     /* bad handle, code or size at this interface */
    CAMEL_TENSOR_ERR_RESOLVE = 4  /* no overload accepts the argument types     */
};

/* Type codes (same values as the reference's TypeCode). */
#define CAMEL_TC_INT32 0x00000000u
#define CAMEL_TC_INT64 0x00000001u
#define CAMEL_TC_FLOAT32 0x00000002u
#define CAMEL_TC_FLOAT64 0x00000003u
#define CAMEL_TC_BOOL 0x00000004u
#define CAMEL_TC_VOID 0x00000006u
#define CAMEL_TC_ARRAY 0x60000008u
/* "Tensor" is an OtherType the reference numbers at run time
 * (modules/tensor/type.cpp:38-40); this layer fixes it here. */
#define CAMEL_TC_TENSOR 0xE0000001u

/* One operator argument or result. */
typedef struct camel_value {
    uint32_t code; /* CAMEL_TC_* */
    uint64_t slot; /* scalar bits in the low bytes, or a handle */
} camel_value;

const char *camel_tensor_last_error(void);

/* ---- tensors ------------------------------------------------------------- */
/* A host tensor of dtype (FLOAT32 / INT64 / BOOL; FLOAT64 and INT32 are
 * normalised as the reference does) copied from `data` (numel * element size
 * bytes; may be NULL for numel == 0).  It is uploaded at its first device use. */
int camel_tensor_from_host(uint32_t dtype, int64_t rank, const int64_t *shape, const void *data,
                           uint64_t *handle);
/* Copies the payload to `dst` (exactly byte_size bytes), downloading once. */
int camel_tensor_to_host(uint64_t handle, void *dst, size_t bytes);
/* dtype, rank and up to `cap` dims. */
int camel_tensor_meta(uint64_t handle, uint32_t *dtype, int64_t *rank, int64_t *shape, int64_t cap);
/* Where the payload is currently valid (1/0 each). */
int camel_tensor_residency(uint64_t handle, int *host_valid, int *device_valid);
/* Device address of the payload (uploading if needed), e.g. for DLPack/torch. */
int camel_tensor_device_ptr(uint64_t handle, uint64_t *device_ptr);
int camel_tensor_release(uint64_t handle);
/* Releases every tensor and array this layer has made; returns how many. */
int64_t camel_tensor_release_all(void);
/* Scoped release for a loop whose iterations make temporaries (e.g. the
 * train loop of test/run/nn/mnist.cml:44-58, where the reference frees
 * nothing: no finalizers, include/camel/core/mm/gen.h:224).  camel_tensor_mark
 * returns a mark; camel_tensor_release_since releases every tensor and array
 * handle made after that mark except the n_keep handles in keep (e.g. the
 * updated weights a later iteration reads), and reports how many it released.
 * Views share their payload, so a kept view keeps it alive.  No reference
 * counterpart: the reference never releases tensors. */
uint64_t camel_tensor_mark(void);
int camel_tensor_release_since(uint64_t mark, int64_t n_keep, const uint64_t *keep,
                               int64_t *released);
int64_t camel_tensor_live_count(void);
/* Writes the reference print form (TensorObject::print) into buf. */
int camel_tensor_format(uint64_t handle, char *buf, size_t cap, size_t *needed);
/* TensorObject::equals: same dtype, shape and bytes. */
int camel_tensor_equals(uint64_t a, uint64_t b, int *equal);
/* TensorObject::clone (runtime.cpp:407-417): a new handle with a deep copy of
 * the payload (made on the device when the source has a device copy). */
int camel_tensor_clone(uint64_t handle, uint64_t *copy);

/* ---- DLPack (tensorToDLPackCopy / tensorFromDLPackCopy, runtime.cpp:1079-1124) */
/* Exports a tensor as a DLManagedTensor; the consumer calls its deleter.
 * on_device = 0: a host copy (kDLCPU), as tensorToDLPackCopy does
 *   (runtime.cpp:1079-1105).
 * on_device = 1: the device payload itself (kDLROCM, device_id = the
 *   library's device), without a copy.  The managed tensor holds a reference
 *   to the payload, so the handle may be released before the deleter runs.
 *   The library stream is synchronised first, so the data is complete for a
 *   consumer on any stream.  Tensors are immutable: the consumer must not
 *   write through it.
 * Float32, Int64 and Bool tensors only ("Unsupported dtype for DLPack
 * export" otherwise, as the reference). */
int camel_tensor_to_dlpack(uint64_t handle, int on_device, DLManagedTensor **managed);
/* Imports a copy of a DLPack tensor (tensorFromDLPackCopy,
 * runtime.cpp:1107-1124), from kDLCPU or from kDLROCM memory of the
 * library's device.  Float32 / Int64 / Bool with lanes 1; row-major with
 * strides NULL or equal to the compact strides (what PyTorch exports),
 * byte_offset 0; the reference's error texts otherwise.  A device source
 * must be complete (its producer synchronised); the copy is finished when
 * this returns.  The caller keeps `managed` (its deleter is not called). */
int camel_tensor_from_dlpack(const DLManagedTensor *managed, uint64_t *handle);

/* ---- arrays (shape arguments, array operands, shape() results) ----------- */
int camel_array_create(uint32_t elem_code, int64_t count, const uint64_t *slots, uint64_t *handle);
int camel_array_read(uint64_t handle, uint32_t *elem_code, int64_t *count, uint64_t *slots,
                     int64_t cap);
int camel_array_release(uint64_t handle);

/* ---- operators ----------------------------------------------------------- */
/* Calls the operator registered under `uri` ("tensor:matmul" or "matmul")
 * with bind arguments `with` and normal arguments `norm`; the result's type
 * is the one the operator group resolves for these argument types. */
int camel_tensor_invoke(const char *uri, int64_t n_with, const camel_value *with, int64_t n_norm,
                        const camel_value *norm, camel_value *result);
/* Overload resolution of a group ("__mat__", "sum", "dense", ...): writes the
 * chosen URI, the result type code and the result's element type: the dtype
 * of a Tensor result as the reference's resolvers give it (Float32 by default,
 * modules/tensor/operators.cpp:41-43; Bool for the comparisons, 137; Int64
 * for range and argmax, 382 and 458), the element type of an Array result
 * (Int64 for shape, 45-48), and the result code itself otherwise.  Either
 * output pointer may be NULL. */
int camel_tensor_resolve(const char *group, int64_t n_with, const uint32_t *with_codes,
                         int64_t n_norm, const uint32_t *norm_codes, char *uri, size_t cap,
                         uint32_t *result_code, uint32_t *result_elem);

/* ---- TensorType (modules/tensor/type.h:32-59, type.cpp:21-145) ----------- */
/* A tensor type is an element dtype (a CAMEL_TC_* primitive code) and a static
 * shape of `rank` extents; rank 0 means dynamic (any shape), as an empty
 * shape does in the reference. */
/* TensorType::toString (mangled = 0, e.g. "Tensor", "Tensor<bool>",
 * "Tensor<[2, 3], i64>"; type.cpp:64-81) or TensorType::mangle (mangled = 1,
 * e.g. "T_;f32", "T2,3;i"; type.cpp:83-98), NUL-terminated into buf;
 * *needed receives the size including the NUL. */
int camel_tensor_type_string(uint32_t dtype, int64_t rank, const int64_t *shape, int mangled,
                             char *buf, size_t cap, size_t *needed);
/* TensorType::assignableFrom and equals (type.cpp:105-131): whether a value of
 * type src may be assigned to dst (a Float32 dst takes any dtype; a dynamic
 * shape on either side matches any shape), and whether the types are equal. */
int camel_tensor_type_relation(uint32_t dst_dtype, int64_t dst_rank, const int64_t *dst_shape,
                               uint32_t src_dtype, int64_t src_rank, const int64_t *src_shape,
                               int *assignable, int *equal);
/* Registered URI suffixes and group names. */
int64_t camel_tensor_op_count(void);
const char *camel_tensor_op_name(int64_t index);
int64_t camel_tensor_group_count(void);
const char *camel_tensor_group_name(int64_t index);

/* ---- composed layer chains --------------------------------------------- */
/* A chain is what `dense<w1, b1>..relu..dense<w2, b2>..softmax` denotes
 * (README.md:40-46): layer operators with their bind arguments, applied in
 * order; `x->chain` is camel_chain_apply.  The reference's compose operator
 * `..` is a stub (src/builtin/operators/macro.cpp:30): this is the object a
 * compose over this module's layer operators builds.  Apply runs adjacent
 * layers as one fused kernel where that computes the same values (dense +
 * relu, dense + softmax, conv2d + relu, conv2d + maxpool2d(2, 2), and a
 * conv2d feeding a conv2d through an NHWC intermediate). */
int camel_chain_create(uint64_t *chain);
/* Appends a layer: uri "dense", "dense_relu", "relu", "softmax", "conv2d",
 * "conv2d_relu", "maxpool2d" or "reshape" ("tensor:" prefix optional) with
 * its bind arguments as the operator takes them: tensors (weights, then
 * bias; Void for none), then integers (conv2d stride, pad; maxpool2d kernel,
 * stride; reshape the shape, as integers or one Array).  Weights are
 * borrowed: they must stay live while the chain is applied. */
int camel_chain_append(uint64_t chain, const char *uri, int64_t n_with, const camel_value *with);
/* x -> chain: a new tensor handle.  Errors carry the failing layer's text. */
int camel_chain_apply(uint64_t chain, uint64_t x, uint64_t *result);
/* The kernel groups apply would run for an input of this shape and dtype (a
 * CAMEL_TC_* code; the fused kernels serve Float32 only), one per line (e.g.
 * "conv2d_relu+maxpool2d(2,2) x=nchw4"), NUL-terminated into buf. */
int camel_chain_plan(uint64_t chain, int64_t rank, const int64_t *shape, uint32_t dtype, char *buf,
                     size_t cap, size_t *needed);
int camel_chain_release(uint64_t chain);

/* The plugin ABI version the reference's module loader checks before it calls
 * camel_module_create: CAMEL_MODULE_ABI_VERSION = 1
 * (include/camel/core/module/dynamic.h:29,38; modules/camel_module_abi.cpp:22;
 * checked in src/core/module/dynamic.cpp:118-178).  camel_module_create itself
 * returns a C++ Module object of libcamel and belongs to the .cmo glue that
 * is compiled against libcamel's headers (see the integration notes). */
int camel_module_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif
