/*
 * camel_dlpack.h -- the DLPack exchange structs (DLPack ABI v0.8, the public
 * dmlc/dlpack standard) that the tensor module's tensorToDLPackCopy /
 * tensorFromDLPackCopy use (modules/tensor/dlpack.h:7-36,
 * modules/tensor/runtime.cpp:1079-1124), with the ROCm device type that a
 * device-resident tensor is exported under.  The layout is fixed by the
 * standard; when the standard header was included first (it defines
 * DLPACK_VERSION) its definitions are used instead.
 */
#ifndef CAMEL_DLPACK_H
#define CAMEL_DLPACK_H

#include <stdint.h>

#ifndef DLPACK_VERSION

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    kDLCPU = 1,  /* host memory */
    kDLROCM = 10 /* HIP device memory; device_id = HIP device ordinal */
} DLDeviceType;

typedef struct {
    DLDeviceType device_type;
    int32_t device_id;
} DLDevice;

typedef enum { kDLInt = 0, kDLUInt = 1, kDLFloat = 2, kDLBfloat = 4, kDLBool = 6 } DLDataTypeCode;

typedef struct {
    uint8_t code;   /* DLDataTypeCode */
    uint8_t bits;
    uint16_t lanes;
} DLDataType;

typedef struct {
    void *data;
    DLDevice device;
    int32_t ndim;
    DLDataType dtype;
    int64_t *shape;
    int64_t *strides; /* NULL: compact row-major */
    uint64_t byte_offset;
} DLTensor;

typedef struct DLManagedTensor {
    DLTensor dl_tensor;
    void *manager_ctx;
    void (*deleter)(struct DLManagedTensor *self);
} DLManagedTensor;

#ifdef __cplusplus
}
#endif

#endif /* DLPACK_VERSION */

#endif /* CAMEL_DLPACK_H */
