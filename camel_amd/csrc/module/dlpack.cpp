// DLPack exchange of TensorObjects (modules/tensor/runtime.cpp:1079-1124).
//
// The reference copies in both directions and handles host memory only.
// Here a tensor can also be exported without a copy from HBM (kDLROCM): the
// managed tensor holds a reference to the payload's Storage, so the device
// block outlives the tensor handle until the consumer's deleter runs, and the
// Storage is marked shared, so its block is reused only after a later
// device-wide wait (the consumer reads it on its own streams).  Imports
// copy, from host memory or from device memory on the library's device.
#include "tensor_object.h"

#include "camel_hip.h"

#include <cstring>
#include <mutex>
#include <stdexcept>
#include <vector>

namespace camel_amd::tensor {

namespace {

// runtime.cpp:221-232
DLDataType toDLPackType(TypeCode dtype) {
    switch (dtype) {
    case TypeCode::Float32:
        return DLDataType{kDLFloat, 32, 1};
    case TypeCode::Int64:
        return DLDataType{kDLInt, 64, 1};
    case TypeCode::Bool:
        return DLDataType{kDLBool, 8, 1};
    default:
        throw std::invalid_argument("Unsupported dtype for DLPack export");
    }
}

// runtime.cpp:234-248
TypeCode fromDLPackType(const DLDataType &dtype) {
    if (dtype.lanes != 1) throw std::invalid_argument("Only lanes=1 DLPack tensors are supported");
    if (dtype.code == kDLFloat && dtype.bits == 32) return TypeCode::Float32;
    if (dtype.code == kDLInt && dtype.bits == 64) return TypeCode::Int64;
    if (dtype.code == kDLBool && dtype.bits == 8) return TypeCode::Bool;
    throw std::invalid_argument("Unsupported DLPack dtype");
}

// What an exported DLManagedTensor owns: its shape array, and either a host
// copy of the payload or a reference to the device payload.
struct ExportContext {
    std::vector<int64_t> shape;
    std::vector<std::byte> host;
    std::shared_ptr<Storage> storage;
};

void deleteExport(DLManagedTensor *self) {
    if (!self) return;
    delete static_cast<ExportContext *>(self->manager_ctx);
    delete self;
}

int libraryDevice() {
    int device = 0;
    checkHip(camel_hip_current_device(&device));
    return device;
}

} // namespace

DLManagedTensor *tensorToDLPack(const TensorObject *tensor, bool onDevice) {
    const DLDataType dtype = toDLPackType(tensor->dtype());
    auto ctx = std::make_unique<ExportContext>();
    ctx->shape.assign(tensor->shape(), tensor->shape() + tensor->rank());
    DLDevice device{kDLCPU, 0};
    void *data = nullptr;
    if (onDevice) {
        data = const_cast<void *>(tensor->deviceData());
        ctx->storage = tensor->storage();
        {
            std::lock_guard<std::mutex> lock(ctx->storage->mutex);
            ctx->storage->shared = true;
        }
        device = DLDevice{kDLROCM, libraryDevice()};
        // The consumer may read on any stream: finish every pending writer.
        checkHip(camel_hip_sync());
    } else {
        ctx->host.resize(tensor->byteSize());
        if (tensor->byteSize() > 0)
            std::memcpy(ctx->host.data(), tensor->hostData(), tensor->byteSize());
        data = ctx->host.data();
    }
    auto *managed = new DLManagedTensor{};
    managed->dl_tensor.data = data;
    managed->dl_tensor.device = device;
    managed->dl_tensor.ndim = static_cast<int32_t>(tensor->rank());
    managed->dl_tensor.dtype = dtype;
    managed->dl_tensor.shape = ctx->shape.data();
    managed->dl_tensor.strides = nullptr;
    managed->dl_tensor.byte_offset = 0;
    managed->manager_ctx = ctx.release();
    managed->deleter = deleteExport;
    return managed;
}

TensorObject *tensorFromDLPack(const DLManagedTensor *managed) {
    if (!managed) throw std::invalid_argument("Null DLPack tensor");
    const DLTensor &dl = managed->dl_tensor;
    const bool onDevice = dl.device.device_type == kDLROCM;
    if (dl.device.device_type != kDLCPU && !onDevice)
        throw std::invalid_argument("Only CPU and ROCm DLPack tensors are supported");
    if (onDevice && dl.device.device_id != libraryDevice())
        throw std::invalid_argument("DLPack tensor is on another device");
    if (dl.ndim < 0 || (dl.ndim > 0 && !dl.shape))
        throw std::invalid_argument("Invalid DLPack tensor shape");
    // The reference accepts strides == NULL only; compact strides describe
    // the same layout (PyTorch always sets them), so they are accepted too.
    bool contiguous = dl.byte_offset == 0;
    if (contiguous && dl.strides) {
        int64_t expect = 1;
        for (int32_t i = dl.ndim - 1; i >= 0; --i) {
            if (dl.shape[i] != 1 && dl.strides[i] != expect) contiguous = false;
            expect *= dl.shape[i];
        }
    }
    if (!contiguous) throw std::invalid_argument("Only contiguous DLPack tensors are supported");
    const TypeCode dtype = fromDLPackType(dl.dtype);
    std::vector<int64_t> shape(dl.shape, dl.shape + dl.ndim);
    TensorObject *tensor =
        TensorObject::create(dtype, shape, onDevice ? Residence::Device : Residence::Host);
    try {
        const size_t bytes = tensor->byteSize();
        if (bytes > 0 && !dl.data) throw std::invalid_argument("Null DLPack tensor data");
        if (bytes > 0 && onDevice) {
            checkHip(camel_hip_d2d(tensor->deviceOutput(), dl.data, bytes));
            // The source may be freed as soon as this returns.
            checkHip(camel_hip_sync());
        } else if (bytes > 0) {
            std::memcpy(tensor->hostOutput(), dl.data, bytes);
        }
    } catch (...) {
        releaseTensor(tensor);
        throw;
    }
    return tensor;
}

} // namespace camel_amd::tensor
