// TensorObject with device residency: the Tensor value of the reference's
// tensor module (modules/tensor/runtime.h:55-109) re-laid out for a GPU.
//
// The reference keeps the payload inline behind the header in GC memory
// (runtime.cpp:256-279, 482-485).  Here the header keeps the same fields
// (dtype, rank, numel, byteSize, shape) and the payload lives in a Storage
// block that has a device copy (HBM, from libcamel_hip's pool) and/or a host
// copy.  Tensors are immutable once an operator has produced them (the
// reference's operators never mutate their inputs), so the two copies are
// kept coherent by validity flags alone:
//   * operator outputs are born on the device (dev_valid only);
//   * tensors built from host data are born on the host and uploaded at the
//     first device use (then both are valid);
//   * host reads (index, print, equals, to_host) download once and cache.
// reshape returns a view that shares the Storage (the reference copies; the
// values are the same because neither copy is ever written again).
#pragma once

#include "camel_core.h"
#include "camel_dlpack.h"

#include <atomic>
#include <cstddef>
#include <iosfwd>
#include <memory>
#include <mutex>
#include <span>
#include <utility>
#include <vector>

namespace camel_amd::tensor {

// modules/tensor/runtime.h:39-53
enum class BinaryOp { Add, Subtract, Multiply, Divide, Power };
enum class CompareOp { Less, LessEqual, Greater, GreaterEqual, Equal };

// Where a new tensor's payload is first materialised.
enum class Residence { Device, Host };

// Throws RuntimeFault with the shim's message when a libcamel_hip call fails.
void checkHip(int status);

struct Storage {
    explicit Storage(size_t bytes) : bytes(bytes) {}
    ~Storage();
    Storage(const Storage &) = delete;
    Storage &operator=(const Storage &) = delete;

    size_t bytes;
    void *dev = nullptr;
    std::unique_ptr<std::byte[]> host;
    bool devValid = false;
    bool hostValid = false;
    // Set when the device block was handed out without a copy (DLPack
    // export): a consumer may still read it on its own stream when the last
    // reference goes, so the block returns to the pool, where the library
    // stream could reuse it, only after a later device-wide wait.
    bool shared = false;
    std::mutex mutex; // residency transitions may race under a thread-pool scheduler
};

class TensorObject {
  public:
    TensorObject(const TensorObject &) = delete;
    TensorObject &operator=(const TensorObject &) = delete;

    // TensorObject::create (runtime.cpp:256-279).  dtype is normalised
    // (Float64 -> Float32, Int32 -> Int64).  zeroInit fills with zeros.
    static TensorObject *create(TypeCode dtype, std::span<const int64_t> shape, Residence where,
                                bool zeroInit = false);
    // A tensor of `shape` sharing `src`'s payload (numel must match).
    static TensorObject *view(const TensorObject *src, std::span<const int64_t> shape);
    // The transpose of a rank-2 Float32 tensor as a view: shape [c, r] over
    // src's [r, c] payload, no copy.  Kernels that read the stored layout
    // (the GEMM's transposed-A loaders) take it as is (storedDeviceData); any
    // other access first makes this tensor's payload contiguous, once, with a
    // device transpose into a block of its own, so every other reader sees
    // the reference's row-major contents (tensorTranspose2D copies,
    // runtime.cpp:704-720; for Float32 the copy through double is exact).
    static TensorObject *transposedView(const TensorObject *src);

    size_t rank() const { return shape_.size(); }
    uint64_t numel() const { return numel_; }
    TypeCode dtype() const { return dtype_; }
    size_t byteSize() const { return byteSize_; }
    const int64_t *shape() const { return shape_.data(); }
    int64_t dim(size_t index) const;
    bool sameShape(const TensorObject *other) const;

    // Device pointer of a valid device copy (uploads a host-only payload).
    const void *deviceData() const;
    // Device pointer for an operator that fills the payload on the device:
    // the device copy becomes the only valid one.
    void *deviceOutput();
    // Host pointer of a valid host copy (downloads a device-only payload).
    const void *hostData() const;
    // Host pointer for a writer that fills the payload on the host.
    void *hostOutput();

    bool hostValid() const;
    bool deviceValid() const;
    // The payload block, shared with views and with DLPack exports (a
    // transposed view is made contiguous first).
    const std::shared_ptr<Storage> &storage() const;

    // True while the payload is stored transposed ([dim1, dim0] row-major).
    bool storedTransposed() const { return transposed_.load(std::memory_order_acquire); }
    // The device payload as stored (uploading if needed), without making a
    // transposed view contiguous; `keep` holds the block for the caller and
    // `transposed` tells which layout the pointer has.
    const void *storedDeviceData(std::shared_ptr<Storage> &keep, bool &transposed) const;

    // Element access with the reference's conversions (runtime.cpp:298-389).
    // A device-only tensor is not downloaded whole: one element is copied.
    double getAsDouble(uint64_t flatIndex) const;
    int64_t getAsInt64(uint64_t flatIndex) const;
    bool getAsBool(uint64_t flatIndex) const;

    // rtdata::Object behaviour (runtime.cpp:391-420, 422-500).
    bool equals(const TensorObject *other) const;
    TensorObject *clone() const;
    void print(std::ostream &os) const;

  private:
    TensorObject(TypeCode dtype, std::vector<int64_t> shape, uint64_t numel, size_t byteSize,
                 std::shared_ptr<Storage> storage)
        : dtype_(dtype), shape_(std::move(shape)), numel_(numel), byteSize_(byteSize),
          storage_(std::move(storage)) {}
    void readElement(uint64_t flatIndex, void *dst) const;
    // Replaces a transposed view's shared payload by a contiguous block of
    // its own (no-op otherwise); thread-safe, runs at most once.
    void makeContiguous() const;
    void printRecursive(std::ostream &os, size_t dimIndex, uint64_t &flatIndex,
                        const std::string &indent, const std::byte *data) const;
    std::string formatElement(const std::byte *data, uint64_t flatIndex) const;

    TypeCode dtype_;
    std::vector<int64_t> shape_;
    uint64_t numel_;
    size_t byteSize_;
    // Replaced only by makeContiguous (under layoutMutex_), before which no
    // accessor other than storedDeviceData reads it.
    mutable std::shared_ptr<Storage> storage_;
    mutable std::atomic<bool> transposed_{false};
    mutable std::mutex layoutMutex_;
};

// modules/tensor/runtime.cpp:530-580
size_t elementSize(TypeCode dtype);
bool isSupportedTensorScalar(TypeCode code);
bool isFloatingTensorType(TypeCode code);
TypeCode normalizeTensorDType(TypeCode code);
TypeCode tensorDTypeFromValueType(TypeCode code);
TypeCode promoteTensorTypes(TypeCode lhs, TypeCode rhs);
// dtype code of libcamel_hip (CAMEL_DT_*) for a storage dtype.
int hipDType(TypeCode dtype);

// Scalar conversions of runtime.cpp:62-111.
double scalarToDouble(TypeCode code, slot_t value);

// Tensor <-> Array values (runtime.cpp:152-226, 582-612, 1067-1077).
std::vector<int64_t> parseShapeArray(const ArrayObject *shapeArray, TypeCode shapeCode);
ArrayObject *makeShapeArray(const TensorObject *tensor);
TensorObject *tensorFromArray(slot_t slot, TypeCode valueCode);

// DLPack exchange (runtime.cpp:1079-1124): host copy or zero-copy device
// export, and a copying import from host or device memory.
DLManagedTensor *tensorToDLPack(const TensorObject *tensor, bool onDevice);
TensorObject *tensorFromDLPack(const DLManagedTensor *managed);

// Tensor-lifetime bookkeeping: every TensorObject / ArrayObject made by this
// layer is registered so a host program (or a graph's end) can release it.
// The reference never frees tensors (no finalizers, GC roots unset).
void registerObject(TensorObject *t);
void registerObject(ArrayObject *a);
bool releaseTensor(TensorObject *t);
bool releaseArray(ArrayObject *a);
bool isLiveTensor(const TensorObject *t);
bool isLiveArray(const ArrayObject *a);
size_t liveTensorCount();
// Releases every registered tensor and array; returns how many objects.
size_t releaseAll();
// The registry's serial counter: every object registered later has a larger
// serial number.
uint64_t registryMark();
// Releases every tensor and array registered after `mark` except the objects
// (tensors or arrays) in `keep`; returns how many objects were released.
size_t releaseSince(uint64_t mark, std::span<const void *const> keep);

// Cleanup of an operator that throws: while a scope is active on a thread,
// every tensor and array registered on that thread is recorded in it.  When
// an exception leaves the scope, the recorded objects that are still live
// are released (outputs and temporaries of the failed call, which the caller
// never receives: the reference abandons its output when it throws).  When
// the scope ends normally its records pass to the enclosing scope, so the
// outputs of a nested operator are released too if the outer call fails
// later.
class CreationScope {
  public:
    CreationScope();
    ~CreationScope();
    CreationScope(const CreationScope &) = delete;
    CreationScope &operator=(const CreationScope &) = delete;

    // Records a new object (with its registry serial number) in the
    // innermost active scope of this thread.
    static void record(TensorObject *t, uint64_t serial);
    static void record(ArrayObject *a, uint64_t serial);

  private:
    CreationScope *parent_;
    int uncaught_;
    std::vector<std::pair<TensorObject *, uint64_t>> tensors_;
    std::vector<std::pair<ArrayObject *, uint64_t>> arrays_;
};

} // namespace camel_amd::tensor
