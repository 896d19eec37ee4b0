// Internal header of libcamel_hip.so: runtime state, status plumbing and the
// device-side dtype helpers shared by every kernel file.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <initializer_list>
#include <mutex>
#include <string>

#include "camel_hip.h"

namespace camel_hip {

// One library-wide lock: the shim owns a single stream and pool, and the
// reference may call operators from Taskflow worker threads.
std::recursive_mutex &lib_mutex();

// Sets the thread's last-error text and returns `status`.
int fail(int status, const std::string &message);
// Clears the last-error text and returns CAMEL_HIP_OK.
int ok();
// Maps a HIP error to CAMEL_HIP_ERR_RUNTIME with its text (OK passes through).
int check_hip(hipError_t err, const char *what);
// Checks the launch just made on the library stream.
int check_launch(const char *kernel);

// Lazily initialises device 0; returns a status.
int ensure_init();
// True once a device has been initialised (no initialisation is attempted).
bool initialised();
hipStream_t stream();
int device_cu_count();

// The allocation-free entry points' scratch: the device address of the
// library's static scratch array on the current device (CAMEL_HIP_NOALLOC_
// SCRATCH_BYTES long, 256-byte aligned), looked up once per device at
// initialisation; nullptr before that.
float *noalloc_scratch();

// Device error flag: cleared by a fill kernel before a checked launch and read
// back (synchronously) after it.
int *error_flag();
int clear_error_flag();
// Reads the flag; returns its value through `value`.
int read_error_flag(int *value);

// True when the product of non-negative factors is at most `limit`, checked
// at every step so that huge factors cannot wrap around into range.
inline bool product_fits(std::initializer_list<int64_t> factors, int64_t limit = INT32_MAX) {
    int64_t p = 1;
    for (int64_t f : factors)
        if (__builtin_mul_overflow(p, f, &p) || p > limit) return false;
    return true;
}

// Bytes of one element of a storage dtype (0 for an unknown dtype).
inline size_t dtype_size(int dt) {
    switch (dt) {
    case CAMEL_DT_F32:
        return 4;
    case CAMEL_DT_I64:
        return 8;
    case CAMEL_DT_BOOL:
        return 1;
    default:
        return 0;
    }
}
inline bool valid_dtype(int dt) { return dtype_size(dt) != 0; }

// Grid size for a grid-stride kernel over `work` items of `per_block` each,
// capped so the grid stays a few waves over the chip.
inline unsigned grid_for(int64_t work, int per_block, int max_blocks_per_cu = 8) {
    int64_t blocks = (work + per_block - 1) / per_block;
    int64_t cap = (int64_t)device_cu_count() * max_blocks_per_cu;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    return (unsigned)blocks;
}

// ---- device helpers ----------------------------------------------------------

// TensorObject::getAsDouble (modules/tensor/runtime.cpp:298-310).
__device__ __forceinline__ double load_as_double(int dt, const void *p, int64_t i) {
    if (dt == CAMEL_DT_F32) return (double)static_cast<const float *>(p)[i];
    if (dt == CAMEL_DT_I64) return (double)static_cast<const int64_t *>(p)[i];
    return static_cast<const uint8_t *>(p)[i] != 0 ? 1.0 : 0.0;
}

// static_cast<int64_t>(double) as the x86-64 reference build executes it
// (cvttsd2si): truncation, INT64_MIN for NaN and out-of-range values.
__device__ __forceinline__ int64_t double_to_i64_x86(double v) {
    if (v >= -9223372036854775808.0 && v < 9223372036854775808.0) return (int64_t)v;
    return INT64_MIN;
}

// TensorObject::setFromDouble (modules/tensor/runtime.cpp:340-355).
__device__ __forceinline__ void store_from_double(int dt, void *p, int64_t i, double v) {
    if (dt == CAMEL_DT_F32)
        static_cast<float *>(p)[i] = (float)v;
    else if (dt == CAMEL_DT_I64)
        static_cast<int64_t *>(p)[i] = double_to_i64_x86(v);
    else
        static_cast<uint8_t *>(p)[i] = v != 0.0 ? 1 : 0;
}

// relu(x) = x * (x > 0), the idiom of test/run/nn/svm.cml:31: keeps the sign
// of zero, maps negative values to -0.0 and -inf / NaN to NaN.
__device__ __forceinline__ float relu_idiom(float x) { return x * (x > 0.0f ? 1.0f : 0.0f); }

} // namespace camel_hip

#define CAMEL_LOCK() std::lock_guard<std::recursive_mutex> camel_lock_guard_(camel_hip::lib_mutex())

#define CAMEL_INIT_OR_RETURN()                                                                     \
    do {                                                                                           \
        int camel_init_rc_ = camel_hip::ensure_init();                                             \
        if (camel_init_rc_ != CAMEL_HIP_OK) return camel_init_rc_;                                 \
    } while (0)

#define CAMEL_RETURN_IF(rc_expr)                                                                   \
    do {                                                                                           \
        int camel_rc_ = (rc_expr);                                                                 \
        if (camel_rc_ != CAMEL_HIP_OK) return camel_rc_;                                           \
    } while (0)
