// Runtime part of libcamel_hip.so: device selection, the single stream, the
// pooled device allocator, boundary copies, events and the creation kernels.
#include "common.h"
#include "host_copy.h"

#include <cstdio>
#include <cstring>
#include <unordered_map>
#include <vector>

namespace camel_hip {

namespace {

struct State {
    bool initialised = false;
    int device = -1;
    int cu_count = 256;
    hipStream_t stream = nullptr;
    int *flag = nullptr;
    // Device address of `scratch` on each device the library initialised.
    std::unordered_map<int, float *> scratch_by_device;
    // Pool: exact-size free lists over rounded sizes; blocks never shrink.
    std::unordered_map<size_t, std::vector<void *>> free_lists;
    std::unordered_map<void *, size_t> live;
    // Blocks released while a consumer may still read them on its own
    // streams (zero-copy DLPack exports): held back from the free lists until
    // a device-wide synchronisation has completed (drain_deferred).
    std::vector<std::pair<void *, size_t>> deferred;
    bool deferred_warned = false;
    size_t in_use = 0;
    size_t cached = 0;
    // Pinned staging ring of the boundary copies (made at the first large
    // copy; null if pinned memory could not be had: copies then go direct).
    char *staging = nullptr;
    hipEvent_t slot_done[3] = {};
    bool staging_tried = false;
    CopyPool *copy_pool = nullptr;
};

// Staged boundary copies: 3 pinned slots of 8 MiB (measured on MI355X with
// 64 MiB copies: 44-48 GB/s each way for 3-6 slots of 4-16 MiB and 1-7 copy
// threads beside the caller; pinned DMA alone 57 GB/s, pageable 17-29 GB/s);
// copies below 2 MiB go direct (the staging's per-slot waits would dominate
// them).
constexpr int STAGING_SLOTS = 3;
constexpr size_t STAGING_SLOT_BYTES = size_t(8) << 20;
constexpr size_t STAGING_MIN_BYTES = size_t(2) << 20;
static_assert(sizeof(State::slot_done) / sizeof(hipEvent_t) == STAGING_SLOTS,
              "one completion event per staging slot");

State &state() {
    static State s;
    return s;
}

thread_local std::string t_last_error;

} // namespace

// Scratch of the allocation-free entry points (camel_hip_sgemm_noalloc):
// their split-K partial sums live here instead of in pool blocks.  Every
// device the library runs on holds its own copy of this array until the
// process ends; host code never uses this name as an address, only the
// per-device address hipGetSymbolAddress gives for it at initialisation.
static __device__ __align__(256) float scratch[CAMEL_HIP_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace {

// Rounded block size: 512 B granules below 1 MiB, 2 MiB granules above, so
// tensors of one shape reuse one block and large tensors do not fragment.
size_t round_size(size_t bytes) {
    if (bytes == 0) bytes = 1;
    if (bytes < (1u << 20)) return (bytes + 511) & ~size_t(511);
    const size_t g = size_t(2) << 20;
    return (bytes + g - 1) / g * g;
}

} // namespace

std::recursive_mutex &lib_mutex() {
    static std::recursive_mutex m;
    return m;
}

int fail(int status, const std::string &message) {
    t_last_error = message;
    return status;
}

int ok() {
    t_last_error.clear();
    return CAMEL_HIP_OK;
}

int check_hip(hipError_t err, const char *what) {
    if (err == hipSuccess) return CAMEL_HIP_OK;
    return fail(CAMEL_HIP_ERR_RUNTIME, std::string(what) + ": " + hipGetErrorString(err));
}

int check_launch(const char *kernel) { return check_hip(hipGetLastError(), kernel); }

hipStream_t stream() { return state().stream; }
int device_cu_count() { return state().cu_count; }
int *error_flag() { return state().flag; }

namespace {

__global__ void fill_i32_kernel(int *p, int n, int v) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

int init_device(int device) {
    State &s = state();
    if (s.initialised) {
        if (device == s.device) return CAMEL_HIP_OK;
        return fail(CAMEL_HIP_ERR_ARG, "camel_hip_init: already initialised on another device");
    }
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0)
        return fail(CAMEL_HIP_ERR_NO_DEVICE, "camel_hip_init: no HIP device visible");
    if (device < 0 || device >= count)
        return fail(CAMEL_HIP_ERR_ARG, "camel_hip_init: device index out of range");
    CAMEL_RETURN_IF(check_hip(hipSetDevice(device), "hipSetDevice"));
    hipDeviceProp_t prop;
    CAMEL_RETURN_IF(check_hip(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties"));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(CAMEL_HIP_ERR_NO_DEVICE,
                    std::string("camel_hip_init: built for gfx950, device is ") + prop.gcnArchName);
    s.cu_count = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    // Default priority, non-blocking with respect to the legacy null stream.
    CAMEL_RETURN_IF(check_hip(hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking),
                              "hipStreamCreateWithFlags"));
    CAMEL_RETURN_IF(check_hip(hipMalloc(&s.flag, 256), "hipMalloc(error flag)"));
    // The static scratch's address on this device (the device is current).
    void *scratch_ptr = nullptr;
    CAMEL_RETURN_IF(check_hip(hipGetSymbolAddress(&scratch_ptr, HIP_SYMBOL(scratch)),
                              "hipGetSymbolAddress(scratch)"));
    if (!scratch_ptr || (reinterpret_cast<uintptr_t>(scratch_ptr) & 255) != 0)
        return fail(CAMEL_HIP_ERR_RUNTIME, "camel_hip_init: static scratch is not 256-byte aligned");
    s.scratch_by_device[device] = static_cast<float *>(scratch_ptr);
    s.device = device;
    s.initialised = true;
    return clear_error_flag();
}

// Returns the deferred blocks to the free lists once every stream of the
// device has drained.  A release never synchronises by itself (it may run in
// a garbage collector, or while another library captures a graph, where a
// device-wide wait fails); the wait happens here, at the library's own
// allocation misses and synchronisation points, and a failed wait keeps the
// blocks deferred for the next attempt.
void drain_deferred() {
    State &s = state();
    if (s.deferred.empty()) return;
    if (hipDeviceSynchronize() != hipSuccess) {
        (void)hipGetLastError();
        if (!s.deferred_warned) {
            std::fprintf(stderr, "camel_hip: %zu exported block(s) held back: the device-wide "
                                 "wait before their reuse failed; retrying later\n",
                         s.deferred.size());
            s.deferred_warned = true;
        }
        return;
    }
    for (const auto &[ptr, size] : s.deferred) {
        s.in_use -= size;
        s.free_lists[size].push_back(ptr);
        s.cached += size;
    }
    s.deferred.clear();
}

} // namespace

int ensure_init() {
    CAMEL_LOCK();
    if (state().initialised) return CAMEL_HIP_OK;
    return init_device(0);
}

bool initialised() {
    CAMEL_LOCK();
    return state().initialised;
}

float *noalloc_scratch() {
    CAMEL_LOCK();
    const State &s = state();
    if (!s.initialised) return nullptr;
    auto it = s.scratch_by_device.find(s.device);
    return it == s.scratch_by_device.end() ? nullptr : it->second;
}

int clear_error_flag() {
    hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(64), 0, stream(), error_flag(), 1, 0);
    return check_launch("fill_i32_kernel");
}

int read_error_flag(int *value) {
    CAMEL_RETURN_IF(check_hip(
        hipMemcpyAsync(value, error_flag(), sizeof(int), hipMemcpyDeviceToHost, stream()),
        "hipMemcpyAsync(error flag)"));
    return check_hip(hipStreamSynchronize(stream()), "hipStreamSynchronize");
}

// ---- creation kernels -------------------------------------------------------------

namespace {

__global__ void fill_f32_kernel(float4 *p4, float *p, int64_t n, float v) {
    int64_t n4 = n / 4;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (int64_t i = tid; i < n4; i += stride) p4[i] = make_float4(v, v, v, v);
    for (int64_t i = n4 * 4 + tid; i < n; i += stride) p[i] = v;
}

__global__ void fill_generic_kernel(int dt, void *p, int64_t n, double v) {
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        store_from_double(dt, p, i, v);
}

__global__ void eye_kernel(float *p, int64_t n) {
    int64_t total = n * n;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride)
        p[i] = (i / n == i % n) ? 1.0f : 0.0f;
}

__global__ void arange_kernel(int64_t *p, int64_t start, int64_t step, int64_t count) {
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride)
        p[i] = start + i * step;
}

} // namespace

namespace {

// The staging ring and its copy threads, made on first use (library mutex
// held).  False when pinned memory or events could not be had.
bool staging_ready() {
    State &s = state();
    if (s.staging) return true;
    if (s.staging_tried) return false;
    s.staging_tried = true;
    void *p = nullptr;
    if (hipHostMalloc(&p, STAGING_SLOTS * STAGING_SLOT_BYTES, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    for (int k = 0; k < STAGING_SLOTS; ++k) {
        if (hipEventCreateWithFlags(&s.slot_done[k], hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            for (int j = 0; j < k; ++j) (void)hipEventDestroy(s.slot_done[j]);
            (void)hipHostFree(p);
            return false;
        }
    }
    // three threads beside the caller: four host copies in parallel
    const unsigned hw = std::thread::hardware_concurrency();
    s.copy_pool = new CopyPool(hw >= 8 ? 3 : (hw > 1 ? (int)hw - 1 : 0));
    s.staging = static_cast<char *>(p);
    return true;
}

// Host -> device through the pinned slots: slot k is refilled once its
// previous DMA has completed, while the DMA of the slot before runs.
int staged_h2d(char *dst, const char *src, size_t bytes) {
    State &s = state();
    bool busy[STAGING_SLOTS] = {};
    int rc = CAMEL_HIP_OK;
    for_each_chunk(bytes, STAGING_SLOT_BYTES, [&](size_t i, size_t off, size_t m) {
        if (rc != CAMEL_HIP_OK) return;
        const int k = (int)(i % STAGING_SLOTS);
        char *slot = s.staging + k * STAGING_SLOT_BYTES;
        if (busy[k] && (rc = check_hip(hipEventSynchronize(s.slot_done[k]), "hipEventSynchronize")))
            return;
        s.copy_pool->copy(slot, src + off, m);
        if ((rc = check_hip(hipMemcpyAsync(dst + off, slot, m, hipMemcpyHostToDevice, stream()),
                            "hipMemcpyAsync(H2D)")))
            return;
        rc = check_hip(hipEventRecord(s.slot_done[k], stream()), "hipEventRecord");
        busy[k] = true;
    });
    // every DMA that was enqueued has finished reading its slot before return
    const int sync = check_hip(hipStreamSynchronize(stream()), "hipStreamSynchronize");
    return rc != CAMEL_HIP_OK ? rc : sync;
}

// Device -> host: the DMAs of the next slots run while the host copies the
// slot that has landed out to the destination.
int staged_d2h(char *dst, const char *src, size_t bytes) {
    State &s = state();
    struct Chunk {
        size_t off, size;
    };
    std::vector<Chunk> chunks;
    for_each_chunk(bytes, STAGING_SLOT_BYTES,
                   [&](size_t, size_t off, size_t m) { chunks.push_back({off, m}); });
    auto issue = [&](size_t i) {
        const int k = (int)(i % STAGING_SLOTS);
        CAMEL_RETURN_IF(check_hip(hipMemcpyAsync(s.staging + k * STAGING_SLOT_BYTES,
                                                 src + chunks[i].off, chunks[i].size,
                                                 hipMemcpyDeviceToHost, stream()),
                                  "hipMemcpyAsync(D2H)"));
        return check_hip(hipEventRecord(s.slot_done[k], stream()), "hipEventRecord");
    };
    int rc = CAMEL_HIP_OK;
    for (size_t i = 0; i < chunks.size() && i < (size_t)STAGING_SLOTS && rc == CAMEL_HIP_OK; ++i)
        rc = issue(i);
    for (size_t i = 0; i < chunks.size() && rc == CAMEL_HIP_OK; ++i) {
        const int k = (int)(i % STAGING_SLOTS);
        rc = check_hip(hipEventSynchronize(s.slot_done[k]), "hipEventSynchronize");
        if (rc != CAMEL_HIP_OK) break;
        s.copy_pool->copy(dst + chunks[i].off, s.staging + k * STAGING_SLOT_BYTES, chunks[i].size);
        if (i + STAGING_SLOTS < chunks.size()) rc = issue(i + STAGING_SLOTS);
    }
    const int sync = check_hip(hipStreamSynchronize(stream()), "hipStreamSynchronize");
    return rc != CAMEL_HIP_OK ? rc : sync;
}

} // namespace

} // namespace camel_hip

using namespace camel_hip;

extern "C" {

int camel_hip_init(int device) {
    CAMEL_LOCK();
    int rc = init_device(device);
    return rc == CAMEL_HIP_OK ? ok() : rc;
}

int camel_hip_device_count(int *count) {
    if (!count) return fail(CAMEL_HIP_ERR_ARG, "camel_hip_device_count: null output");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    *count = n;
    return ok();
}

const char *camel_hip_last_error(void) { return t_last_error.c_str(); }

int camel_hip_sync(void) {
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    CAMEL_RETURN_IF(check_hip(hipStreamSynchronize(stream()), "hipStreamSynchronize"));
    return ok();
}

int camel_hip_device_sync(void) {
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    CAMEL_RETURN_IF(check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize"));
    drain_deferred();
    return ok();
}

int camel_hip_current_device(int *device) {
    if (!device) return fail(CAMEL_HIP_ERR_ARG, "camel_hip_current_device: null pointer");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    *device = state().device;
    return ok();
}

void *camel_hip_stream(void) {
    CAMEL_LOCK();
    if (ensure_init() != CAMEL_HIP_OK) return nullptr;
    return (void *)stream();
}

int camel_hip_malloc(void **ptr, size_t bytes) {
    if (!ptr) return fail(CAMEL_HIP_ERR_ARG, "camel_hip_malloc: null output");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    State &s = state();
    size_t size = round_size(bytes);
    auto it = s.free_lists.find(size);
    if (it != s.free_lists.end() && !it->second.empty()) {
        *ptr = it->second.back();
        it->second.pop_back();
        s.cached -= size;
    } else {
        drain_deferred();
        auto again = s.free_lists.find(size);
        if (again != s.free_lists.end() && !again->second.empty()) {
            *ptr = again->second.back();
            again->second.pop_back();
            s.cached -= size;
            s.live[*ptr] = size;
            s.in_use += size;
            return ok();
        }
        void *p = nullptr;
        hipError_t err = hipMalloc(&p, size);
        if (err != hipSuccess) {
            (void)hipGetLastError();
            camel_hip_pool_trim();
            err = hipMalloc(&p, size);
        }
        if (err != hipSuccess) {
            (void)hipGetLastError();
            return fail(CAMEL_HIP_ERR_OOM, "camel_hip_malloc: out of device memory for " +
                                               std::to_string(bytes) + " bytes");
        }
        *ptr = p;
    }
    s.live[*ptr] = size;
    s.in_use += size;
    return ok();
}

int camel_hip_free(void *ptr) {
    if (!ptr) return ok();
    CAMEL_LOCK();
    State &s = state();
    auto it = s.live.find(ptr);
    if (it == s.live.end()) return fail(CAMEL_HIP_ERR_ARG, "camel_hip_free: unknown pointer");
    size_t size = it->second;
    s.live.erase(it);
    s.in_use -= size;
    // Work already enqueued on the single stream may still read the block; a
    // later allocation reuses it only through that same stream, so stream
    // order keeps the reuse safe without a synchronisation here.
    s.free_lists[size].push_back(ptr);
    s.cached += size;
    return ok();
}

int camel_hip_free_shared(void *ptr) {
    if (!ptr) return ok();
    CAMEL_LOCK();
    State &s = state();
    auto it = s.live.find(ptr);
    if (it == s.live.end()) return fail(CAMEL_HIP_ERR_ARG, "camel_hip_free_shared: unknown pointer");
    // Still counted in use until drain_deferred returns it to the pool.
    s.deferred.emplace_back(ptr, it->second);
    s.live.erase(it);
    return ok();
}

int camel_hip_pool_trim(void) {
    CAMEL_LOCK();
    State &s = state();
    if (!s.initialised) return ok();
    drain_deferred();
    CAMEL_RETURN_IF(check_hip(hipStreamSynchronize(s.stream), "hipStreamSynchronize"));
    for (auto &kv : s.free_lists) {
        for (void *p : kv.second) (void)hipFree(p);
        kv.second.clear();
    }
    s.cached = 0;
    return ok();
}

int camel_hip_pool_stats(size_t *in_use, size_t *cached) {
    CAMEL_LOCK();
    if (in_use) *in_use = state().in_use;
    if (cached) *cached = state().cached;
    return ok();
}

int camel_hip_h2d(void *dst, const void *src, size_t bytes) {
    if (bytes == 0) return ok();
    if (!dst || !src) return fail(CAMEL_HIP_ERR_ARG, "camel_hip_h2d: null pointer");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    if (bytes >= STAGING_MIN_BYTES && staging_ready()) {
        CAMEL_RETURN_IF(staged_h2d(static_cast<char *>(dst), static_cast<const char *>(src), bytes));
        return ok();
    }
    CAMEL_RETURN_IF(check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream()),
                              "hipMemcpyAsync(H2D)"));
    CAMEL_RETURN_IF(check_hip(hipStreamSynchronize(stream()), "hipStreamSynchronize"));
    return ok();
}

int camel_hip_d2h(void *dst, const void *src, size_t bytes) {
    if (bytes == 0) return ok();
    if (!dst || !src) return fail(CAMEL_HIP_ERR_ARG, "camel_hip_d2h: null pointer");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    if (bytes >= STAGING_MIN_BYTES && staging_ready()) {
        CAMEL_RETURN_IF(staged_d2h(static_cast<char *>(dst), static_cast<const char *>(src), bytes));
        return ok();
    }
    CAMEL_RETURN_IF(check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, stream()),
                              "hipMemcpyAsync(D2H)"));
    CAMEL_RETURN_IF(check_hip(hipStreamSynchronize(stream()), "hipStreamSynchronize"));
    return ok();
}

int camel_hip_d2d(void *dst, const void *src, size_t bytes) {
    if (bytes == 0) return ok();
    if (!dst || !src) return fail(CAMEL_HIP_ERR_ARG, "camel_hip_d2d: null pointer");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    CAMEL_RETURN_IF(check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream()),
                              "hipMemcpyAsync(D2D)"));
    return ok();
}

int camel_hip_fill(int dtype, void *out, int64_t n, double value) {
    if (!valid_dtype(dtype)) return fail(CAMEL_HIP_ERR_DTYPE, "camel_hip_fill: unknown dtype");
    if (n < 0) return fail(CAMEL_HIP_ERR_ARG, "camel_hip_fill: negative size");
    if (n == 0) return ok();
    if (!out) return fail(CAMEL_HIP_ERR_ARG, "camel_hip_fill: null output");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    if (dtype == CAMEL_DT_F32 && (reinterpret_cast<uintptr_t>(out) & 15) == 0) {
        hipLaunchKernelGGL(fill_f32_kernel, dim3(grid_for(n / 4 + 1, 256)), dim3(256), 0, stream(),
                           static_cast<float4 *>(out), static_cast<float *>(out), n, (float)value);
        CAMEL_RETURN_IF(check_launch("fill_f32_kernel"));
    } else {
        hipLaunchKernelGGL(fill_generic_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream(),
                           dtype, out, n, value);
        CAMEL_RETURN_IF(check_launch("fill_generic_kernel"));
    }
    return ok();
}

int camel_hip_eye(float *out, int64_t n) {
    if (n < 0) return fail(CAMEL_HIP_ERR_ARG, "eye size cannot be negative");
    if (n == 0) return ok();
    if (!out) return fail(CAMEL_HIP_ERR_ARG, "camel_hip_eye: null output");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    hipLaunchKernelGGL(eye_kernel, dim3(grid_for(n * n, 256)), dim3(256), 0, stream(), out, n);
    CAMEL_RETURN_IF(check_launch("eye_kernel"));
    return ok();
}

int camel_hip_arange(int64_t *out, int64_t start, int64_t step, int64_t count) {
    if (step == 0) return fail(CAMEL_HIP_ERR_ARG, "range step cannot be zero");
    if (count < 0) return fail(CAMEL_HIP_ERR_ARG, "camel_hip_arange: negative count");
    if (count == 0) return ok();
    if (!out) return fail(CAMEL_HIP_ERR_ARG, "camel_hip_arange: null output");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    hipLaunchKernelGGL(arange_kernel, dim3(grid_for(count, 256)), dim3(256), 0, stream(), out,
                       start, step, count);
    CAMEL_RETURN_IF(check_launch("arange_kernel"));
    return ok();
}

int camel_hip_event_create(void **event) {
    if (!event) return fail(CAMEL_HIP_ERR_ARG, "camel_hip_event_create: null output");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    hipEvent_t e;
    CAMEL_RETURN_IF(check_hip(hipEventCreate(&e), "hipEventCreate"));
    *event = (void *)e;
    return ok();
}

int camel_hip_event_record(void *event) {
    if (!event) return fail(CAMEL_HIP_ERR_ARG, "camel_hip_event_record: null event");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    CAMEL_RETURN_IF(check_hip(hipEventRecord((hipEvent_t)event, stream()), "hipEventRecord"));
    return ok();
}

int camel_hip_event_elapsed_ms(void *start, void *stop, float *ms) {
    if (!start || !stop || !ms) return fail(CAMEL_HIP_ERR_ARG, "camel_hip_event_elapsed_ms: null");
    CAMEL_LOCK();
    CAMEL_RETURN_IF(check_hip(hipEventSynchronize((hipEvent_t)stop), "hipEventSynchronize"));
    CAMEL_RETURN_IF(
        check_hip(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop), "hipEventElapsed"));
    return ok();
}

int camel_hip_event_destroy(void *event) {
    if (!event) return ok();
    CAMEL_LOCK();
    CAMEL_RETURN_IF(check_hip(hipEventDestroy((hipEvent_t)event), "hipEventDestroy"));
    return ok();
}

} // extern "C"
