// Host harness of the operator layer: the extern "C" entry points of
// include/camel_tensor.h.  It builds ArgsViews from {code, slot} pairs and
// calls the registered operator_t exactly as the reference's executors do
// (modules/tensor/executor.cpp:36-56: look the URI suffix up in the ops map,
// call op(with, norm, ctx), store the result slot).
#include "camel_tensor.h"

#include "chain.h"
#include "operators.h"
#include "runtime.h"
#include "tensor_type.h"

#include <algorithm>
#include <memory>
#include <mutex>
#include <sstream>
#include <unordered_map>

using namespace camel_amd;
using namespace camel_amd::tensor;

namespace {

thread_local std::string t_error;

int fail(int status, std::string msg) {
    t_error = std::move(msg);
    return status;
}

int ok() {
    t_error.clear();
    return CAMEL_TENSOR_OK;
}

const std::unordered_map<std::string, operator_t> &opsMap() {
    static const auto map = getTensorOpsMap();
    return map;
}

const std::vector<std::string> &opNames() {
    static const std::vector<std::string> names = [] {
        std::vector<std::string> v;
        for (const auto &kv : opsMap()) v.push_back(kv.first);
        std::sort(v.begin(), v.end());
        return v;
    }();
    return names;
}

TensorObject *tensorOf(uint64_t handle) {
    auto *t = fromSlot<TensorObject *>(handle);
    return t && isLiveTensor(t) ? t : nullptr;
}

ArrayObject *arrayOf(uint64_t handle) {
    auto *a = fromSlot<ArrayObject *>(handle);
    return a && isLiveArray(a) ? a : nullptr;
}

// Builds a view over caller values, checking every handle is a live object
// of the kind its code names.
bool buildView(int64_t n, const camel_value *values, VectorArgsView &view, std::string &err) {
    for (int64_t i = 0; i < n; ++i) {
        const TypeCode code = static_cast<TypeCode>(values[i].code);
        if (code == TypeCode::Tensor && values[i].slot != 0 && !tensorOf(values[i].slot)) {
            err = "argument " + std::to_string(i) + " is not a live tensor handle";
            return false;
        }
        if (code == TypeCode::Array && values[i].slot != 0 && !arrayOf(values[i].slot)) {
            err = "argument " + std::to_string(i) + " is not a live array handle";
            return false;
        }
        view.push(code, values[i].slot);
    }
    return true;
}

// Live chains by handle (the address of the chain object).
std::mutex g_chain_mutex;
std::unordered_map<uint64_t, std::unique_ptr<LayerChain>> g_chains;

LayerChain *chainOf(uint64_t handle) {
    std::lock_guard<std::mutex> lock(g_chain_mutex);
    auto it = g_chains.find(handle);
    return it == g_chains.end() ? nullptr : it->second.get();
}

template <typename Fn> int guarded(Fn &&fn) {
    try {
        // Objects made by a call that throws never reach the caller.
        CreationScope scope;
        return fn();
    } catch (const RuntimeFault &e) {
        return fail(CAMEL_TENSOR_ERR_RUNTIME, e.what());
    } catch (const std::exception &e) {
        return fail(CAMEL_TENSOR_ERR_RUNTIME, e.what());
    }
}

} // namespace

extern "C" {

const char *camel_tensor_last_error(void) { return t_error.c_str(); }

int camel_module_abi_version(void) { return 1; }

namespace {

// A TensorType from C-ABI arguments (shape extents must be non-negative).
bool tensorTypeOf(uint32_t dtype, int64_t rank, const int64_t *shape, TensorType &out) {
    if (rank < 0 || (rank > 0 && !shape)) return false;
    std::vector<size_t> dims;
    for (int64_t i = 0; i < rank; ++i) {
        if (shape[i] < 0) return false;
        dims.push_back(static_cast<size_t>(shape[i]));
    }
    out = TensorType(std::move(dims), static_cast<TypeCode>(dtype));
    return true;
}

} // namespace

int camel_tensor_type_string(uint32_t dtype, int64_t rank, const int64_t *shape, int mangled,
                             char *buf, size_t cap, size_t *needed) {
    TensorType t;
    if (!tensorTypeOf(dtype, rank, shape, t))
        return fail(CAMEL_TENSOR_ERR_ARG, "camel_tensor_type_string: bad shape");
    return guarded([&] {
        const std::string text = mangled ? t.mangle() : t.toString();
        if (needed) *needed = text.size() + 1;
        if (buf && cap > 0) {
            const size_t n = std::min(cap - 1, text.size());
            std::memcpy(buf, text.data(), n);
            buf[n] = '\0';
        }
        return ok();
    });
}

int camel_tensor_type_relation(uint32_t dst_dtype, int64_t dst_rank, const int64_t *dst_shape,
                               uint32_t src_dtype, int64_t src_rank, const int64_t *src_shape,
                               int *assignable, int *equal) {
    TensorType dst, src;
    if (!tensorTypeOf(dst_dtype, dst_rank, dst_shape, dst) ||
        !tensorTypeOf(src_dtype, src_rank, src_shape, src))
        return fail(CAMEL_TENSOR_ERR_ARG, "camel_tensor_type_relation: bad shape");
    if (assignable) *assignable = dst.assignableFrom(src) ? 1 : 0;
    if (equal) *equal = dst.equals(src) ? 1 : 0;
    return ok();
}

int camel_tensor_from_host(uint32_t dtype, int64_t rank, const int64_t *shape, const void *data,
                           uint64_t *handle) {
    if (!handle || rank < 0 || (rank > 0 && !shape))
        return fail(CAMEL_TENSOR_ERR_ARG, "camel_tensor_from_host: bad arguments");
    return guarded([&] {
        TensorObject *t = TensorObject::create(static_cast<TypeCode>(dtype),
                                               std::span<const int64_t>(shape, (size_t)rank),
                                               Residence::Host);
        if (t->byteSize() > 0) {
            if (!data) {
                releaseTensor(t);
                return fail(CAMEL_TENSOR_ERR_ARG, "camel_tensor_from_host: null data");
            }
            std::memcpy(t->hostOutput(), data, t->byteSize());
        }
        *handle = toSlot(t);
        return ok();
    });
}

int camel_tensor_to_host(uint64_t handle, void *dst, size_t bytes) {
    TensorObject *t = tensorOf(handle);
    if (!t) return fail(CAMEL_TENSOR_ERR_ARG, "camel_tensor_to_host: not a live tensor");
    if (bytes != t->byteSize() || (bytes > 0 && !dst))
        return fail(CAMEL_TENSOR_ERR_ARG, "camel_tensor_to_host: size mismatch");
    return guarded([&] {
        if (bytes > 0) std::memcpy(dst, t->hostData(), bytes);
        return ok();
    });
}

int camel_tensor_meta(uint64_t handle, uint32_t *dtype, int64_t *rank, int64_t *shape, int64_t cap) {
    TensorObject *t = tensorOf(handle);
    if (!t) return fail(CAMEL_TENSOR_ERR_ARG, "camel_tensor_meta: not a live tensor");
    if (dtype) *dtype = static_cast<uint32_t>(t->dtype());
    if (rank) *rank = (int64_t)t->rank();
    for (int64_t i = 0; shape && i < cap && i < (int64_t)t->rank(); ++i) shape[i] = t->dim(i);
    return ok();
}

int camel_tensor_residency(uint64_t handle, int *host_valid, int *device_valid) {
    TensorObject *t = tensorOf(handle);
    if (!t) return fail(CAMEL_TENSOR_ERR_ARG, "camel_tensor_residency: not a live tensor");
    if (host_valid) *host_valid = t->hostValid() ? 1 : 0;
    if (device_valid) *device_valid = t->deviceValid() ? 1 : 0;
    return ok();
}

int camel_tensor_device_ptr(uint64_t handle, uint64_t *device_ptr) {
    TensorObject *t = tensorOf(handle);
    if (!t || !device_ptr) return fail(CAMEL_TENSOR_ERR_ARG, "camel_tensor_device_ptr: bad arguments");
    return guarded([&] {
        *device_ptr = toSlot(t->deviceData());
        return ok();
    });
}

int camel_tensor_release(uint64_t handle) {
    auto *t = fromSlot<TensorObject *>(handle);
    if (!t || !releaseTensor(t)) return fail(CAMEL_TENSOR_ERR_ARG, "camel_tensor_release: not a live tensor");
    return ok();
}

int camel_tensor_to_dlpack(uint64_t handle, int on_device, DLManagedTensor **managed) {
    TensorObject *t = tensorOf(handle);
    if (!t || !managed) return fail(CAMEL_TENSOR_ERR_ARG, "camel_tensor_to_dlpack: bad arguments");
    return guarded([&] {
        *managed = tensorToDLPack(t, on_device != 0);
        return ok();
    });
}

int camel_tensor_from_dlpack(const DLManagedTensor *managed, uint64_t *handle) {
    if (!handle) return fail(CAMEL_TENSOR_ERR_ARG, "camel_tensor_from_dlpack: bad arguments");
    return guarded([&] {
        *handle = toSlot(tensorFromDLPack(managed));
        return ok();
    });
}

int64_t camel_tensor_live_count(void) { return (int64_t)liveTensorCount(); }

int64_t camel_tensor_release_all(void) { return (int64_t)releaseAll(); }

uint64_t camel_tensor_mark(void) { return registryMark(); }

int camel_tensor_release_since(uint64_t mark, int64_t n_keep, const uint64_t *keep,
                               int64_t *released) {
    if (n_keep < 0 || (n_keep > 0 && !keep))
        return fail(CAMEL_TENSOR_ERR_ARG, "camel_tensor_release_since: bad arguments");
    std::vector<const void *> kept;
    kept.reserve((size_t)n_keep);
    for (int64_t i = 0; i < n_keep; ++i) kept.push_back(reinterpret_cast<const void *>(keep[i]));
    const size_t n = releaseSince(mark, kept);
    if (released) *released = (int64_t)n;
    return ok();
}

int camel_tensor_format(uint64_t handle, char *buf, size_t cap, size_t *needed) {
    TensorObject *t = tensorOf(handle);
    if (!t) return fail(CAMEL_TENSOR_ERR_ARG, "camel_tensor_format: not a live tensor");
    return guarded([&] {
        std::ostringstream os;
        t->print(os);
        const std::string s = os.str();
        if (needed) *needed = s.size() + 1;
        if (buf && cap > 0) {
            const size_t n = std::min(cap - 1, s.size());
            std::memcpy(buf, s.data(), n);
            buf[n] = '\0';
        }
        return ok();
    });
}

int camel_tensor_clone(uint64_t handle, uint64_t *copy) {
    TensorObject *t = tensorOf(handle);
    if (!t || !copy) return fail(CAMEL_TENSOR_ERR_ARG, "camel_tensor_clone: bad arguments");
    return guarded([&] {
        *copy = toSlot(t->clone());
        return ok();
    });
}

int camel_tensor_equals(uint64_t a, uint64_t b, int *equal) {
    TensorObject *ta = tensorOf(a), *tb = tensorOf(b);
    if (!ta || !tb || !equal) return fail(CAMEL_TENSOR_ERR_ARG, "camel_tensor_equals: bad arguments");
    return guarded([&] {
        *equal = ta->equals(tb) ? 1 : 0;
        return ok();
    });
}

int camel_array_create(uint32_t elem_code, int64_t count, const uint64_t *slots, uint64_t *handle) {
    if (!handle || count < 0 || (count > 0 && !slots))
        return fail(CAMEL_TENSOR_ERR_ARG, "camel_array_create: bad arguments");
    const TypeCode elem = static_cast<TypeCode>(elem_code);
    for (int64_t i = 0; elem == TypeCode::Array && i < count; ++i)
        if (!arrayOf(slots[i])) return fail(CAMEL_TENSOR_ERR_ARG, "camel_array_create: bad nested array");
    auto *a = new ArrayObject{elem, std::vector<slot_t>(slots, slots + count)};
    registerObject(a);
    *handle = toSlot(a);
    return ok();
}

int camel_array_read(uint64_t handle, uint32_t *elem_code, int64_t *count, uint64_t *slots,
                     int64_t cap) {
    ArrayObject *a = arrayOf(handle);
    if (!a) return fail(CAMEL_TENSOR_ERR_ARG, "camel_array_read: not a live array");
    if (elem_code) *elem_code = static_cast<uint32_t>(a->elem);
    if (count) *count = (int64_t)a->size();
    for (int64_t i = 0; slots && i < cap && i < (int64_t)a->size(); ++i) slots[i] = a->items[i];
    return ok();
}

int camel_array_release(uint64_t handle) {
    auto *a = fromSlot<ArrayObject *>(handle);
    if (!a || !releaseArray(a)) return fail(CAMEL_TENSOR_ERR_ARG, "camel_array_release: not a live array");
    return ok();
}

int camel_tensor_invoke(const char *uri, int64_t n_with, const camel_value *with, int64_t n_norm,
                        const camel_value *norm, camel_value *result) {
    if (!uri || !result || n_with < 0 || n_norm < 0 || (n_with > 0 && !with) || (n_norm > 0 && !norm))
        return fail(CAMEL_TENSOR_ERR_ARG, "camel_tensor_invoke: bad arguments");
    std::string key(uri);
    if (key.rfind("tensor:", 0) == 0) key = key.substr(7);
    auto it = opsMap().find(key);
    if (it == opsMap().end()) return fail(CAMEL_TENSOR_ERR_URI, "Unrecognized operator URI: " + std::string(uri));
    VectorArgsView withView, normView;
    std::string err;
    if (!buildView(n_with, with, withView, err) || !buildView(n_norm, norm, normView, err))
        return fail(CAMEL_TENSOR_ERR_ARG, err);
    // The result type is the one the operator's group resolves for these
    // argument codes (the compiler fixes it in the reference).
    std::vector<TypeCode> wc, nc;
    for (int64_t i = 0; i < n_with; ++i) wc.push_back(static_cast<TypeCode>(with[i].code));
    for (int64_t i = 0; i < n_norm; ++i) nc.push_back(static_cast<TypeCode>(norm[i].code));
    std::optional<ResultType> rtype;
    const std::string full = "tensor:" + key;
    for (const auto &g : getTensorOperatorGroups()) {
        for (const auto &[guri, fn] : g.overloads) {
            if (guri != full) continue;
            if (auto t = fn(wc, nc)) rtype = t;
            if (rtype) break;
        }
        if (rtype) break;
    }
    if (!rtype)
        return fail(CAMEL_TENSOR_ERR_RESOLVE, "no overload of " + full + " accepts these argument types");
    return guarded([&] {
        Context ctx;
        const slot_t out = it->second(withView, normView, ctx);
        result->code = static_cast<uint32_t>(rtype->code);
        result->slot = out;
        return ok();
    });
}

int camel_tensor_resolve(const char *group, int64_t n_with, const uint32_t *with_codes,
                         int64_t n_norm, const uint32_t *norm_codes, char *uri, size_t cap,
                         uint32_t *result_code, uint32_t *result_elem) {
    if (!group || n_with < 0 || n_norm < 0 || (n_with > 0 && !with_codes) ||
        (n_norm > 0 && !norm_codes))
        return fail(CAMEL_TENSOR_ERR_ARG, "camel_tensor_resolve: bad arguments");
    std::vector<TypeCode> wc, nc;
    for (int64_t i = 0; i < n_with; ++i) wc.push_back(static_cast<TypeCode>(with_codes[i]));
    for (int64_t i = 0; i < n_norm; ++i) nc.push_back(static_cast<TypeCode>(norm_codes[i]));
    bool found = false;
    for (const auto &g : getTensorOperatorGroups()) {
        if (g.name != group) continue;
        found = true;
        if (auto r = g.resolve(wc, nc)) {
            if (uri && cap > 0) {
                const size_t n = std::min(cap - 1, r->first.size());
                std::memcpy(uri, r->first.data(), n);
                uri[n] = '\0';
            }
            if (result_code) *result_code = static_cast<uint32_t>(r->second.code);
            if (result_elem) *result_elem = static_cast<uint32_t>(r->second.elem);
            return ok();
        }
    }
    if (!found) return fail(CAMEL_TENSOR_ERR_URI, "Unknown operator group: " + std::string(group));
    return fail(CAMEL_TENSOR_ERR_RESOLVE, "no overload of " + std::string(group) + " accepts these argument types");
}

int camel_chain_create(uint64_t *chain) {
    if (!chain) return fail(CAMEL_TENSOR_ERR_ARG, "camel_chain_create: null handle");
    auto c = std::make_unique<LayerChain>();
    const uint64_t h = reinterpret_cast<uint64_t>(c.get());
    std::lock_guard<std::mutex> lock(g_chain_mutex);
    g_chains.emplace(h, std::move(c));
    *chain = h;
    return ok();
}

int camel_chain_append(uint64_t chain, const char *uri, int64_t n_with, const camel_value *with) {
    LayerChain *c = chainOf(chain);
    if (!c || !uri || n_with < 0 || (n_with > 0 && !with))
        return fail(CAMEL_TENSOR_ERR_ARG, "camel_chain_append: bad arguments");
    // Bind arguments as LayerOperands reads them: tensors (Void for "no
    // bias") first, then integers (an Array of integers counts as its items).
    std::vector<const TensorObject *> tensors;
    std::vector<int64_t> ints;
    int64_t i = 0;
    for (; i < n_with; ++i) {
        const TypeCode code = static_cast<TypeCode>(with[i].code);
        if (code == TypeCode::Void) {
            tensors.push_back(nullptr);
        } else if (code == TypeCode::Tensor) {
            TensorObject *t = tensorOf(with[i].slot);
            if (!t) return fail(CAMEL_TENSOR_ERR_ARG, "argument " + std::to_string(i) + " is not a live tensor handle");
            tensors.push_back(t);
        } else {
            break;
        }
    }
    for (; i < n_with; ++i) {
        const TypeCode code = static_cast<TypeCode>(with[i].code);
        if (code == TypeCode::Int32) {
            ints.push_back(static_cast<int32_t>(static_cast<uint32_t>(with[i].slot)));
        } else if (code == TypeCode::Int64) {
            ints.push_back(static_cast<int64_t>(with[i].slot));
        } else if (code == TypeCode::Array) {
            ArrayObject *a = arrayOf(with[i].slot);
            if (!a) return fail(CAMEL_TENSOR_ERR_ARG, "argument " + std::to_string(i) + " is not a live array handle");
            return guarded([&] {
                for (int64_t d : parseShapeArray(a, TypeCode::Array)) ints.push_back(d);
                c->append(uri, tensors, ints);
                return ok();
            });
        } else {
            return fail(CAMEL_TENSOR_ERR_RUNTIME, "Expected integer argument");
        }
    }
    return guarded([&] {
        c->append(uri, tensors, ints);
        return ok();
    });
}

int camel_chain_apply(uint64_t chain, uint64_t x, uint64_t *result) {
    LayerChain *c = chainOf(chain);
    TensorObject *t = tensorOf(x);
    if (!c || !t || !result) return fail(CAMEL_TENSOR_ERR_ARG, "camel_chain_apply: bad arguments");
    return guarded([&] {
        *result = toSlot(c->apply(t));
        return ok();
    });
}

int camel_chain_plan(uint64_t chain, int64_t rank, const int64_t *shape, uint32_t dtype, char *buf,
                     size_t cap, size_t *needed) {
    LayerChain *c = chainOf(chain);
    if (!c || rank < 0 || (rank > 0 && !shape))
        return fail(CAMEL_TENSOR_ERR_ARG, "camel_chain_plan: bad arguments");
    if (dtype != CAMEL_TC_FLOAT32 && dtype != CAMEL_TC_INT64 && dtype != CAMEL_TC_BOOL &&
        dtype != CAMEL_TC_FLOAT64 && dtype != CAMEL_TC_INT32)
        return fail(CAMEL_TENSOR_ERR_ARG, "camel_chain_plan: not a tensor dtype");
    const std::string text = c->plan(std::span<const int64_t>(shape, (size_t)rank),
                                     normalizeTensorDType(static_cast<TypeCode>(dtype)));
    if (needed) *needed = text.size() + 1;
    if (buf && cap > 0) {
        const size_t n = std::min(cap - 1, text.size());
        std::memcpy(buf, text.data(), n);
        buf[n] = '\0';
    }
    return ok();
}

int camel_chain_release(uint64_t chain) {
    std::lock_guard<std::mutex> lock(g_chain_mutex);
    if (g_chains.erase(chain) == 0) return fail(CAMEL_TENSOR_ERR_ARG, "camel_chain_release: not a live chain");
    return ok();
}

int64_t camel_tensor_op_count(void) { return (int64_t)opNames().size(); }

const char *camel_tensor_op_name(int64_t index) {
    if (index < 0 || index >= (int64_t)opNames().size()) return nullptr;
    return opNames()[(size_t)index].c_str();
}

int64_t camel_tensor_group_count(void) { return (int64_t)getTensorOperatorGroups().size(); }

const char *camel_tensor_group_name(int64_t index) {
    const auto &g = getTensorOperatorGroups();
    if (index < 0 || index >= (int64_t)g.size()) return nullptr;
    return g[(size_t)index].name.c_str();
}

} // extern "C"
