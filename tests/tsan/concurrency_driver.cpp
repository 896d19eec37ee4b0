// Concurrency driver for ThreadSanitizer: worker threads drive the operator
// layer's host-side paths at once, the way the reference's Taskflow scheduler
// calls operators from worker threads (src/passes/sched/taskflow/taskflow.cpp:
// 157-181, 474-513).  Every path here stays on the host (host-born tensors,
// views, shape arrays, element reads, equality, printing, layer-chain
// planning, release), so it runs without a GPU; what it exercises is the
// layer's shared state: the object and chain registries, the Storage
// residency state and the per-thread error text.
//
// Usage: concurrency_driver [threads] [iterations]; exit status 0 when every
// result matched (ThreadSanitizer reports separately on stderr).
#include "camel_tensor.h"

#include <atomic>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

namespace {

std::atomic<int> g_failures{0};

void fail(int id, const char *what) {
    std::fprintf(stderr, "thread %d: %s: %s\n", id, what, camel_tensor_last_error());
    ++g_failures;
}

uint64_t f64_bits(double v) {
    uint64_t u;
    std::memcpy(&u, &v, sizeof u);
    return u;
}

double bits_f64(uint64_t u) {
    double v;
    std::memcpy(&v, &u, sizeof v);
    return v;
}

void worker(int id, int iterations) {
    const int64_t rows = 3, cols = 4 + id;
    std::vector<float> data((size_t)(rows * cols));
    for (int it = 0; it < iterations; ++it) {
        for (size_t i = 0; i < data.size(); ++i) data[i] = (float)(id * 1000 + it) + 0.25f * (float)i;
        const int64_t shape[2] = {rows, cols};
        uint64_t t = 0;
        if (camel_tensor_from_host(CAMEL_TC_FLOAT32, 2, shape, data.data(), &t)) {
            fail(id, "from_host");
            continue;
        }
        // shape(t) -> [rows, cols]
        camel_value arg{CAMEL_TC_TENSOR, t}, res{};
        if (camel_tensor_invoke("tensor:shape", 0, nullptr, 1, &arg, &res) ||
            res.code != CAMEL_TC_ARRAY) {
            fail(id, "shape");
        } else {
            uint32_t elem = 0;
            int64_t count = 0;
            uint64_t dims[2] = {0, 0};
            if (camel_array_read(res.slot, &elem, &count, dims, 2) || count != 2 ||
                (int64_t)dims[0] != rows || (int64_t)dims[1] != cols)
                fail(id, "shape values");
            camel_array_release(res.slot);
        }
        // reshape(t, [cols, rows]) -> a view sharing t's storage
        const uint64_t new_dims[2] = {(uint64_t)cols, (uint64_t)rows};
        uint64_t arr = 0;
        if (camel_array_create(CAMEL_TC_INT64, 2, new_dims, &arr)) {
            fail(id, "array_create");
        } else {
            camel_value args[2] = {{CAMEL_TC_TENSOR, t}, {CAMEL_TC_ARRAY, arr}};
            camel_value view{};
            if (camel_tensor_invoke("tensor:reshape", 0, nullptr, 2, args, &view) ||
                view.code != CAMEL_TC_TENSOR) {
                fail(id, "reshape");
            } else {
                // view[1][2] is flat element 1*rows + 2
                camel_value ij[3] = {{CAMEL_TC_TENSOR, view.slot}, {CAMEL_TC_INT64, 1},
                                     {CAMEL_TC_INT64, 2}};
                camel_value got{};
                if (camel_tensor_invoke("tensor:idx2d", 0, nullptr, 3, ij, &got) ||
                    got.code != CAMEL_TC_FLOAT64 ||
                    bits_f64(got.slot) != (double)data[(size_t)(1 * rows + 2)])
                    fail(id, "idx2d");
                int equal = 0;
                if (camel_tensor_equals(t, t, &equal) || !equal) fail(id, "equals");
                std::vector<float> back(data.size());
                if (camel_tensor_to_host(view.slot, back.data(), back.size() * sizeof(float)) ||
                    std::memcmp(back.data(), data.data(), back.size() * sizeof(float)) != 0)
                    fail(id, "to_host");
                size_t need = 0;
                if (camel_tensor_format(view.slot, nullptr, 0, &need) || need < 8) fail(id, "format");
                if (camel_tensor_release(view.slot)) fail(id, "release view");
            }
            camel_array_release(arr);
        }
        // A layer chain over host-born weights: created, extended, planned and
        // released on every thread at once (the chain registry is shared).
        {
            const int64_t wshape[2] = {cols, 5};
            std::vector<float> wdata((size_t)(cols * 5), 0.5f);
            uint64_t w = 0, chain = 0;
            if (camel_tensor_from_host(CAMEL_TC_FLOAT32, 2, wshape, wdata.data(), &w) ||
                camel_chain_create(&chain)) {
                fail(id, "chain setup");
            } else {
                camel_value wv{CAMEL_TC_TENSOR, w};
                if (camel_chain_append(chain, "tensor:dense", 1, &wv) ||
                    camel_chain_append(chain, "relu", 0, nullptr) ||
                    camel_chain_append(chain, "softmax", 0, nullptr))
                    fail(id, "chain append");
                char plan[128];
                size_t need = 0;
                if (camel_chain_plan(chain, 2, shape, CAMEL_TC_FLOAT32, plan, sizeof plan, &need) ||
                    std::strcmp(plan, "dense_relu+softmax\n") != 0)
                    fail(id, "chain plan");
                if (camel_chain_release(chain)) fail(id, "chain release");
                if (camel_tensor_release(w)) fail(id, "release weights");
            }
        }
        // An error on this thread must not leak into another thread's text.
        camel_value bad{CAMEL_TC_TENSOR, t}, out{};
        camel_value two[2] = {bad, {CAMEL_TC_FLOAT64, f64_bits(1.0)}};
        if (camel_tensor_invoke("tensor:reshape", 0, nullptr, 2, two, &out) == CAMEL_TENSOR_OK)
            fail(id, "bad reshape accepted");
        else if (std::strlen(camel_tensor_last_error()) == 0)
            fail(id, "error text missing");
        if (camel_tensor_release(t)) fail(id, "release");
    }
}

} // namespace

int main(int argc, char **argv) {
    const int threads = argc > 1 ? std::atoi(argv[1]) : 8;
    const int iterations = argc > 2 ? std::atoi(argv[2]) : 200;
    std::vector<std::thread> pool;
    for (int i = 0; i < threads; ++i) pool.emplace_back(worker, i, iterations);
    for (auto &th : pool) th.join();
    if (camel_tensor_live_count() != 0) {
        std::fprintf(stderr, "%lld objects still live\n", (long long)camel_tensor_live_count());
        ++g_failures;
    }
    std::printf("threads=%d iterations=%d failures=%d\n", threads, iterations, g_failures.load());
    return g_failures.load() == 0 ? 0 : 1;
}
