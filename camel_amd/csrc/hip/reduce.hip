// Row softmax and the rank-2 reductions (sum / max / argmax along an axis,
// whole-tensor sum).
//
// Softmax fuses the nine-operator composition of test/run/nn/mnist.cml:13-25
// into one pass, op for op:
//   m  = first strict-'>' row max (tensorMaxAxis, runtime.cpp:924-963)
//   mb = fl32(0.0 + m*1.0)         (reshape(m) @ ones([1,k]) broadcast)
//   e  = fl32(exp(fl32(x - mb)))   (subtract, tensorExp 1013-1026; fp32 expf
//                                   here, within 1 ulp of the fp64 libm exp)
//   s  = fl32(sum_j double(e_j))   (tensorSumAxis 887-922, fp64 accumulation)
//   y  = fl32(e / s)               (divide, bit-exact through 1/s in fp64)
// One wave owns one row; rows up to 64*4*ITEMS columns stay in registers, so
// HBM sees one read and one write per element (8 B/elem).  The fp64 sum
// differs from the reference's sequential order only in the last bits of
// the double, below the fp32 rounding of s.
//
// Max/argmax reductions across lanes keep (value, index) pairs and prefer the
// lower index on ties, which reproduces "first element, then strict '>'",
// including the order of +0/-0; NaN never wins except as element 0.
#include "common.h"
#include "row_softmax.h"

#include <cmath>

namespace camel_hip {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;

// One wave per row, the whole row in registers: ITEMS float4 per lane (VEC,
// cols % 4 == 0 and 16-byte aligned rows) or ITEMS*4 scalars per lane.  Slots
// past the end of the row hold -inf, which never wins the max and adds an
// exact 0 to the sum, so only the loads and stores are guarded.
template <int ITEMS, bool VEC>
__device__ __forceinline__ void softmax_row(const float *__restrict__ xr, float *__restrict__ yr,
                                            int cols, int lane) {
    constexpr int NV = ITEMS * 4;
    float v[NV];
    if constexpr (VEC) {
        const int nq = cols >> 2;
#pragma unroll
        for (int it = 0; it < ITEMS; ++it) {
            const int q = lane + WAVE * it;
            f4 t = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
            if (q < nq) t = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(xr) + q);
#pragma unroll
            for (int c = 0; c < 4; ++c) v[4 * it + c] = t[c];
        }
    } else {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int c = lane + WAVE * j;
            v[j] = c < cols ? xr[c] : -INFINITY;
        }
    }
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < NV; ++j) m = max_gt(m, v[j]);
    m = wave_max_gt(m);
    const float x0 = __shfl(v[0], 0); // column 0 sits in lane 0, slot 0, in both layouts
    if (x0 != x0) m = x0;
    const float mb = m + 0.0f; // fl32(0.0 + m * 1.0): the ones-matmul broadcast
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        v[j] = softmax_exp(v[j], mb);
        s += (double)v[j];
    }
    s = wave_sum(s);
    // s >= 1 (the max element contributes exp(0) = 1) or NaN, so the
    // reference's "Division by zero" cannot occur here.
    const double rcp = 1.0 / (double)(float)s;
    if constexpr (VEC) {
        const int nq = cols >> 2;
#pragma unroll
        for (int it = 0; it < ITEMS; ++it) {
            const int q = lane + WAVE * it;
            if (q < nq) {
                f4 t;
#pragma unroll
                for (int c = 0; c < 4; ++c) t[c] = softmax_div(v[4 * it + c], rcp);
                __builtin_nontemporal_store(t, reinterpret_cast<f4 *>(yr) + q);
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int c = lane + WAVE * j;
            if (c < cols) yr[c] = softmax_div(v[j], rcp);
        }
    }
}

// Row indices of the one-wave-per-row kernels: a grid of at most
// ROW_GRID_CAP blocks of 4 waves strides over the rows, so any row count
// fits the launch's 32-bit grid (one row per wave up to 4 * ROW_GRID_CAP rows).
constexpr int64_t ROW_GRID_CAP = 1 << 20;

inline unsigned row_grid(int64_t rows) {
    return (unsigned)std::min<int64_t>((rows + 3) / 4, ROW_GRID_CAP);
}

__device__ __forceinline__ int64_t first_row() {
    return (int64_t)blockIdx.x * (blockDim.x / WAVE) + (threadIdx.x >> 6);
}

__device__ __forceinline__ int64_t row_step() { return (int64_t)gridDim.x * (blockDim.x / WAVE); }

template <int ITEMS, bool VEC>
__global__ __launch_bounds__(256) void softmax_rows_kernel(const float *__restrict__ x,
                                                           float *__restrict__ y, int64_t rows,
                                                           int cols) {
    const int lane = threadIdx.x & 63;
    for (int64_t row = first_row(); row < rows; row += row_step())
        softmax_row<ITEMS, VEC>(x + row * cols, y + row * cols, cols, lane);
}

// Rows longer than the register budget: max pass, sum pass, write pass.
__global__ __launch_bounds__(256) void softmax_rows_long_kernel(const float *__restrict__ x,
                                                                float *__restrict__ y,
                                                                int64_t rows, int64_t cols) {
    const int lane = threadIdx.x & 63;
    for (int64_t row = first_row(); row < rows; row += row_step()) {
    const float *xr = x + row * cols;
    float *yr = y + row * cols;
    float m = -INFINITY;
    for (int64_t c = lane; c < cols; c += WAVE) m = max_gt(m, xr[c]);
    m = wave_max_gt(m);
    const float x0 = xr[0];
    if (x0 != x0) m = x0;
    const float mb = m + 0.0f;
    double s = 0.0;
    for (int64_t c = lane; c < cols; c += WAVE) s += (double)softmax_exp(xr[c], mb);
    s = wave_sum(s);
    const double rcp = 1.0 / (double)(float)s;
    for (int64_t c = lane; c < cols; c += WAVE) yr[c] = softmax_div(softmax_exp(xr[c], mb), rcp);
    }
}

// axis = 1: one wave per row.  kind 0 = sum, 1 = max, 2 = argmax.
__global__ __launch_bounds__(256) void reduce_rows_kernel(int kind, int dt, const void *x,
                                                          int64_t rows, int64_t cols, void *out) {
    const int lane = threadIdx.x & 63;
    for (int64_t row = first_row(); row < rows; row += row_step()) {
    const int64_t base = row * cols;
    if (kind == 0) {
        double s = 0.0;
        for (int64_t c = lane; c < cols; c += WAVE) s += load_as_double(dt, x, base + c);
        s = wave_sum(s);
        if (lane == 0) static_cast<float *>(out)[row] = (float)s;
        continue;
    }
    // Values compare as doubles (exact for fp32 and bool; int64 as the
    // reference converts it).  Track them as double to keep int64 order.
    double bv = 0.0;
    int64_t bi = INT64_MAX;
    for (int64_t c = lane; c < cols; c += WAVE) {
        const double v = load_as_double(dt, x, base + c);
        if (v != v) continue;
        if (bi == INT64_MAX || v > bv) {
            bv = v;
            bi = c;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const double ov = __shfl_xor(bv, off);
        const int64_t oi = __shfl_xor(bi, off);
        if (oi != INT64_MAX && (bi == INT64_MAX || ov > bv || (ov == bv && oi < bi))) {
            bv = ov;
            bi = oi;
        }
    }
    if (lane == 0) {
        const double x0 = load_as_double(dt, x, base);
        if (x0 != x0 || bi == INT64_MAX) {
            bv = x0;
            bi = 0;
        }
        if (kind == 1)
            static_cast<float *>(out)[row] = (float)bv;
        else
            static_cast<int64_t *>(out)[row] = bi;
    }
    }
}

// axis = 0: one thread per column, rows in the reference's order (exact).
__global__ void reduce_cols_kernel(int kind, int dt, const void *x, int64_t rows, int64_t cols,
                                   void *out) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < cols; j += stride) {
        if (kind == 0) {
            double acc = 0.0;
            for (int64_t i = 0; i < rows; ++i) acc += load_as_double(dt, x, i * cols + j);
            static_cast<float *>(out)[j] = (float)acc;
        } else {
            double best = load_as_double(dt, x, j);
            int64_t best_i = 0;
            for (int64_t i = 1; i < rows; ++i) {
                const double v = load_as_double(dt, x, i * cols + j);
                if (v > best) {
                    best = v;
                    best_i = i;
                }
            }
            if (kind == 1)
                static_cast<float *>(out)[j] = (float)best;
            else
                static_cast<int64_t *>(out)[j] = best_i;
        }
    }
}

// Whole-tensor sum: per-block fp64 partials, then one block folds them.
__global__ __launch_bounds__(256) void sum_partial_kernel(int dt, const void *x, int64_t n,
                                                          double *partial) {
    __shared__ double lds[256 / WAVE];
    double s = 0.0;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        s += load_as_double(dt, x, i);
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int w = 0; w < (int)(blockDim.x / WAVE); ++w) t += lds[w];
        partial[blockIdx.x] = t;
    }
}

__global__ __launch_bounds__(256) void sum_final_kernel(const double *partial, int count,
                                                        double *result) {
    __shared__ double lds[256 / WAVE];
    double s = 0.0;
    for (int i = threadIdx.x; i < count; i += blockDim.x) s += partial[i];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int w = 0; w < (int)(blockDim.x / WAVE); ++w) t += lds[w];
        *result = t;
    }
}

template <int ITEMS> int launch_softmax(const float *x, float *y, int64_t rows, int cols, bool vec) {
    dim3 grid(row_grid(rows)), block(256);
    if (vec)
        hipLaunchKernelGGL((softmax_rows_kernel<ITEMS, true>), grid, block, 0, stream(), x, y, rows,
                           cols);
    else
        hipLaunchKernelGGL((softmax_rows_kernel<ITEMS, false>), grid, block, 0, stream(), x, y,
                           rows, cols);
    return check_launch("softmax_rows_kernel");
}

int check_axis(int64_t rows, int64_t cols, int64_t &axis, const char *what) {
    if (rows < 0 || cols < 0) return fail(CAMEL_HIP_ERR_SHAPE, std::string(what) + ": negative shape");
    if (!product_fits({rows, cols, 8}, INT64_MAX))
        return fail(CAMEL_HIP_ERR_SHAPE, std::string(what) + ": tensor too large");
    if (axis < 0) axis += 2;
    if (axis != 0 && axis != 1)
        return fail(CAMEL_HIP_ERR_SHAPE,
                    std::string(what) + "(axis): axis must be 0 or 1 for rank-2 tensors");
    return CAMEL_HIP_OK;
}

int reduce_axis(int kind, int dt, const void *x, int64_t rows, int64_t cols, int64_t axis,
                void *out, const char *what) {
    if (!valid_dtype(dt)) return fail(CAMEL_HIP_ERR_DTYPE, std::string(what) + ": unsupported dtype");
    CAMEL_RETURN_IF(check_axis(rows, cols, axis, what));
    const int64_t out_n = axis == 0 ? cols : rows;
    const int64_t red_n = axis == 0 ? rows : cols;
    if (out_n == 0) return ok();
    if (red_n == 0 && kind != 0)
        return fail(CAMEL_HIP_ERR_SHAPE, std::string(what) + ": reduction over an empty axis");
    if (!out || (red_n > 0 && !x)) return fail(CAMEL_HIP_ERR_ARG, std::string(what) + ": null pointer");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    if (axis == 1) {
        hipLaunchKernelGGL(reduce_rows_kernel, dim3(row_grid(rows)), dim3(256), 0,
                           stream(), kind, dt, x, rows, cols, out);
        CAMEL_RETURN_IF(check_launch("reduce_rows_kernel"));
    } else {
        hipLaunchKernelGGL(reduce_cols_kernel, dim3(grid_for(cols, 256, 16)), dim3(256), 0,
                           stream(), kind, dt, x, rows, cols, out);
        CAMEL_RETURN_IF(check_launch("reduce_cols_kernel"));
    }
    return ok();
}

} // namespace
} // namespace camel_hip

using namespace camel_hip;

extern "C" {

int camel_hip_softmax_rows(const float *x, float *y, int64_t rows, int64_t cols) {
    if (rows < 0 || cols < 0) return fail(CAMEL_HIP_ERR_SHAPE, "softmax: negative shape");
    if (!product_fits({rows, cols, 4}, INT64_MAX))
        return fail(CAMEL_HIP_ERR_SHAPE, "softmax: tensor too large");
    if (rows == 0 || cols == 0) return ok();
    if (!x || !y) return fail(CAMEL_HIP_ERR_ARG, "softmax: null pointer");
    if (cols > INT32_MAX / 2) return fail(CAMEL_HIP_ERR_SHAPE, "softmax: row too long");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    const bool vec = (cols % 4 == 0) && (((uintptr_t)x | (uintptr_t)y) & 15) == 0;
    const int c = (int)cols;
    if (cols <= 64 * 4)
        CAMEL_RETURN_IF(launch_softmax<1>(x, y, rows, c, vec));
    else if (cols <= 64 * 8)
        CAMEL_RETURN_IF(launch_softmax<2>(x, y, rows, c, vec));
    else if (cols <= 64 * 16)
        CAMEL_RETURN_IF(launch_softmax<4>(x, y, rows, c, vec));
    else if (cols <= 64 * 32)
        CAMEL_RETURN_IF(launch_softmax<8>(x, y, rows, c, vec));
    else if (cols <= 64 * 64)
        CAMEL_RETURN_IF(launch_softmax<16>(x, y, rows, c, vec));
    else {
        hipLaunchKernelGGL(softmax_rows_long_kernel, dim3(row_grid(rows)), dim3(256), 0,
                           stream(), x, y, rows, cols);
        CAMEL_RETURN_IF(check_launch("softmax_rows_long_kernel"));
    }
    return ok();
}

int camel_hip_sum_axis(int dt, const void *x, int64_t rows, int64_t cols, int64_t axis,
                       float *out) {
    return reduce_axis(0, dt, x, rows, cols, axis, out, "sum");
}

int camel_hip_max_axis(int dt, const void *x, int64_t rows, int64_t cols, int64_t axis,
                       float *out) {
    return reduce_axis(1, dt, x, rows, cols, axis, out, "max");
}

int camel_hip_argmax_axis(int dt, const void *x, int64_t rows, int64_t cols, int64_t axis,
                          int64_t *out) {
    return reduce_axis(2, dt, x, rows, cols, axis, out, "argmax");
}

int camel_hip_sum(int dt, const void *x, int64_t n, double *result) {
    if (!valid_dtype(dt)) return fail(CAMEL_HIP_ERR_DTYPE, "sum: unsupported dtype");
    if (!result || n < 0) return fail(CAMEL_HIP_ERR_ARG, "sum: bad argument");
    if (n == 0) {
        *result = 0.0;
        return ok();
    }
    if (!x) return fail(CAMEL_HIP_ERR_ARG, "sum: null input");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    const unsigned blocks = grid_for(n, 256, 4);
    void *ws = nullptr;
    CAMEL_RETURN_IF(camel_hip_malloc(&ws, (blocks + 1) * sizeof(double)));
    double *partial = static_cast<double *>(ws);
    hipLaunchKernelGGL(sum_partial_kernel, dim3(blocks), dim3(256), 0, stream(), dt, x, n, partial);
    int rc = check_launch("sum_partial_kernel");
    if (rc == CAMEL_HIP_OK) {
        hipLaunchKernelGGL(sum_final_kernel, dim3(1), dim3(256), 0, stream(), partial, (int)blocks,
                           partial + blocks);
        rc = check_launch("sum_final_kernel");
    }
    if (rc == CAMEL_HIP_OK)
        rc = camel_hip_d2h(result, partial + blocks, sizeof(double));
    camel_hip_free(ws);
    CAMEL_RETURN_IF(rc);
    return ok();
}

} // extern "C"
