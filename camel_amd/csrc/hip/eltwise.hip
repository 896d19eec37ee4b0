// Elementwise kernels: binary / scalar / compare / relu / exp / log.
//
// Semantics follow modules/tensor/runtime.cpp: each element is widened to
// double, the operation runs once, the result is rounded to the output dtype
// (tensorBinary 775-793, applyBinary 113-130, scalar forms 795-831, compares
// 833-877, exp/log 1013-1045).  For fp32 operands and a single +, -, *, /
// the fp32 instruction gives the same bits as double-then-round (double
// rounding is innocuous for one operation when 53 >= 2*24+2), so the fp32
// fast paths use fp32 arithmetic with contraction off and denormals kept.
//
// Bandwidth layout: the fp32 fast paths move 16-byte vectors, each thread
// handling VEC_PER_THREAD consecutive-in-grid float4s so a wave's accesses
// are contiguous 1 KiB runs; tails are handled by a scalar loop.
#include "common.h"

namespace camel_hip {
namespace {

constexpr int THREADS = 256;
constexpr int VEC_PER_THREAD = 4;

// Native 4-wide vector (the nontemporal builtins take clang vector types).
typedef float f4 __attribute__((ext_vector_type(4)));

template <int OP> __device__ __forceinline__ float op_f32(float a, float b) {
    if constexpr (OP == CAMEL_OP_ADD) return a + b;
    if constexpr (OP == CAMEL_OP_SUB) return a - b;
    if constexpr (OP == CAMEL_OP_MUL) return a * b;
    return a / b; // CAMEL_OP_DIV: IEEE correctly rounded
}

__device__ __forceinline__ double op_f64(int op, double a, double b, int *flag) {
    switch (op) {
    case CAMEL_OP_ADD:
        return a + b;
    case CAMEL_OP_SUB:
        return a - b;
    case CAMEL_OP_MUL:
        return a * b;
    case CAMEL_OP_DIV:
        if (b == 0.0) *flag = 1;
        return a / b;
    default:
        return pow(a, b);
    }
}

__device__ __forceinline__ bool cmp_f64(int op, double a, double b) {
    switch (op) {
    case CAMEL_CMP_LT:
        return a < b;
    case CAMEL_CMP_LE:
        return a <= b;
    case CAMEL_CMP_GT:
        return a > b;
    case CAMEL_CMP_GE:
        return a >= b;
    default:
        return a == b;
    }
}

// fp32 (op) fp32 -> fp32, vectorised.
template <int OP>
__global__ __launch_bounds__(THREADS) void binary_f32_kernel(const float *__restrict__ l,
                                                             const float *__restrict__ r,
                                                             float *__restrict__ out, int64_t n,
                                                             int *flag) {
    const int64_t n4 = n >> 2;
    const f4 *l4 = reinterpret_cast<const f4 *>(l);
    const f4 *r4 = reinterpret_cast<const f4 *>(r);
    f4 *o4 = reinterpret_cast<f4 *>(out);
    const int64_t base = (int64_t)blockIdx.x * THREADS * VEC_PER_THREAD + threadIdx.x;
    f4 a[VEC_PER_THREAD], b[VEC_PER_THREAD];
#pragma unroll
    for (int v = 0; v < VEC_PER_THREAD; ++v) {
        const int64_t i = base + (int64_t)v * THREADS;
        if (i < n4) {
            a[v] = __builtin_nontemporal_load(l4 + i);
            b[v] = __builtin_nontemporal_load(r4 + i);
        }
    }
    bool zero = false;
#pragma unroll
    for (int v = 0; v < VEC_PER_THREAD; ++v) {
        const int64_t i = base + (int64_t)v * THREADS;
        if (i < n4) {
            if constexpr (OP == CAMEL_OP_DIV)
                zero |= (b[v].x == 0.0f) | (b[v].y == 0.0f) | (b[v].z == 0.0f) | (b[v].w == 0.0f);
            f4 o;
            o.x = op_f32<OP>(a[v].x, b[v].x);
            o.y = op_f32<OP>(a[v].y, b[v].y);
            o.z = op_f32<OP>(a[v].z, b[v].z);
            o.w = op_f32<OP>(a[v].w, b[v].w);
            __builtin_nontemporal_store(o, o4 + i);
        }
    }
    // Tail (n % 4 elements), handled by the first block.
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
        const int64_t i = n4 * 4 + threadIdx.x;
        if constexpr (OP == CAMEL_OP_DIV) zero |= r[i] == 0.0f;
        out[i] = op_f32<OP>(l[i], r[i]);
    }
    if constexpr (OP == CAMEL_OP_DIV)
        if (zero) *flag = 1;
}

// Any dtypes, through double (pow and mixed-dtype operands).
__global__ void binary_generic_kernel(int op, int ldt, const void *l, int rdt, const void *r,
                                      int odt, void *out, int64_t n, int *flag) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int err = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        store_from_double(odt, out, i,
                          op_f64(op, load_as_double(ldt, l, i), load_as_double(rdt, r, i), &err));
    if (err) *flag = 1;
}

// Tensor (op) scalar, fp32 tensor and output: double op then one rounding.
__global__ __launch_bounds__(THREADS) void scalar_f32_kernel(int op, int side,
                                                             const float *__restrict__ t, double s,
                                                             float *__restrict__ out, int64_t n,
                                                             int *flag) {
    const int64_t n4 = n >> 2;
    const f4 *t4 = reinterpret_cast<const f4 *>(t);
    f4 *o4 = reinterpret_cast<f4 *>(out);
    const int64_t base = (int64_t)blockIdx.x * THREADS * VEC_PER_THREAD + threadIdx.x;
    int err = 0;
#pragma unroll
    for (int v = 0; v < VEC_PER_THREAD; ++v) {
        const int64_t i = base + (int64_t)v * THREADS;
        if (i < n4) {
            const f4 a = __builtin_nontemporal_load(t4 + i);
            f4 o;
            if (side == 0) {
                o.x = (float)op_f64(op, (double)a.x, s, &err);
                o.y = (float)op_f64(op, (double)a.y, s, &err);
                o.z = (float)op_f64(op, (double)a.z, s, &err);
                o.w = (float)op_f64(op, (double)a.w, s, &err);
            } else {
                o.x = (float)op_f64(op, s, (double)a.x, &err);
                o.y = (float)op_f64(op, s, (double)a.y, &err);
                o.z = (float)op_f64(op, s, (double)a.z, &err);
                o.w = (float)op_f64(op, s, (double)a.w, &err);
            }
            __builtin_nontemporal_store(o, o4 + i);
        }
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
        const int64_t i = n4 * 4 + threadIdx.x;
        out[i] = side == 0 ? (float)op_f64(op, (double)t[i], s, &err)
                           : (float)op_f64(op, s, (double)t[i], &err);
    }
    if (err) *flag = 1;
}

__global__ void scalar_generic_kernel(int op, int side, int tdt, const void *t, double s, int odt,
                                      void *out, int64_t n, int *flag) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int err = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const double x = load_as_double(tdt, t, i);
        store_from_double(odt, out, i, side == 0 ? op_f64(op, x, s, &err) : op_f64(op, s, x, &err));
    }
    if (err) *flag = 1;
}

__global__ void compare_generic_kernel(int op, int ldt, const void *l, int rdt, const void *r,
                                       uint8_t *out, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = cmp_f64(op, load_as_double(ldt, l, i), load_as_double(rdt, r, i)) ? 1 : 0;
}

__global__ void compare_scalar_kernel(int op, int side, int tdt, const void *t, double s,
                                      uint8_t *out, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const double x = load_as_double(tdt, t, i);
        out[i] = (side == 0 ? cmp_f64(op, x, s) : cmp_f64(op, s, x)) ? 1 : 0;
    }
}

__global__ __launch_bounds__(THREADS) void relu_kernel(const float *__restrict__ x,
                                                       float *__restrict__ y, int64_t n) {
    const int64_t n4 = n >> 2;
    const f4 *x4 = reinterpret_cast<const f4 *>(x);
    f4 *y4 = reinterpret_cast<f4 *>(y);
    const int64_t base = (int64_t)blockIdx.x * THREADS * VEC_PER_THREAD + threadIdx.x;
    f4 a[VEC_PER_THREAD];
#pragma unroll
    for (int v = 0; v < VEC_PER_THREAD; ++v) {
        const int64_t i = base + (int64_t)v * THREADS;
        if (i < n4) a[v] = __builtin_nontemporal_load(x4 + i);
    }
#pragma unroll
    for (int v = 0; v < VEC_PER_THREAD; ++v) {
        const int64_t i = base + (int64_t)v * THREADS;
        if (i < n4) {
            f4 o;
            o.x = relu_idiom(a[v].x);
            o.y = relu_idiom(a[v].y);
            o.z = relu_idiom(a[v].z);
            o.w = relu_idiom(a[v].w);
            __builtin_nontemporal_store(o, y4 + i);
        }
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
        const int64_t i = n4 * 4 + threadIdx.x;
        y[i] = relu_idiom(x[i]);
    }
}

__global__ void relu_scalar_kernel(const float *x, float *y, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        y[i] = relu_idiom(x[i]);
}

// exp (is_log = 0) or log (is_log = 1) in double, rounded to fp32.
__global__ void unary_kernel(int is_log, const float *__restrict__ x, float *__restrict__ y,
                             int64_t n, int *flag) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int err = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const double v = (double)x[i];
        if (is_log) {
            if (v <= 0.0) err = 1;
            y[i] = (float)log(v);
        } else {
            y[i] = (float)exp(v);
        }
    }
    if (err) *flag = 1;
}

unsigned vec_grid(int64_t n) {
    const int64_t per_block = (int64_t)THREADS * VEC_PER_THREAD;
    int64_t blocks = ((n >> 2) + per_block - 1) / per_block;
    return (unsigned)(blocks < 1 ? 1 : blocks);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Runs a launch that may raise a device-side error, then maps the flag.
template <class Launch> int checked(Launch &&launch, int err_status, const char *msg) {
    CAMEL_RETURN_IF(clear_error_flag());
    CAMEL_RETURN_IF(launch());
    int flag = 0;
    CAMEL_RETURN_IF(read_error_flag(&flag));
    if (flag) return fail(err_status, msg);
    return CAMEL_HIP_OK;
}

int check_elementwise(int64_t n, const void *a, const void *b, const void *out) {
    if (n < 0) return fail(CAMEL_HIP_ERR_ARG, "elementwise: negative size");
    if (n > 0 && (!a || !b || !out)) return fail(CAMEL_HIP_ERR_ARG, "elementwise: null pointer");
    return CAMEL_HIP_OK;
}

} // namespace
} // namespace camel_hip

using namespace camel_hip;

extern "C" {

int camel_hip_binary(int op, int ldt, const void *l, int rdt, const void *r, int odt, void *out,
                     int64_t n) {
    if (op < CAMEL_OP_ADD || op > CAMEL_OP_POW) return fail(CAMEL_HIP_ERR_ARG, "binary: bad op");
    if (!valid_dtype(ldt) || !valid_dtype(rdt) || !valid_dtype(odt))
        return fail(CAMEL_HIP_ERR_DTYPE, "binary: unsupported dtype");
    CAMEL_RETURN_IF(check_elementwise(n, l, r, out));
    if (n == 0) return ok();
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    const bool fast = op != CAMEL_OP_POW && ldt == CAMEL_DT_F32 && rdt == CAMEL_DT_F32 &&
                      odt == CAMEL_DT_F32 && aligned16(l) && aligned16(r) && aligned16(out);
    auto launch = [&]() -> int {
        if (fast) {
            const float *lf = static_cast<const float *>(l);
            const float *rf = static_cast<const float *>(r);
            float *of = static_cast<float *>(out);
            dim3 grid(vec_grid(n)), block(THREADS);
            switch (op) {
            case CAMEL_OP_ADD:
                hipLaunchKernelGGL(binary_f32_kernel<CAMEL_OP_ADD>, grid, block, 0, stream(), lf,
                                   rf, of, n, error_flag());
                break;
            case CAMEL_OP_SUB:
                hipLaunchKernelGGL(binary_f32_kernel<CAMEL_OP_SUB>, grid, block, 0, stream(), lf,
                                   rf, of, n, error_flag());
                break;
            case CAMEL_OP_MUL:
                hipLaunchKernelGGL(binary_f32_kernel<CAMEL_OP_MUL>, grid, block, 0, stream(), lf,
                                   rf, of, n, error_flag());
                break;
            default:
                hipLaunchKernelGGL(binary_f32_kernel<CAMEL_OP_DIV>, grid, block, 0, stream(), lf,
                                   rf, of, n, error_flag());
                break;
            }
            return check_launch("binary_f32_kernel");
        }
        hipLaunchKernelGGL(binary_generic_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream(), op,
                           ldt, l, rdt, r, odt, out, n, error_flag());
        return check_launch("binary_generic_kernel");
    };
    if (op == CAMEL_OP_DIV) {
        CAMEL_RETURN_IF(checked(launch, CAMEL_HIP_ERR_DIV_ZERO, "Division by zero"));
    } else {
        CAMEL_RETURN_IF(launch());
    }
    return ok();
}

int camel_hip_binary_scalar(int op, int side, int tdt, const void *t, double s, int odt,
                            void *out, int64_t n) {
    if (op < CAMEL_OP_ADD || op > CAMEL_OP_POW || (side != 0 && side != 1))
        return fail(CAMEL_HIP_ERR_ARG, "binary_scalar: bad op or side");
    if (!valid_dtype(tdt) || !valid_dtype(odt))
        return fail(CAMEL_HIP_ERR_DTYPE, "binary_scalar: unsupported dtype");
    CAMEL_RETURN_IF(check_elementwise(n, t, t, out));
    if (n == 0) return ok();
    // Scalar divisor: the reference's per-element check fails on element 0.
    if (op == CAMEL_OP_DIV && side == 0 && s == 0.0) return fail(CAMEL_HIP_ERR_DIV_ZERO, "Division by zero");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    const bool fast = op != CAMEL_OP_POW && tdt == CAMEL_DT_F32 && odt == CAMEL_DT_F32 &&
                      aligned16(t) && aligned16(out);
    auto launch = [&]() -> int {
        if (fast) {
            hipLaunchKernelGGL(scalar_f32_kernel, dim3(vec_grid(n)), dim3(THREADS), 0, stream(), op,
                               side, static_cast<const float *>(t), s, static_cast<float *>(out), n,
                               error_flag());
            return check_launch("scalar_f32_kernel");
        }
        hipLaunchKernelGGL(scalar_generic_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream(), op,
                           side, tdt, t, s, odt, out, n, error_flag());
        return check_launch("scalar_generic_kernel");
    };
    if (op == CAMEL_OP_DIV && side == 1) {
        CAMEL_RETURN_IF(checked(launch, CAMEL_HIP_ERR_DIV_ZERO, "Division by zero"));
    } else {
        CAMEL_RETURN_IF(launch());
    }
    return ok();
}

int camel_hip_compare(int op, int ldt, const void *l, int rdt, const void *r, uint8_t *out,
                      int64_t n) {
    if (op < CAMEL_CMP_LT || op > CAMEL_CMP_EQ) return fail(CAMEL_HIP_ERR_ARG, "compare: bad op");
    if (!valid_dtype(ldt) || !valid_dtype(rdt))
        return fail(CAMEL_HIP_ERR_DTYPE, "compare: unsupported dtype");
    CAMEL_RETURN_IF(check_elementwise(n, l, r, out));
    if (n == 0) return ok();
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    hipLaunchKernelGGL(compare_generic_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream(), op,
                       ldt, l, rdt, r, out, n);
    CAMEL_RETURN_IF(check_launch("compare_generic_kernel"));
    return ok();
}

int camel_hip_compare_scalar(int op, int side, int tdt, const void *t, double s, uint8_t *out,
                             int64_t n) {
    if (op < CAMEL_CMP_LT || op > CAMEL_CMP_EQ || (side != 0 && side != 1))
        return fail(CAMEL_HIP_ERR_ARG, "compare_scalar: bad op or side");
    if (!valid_dtype(tdt)) return fail(CAMEL_HIP_ERR_DTYPE, "compare_scalar: unsupported dtype");
    CAMEL_RETURN_IF(check_elementwise(n, t, t, out));
    if (n == 0) return ok();
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    hipLaunchKernelGGL(compare_scalar_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream(), op,
                       side, tdt, t, s, out, n);
    CAMEL_RETURN_IF(check_launch("compare_scalar_kernel"));
    return ok();
}

int camel_hip_relu(const float *x, float *y, int64_t n) {
    CAMEL_RETURN_IF(check_elementwise(n, x, x, y));
    if (n == 0) return ok();
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    if (aligned16(x) && aligned16(y)) {
        hipLaunchKernelGGL(relu_kernel, dim3(vec_grid(n)), dim3(THREADS), 0, stream(), x, y, n);
        CAMEL_RETURN_IF(check_launch("relu_kernel"));
    } else {
        hipLaunchKernelGGL(relu_scalar_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream(), x, y,
                           n);
        CAMEL_RETURN_IF(check_launch("relu_scalar_kernel"));
    }
    return ok();
}

int camel_hip_exp(const float *x, float *y, int64_t n) {
    CAMEL_RETURN_IF(check_elementwise(n, x, x, y));
    if (n == 0) return ok();
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    hipLaunchKernelGGL(unary_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream(), 0, x, y, n,
                       error_flag());
    CAMEL_RETURN_IF(check_launch("unary_kernel"));
    return ok();
}

int camel_hip_log(const float *x, float *y, int64_t n) {
    CAMEL_RETURN_IF(check_elementwise(n, x, x, y));
    if (n == 0) return ok();
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    auto launch = [&]() -> int {
        hipLaunchKernelGGL(unary_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream(), 1, x, y, n,
                           error_flag());
        return check_launch("unary_kernel");
    };
    CAMEL_RETURN_IF(checked(launch, CAMEL_HIP_ERR_LOG_DOMAIN, "log: input must be positive"));
    return ok();
}

} // extern "C"
