// Layout kernels: 2-D transpose, concat and NCHW max pooling.
#include "common.h"

namespace camel_hip {
namespace {

constexpr int TT = 32; // transpose tile edge

// tensorTranspose2D (runtime.cpp:704-720) copies each element through
// getAsDouble/setFromDouble: int64 values pass through a double and bool
// bytes are normalised to 0/1; fp32 round-trips exactly (raw bits move).
enum { COPY_RAW = 0, COPY_I64_VIA_DOUBLE = 1, COPY_BOOL_NORMALISE = 2 };

template <class T, int MODE>
__global__ __launch_bounds__(TT * 8) void transpose_kernel(const T *__restrict__ x,
                                                           T *__restrict__ y, int64_t rows,
                                                           int64_t cols) {
    __shared__ T tile[TT][TT + 1];
    const int64_t c0 = (int64_t)blockIdx.x * TT, r0 = (int64_t)blockIdx.y * TT;
    const int tx = threadIdx.x % TT, ty = threadIdx.x / TT;
    for (int k = ty; k < TT; k += 8) {
        const int64_t r = r0 + k, c = c0 + tx;
        if (r < rows && c < cols) tile[k][tx] = x[r * cols + c];
    }
    __syncthreads();
    for (int k = ty; k < TT; k += 8) {
        const int64_t c = c0 + k, r = r0 + tx; // output row c, column r
        if (r < rows && c < cols) {
            T v = tile[tx][k];
            if constexpr (MODE == COPY_I64_VIA_DOUBLE) v = (T)double_to_i64_x86((double)v);
            if constexpr (MODE == COPY_BOOL_NORMALISE) v = v != 0 ? 1 : 0;
            y[c * rows + r] = v;
        }
    }
}

// Max pool: window scanned (kh, kw) ascending, first element then strict '>'
// (the tensorMaxAxis rule, runtime.cpp:953-958).  One thread per output.
__global__ void maxpool_kernel(const float *__restrict__ x, float *__restrict__ y, int64_t planes,
                               int H, int W, int OH, int OW, int KH, int KW, int stride) {
    const int64_t total = planes * OH * OW;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += step) {
        const int ow = (int)(o % OW);
        const int64_t t = o / OW;
        const int oh = (int)(t % OH);
        const int64_t p = t / OH;
        const float *src = x + p * H * W + (int64_t)(oh * stride) * W + ow * stride;
        float best = src[0];
        for (int kh = 0; kh < KH; ++kh)
            for (int kw = 0; kw < KW; ++kw) {
                const float v = src[kh * W + kw];
                if (v > best) best = v;
            }
        y[o] = best;
    }
}

// 2x2 stride-2 specialisation: each thread produces two adjacent outputs from
// two 16-byte row loads when W is a multiple of 4.
__global__ void maxpool2x2_kernel(const float *__restrict__ x, float *__restrict__ y,
                                  int64_t planes, int H, int W, int OH, int OW) {
    const int64_t pairs = planes * OH * (OW / 2);
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < pairs; q += step) {
        const int pw = (int)(q % (OW / 2));
        const int64_t t = q / (OW / 2);
        const int oh = (int)(t % OH);
        const int64_t p = t / OH;
        const float *src = x + p * H * W + (int64_t)(2 * oh) * W + 4 * pw;
        const float4 a = *reinterpret_cast<const float4 *>(src);
        const float4 b = *reinterpret_cast<const float4 *>(src + W);
        float m0 = a.x, m1 = a.z;
        if (a.y > m0) m0 = a.y;
        if (b.x > m0) m0 = b.x;
        if (b.y > m0) m0 = b.y;
        if (a.w > m1) m1 = a.w;
        if (b.z > m1) m1 = b.z;
        if (b.w > m1) m1 = b.w;
        *reinterpret_cast<float2 *>(y + (p * OH + oh) * OW + 2 * pw) = make_float2(m0, m1);
    }
}

} // namespace
} // namespace camel_hip

using namespace camel_hip;

extern "C" {

int camel_hip_transpose2d(int dt, const void *x, void *y, int64_t rows, int64_t cols) {
    if (!valid_dtype(dt)) return fail(CAMEL_HIP_ERR_DTYPE, "transpose: unsupported dtype");
    if (rows < 0 || cols < 0) return fail(CAMEL_HIP_ERR_SHAPE, "transpose: negative shape");
    if (rows == 0 || cols == 0) return ok();
    if (!x || !y) return fail(CAMEL_HIP_ERR_ARG, "transpose: null pointer");
    if ((cols + TT - 1) / TT > INT32_MAX || (rows + TT - 1) / TT > 65535)
        return fail(CAMEL_HIP_ERR_SHAPE, "transpose: tensor too large");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    dim3 grid((unsigned)((cols + TT - 1) / TT), (unsigned)((rows + TT - 1) / TT)), block(TT * 8);
    if (dt == CAMEL_DT_F32)
        hipLaunchKernelGGL((transpose_kernel<float, COPY_RAW>), grid, block, 0, stream(),
                           static_cast<const float *>(x), static_cast<float *>(y), rows, cols);
    else if (dt == CAMEL_DT_I64)
        hipLaunchKernelGGL((transpose_kernel<int64_t, COPY_I64_VIA_DOUBLE>), grid, block, 0, stream(),
                           static_cast<const int64_t *>(x), static_cast<int64_t *>(y), rows, cols);
    else
        hipLaunchKernelGGL((transpose_kernel<uint8_t, COPY_BOOL_NORMALISE>), grid, block, 0, stream(),
                           static_cast<const uint8_t *>(x), static_cast<uint8_t *>(y), rows, cols);
    CAMEL_RETURN_IF(check_launch("transpose_kernel"));
    return ok();
}

int camel_hip_concat(int dt, const void *l, const void *r, void *out, int64_t outer,
                     int64_t l_axis, int64_t r_axis, int64_t inner) {
    if (!valid_dtype(dt)) return fail(CAMEL_HIP_ERR_DTYPE, "concat: unsupported dtype");
    if (outer < 0 || l_axis < 0 || r_axis < 0 || inner < 0)
        return fail(CAMEL_HIP_ERR_SHAPE, "concat: negative extent");
    if (!product_fits({outer, l_axis, inner, 8}, INT64_MAX / 2) ||
        !product_fits({outer, r_axis, inner, 8}, INT64_MAX / 2))
        return fail(CAMEL_HIP_ERR_SHAPE, "concat: tensor too large");
    const size_t item = dtype_size(dt);
    const size_t lw = (size_t)(l_axis * inner) * item, rw = (size_t)(r_axis * inner) * item;
    const size_t ow = lw + rw;
    if (outer == 0 || ow == 0) return ok();
    if (!out || (lw && !l) || (rw && !r)) return fail(CAMEL_HIP_ERR_ARG, "concat: null pointer");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    if (lw)
        CAMEL_RETURN_IF(check_hip(hipMemcpy2DAsync(out, ow, l, lw, lw, (size_t)outer,
                                                   hipMemcpyDeviceToDevice, stream()),
                                  "hipMemcpy2DAsync(concat lhs)"));
    if (rw)
        CAMEL_RETURN_IF(check_hip(hipMemcpy2DAsync(static_cast<char *>(out) + lw, ow, r, rw, rw,
                                                   (size_t)outer, hipMemcpyDeviceToDevice, stream()),
                                  "hipMemcpy2DAsync(concat rhs)"));
    return ok();
}

int camel_hip_maxpool2d(const float *x, float *y, int64_t N, int64_t C, int64_t H, int64_t W,
                        int64_t KH, int64_t KW, int64_t stride) {
    if (N < 0 || C < 0 || H <= 0 || W <= 0 || KH <= 0 || KW <= 0 || stride <= 0 || H < KH ||
        W < KW)
        return fail(CAMEL_HIP_ERR_SHAPE, "maxpool2d: invalid geometry");
    if (H > INT32_MAX / 2 || W > INT32_MAX / 2 || !product_fits({N, C, H, W}, INT64_MAX / 4))
        return fail(CAMEL_HIP_ERR_SHAPE, "maxpool2d: tensor too large");
    const int64_t OH = (H - KH) / stride + 1, OW = (W - KW) / stride + 1;
    const int64_t planes = N * C;
    if (planes == 0) return ok();
    if (!x || !y) return fail(CAMEL_HIP_ERR_ARG, "maxpool2d: null pointer");
    CAMEL_LOCK();
    CAMEL_INIT_OR_RETURN();
    const bool fast = KH == 2 && KW == 2 && stride == 2 && W % 4 == 0 && OW % 2 == 0 &&
                      (((uintptr_t)x & 15) == 0) && (((uintptr_t)y & 7) == 0);
    if (fast) {
        hipLaunchKernelGGL(maxpool2x2_kernel, dim3(grid_for(planes * OH * OW / 2, 256)), dim3(256),
                           0, stream(), x, y, planes, (int)H, (int)W, (int)OH, (int)OW);
        CAMEL_RETURN_IF(check_launch("maxpool2x2_kernel"));
    } else {
        hipLaunchKernelGGL(maxpool_kernel, dim3(grid_for(planes * OH * OW, 256)), dim3(256), 0,
                           stream(), x, y, planes, (int)H, (int)W, (int)OH, (int)OW, (int)KH,
                           (int)KW, (int)stride);
        CAMEL_RETURN_IF(check_launch("maxpool_kernel"));
    }
    return ok();
}

} // extern "C"
