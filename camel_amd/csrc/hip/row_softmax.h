// Device helpers of the row softmax (the composition of
// test/run/nn/mnist.cml:13-25), shared by the softmax kernels and by the
// GEMM kernels that fuse a softmax into their epilogue, so that both compute
// every row with the same operations in the same order.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>

namespace camel_hip {
namespace {

__device__ __forceinline__ double wave_sum(double s) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    return s;
}

// Row max with the reference's rule (first element, then strict '>'), value
// only: NaNs never win unless the row starts with one.  Which of several
// equal maxima wins cannot change the softmax (m is only used as m + 0.0,
// which also maps -0.0 to +0.0), so no index is tracked.
__device__ __forceinline__ float max_gt(float best, float v) { return v > best ? v : best; }

__device__ __forceinline__ float wave_max_gt(float m) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = max_gt(m, __shfl_xor(m, off));
    return m;
}

// e = exp(x - mb) rounded to fp32.  The device expf is within 1 ulp of the
// reference's (float)std::exp((double)d); the softmax bar is rel-err 1e-6
// (about 16 ulp), and fp32 exp keeps the kernel at HBM speed where the fp64
// exp made it ALU-bound.
__device__ __forceinline__ float softmax_exp(float v, float mb) { return expf(v - mb); }

// y = fl32(e / s) bit-exactly, computed as fl32(e * fl64(1 / s)): the relative
// error of the double product is <= 2^-52, while a quotient of two fp32 values
// is never closer than 2^-49 (relative) to an fp32 rounding midpoint, so both
// round to the same fp32 value.  This replaces a per-element fp32 division.
__device__ __forceinline__ float softmax_div(float e, double rcp) {
    return (float)((double)e * rcp);
}

// Softmax of a row of at most 64 columns held one value per lane (lane c
// holds column c, lanes past the row hold -inf): the steps of the softmax
// kernel for such rows, in the same order (the kernel's other register slots
// of these rows hold -inf, which leave the max alone and add exact zeros to
// the sum), so a fused GEMM epilogue and the stand-alone kernel agree bit for
// bit.  Every lane of the wave must call it.
__device__ __forceinline__ float softmax_row_lanes(float v) {
    float m = wave_max_gt(max_gt(-INFINITY, v));
    const float x0 = __shfl(v, 0);
    if (x0 != x0) m = x0;
    const float mb = m + 0.0f;
    const float e = softmax_exp(v, mb);
    const double s = wave_sum(0.0 + (double)e);
    const double rcp = 1.0 / (double)(float)s;
    return softmax_div(e, rcp);
}

} // namespace
} // namespace camel_hip
