/*
 * camel_hip.h -- C-ABI of libcamel_hip.so, the MI355X (gfx950) backend of the
 * Camel `tensor` module.
 *
 * Plain C: pointers, int64 sizes, double scalars, int status codes.  No C++
 * or HIP types cross this boundary, so the reference's tensor module
 * (modules/tensor, C++) or any FFI can bind it.  Device pointers are opaque
 * `void *` handed out by camel_hip_malloc.  All work is enqueued on the
 * library's single HIP stream, in call order; the calls are thread-safe
 * (one library mutex), matching the Taskflow scheduler that runs operators on
 * worker threads (src/passes/sched/taskflow/taskflow.cpp:157-181).
 *
 * Every compute entry point names the reference function whose CPU loop it
 * replaces (paths relative to the OpenCML/Camel 0.1.19 tree).  Shape, rank
 * and dtype errors are detected on the host before anything is launched;
 * value-dependent errors (division by zero, log of a non-positive value) are
 * raised by a device flag read back after the kernel, and the output is then
 * undefined, as the reference abandons its output when it throws.
 */
#ifndef CAMEL_HIP_H
#define CAMEL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
enum camel_hip_status {
    CAMEL_HIP_OK = 0,
    CAMEL_HIP_ERR_ARG = 1,        /* bad pointer / size / enum value          */
    CAMEL_HIP_ERR_SHAPE = 2,      /* shape, rank or axis rejected             */
    CAMEL_HIP_ERR_DIV_ZERO = 3,   /* "Division by zero", runtime.cpp:122-124  */
    CAMEL_HIP_ERR_LOG_DOMAIN = 4, /* "log: input must be positive", 1039-1041 */
    CAMEL_HIP_ERR_DTYPE = 5,      /* dtype not supported by the op            */
    CAMEL_HIP_ERR_OOM = 6,        /* device allocation failed                 */
    CAMEL_HIP_ERR_RUNTIME = 7,    /* HIP runtime error (message via last_error) */
    CAMEL_HIP_ERR_NO_DEVICE = 8   /* no usable gfx950 device                  */
};

/* Storage dtypes of a tensor: Float32, Int64, Bool(u8) -- the only three the
 * reference stores (elementSize, modules/tensor/runtime.cpp:530-541). */
enum camel_hip_dtype { CAMEL_DT_F32 = 0, CAMEL_DT_I64 = 1, CAMEL_DT_BOOL = 2 };

/* BinaryOp and CompareOp in the order of modules/tensor/runtime.h:39-53. */
enum camel_hip_binary_op {
    CAMEL_OP_ADD = 0, CAMEL_OP_SUB = 1, CAMEL_OP_MUL = 2, CAMEL_OP_DIV = 3, CAMEL_OP_POW = 4
};
enum camel_hip_compare_op {
    CAMEL_CMP_LT = 0, CAMEL_CMP_LE = 1, CAMEL_CMP_GT = 2, CAMEL_CMP_GE = 3, CAMEL_CMP_EQ = 4
};

/* Epilogue flags of the GEMM / conv entry points. */
enum camel_hip_epilogue { CAMEL_EPI_NONE = 0, CAMEL_EPI_BIAS = 1, CAMEL_EPI_RELU = 2 };
/* Operand layout flag of camel_hip_sgemm / camel_hip_sgemm_noalloc: A is given
 * transposed, as At[K, M] row-major (A[m][k] = At[k][m]), and read in place by
 * the MFMA tile loaders: transpose(X) @ E (test/run/nn/mnist.cml:39,
 * test/run/nn/lr.cml:28; tensorTranspose2D runtime.cpp:704-720 followed by
 * the matmul of operators.cpp:740-769) without a copy of X. */
enum camel_hip_gemm_layout { CAMEL_GEMM_A_T = 0x10 };
/* Layout bits of the conv2d flags, for a fused layer chain that keeps an
 * intermediate in the layout its consumer reads: x given as [N, H, W, C],
 * y written as [N, OH, OW, Co], w given as [Co, KH, KW, C] (packed once by
 * camel_hip_conv2d_pack_weights), x given / y written as NCHW4
 * [N, C/4, H, W, 4] (channel quads interleaved: C % 4 == 0 and 16-byte
 * alignment; at most one input and one output layout bit).  Each is only
 * an addressing change. */
enum camel_hip_conv_layout {
    CAMEL_CONV_X_NHWC = 0x100,
    CAMEL_CONV_Y_NHWC = 0x200,
    CAMEL_CONV_W_PACKED = 0x400,
    CAMEL_CONV_X_NCHW4 = 0x800,
    CAMEL_CONV_Y_NCHW4 = 0x1000
};

/* ---- runtime ------------------------------------------------------------- */
/* Selects the device and creates the stream and device-side error flag.
 * Idempotent; every other entry point calls it lazily with device 0.
 * No reference counterpart (the reference is CPU-only). */
int camel_hip_init(int device);
int camel_hip_device_count(int *count);
/* The device the library runs on (initialising device 0 if nothing chose
 * one), e.g. the device_id of an exported DLPack tensor.  No reference
 * counterpart. */
int camel_hip_current_device(int *device);
/* Text of the last error on this thread ("" when none). */
const char *camel_hip_last_error(void);
/* Blocks until all enqueued work is done. */
int camel_hip_sync(void);
/* Blocks until every stream of the library's device is idle, the library's
 * and other libraries' alike (hipDeviceSynchronize): for payloads handed to
 * consumers that read them on their own streams (zero-copy DLPack export).
 * No reference counterpart (the reference is CPU-only). */
int camel_hip_device_sync(void);
/* The library's hipStream_t, as an opaque handle (for timing by callers). */
void *camel_hip_stream(void);

/* ---- device memory (the Tensor-keyed allocator's backing store) ---------- */
/* Pooled device allocation, 256-byte aligned, never zero-filled.  Replaces
 * the payload part of TensorObject::create (runtime.cpp:256-279). */
int camel_hip_malloc(void **ptr, size_t bytes);
/* Returns a block to the pool (NULL is a no-op). */
int camel_hip_free(void *ptr);
/* Releases a block that other streams may still read (a zero-copy DLPack
 * export whose consumer's deleter ran): it returns to the pool only after a
 * later device-wide synchronisation, which the library runs at its next pool
 * miss, camel_hip_device_sync or camel_hip_pool_trim; the call itself never
 * waits.  No reference counterpart (the reference exports host copies only,
 * runtime.cpp:1079-1100). */
int camel_hip_free_shared(void *ptr);
/* Releases every cached free block to the driver. */
int camel_hip_pool_trim(void);
/* Bytes currently handed out / cached, for leak checks. */
int camel_hip_pool_stats(size_t *in_use, size_t *cached);
/* Synchronous copies at a graph boundary (host memory may be pageable and
 * only 8-byte aligned, as the reference's inline tensor payload is,
 * runtime.cpp:482-485). */
int camel_hip_h2d(void *dst, const void *src, size_t bytes);
int camel_hip_d2h(void *dst, const void *src, size_t bytes);
int camel_hip_d2d(void *dst, const void *src, size_t bytes);

/* ---- creation (tensorZeros/Ones/Full/Eye/Arange, runtime.cpp:614-690) ---- */
/* out[i] = value converted to dtype as setFromDouble does (runtime.cpp:340-355). */
int camel_hip_fill(int dtype, void *out, int64_t n, double value);
/* Float32 identity n x n (tensorEye, runtime.cpp:679-690). */
int camel_hip_eye(float *out, int64_t n);
/* Int64 out[i] = start + i*step, i < count (tensorArange, runtime.cpp:656-677). */
int camel_hip_arange(int64_t *out, int64_t start, int64_t step, int64_t count);

/* ---- GEMM (tensor:matmul and dense) -------------------------------------- */
/* C[M,N] = A[M,K] . B[K,N], fp32 row-major contiguous, on fp32 MFMA.
 * Replaces the ijk loop of __tensor_matmul__ (operators.cpp:740-769).
 * flags: CAMEL_EPI_BIAS adds bias[N] to every row (the ones@b broadcast idiom,
 * test/run/nn/mnist.cml:18, then add), CAMEL_EPI_RELU applies x*(x>0)
 * (test/run/nn/svm.cml:31), both fused in the GEMM epilogue;
 * CAMEL_GEMM_A_T: A given as At[K, M] (see camel_hip_gemm_layout).  Other
 * flag bits are refused (CAMEL_HIP_ERR_ARG). */
int camel_hip_sgemm(const float *A, const float *B, float *C, int64_t M, int64_t N, int64_t K,
                    const float *bias, int flags);
/* Bytes of the static scratch of the allocation-free entry points (one copy
 * per device the library runs on, held until the process ends). */
#define CAMEL_HIP_NOALLOC_SCRATCH_BYTES (64u << 20)
/* camel_hip_sgemm without any device allocation: the same kernels and the
 * same results bit for bit, with split-K partial sums kept in the library's
 * static scratch (CAMEL_HIP_NOALLOC_SCRATCH_BYTES) instead of pool blocks.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  camel_hip_init must have run first (initialisation allocates).
 * A shape whose split-K partials need more than the scratch is refused with
 * CAMEL_HIP_ERR_SHAPE before anything is launched (no benchmark shape comes
 * near it: the most any GEMM schedule uses is 64 MiB, a full round of split
 * 256x256 tiles).  Every call on a device shares that device's scratch, which
 * keeps the last call's contents (nothing in it needs to start at zero).
 * Library calls run in order on the library stream, but work that overlaps
 * on one device -- e.g. a graph captured from this entry point replayed on
 * another stream while the library stream runs another such call -- races
 * on the scratch. */
int camel_hip_sgemm_noalloc(const float *A, const float *B, float *C, int64_t M, int64_t N,
                            int64_t K, const float *bias, int flags);
/* C[M,N] = softmax_rows(A . B (+bias) (relu)): the dense..softmax of a
 * classifier layer (README.md:43, `dense<w3, b3>..softmax`; softmax as in
 * test/run/nn/mnist.cml:13-25) fused into one pass when N <= 32 (each row's
 * softmax runs on the GEMM's own wave); equals camel_hip_sgemm followed by
 * camel_hip_softmax_rows.  No reference operator: the reference's compose
 * (`..`, src/builtin/operators/macro.cpp:30) is a stub. */
int camel_hip_dense_softmax(const float *A, const float *B, const float *bias, float *C, int64_t M,
                            int64_t N, int64_t K, int flags);
/* y[M,N2] = [softmax_rows]( H . W2 (+b2) (relu) ) with H = x[M,K1] . W1[K1,N1]
 * (+b1) (relu): the two dense layers of a classifier head
 * (`dense<w1, b1>..relu..dense<w2, b2>..softmax`, README.md:40-46); flags1 /
 * flags2 are each layer's CAMEL_EPI_* bits, softmax != 0 adds the row
 * softmax.  Equals camel_hip_sgemm(x, W1) into H followed by
 * camel_hip_dense_softmax (softmax) or camel_hip_sgemm (no softmax) on H, bit
 * for bit.  When layer 1 runs as a split-K GEMM and N2 <= 16, layer 2's kernel
 * adds layer 1's partial sums itself (no reduce launch, H never reaches HBM).
 * No reference operator: the reference's compose is a stub
 * (src/builtin/operators/macro.cpp:30). */
int camel_hip_dense_head(const float *x, const float *w1, const float *b1, const float *w2,
                         const float *b2, float *y, int64_t M, int64_t K1, int64_t N1, int64_t N2,
                         int flags1, int flags2, int softmax);
/* Mixed-dtype matmul through double (Int64 / Bool operands, promoted output
 * dtype, promoteTensorTypes runtime.cpp:570-580). */
int camel_hip_matmul_generic(int adt, const void *A, int bdt, const void *B, int odt, void *C,
                             int64_t M, int64_t N, int64_t K);

/* ---- conv2d / pooling (no reference op; defined by composition) --------- */
/* y[N,Co,OH,OW] = conv(x[N,C,H,W], w[Co,C,KH,KW]) (+bias[Co]) (relu), NCHW,
 * implicit GEMM on the same MFMA core.  OH = (H+2*pad-KH)/stride+1.
 * flags may add the camel_hip_conv_layout bits (same values, other
 * addressing). */
int camel_hip_conv2d(const float *x, const float *w, const float *bias, float *y, int64_t N,
                     int64_t C, int64_t H, int64_t W, int64_t Co, int64_t KH, int64_t KW,
                     int64_t stride, int64_t pad, int flags);
/* wp[Co,KH,KW,C] = w[Co,C,KH,KW] reordered: the weight layout the NHWC
 * implicit GEMM reads.  A caller that applies the same weights many times
 * packs them once and passes CAMEL_CONV_W_PACKED (no reference counterpart:
 * weight pre-packing of a layer chain). */
int camel_hip_conv2d_pack_weights(const float *w, float *wp, int64_t Co, int64_t C, int64_t KH,
                                  int64_t KW);
/* y[N,Co,OH/2,OW/2] = maxpool2x2(conv2d(x) (+bias) (relu)), the
 * conv2d_relu..maxpool2d of a CNN fused: the 2x2 stride-2 max (the rule of
 * camel_hip_maxpool2d) is taken in the convolution's epilogue, so the
 * full-size result never reaches HBM.  No reference operator (compose is a
 * stub, src/builtin/operators/macro.cpp:30).  flags may add
 * CAMEL_CONV_X_NHWC / CAMEL_CONV_X_NCHW4 / CAMEL_CONV_W_PACKED; OH, OW >= 2. */
int camel_hip_conv2d_pool2(const float *x, const float *w, const float *bias, float *y, int64_t N,
                           int64_t C, int64_t H, int64_t W, int64_t Co, int64_t KH, int64_t KW,
                           int64_t stride, int64_t pad, int flags);
/* y[N,Co2,(H-4)/2,(W-4)/2] = maxpool2x2(conv2(conv1(x))): the
 * conv2d..conv2d..maxpool2d(2, 2) opening of an image CNN
 * (`conv2d<w1,b1>..relu..conv2d<w2,b2>..relu..maxpool2d`) in one kernel, with
 * conv1 = x[N,1,H,W] * w1[C1,1,3,3] (+b1) (relu) and conv2 = conv1 *
 * w2[Co2,C1,3,3] (+b2) (relu), both stride 1 and unpadded; flags1 / flags2
 * carry each conv's CAMEL_EPI_* bits, flags2 may add CAMEL_CONV_W_PACKED (w2
 * as [Co2,3,3,C1]).  conv1's output never reaches HBM: each work-group
 * computes the rows its band of conv2 reads into LDS.  Equals
 * camel_hip_conv2d(conv1, CAMEL_CONV_Y_NCHW4) followed by
 * camel_hip_conv2d_pool2(conv2, CAMEL_CONV_X_NCHW4) bit for bit.  Served
 * shapes: W = 28, C1 = 32, Co2 % 64 == 0, (H - 4) % 8 == 0 (MNIST-style
 * 28 x 28 inputs); others return CAMEL_HIP_ERR_SHAPE.  No reference operator:
 * the reference's compose is a stub (src/builtin/operators/macro.cpp:30). */
int camel_hip_conv2d_pair_pool2(const float *x, const float *w1, const float *b1, const float *w2,
                                const float *b2, float *y, int64_t N, int64_t H, int64_t W,
                                int64_t C1, int64_t Co2, int flags1, int flags2);
/* Max pool, NCHW, window KH x KW, first-then-strict-'>' rule of tensorMaxAxis
 * (runtime.cpp:953-958).  OH = (H-KH)/stride+1. */
int camel_hip_maxpool2d(const float *x, float *y, int64_t N, int64_t C, int64_t H, int64_t W,
                        int64_t KH, int64_t KW, int64_t stride);

/* ---- elementwise ----------------------------------------------------------- */
/* out[i] = op(l[i], r[i]) computed as (odt)op((double)l, (double)r).
 * Replaces tensorBinary (runtime.cpp:775-793, applyBinary 113-130). */
int camel_hip_binary(int op, int ldt, const void *l, int rdt, const void *r, int odt, void *out,
                     int64_t n);
/* Tensor (op) scalar: side 0 = tensor on the left (tensorBinaryScalarRight,
 * runtime.cpp:795-812), side 1 = scalar on the left (tensorBinaryScalarLeft,
 * 814-831).  The scalar is the double of scalarToDouble (runtime.cpp:62-77). */
int camel_hip_binary_scalar(int op, int side, int tdt, const void *t, double s, int odt,
                            void *out, int64_t n);
/* out[i] = (u8)cmp((double)l[i], (double)r[i])  (tensorCompare, runtime.cpp:863-877). */
int camel_hip_compare(int op, int ldt, const void *l, int rdt, const void *r, uint8_t *out,
                      int64_t n);
/* Scalar comparisons (tensorCompareScalarRight/Left, runtime.cpp:833-861). */
int camel_hip_compare_scalar(int op, int side, int tdt, const void *t, double s, uint8_t *out,
                             int64_t n);
/* relu(x) = x * (x > 0) bit-exactly (-0.0 for x<0, NaN for -inf / NaN). */
int camel_hip_relu(const float *x, float *y, int64_t n);
/* (float)exp((double)x)  (tensorExp, runtime.cpp:1013-1026). */
int camel_hip_exp(const float *x, float *y, int64_t n);
/* (float)log((double)x), CAMEL_HIP_ERR_LOG_DOMAIN if any x <= 0
 * (tensorLog, runtime.cpp:1028-1045). */
int camel_hip_log(const float *x, float *y, int64_t n);

/* ---- reductions ---------------------------------------------------------- */
/* Row softmax of x[rows, cols]: the op-for-op composition of
 * test/run/nn/mnist.cml:13-25 fused in one pass (fp64 exp and row sum). */
int camel_hip_softmax_rows(const float *x, float *y, int64_t rows, int64_t cols);
/* Rank-2 reductions along axis 0 or 1 (negative axis += 2):
 *   sum    -> Float32 out (tensorSumAxis,    runtime.cpp:887-922)
 *   max    -> Float32 out (tensorMaxAxis,    runtime.cpp:924-963)
 *   argmax -> Int64 out   (tensorArgmaxAxis, runtime.cpp:965-1011) */
int camel_hip_sum_axis(int dt, const void *x, int64_t rows, int64_t cols, int64_t axis,
                       float *out);
int camel_hip_max_axis(int dt, const void *x, int64_t rows, int64_t cols, int64_t axis,
                       float *out);
int camel_hip_argmax_axis(int dt, const void *x, int64_t rows, int64_t cols, int64_t axis,
                          int64_t *out);
/* Whole-tensor double sum (tensorSum, runtime.cpp:879-885). */
int camel_hip_sum(int dt, const void *x, int64_t n, double *result);

/* ---- layout ---------------------------------------------------------------- */
/* tensorTranspose2D (runtime.cpp:704-720). */
int camel_hip_transpose2d(int dt, const void *x, void *y, int64_t rows, int64_t cols);
/* tensorConcat (runtime.cpp:722-773): per outer index, l_axis*inner items of
 * l then r_axis*inner items of r. */
int camel_hip_concat(int dt, const void *l, const void *r, void *out, int64_t outer,
                     int64_t l_axis, int64_t r_axis, int64_t inner);

/* ---- timing (HIP events on the library stream) ----------------------------- */
int camel_hip_event_create(void **event);
int camel_hip_event_record(void *event);
int camel_hip_event_elapsed_ms(void *start, void *stop, float *ms);
int camel_hip_event_destroy(void *event);

#ifdef __cplusplus
}
#endif

#endif
