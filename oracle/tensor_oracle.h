/*
 * tensor_oracle.h -- CPU restatement of the Camel `tensor` module kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path and
 * the timed CPU baseline in bench.py; the product (libcamel_hip.so and the
 * operator layer) never links, loads or calls it.  Only tests/, the smoke()
 * entry of __graft_entry__.py and bench.py's cpu_baseline leg may use it.
 *
 * Every function restates the reference algorithm loop for loop (same loop
 * order, fp64 accumulation, one fp32 rounding per reference operation) and
 * cites the reference file:line it follows (paths relative to the reference
 * tree, OpenCML/Camel 0.1.19).  The ops the reference lacks (relu, softmax,
 * dense, conv2d, maxpool) are defined as compositions of reference kernels,
 * as named in each comment.
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off, no fast-math), matching
 * the module flags of modules/camel_module.cmake:68-73 (no -march, so no FMA).
 */
#ifndef CAMEL_TENSOR_ORACLE_H
#define CAMEL_TENSOR_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Storage dtypes of TensorObject (modules/tensor/runtime.cpp:530-541). */
enum { OT_F32 = 0, OT_I64 = 1, OT_BOOL = 2 };

/* BinaryOp / CompareOp, same order as modules/tensor/runtime.h:39-53. */
enum { OT_ADD = 0, OT_SUB = 1, OT_MUL = 2, OT_DIV = 3, OT_POW = 4 };
enum { OT_LT = 0, OT_LE = 1, OT_GT = 2, OT_GE = 3, OT_EQ = 4 };

/* Return codes; each maps to the std::invalid_argument the reference throws. */
enum {
    OT_OK = 0,
    OT_ERR_DIV_ZERO = 1,   /* "Division by zero"             runtime.cpp:122-124 */
    OT_ERR_LOG_DOMAIN = 2, /* "log: input must be positive"   runtime.cpp:1039-1041 */
    OT_ERR_SHAPE = 3,      /* shape / axis / rank errors                          */
    OT_ERR_DTYPE = 4       /* "exp/log requires floating-point tensor"            */
};

int ot_promote(int lhs, int rhs);
double ot_get(int dt, const void *p, uint64_t i);
void ot_set(int dt, void *p, uint64_t i, double v);
double ot_apply_binary(int op, double l, double r, int *err);

int ot_binary(int op, int ldt, const void *l, int rdt, const void *r, int odt, void *out,
              uint64_t n);
int ot_binary_scalar_right(int op, int ldt, const void *l, double s, int odt, void *out,
                           uint64_t n);
int ot_binary_scalar_left(int op, double s, int rdt, const void *r, int odt, void *out,
                          uint64_t n);
void ot_compare(int op, int ldt, const void *l, int rdt, const void *r, uint8_t *out, uint64_t n);
void ot_compare_scalar_right(int op, int ldt, const void *l, double s, uint8_t *out, uint64_t n);
void ot_compare_scalar_left(int op, double s, int rdt, const void *r, uint8_t *out, uint64_t n);

int ot_matmul(int adt, const void *A, int bdt, const void *B, int odt, void *C, int64_t M,
              int64_t K, int64_t N);
int64_t ot_matmul_rows(const float *A, const float *B, float *C, int64_t M, int64_t K, int64_t N,
                       int64_t row_begin, int64_t row_end);

double ot_sum(int dt, const void *x, uint64_t n);
int ot_sum_axis(int dt, const void *x, int64_t rows, int64_t cols, int64_t axis, float *out);
int ot_max_axis(int dt, const void *x, int64_t rows, int64_t cols, int64_t axis, float *out);
int ot_argmax_axis(int dt, const void *x, int64_t rows, int64_t cols, int64_t axis, int64_t *out);
int ot_exp(int dt, const void *x, float *out, uint64_t n);
int ot_log(int dt, const void *x, float *out, uint64_t n);
void ot_transpose2d(int dt, const void *x, void *out, int64_t rows, int64_t cols);
void ot_concat(int dt, const void *l, const void *r, void *out, uint64_t outer, uint64_t l_axis,
               uint64_t r_axis, uint64_t inner);

/* Compositions for the ops the reference has no kernel for. */
void ot_relu(const float *x, float *out, uint64_t n);
int ot_softmax_rows(const float *x, float *out, int64_t n, int64_t k);
int ot_dense(const float *x, const float *W, const float *b, int relu, float *out, int64_t M,
             int64_t K, int64_t N);
int ot_conv2d(const float *x, const float *w, const float *b, int relu, float *y, int64_t N,
              int64_t C, int64_t H, int64_t W, int64_t Co, int64_t KH, int64_t KW, int64_t stride,
              int64_t pad);
int64_t ot_conv2d_images(const float *x, const float *w, const float *b, int relu, float *y,
                         int64_t n_begin, int64_t n_end, int64_t C, int64_t H, int64_t W,
                         int64_t Co, int64_t KH, int64_t KW, int64_t stride, int64_t pad);
int ot_maxpool2d(const float *x, float *y, int64_t N, int64_t C, int64_t H, int64_t W, int64_t KH,
                 int64_t KW, int64_t stride);

/* Seeded inputs: counter-based SplitMix64 (public domain, S. Vigna). */
uint64_t ot_splitmix64(uint64_t seed, uint64_t index);
void ot_fill_uniform(float *out, uint64_t n, uint64_t seed, float lo, float hi);

#ifdef __cplusplus
}
#endif

#endif
