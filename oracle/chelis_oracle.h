/*
 * CPU oracle for the fused-DAG execution path: TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker or the timed CPU baseline.
 * The product library (chelis_amd/csrc) never links or calls it.
 *
 * It restates, in plain C, what the reference C backend computes for the
 * configurations of this path (crates/chelis-backend-c/src/emit.rs), under
 * the reference's pinned toolchain profile
 * `-O2 -ffp-contract=off -fno-fast-math -fopenmp`
 * (crates/chelis-backend-c/src/toolchain.rs:229-260).
 *
 * Correctly rounded transcendentals are not restated: they are the vendored
 * CORE-MATH library (MIT, upstream commit
 * 284b3b0e198042c38f5c30316f696786b10816b0, see
 * crates/chelis-crmath/vendor/core-math/VENDOR.toml), compiled from the
 * reference's own source into oracle/_ref/ by oracle/Makefile and reached
 * through its `chelis_crmath_ffi_*` shims (crates/chelis-crmath/csrc/crmath_ffi.c),
 * which already finalize NaN to the canonical quiet NaN.
 *
 * Parity pins (tests/test_oracle_*.py): every function below is checked
 * against a golden vector, a known-answer test or an independent
 * restatement; see the header comment of each test file.
 */
#ifndef CHELIS_ORACLE_H
#define CHELIS_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- keyed RNG ([05-RNG-1], [05-RNG-2], [05-OP-69..72]) ---- */
uint64_t orc_splitmix64(uint64_t x);
uint64_t orc_derive(uint64_t key, uint64_t j);
uint64_t orc_word(uint64_t key, uint64_t index);
double orc_unit(uint64_t key, uint64_t index);
void orc_split(uint64_t key, uint64_t out[2]);
uint64_t orc_fold_in(uint64_t key, int64_t n);
void orc_split_n(uint64_t key, int64_t n, uint64_t *out);
void orc_uniform_like_f32(uint64_t key, float low, float high, float *out, int64_t n);
void orc_uniform_like_f64(uint64_t key, double low, double high, double *out, int64_t n);

/* ---- correctly rounded leaves (CORE-MATH, canonical NaN) ---- */
float orc_expf(float x);
double orc_exp(double x);
float orc_logf(float x);
double orc_log(double x);
float orc_erfcf(float x);
double orc_erfc(double x);
float orc_tanhf(float x);
double orc_tanh(double x);

/* OpenMP threads of the parallel loops; returns the previous setting. */
int orc_set_threads(int n);

/* ---- canonical reductions ([05-OP-30], [05-OP-12], [05-OP-29]) ---- */
float orc_tree_sum_f32(const float *x, int64_t n, int64_t stride);
double orc_tree_sum_f64(const double *x, int64_t n, int64_t stride);
/* Reference pass-by-pass tree (spec/05 section 2.3 "Reduction order"). */
float orc_level_sum_f32(const float *x, int64_t n);
double orc_level_sum_f64(const double *x, int64_t n);
float orc_max_reduce_f32(const float *x, int64_t n, int64_t stride);
double orc_max_reduce_f64(const double *x, int64_t n, int64_t stride);
/* Sum of `x` viewed as [outer, n, inner] over the middle axis. */
void orc_sum_axis_f32(const float *x, int64_t outer, int64_t n, int64_t inner, float *out);
void orc_sum_axis_f64(const double *x, int64_t outer, int64_t n, int64_t inner, double *out);
void orc_max_axis_f32(const float *x, int64_t outer, int64_t n, int64_t inner, float *out);
void orc_max_axis_f64(const double *x, int64_t outer, int64_t n, int64_t inner, double *out);
/* ProdReduce over [outer, n, inner]: the C lane's left fold from 1
 * (crates/chelis-backend-c/src/emit.rs:2551-2561, 8817-8912), NaN-finalized.
 * The C lane admits f32 only (emit.rs:8838-8855); the f64 form is the same
 * fold at binary64, as the reference HIP lane's reduce_prod computes it
 * (crates/chelis-backend-hip/src/kernels.rs:1888-1925). */
void orc_prod_axis_f32(const float *x, int64_t outer, int64_t n, int64_t inner, float *out);
void orc_prod_axis_f64(const double *x, int64_t outer, int64_t n, int64_t inner, double *out);
/* Bool8 count over [outer, n, inner]; returns 0 or the reference error
 * code 1 (a byte that is not 0 or 1). */
int32_t orc_count_axis(const uint8_t *x, int64_t outer, int64_t n, int64_t inner, int64_t *out);

/* ---- row regions ---- */
void orc_softmax_rows_f32(const float *x, float *y, int64_t rows, int64_t n);
void orc_softmax_rows_f64(const double *x, double *y, int64_t rows, int64_t n);
void orc_softmax_adjoint_rows_f32(const float *y, const float *g, float *dx, int64_t rows, int64_t n);
void orc_softmax_adjoint_rows_f64(const double *y, const double *g, double *dx, int64_t rows, int64_t n);
void orc_layer_norm_rows_f32(const float *x, const float *gamma, const float *beta, float eps,
                             float *y, int64_t rows, int64_t n);
void orc_layer_norm_rows_f64(const double *x, const double *gamma, const double *beta, double eps,
                             double *y, int64_t rows, int64_t n);

/* ---- elementwise ---- */
void orc_gelu_f32(const float *x, float *y, int64_t n);
void orc_gelu_f64(const double *x, double *y, int64_t n);
void orc_relu_f32(const float *x, float *y, int64_t n);
void orc_relu_adjoint_f32(const float *x, const float *g, float *y, int64_t n);
void orc_dropout_f32(uint64_t key, const float *x, float rate, float *y, int64_t n);
void orc_dropout_replay_f32(uint64_t key, const float *g, float rate, float *dx, int64_t n);
void orc_dropout_f64(uint64_t key, const double *x, double rate, double *y, int64_t n);
void orc_dropout_replay_f64(uint64_t key, const double *g, double rate, double *dx, int64_t n);

/* ---- bfloat16 / binary16 storage (kind 0 = bf16, 1 = f16) ----
 * [04-NUM-8]: stored as 16 bits, computed at binary32, finalized once per
 * op (crates/chelis-runtime/include/chelis_runtime.h:664-760). */
void orc_narrow_decode(int kind, const uint16_t *x, float *y, int64_t n);
void orc_narrow_encode(int kind, const float *x, uint16_t *y, int64_t n);
void orc_narrow_sub(int kind, const uint16_t *a, const uint16_t *b, uint16_t *y, int64_t n);
void orc_narrow_max(int kind, const uint16_t *a, const uint16_t *b, uint16_t *y, int64_t n);
void orc_narrow_min(int kind, const uint16_t *a, const uint16_t *b, uint16_t *y, int64_t n);
void orc_narrow_relu(int kind, const uint16_t *x, uint16_t *y, int64_t n);
void orc_narrow_relu_adjoint(int kind, const uint16_t *x, const uint16_t *g, uint16_t *y, int64_t n);
/* C = encode(tree_k(decode(A) * decode(B))) with the binary32 accumulator
 * (spec/04 section 5.7.1); row-major contiguous A [M,K], B [K,N], C [M,N]. */
void orc_matmul_narrow(int kind, const uint16_t *A, const uint16_t *B, uint16_t *C, int64_t M, int64_t N,
                       int64_t K);

/* ---- canonical-tree matmul (inlined product, emit.rs:8431-8560) ----
 * C[i,j] = tree_k(A[i*sa0 + k*sa1] * B[k*sb0 + j*sb1]); strides in elements. */
void orc_matmul_f32(const float *A, int64_t sa0, int64_t sa1, const float *B, int64_t sb0,
                    int64_t sb1, float *C, int64_t M, int64_t N, int64_t K);
void orc_matmul_f64(const double *A, int64_t sa0, int64_t sa1, const double *B, int64_t sb0,
                    int64_t sb1, double *C, int64_t M, int64_t N, int64_t K);

/* ---- configuration programs ---- */
void orc_linreg_step_f64(const double *X, const double *w, const double *y, double *grad,
                         double *loss, int64_t n, int64_t d);
void orc_transformer_block_f32(const float *x, const float *const *params, float *out, int64_t batch,
                               int64_t seq, int64_t dmodel, int64_t heads, int64_t ffn);
void orc_mlp_train_step_f32(const float *x, const float *onehot, float *w1, float *b1, float *w2,
                            float *b2, uint64_t key, float rate, float lr, float *loss,
                            int64_t batch, int64_t din, int64_t dhid, int64_t dout);

/* ---- comparison, logical, where, checked cast and integer arithmetic,
 * gather (flat, equal-length operands; dtype ids of the device packet).
 * Trapping functions return the first failing index or -1 and set *kind
 * (1 overflow, 2 domain, 3 division by zero). ---- */
void orc_compare(int kind, int dt, const void *a, const void *b, uint8_t *out, int64_t n);
void orc_logical(int kind, const uint8_t *a, const uint8_t *b, uint8_t *out, int64_t n);
void orc_where(const uint8_t *cond, const void *a, const void *b, void *out, int64_t width, int64_t n);
void orc_extrema_adjoint(int is_min, int right, int dt, const void *a, const void *b, const void *g, void *out,
                         int64_t n);
int64_t orc_cast(int src, int dst, const void *x, void *y, int64_t n, int32_t *kind);
int64_t orc_int_binary(int op, int dt, const void *a, const void *b, void *y, int64_t n, int32_t *kind);
int64_t orc_int_unary(int op, int dt, const void *x, void *y, int64_t n, int32_t *kind);
int64_t orc_cumsum(int dt, const void *x, void *y, int64_t outer, int64_t n, int64_t inner, int reverse,
                   int32_t *kind);
void orc_pad(int width, const void *x, int rank, const int64_t *src_shape, const int64_t *lo,
             const int64_t *out_shape, uint64_t fill, void *y);
void orc_slice(int width, const void *x, int rank, const int64_t *src_shape, const int64_t *start,
               const int64_t *step, const int64_t *out_shape, void *y);
int64_t orc_scatter(int add, int dt, const void *target, const int64_t *idx, const void *upd, void *out,
                    int64_t before, int64_t axis_size, int64_t after, int64_t index_count, int64_t outer_per_batch,
                    int32_t *kind);
int64_t orc_scatter_elements(int dt, const void *target, const int64_t *idx, const void *upd, void *out, int rank,
                             const int64_t *idx_shape, const int64_t *target_shape, int axis, int32_t *kind);
int64_t orc_gather(const void *values, int64_t width, int64_t before, int64_t axis_size, int64_t after,
                   const void *idx, int idx_dt, int64_t index_count, int64_t batch_count, void *out, int32_t *kind);

#ifdef __cplusplus
}
#endif
#endif
