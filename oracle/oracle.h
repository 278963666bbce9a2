/*
 * oracle.h — CPU restatement of the reference's semantics for the silarray
 * GPU hot path.  TEST INFRASTRUCTURE ONLY: used by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg as the checker
 * and the CPU baseline.  Nothing in the product (libsilgpu.so, the C++
 * headers under silarray_amd/include) links, loads or calls it.
 *
 * Two modes per op where the reference's rounding is not specified:
 *   *_f64  : the mathematical definition evaluated in double ("golden");
 *   *_ref  : the reference's own fp32 evaluation order, restated from the
 *            cited file:line of /root/reference (include/cpu.h, array.h).
 *
 * Each function is pinned in tests/test_oracle.py against the reference's
 * own golden vectors (test/test_array.cpp), closed forms, invariants or an
 * independent brute force, so a dropped term, wrong sign or transposed
 * operand fails a check.
 */
#ifndef SIL_ORACLE_H
#define SIL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- GEMM (include/cpu.h:239-264, include/array.h:2632-2655) ------------- */
/* C64[m*N + n] = sum_k op(A)[m][k] * op(B)[k][n] in double; if Cabs is not
 * NULL also Cabs = sum_k |op(A)[m][k] * op(B)[k][n]| (for per-element
 * rounding bounds).  op(A)[m][k] = ta ? A[k*lda+m] : A[m*lda+k]. */
void oracle_sgemm_f64(int ta, int tb, int64_t M, int64_t N, int64_t K, const float *A,
                      int64_t lda, const float *B, int64_t ldb, double *C64, double *Cabs);

/* Same, only at the (rows[i], cols[i]) entries. */
void oracle_sgemm_sampled_f64(int ta, int tb, int64_t K, const float *A, int64_t lda,
                              const float *B, int64_t ldb, const int64_t *rows,
                              const int64_t *cols, int64_t count, double *out,
                              double *outabs);

/* ---- elementwise (include/cpu.h:76-237, include/gpu_kernels.metal:826-968) */
/* out[i] = a[i % a_len] op b[i % b_len]; op 0..4 = add sub mul div pow. */
void oracle_binary_mod_f32(int op, const float *a, int64_t a_len, const float *b,
                           int64_t b_len, float *out, int64_t n);
void oracle_binary_mod_i32(int op, const int32_t *a, int64_t a_len, const int32_t *b,
                           int64_t b_len, int32_t *out, int64_t n);
/* Broadcast through element strides (0 on broadcast axes). */
void oracle_binary_strided_f32(int op, int ndim, const int64_t *shape, const float *a,
                               const int64_t *sa, const float *b, const int64_t *sb,
                               float *out);
/* cpu.h:290-327 */
void oracle_sigmoid(const float *x, float *out, int64_t n);
void oracle_relu(const float *x, float *out, int64_t n);
void oracle_bias_sigmoid(float *data, const float *bias, int64_t n, int64_t cols);
void oracle_sigmoid_backward(const float *dout, const float *x, float *out, int64_t n);
/* out = fmaf(x, scale, offset) (gpu_kernels.metal:1489-1497, cpu.h:329-350) */
void oracle_affine(const float *x, float *out, int64_t n, float scale, float offset);
/* A chain of `steps` scalar affine nodes evaluated node by node, as
 * sil::eval does after try_affine_reduce folds each node one level
 * (include/array.h:1888-2022): x <- fmaf(x, scale[s], offset[s]). */
void oracle_affine_chain(const float *x, float *out, int64_t n, const float *scale,
                         const float *offset, int steps);

/* ---- reductions ---------------------------------------------------------- */
double oracle_sum_f64(const float *x, int64_t n);
/* Sequential fp32 sum (the order of std::accumulate, include/array.h:1531). */
float oracle_sum_ref(const float *x, int64_t n);
float oracle_min(const float *x, int64_t n);
float oracle_max(const float *x, int64_t n);
/* out[o*inner + i] = sum_a x[(o*axis_len + a)*inner + i] in double. */
void oracle_sum_axis_f64(const float *x, int64_t outer, int64_t axis_len, int64_t inner,
                         double *out);
/* The reference's float path for sum(axis) (include/array.h:1574-1578,
 * 2309-2314): out[o*inner + i] accumulated in float, axis index ascending. */
void oracle_sum_axis_ref(const float *x, int64_t outer, int64_t axis_len, int64_t inner,
                         float *out);
/* First index of the row maximum; NaN never wins (an all-NaN row gives 0). */
void oracle_argmax_rows(const float *x, int64_t rows, int64_t cols, int32_t *out);
/* The reference CPU loop verbatim in meaning (include/array.h:1728-1745):
 * max_val starts at numeric_limits<float>::min() (+1.17549435e-38), strict >.
 * A row whose values are all <= that constant returns 0. */
void oracle_argmax_rows_cpu_ref(const float *x, int64_t rows, int64_t cols, int32_t *out);

/* ---- row ops ------------------------------------------------------------- */
/* exp(x - max) / sum in double. */
void oracle_softmax_rows_f64(const float *x, int64_t rows, int64_t cols, double *out);
/* Reference CPU path (include/array.h:2135-2151): c = row min,
 * e = expf(x - c) in float, s = sequential float sum, out = e / s. */
void oracle_softmax_rows_ref(const float *x, int64_t rows, int64_t cols, float *out);
/* (x - mean) / sqrt(var + eps) * gamma + beta in double, var = mean((x-mean)^2). */
void oracle_layer_norm_f64(const float *x, const float *gamma, const float *beta,
                           int64_t rows, int64_t cols, float eps, double *out);
/* cpu::layer_norm (include/cpu.h:352-373) in float: mean, out = x - mean,
 * ss = sum(out*out), inv = 1/sqrtf(ss/cols + eps), out*inv*gamma + beta. */
void oracle_layer_norm_ref(const float *x, const float *gamma, const float *beta,
                           int64_t rows, int64_t cols, float eps, float *out);

/* ---- CPU baseline helpers ---------------------------------------------- */
/* Scalar single-thread loops for the cpu_baseline leg of bench.py (the
 * reference's vDSP calls restated as plain loops). */
void oracle_gemv_f32(const float *x, const float *B, int64_t N, int64_t K, float *y);

#ifdef __cplusplus
}
#endif

#endif /* SIL_ORACLE_H */
