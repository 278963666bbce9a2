/*
 * oracle.c — CPU restatement of the reference's hot-path semantics.
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for tests/, smoke()
 * and the cpu_baseline leg of bench.py; never linked into the product.
 *
 * Built with -ffp-contract=off so every float expression rounds exactly as
 * written; fmaf() is called explicitly where the reference fuses.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <string.h>

/* ---- GEMM ---------------------------------------------------------------- */

static inline float opA(int ta, const float *A, int64_t lda, int64_t m, int64_t k) {
  return ta ? A[k * lda + m] : A[m * lda + k];
}
static inline float opB(int tb, const float *B, int64_t ldb, int64_t k, int64_t n) {
  return tb ? B[n * ldb + k] : B[k * ldb + n];
}

/* cpu.h:239-264 (cblas_sgemm, RowMajor, alpha 1, beta 0) with the transposes
 * that array.h:2639-2649 derives from strides. */
void oracle_sgemm_f64(int ta, int tb, int64_t M, int64_t N, int64_t K, const float *A,
                      int64_t lda, const float *B, int64_t ldb, double *C64, double *Cabs) {
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      double s = 0.0, sa = 0.0;
      for (int64_t k = 0; k < K; ++k) {
        double p = (double)opA(ta, A, lda, m, k) * (double)opB(tb, B, ldb, k, n);
        s += p;
        sa += fabs(p);
      }
      C64[m * N + n] = s;
      if (Cabs) Cabs[m * N + n] = sa;
    }
  }
}

void oracle_sgemm_sampled_f64(int ta, int tb, int64_t K, const float *A, int64_t lda,
                              const float *B, int64_t ldb, const int64_t *rows,
                              const int64_t *cols, int64_t count, double *out,
                              double *outabs) {
  for (int64_t i = 0; i < count; ++i) {
    double s = 0.0, sa = 0.0;
    for (int64_t k = 0; k < K; ++k) {
      double p = (double)opA(ta, A, lda, rows[i], k) * (double)opB(tb, B, ldb, k, cols[i]);
      s += p;
      sa += fabs(p);
    }
    out[i] = s;
    if (outabs) outabs[i] = sa;
  }
}

/* ---- elementwise ---------------------------------------------------------- */

static inline float binf(int op, float a, float b) {
  switch (op) {
    case 0: return a + b;
    case 1: return a - b;
    case 2: return a * b;
    case 3: return a / b;
    default: return powf(a, b);
  }
}

/* gpu_kernels.metal:826-842 and cpu.h:76-237: out[i] = a[i%len_a] op b[i%len_b]. */
void oracle_binary_mod_f32(int op, const float *a, int64_t a_len, const float *b,
                           int64_t b_len, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = binf(op, a[i % a_len], b[i % b_len]);
}

/* Integer ops: C arithmetic; pow rounds powf of the float operands
 * (gpu_kernels.metal:860-862).  Division by zero yields 0 here (undefined in
 * the reference). */
void oracle_binary_mod_i32(int op, const int32_t *a, int64_t a_len, const int32_t *b,
                           int64_t b_len, int32_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    int32_t x = a[i % a_len], y = b[i % b_len];
    int32_t r;
    switch (op) {
      case 0: r = x + y; break;
      case 1: r = x - y; break;
      case 2: r = x * y; break;
      case 3: r = y == 0 ? 0 : x / y; break;
      default: r = (int32_t)rintf(powf((float)x, (float)y)); break;
    }
    out[i] = r;
  }
}

void oracle_binary_strided_f32(int op, int ndim, const int64_t *shape, const float *a,
                               const int64_t *sa, const float *b, const int64_t *sb,
                               float *out) {
  int64_t n = 1;
  for (int d = 0; d < ndim; ++d) n *= shape[d];
  for (int64_t i = 0; i < n; ++i) {
    int64_t rem = i, oa = 0, ob = 0;
    for (int d = ndim - 1; d >= 0; --d) {
      int64_t idx = rem % shape[d];
      rem /= shape[d];
      oa += idx * sa[d];
      ob += idx * sb[d];
    }
    out[i] = binf(op, a[oa], b[ob]);
  }
}

/* cpu.h:290-297: 1 / (1 + exp(-x)) */
void oracle_sigmoid(const float *x, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = 1.0f / (1.0f + expf(-x[i]));
}

/* cpu.h:324-327: vDSP_vthres(x, 0) = x if x >= 0 else 0 */
void oracle_relu(const float *x, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = x[i] >= 0.0f ? x[i] : 0.0f;
}

/* cpu.h:310-322 */
void oracle_bias_sigmoid(float *data, const float *bias, int64_t n, int64_t cols) {
  for (int64_t i = 0; i < n; ++i) {
    float v = data[i] + bias[i % cols];
    data[i] = 1.0f / (1.0f + expf(-v));
  }
}

/* cpu.h:299-308 */
void oracle_sigmoid_backward(const float *dout, const float *x, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    float s = 1.0f / (1.0f + expf(-x[i]));
    out[i] = dout[i] * s * (1.0f - s);
  }
}

void oracle_affine(const float *x, float *out, int64_t n, float scale, float offset) {
  for (int64_t i = 0; i < n; ++i) out[i] = fmaf(x[i], scale, offset);
}

void oracle_affine_chain(const float *x, float *out, int64_t n, const float *scale,
                         const float *offset, int steps) {
  for (int64_t i = 0; i < n; ++i) {
    float v = x[i];
    for (int s = 0; s < steps; ++s) v = fmaf(v, scale[s], offset[s]);
    out[i] = v;
  }
}

/* ---- reductions ------------------------------------------------------------ */

double oracle_sum_f64(const float *x, int64_t n) {
  double s = 0.0;
  for (int64_t i = 0; i < n; ++i) s += (double)x[i];
  return s;
}

float oracle_sum_ref(const float *x, int64_t n) {
  float s = 0.0f;
  for (int64_t i = 0; i < n; ++i) s += x[i];
  return s;
}

float oracle_min(const float *x, int64_t n) {
  float m = INFINITY;
  for (int64_t i = 0; i < n; ++i) m = fminf(m, x[i]);
  return m;
}

float oracle_max(const float *x, int64_t n) {
  float m = -INFINITY;
  for (int64_t i = 0; i < n; ++i) m = fmaxf(m, x[i]);
  return m;
}

void oracle_sum_axis_f64(const float *x, int64_t outer, int64_t axis_len, int64_t inner,
                         double *out) {
  for (int64_t o = 0; o < outer; ++o)
    for (int64_t i = 0; i < inner; ++i) {
      double s = 0.0;
      for (int64_t a = 0; a < axis_len; ++a) s += (double)x[(o * axis_len + a) * inner + i];
      out[o * inner + i] = s;
    }
}

/* array.h:1574-1578 / 2309-2314: tmp.at(p) += at(pos) over the positions in
 * row-major order, in float: each output sums its inputs in axis order. */
void oracle_sum_axis_ref(const float *x, int64_t outer, int64_t axis_len, int64_t inner,
                         float *out) {
  for (int64_t j = 0; j < outer * inner; ++j) out[j] = 0.0f;
  for (int64_t o = 0; o < outer; ++o)
    for (int64_t a = 0; a < axis_len; ++a) {
      const float *src = x + (o * axis_len + a) * inner;
      float *dst = out + o * inner;
      for (int64_t i = 0; i < inner; ++i) dst[i] += src[i];
    }
}

void oracle_argmax_rows(const float *x, int64_t rows, int64_t cols, int32_t *out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *row = x + r * cols;
    int64_t best = -1;
    for (int64_t c = 0; c < cols; ++c) {
      float v = row[c];
      if (v != v) continue;
      if (best < 0 || v > row[best]) best = c;
    }
    out[r] = (int32_t)(best < 0 ? 0 : best);
  }
}

void oracle_argmax_rows_cpu_ref(const float *x, int64_t rows, int64_t cols, int32_t *out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *row = x + r * cols;
    float max_val = FLT_MIN;
    int64_t max_index = 0;
    for (int64_t c = 0; c < cols; ++c)
      if (row[c] > max_val) {
        max_val = row[c];
        max_index = c;
      }
    out[r] = (int32_t)max_index;
  }
}

/* ---- row ops ---------------------------------------------------------------- */

void oracle_softmax_rows_f64(const float *x, int64_t rows, int64_t cols, double *out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *row = x + r * cols;
    double m = -INFINITY;
    for (int64_t c = 0; c < cols; ++c) m = row[c] > m ? row[c] : m;
    double s = 0.0;
    for (int64_t c = 0; c < cols; ++c) {
      double e = exp((double)row[c] - m);
      out[r * cols + c] = e;
      s += e;
    }
    for (int64_t c = 0; c < cols; ++c) out[r * cols + c] /= s;
  }
}

void oracle_softmax_rows_ref(const float *x, int64_t rows, int64_t cols, float *out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *row = x + r * cols;
    float c = oracle_min(row, cols);
    float s = 0.0f;
    for (int64_t j = 0; j < cols; ++j) {
      out[r * cols + j] = expf(row[j] - c);
      s += out[r * cols + j];
    }
    for (int64_t j = 0; j < cols; ++j) out[r * cols + j] = out[r * cols + j] / s;
  }
}

void oracle_layer_norm_f64(const float *x, const float *gamma, const float *beta,
                           int64_t rows, int64_t cols, float eps, double *out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *row = x + r * cols;
    double mu = 0.0;
    for (int64_t c = 0; c < cols; ++c) mu += row[c];
    mu /= (double)cols;
    double ss = 0.0;
    for (int64_t c = 0; c < cols; ++c) ss += ((double)row[c] - mu) * ((double)row[c] - mu);
    double inv = 1.0 / sqrt(ss / (double)cols + (double)eps);
    for (int64_t c = 0; c < cols; ++c)
      out[r * cols + c] = ((double)row[c] - mu) * inv * (double)gamma[c] + (double)beta[c];
  }
}

void oracle_layer_norm_ref(const float *x, const float *gamma, const float *beta,
                           int64_t rows, int64_t cols, float eps, float *out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *row = x + r * cols;
    float *o = out + r * cols;
    float mu = oracle_sum_ref(row, cols) / (float)cols;   /* vDSP_meanv */
    for (int64_t c = 0; c < cols; ++c) o[c] = row[c] + (-mu); /* vDSP_vsadd(-mu) */
    float ss = 0.0f;
    for (int64_t c = 0; c < cols; ++c) ss += o[c] * o[c];  /* vDSP_dotpr */
    float inv = 1.0f / sqrtf(ss / (float)cols + eps);
    for (int64_t c = 0; c < cols; ++c) o[c] = o[c] * inv;   /* vDSP_vsmul */
    for (int64_t c = 0; c < cols; ++c) o[c] = o[c] * gamma[c]; /* vDSP_vmul */
    for (int64_t c = 0; c < cols; ++c) o[c] = o[c] + beta[c];  /* vDSP_vadd */
  }
}

/* ---- CPU baseline helpers ------------------------------------------------------ */

void oracle_gemv_f32(const float *x, const float *B, int64_t N, int64_t K, float *y) {
  for (int64_t n = 0; n < N; ++n) y[n] = 0.0f;
  for (int64_t k = 0; k < K; ++k) {
    const float xv = x[k];
    const float *row = B + k * N;
    for (int64_t n = 0; n < N; ++n) y[n] += xv * row[n];
  }
}
