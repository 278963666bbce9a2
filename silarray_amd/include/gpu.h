#pragma once
// sil::gpu — the reference's operator boundary (include/gpu.h:266-1036),
// same class name, method names and storage-based signatures, implemented
// over the C ABI of libsilgpu.so (include/silgpu.h).  Each dispatcher makes
// its inputs device-current, launches on the library's single stream and
// marks its outputs device-written; nothing waits until flush().
//
// Semantics follow the reference dispatchers:
//   add/sub/mul/div/pow : OUT[i] = A[i % A.len] op B[i % B.len], i < OUT.len
//   sum_f32/min_f32/max_f32 return the number of partial results written to
//     OUT; here the device finishes the reduction, so that number is 1 and
//     OUT[0] holds the result (the reference's host finish over one partial
//     returns the same value, include/array.h:1535-1545)
//   sgemm* / sgemv / dot_f32_ex: C (ldc = N) = op(A) op(B) [+ bias][sigmoid]
//
// Every dispatcher takes its input pointers (dev_in) in statements of their
// own before it takes the output pointer (dev_out): an in-place call passes
// the same storage as input and output, and dev_out marks the device copy
// current, so an input taken after it (C++ leaves the evaluation order of
// call arguments unspecified) would skip a pending upload.

#include <algorithm>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

#include "device.h"
#include "storage.h"
#include "types.h"

namespace sil {

// The reference's gpu_context (include/gpu.h:49-260): one queue, one command
// buffer, blocking flush.  Here: the library's one HIP stream.
class gpu_context {
 public:
  static gpu_context &instance() {
    static auto *ctx = new gpu_context();
    return *ctx;
  }

  // Launches are submitted as they are issued; nothing to commit.
  void commit() {}

  // Waits for every launch issued so far (include/gpu.h:107-123).
  void flush() {
    detail::check(silgpu_sync(), "flush");
    gpu_pending_ = false;
  }

 private:
  gpu_context() { detail::ensure_init(); }
};

class gpu {
 public:
  // ---- elementwise (include/gpu.h:289-320, 945-1004) ------------------------
  template <value_type T>
  static void add(const storage &A, const storage &B, storage &OUT) {
    arithmetic_<T>(SILGPU_ADD, A, B, OUT);
  }
  template <value_type T>
  static void sub(const storage &A, const storage &B, storage &OUT) {
    arithmetic_<T>(SILGPU_SUB, A, B, OUT);
  }
  template <value_type T>
  static void mul(const storage &A, const storage &B, storage &OUT) {
    arithmetic_<T>(SILGPU_MUL, A, B, OUT);
  }
  template <value_type T>
  static void div(const storage &A, const storage &B, storage &OUT) {
    arithmetic_<T>(SILGPU_DIV, A, B, OUT);
  }
  template <value_type T>
  static void pow(const storage &A, const storage &B, storage &OUT) {
    arithmetic_<T>(SILGPU_POW, A, B, OUT);
  }

  static void sigmoid(const storage &IN, storage &OUT) { unary_(SILGPU_SIGMOID, IN, OUT); }
  static void relu(const storage &IN, storage &OUT) { unary_(SILGPU_RELU, IN, OUT); }

  static void sigmoid_backward(const storage &dout, const storage &x, storage &OUT, size_t n) {
    const float *d = dout.dev_in<float>();
    const float *xv = x.dev_in<float>();
    launched_(silgpu_sigmoid_backward_f32(d, xv, OUT.dev_out<float>(), int64_t(n)),
              "sigmoid_backward");
  }

  static void bias_sigmoid(storage &data, const storage &bias, size_t n, uint32_t cols) {
    const float *b = bias.dev_in<float>();
    launched_(silgpu_bias_sigmoid_f32(data.dev_inout<float>(), b, int64_t(n), int64_t(cols)),
              "bias_sigmoid");
  }

  static void affine(const storage &IN, storage &OUT, size_t n, float scale, float offset) {
    const float *in = IN.dev_in<float>();
    launched_(silgpu_affine_f32(in, OUT.dev_out<float>(), int64_t(n), scale, offset), "affine");
  }

  // ---- reductions (include/gpu.h:323-470, 889-913) --------------------------
  static size_t sum_f32_num_tg(size_t) { return 1; }
  static size_t min_f32_num_tg(size_t) { return 1; }
  static size_t max_f32_num_tg(size_t) { return 1; }

  static size_t sum_f32(const storage &IN, storage &OUT, size_t length) {
    const float *in = IN.dev_in<float>();
    launched_(silgpu_sum_f32(in, int64_t(length), OUT.dev_out<float>()), "sum");
    return 1;
  }
  static size_t min_f32(const storage &IN, storage &OUT, size_t length) {
    const float *in = IN.dev_in<float>();
    launched_(silgpu_min_f32(in, int64_t(length), OUT.dev_out<float>()), "min");
    return 1;
  }
  static size_t max_f32(const storage &IN, storage &OUT, size_t length) {
    const float *in = IN.dev_in<float>();
    launched_(silgpu_max_f32(in, int64_t(length), OUT.dev_out<float>()), "max");
    return 1;
  }

  // Column sums of a [rows, cols] array.  `partial`, `num_row_blocks` and
  // `bm` describe the reference's two-pass scheme and are ignored: the
  // library sizes its own passes.
  static void sum_axis0_f32(const storage &IN, storage &OUT, size_t rows, size_t cols,
                            const storage & /*partial*/ = {}, size_t /*num_row_blocks*/ = 0,
                            size_t /*bm*/ = 0) {
    sum_axis(IN, OUT, 1, rows, cols);
  }

  // Sum over the middle axis of a contiguous [outer, axis_len, inner] array
  // (no reference counterpart: the reference sums axis != 0 on the host).
  static void sum_axis(const storage &IN, storage &OUT, size_t outer, size_t axis_len,
                       size_t inner) {
    const float *in = IN.dev_in<float>();
    launched_(silgpu_sum_axis_f32(in, int64_t(outer), int64_t(axis_len), int64_t(inner),
                                  OUT.dev_out<float>()),
              "sum_axis");
  }

  static void argmax_f32(const storage &IN, storage &OUT, uint32_t rows, uint32_t cols) {
    const float *in = IN.dev_in<float>();
    launched_(silgpu_argmax_rows_f32(in, rows, cols, OUT.dev_out<int32_t>()), "argmax");
  }

  // ---- row ops (include/gpu.h:473-501, 916-942) ------------------------------
  static void layer_norm(const storage &IN, storage &OUT, const storage &gamma,
                         const storage &beta, uint32_t rows, uint32_t cols, float eps) {
    const float *in = IN.dev_in<float>();
    const float *g = gamma.dev_in<float>();
    const float *b = beta.dev_in<float>();
    launched_(silgpu_layer_norm_rows_f32(in, OUT.dev_out<float>(), g, b, rows, cols, eps),
              "layer_norm");
  }

  static void softmax(const storage &IN, storage &OUT, uint32_t rows, uint32_t cols) {
    const float *in = IN.dev_in<float>();
    launched_(silgpu_softmax_rows_f32(in, OUT.dev_out<float>(), rows, cols), "softmax");
  }

  // ---- matrix products (include/gpu.h:509-615, 1296-1328) --------------------
  static void sgemm(const storage &A, const storage &B, storage &C, uint32_t M, uint32_t N,
                    uint32_t K, uint32_t lda, uint32_t ldb, bool transA, bool transB) {
    gemm_(A, B, C, M, N, K, lda, ldb, transA, transB, 1, 0, 0, 0, nullptr, 0, SILGPU_EPI_NONE);
  }

  static void sgemm_batched(const storage &A, const storage &B, storage &C, uint32_t M,
                            uint32_t N, uint32_t K, uint32_t lda, uint32_t ldb, uint32_t batch,
                            uint32_t stride_a, uint32_t stride_b, uint32_t stride_c) {
    gemm_(A, B, C, M, N, K, lda, ldb, false, false, batch, stride_a, stride_b, stride_c, nullptr,
          0, SILGPU_EPI_NONE);
  }

  static void sgemm_steel_batched(const storage &A, const storage &B, storage &C, uint32_t M,
                                  uint32_t N, uint32_t K, uint32_t lda, uint32_t ldb,
                                  uint32_t batch, uint32_t stride_a, uint32_t stride_b,
                                  uint32_t stride_c) {
    sgemm_batched(A, B, C, M, N, K, lda, ldb, batch, stride_a, stride_b, stride_c);
  }

  static void sgemv(const storage &x, const storage &B, storage &y, uint32_t N, uint32_t K) {
    const float *xv = x.dev_in<float>();
    const float *b = B.dev_in<float>();
    launched_(silgpu_sgemv(xv, b, N, y.dev_out<float>(), N, K), "sgemv");
  }

  static void sgemm_steel(const storage &A, const storage &B, storage &C, uint32_t M, uint32_t N,
                          uint32_t K, uint32_t lda, uint32_t ldb) {
    sgemm(A, B, C, M, N, K, lda, ldb, false, false);
  }

  static void sgemm_bias_steel(const storage &A, const storage &B, storage &C,
                               const storage &bias, uint32_t bias_len, uint32_t M, uint32_t N,
                               uint32_t K, uint32_t lda, uint32_t ldb) {
    gemm_(A, B, C, M, N, K, lda, ldb, false, false, 1, 0, 0, 0, &bias, bias_len, SILGPU_EPI_BIAS);
  }

  static void sgemm_bias_sigmoid_steel(const storage &A, const storage &B, storage &C,
                                       const storage &bias, uint32_t bias_len, uint32_t M,
                                       uint32_t N, uint32_t K, uint32_t lda, uint32_t ldb) {
    gemm_(A, B, C, M, N, K, lda, ldb, false, false, 1, 0, 0, 0, &bias, bias_len,
          SILGPU_EPI_BIAS_SIGMOID);
  }

  static void dot_f32_ex(const storage &A, const storage &B, storage &OUT, size_t /*phys_A_rows*/,
                         size_t phys_A_cols, size_t /*phys_B_rows*/, size_t phys_B_cols,
                         size_t M, size_t N, size_t K, bool transA, bool transB) {
    gemm_(A, B, OUT, M, N, K, phys_A_cols, phys_B_cols, transA, transB, 1, 0, 0, 0, nullptr, 0,
          SILGPU_EPI_NONE);
  }

  // General form used by the array front end: leading dimensions, batch
  // strides and an epilogue (no single reference counterpart; it covers all
  // of the above).
  static void gemm_(const storage &A, const storage &B, storage &C, size_t M, size_t N, size_t K,
                    size_t lda, size_t ldb, bool transA, bool transB, size_t batch,
                    size_t stride_a, size_t stride_b, size_t stride_c, const storage *bias,
                    size_t bias_len, int epilogue, size_t ldc = 0) {
    const float *a = A.dev_in<float>();
    const float *b = B.dev_in<float>();
    const float *bs = bias ? bias->dev_in<float>() : nullptr;
    launched_(silgpu_sgemm(transA, transB, int64_t(M), int64_t(N), int64_t(K), a, int64_t(lda),
                           int64_t(stride_a), b, int64_t(ldb), int64_t(stride_b),
                           C.dev_out<float>(), int64_t(ldc ? ldc : N), int64_t(stride_c),
                           int64_t(batch), bs, int64_t(bias_len), epilogue),
              "sgemm");
  }

  // silgpu_gemm with its pointers taken from storages: two-level batch
  // strides and the fused scale / residual epilogue of the eval lowering.
  static void gemm(silgpu_gemm_desc d, const storage &A, const storage &B, storage &C,
                   const storage *bias = nullptr, const storage *residual = nullptr) {
    d.A = A.dev_in<float>();
    d.B = B.dev_in<float>();
    d.bias = bias ? bias->dev_in<float>() : nullptr;
    d.residual = residual ? residual->dev_in<float>() : nullptr;
    d.C = C.dev_out<float>();
    launched_(silgpu_gemm(&d), "gemm");
  }

  // Fused attention (the lowering target of sil::eval for
  // batched_dot(softmax(batched_dot(q, k^T) * s), v)).
  static void attention(silgpu_attn_desc d, const storage &Q, const storage &K,
                        const storage &V, storage &O) {
    d.Q = Q.dev_in<float>();
    d.K = K.dev_in<float>();
    d.V = V.dev_in<float>();
    d.O = O.dev_out<float>();
    launched_(silgpu_attention_f32(&d), "attention");
  }

  // Fused elementwise program (the lowering target of sil::eval).
  static void program(const silgpu_program &p, storage &OUT) {
    launched_(silgpu_program_f32(&p, OUT.dev_out<float>()), "program");
  }

  // NHWC input, OHWI weight, NHWC output; stride 1, padding K / 2
  // (include/gpu.h:815-833 of the reference).
  static void conv2d(const storage &input, const storage &weight, storage &output, uint32_t N,
                     uint32_t H, uint32_t W, uint32_t C_in, uint32_t K, uint32_t C_out) {
    const float *in = input.dev_in<float>();
    const float *w = weight.dev_in<float>();
    launched_(silgpu_conv2d_f32(in, w, output.dev_out<float>(), N, H, W, C_in, K, C_out),
              "conv2d");
  }

  static void launched_(int rc, const char *what) {
    detail::check(rc, what);
    gpu_pending_ = true;
  }

 private:
  template <value_type T>
  static void arithmetic_(int op, const storage &A, const storage &B, storage &OUT) {
    if constexpr (std::is_same_v<T, float>) {
      const float *a = A.dev_in<float>();
      const float *b = B.dev_in<float>();
      launched_(silgpu_binary_f32(op, a, int64_t(A.len), b, int64_t(B.len),
                                  OUT.dev_out<float>(), int64_t(OUT.len)),
                "arithmetic");
    } else if constexpr (std::is_same_v<T, int>) {
      const int32_t *a = A.dev_in<int32_t>();
      const int32_t *b = B.dev_in<int32_t>();
      launched_(silgpu_binary_i32(op, a, int64_t(A.len), b, int64_t(B.len),
                                  OUT.dev_out<int32_t>(), int64_t(OUT.len)),
                "arithmetic");
    } else {
      throw std::runtime_error("gpu: arithmetic on bool storage");
    }
  }

  static void unary_(int op, const storage &IN, storage &OUT) {
    const float *in = IN.dev_in<float>();
    launched_(silgpu_unary_f32(op, in, OUT.dev_out<float>(), int64_t(OUT.len)), "unary");
  }
};

// The reference's aliases (include/gpu.h:1372-1373).
using msl = gpu;
using mps = gpu;

// Waits for the GPU and brings every kernel result back to its host mirror,
// so raw storage users can read `data` (include/gpu.h:1375-1377).
inline void synchronize() {
  gpu_context::instance().flush();
  auto &d = detail::dirty_set::instance();
  std::vector<detail::block *> blocks;
  {
    std::lock_guard<std::mutex> lk(d.mu);
    blocks.assign(d.blocks.begin(), d.blocks.end());
  }
  for (auto *b : blocks) b->host_read();
}

}  // namespace sil
