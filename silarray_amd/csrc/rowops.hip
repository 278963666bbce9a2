// Row softmax and row layer_norm over a contiguous [rows, cols] array.
//
// Both are HBM-bound: the optimum is one read and one write of the array
// (8 bytes per element).  A row of up to 16384 floats is held in registers
// by one workgroup (256 or 512 threads x up to 8 float4) or, for rows up to
// 2048, by one wavefront, so the row is read from HBM exactly once and every
// reduction (max, sum, mean, variance) runs over registers with wave64
// butterflies and one LDS exchange.  Inputs are read and outputs written
// with non-temporal (streaming) accesses.  Longer rows take a looped variant
// that reads the row twice.
//
// Numerics: softmax subtracts the row maximum and scales by the reciprocal
// of an fp64-accumulated sum; layer_norm uses the two-pass form of cpu::layer_norm
// (include/cpu.h:352-373): mean, then sum of squared deviations, then
// 1/sqrtf(ss/cols + eps), then *gamma + beta; the sums are fp64 and each
// deviation is taken from the fp64 mean (mean_split), not its float
// rounding.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>

#include "internal.h"

namespace silgpu {
namespace {

// exp(m - M) for a partial sum exponentiated against its own maximum m
// (m <= M); a partial with no finite maximum contributes nothing.
__device__ __forceinline__ float rescale(float m, float M) {
  return m == -INFINITY ? 0.0f : expf(m - M);
}

// The row mean as an unevaluated sum hi + lo of two floats (hi the fp64 mean
// rounded to float, lo the rest), so a deviation x - mean is formed as
// (x - hi) - lo: x - hi is exact wherever x lies within a factor of two of
// the mean (Sterbenz), and the result then carries one float rounding of the
// deviation itself.  Subtracting the float-rounded mean instead errs by up
// to half an ulp of the mean, which for a row whose spread is small against
// its mean (values 1000 +- 0.01) is most of the deviation.
struct mean_split {
  float hi, lo;
  __device__ explicit mean_split(double m)
      : hi(static_cast<float>(m)), lo(static_cast<float>(m - static_cast<double>(hi))) {}
  __device__ float deviation(float x) const { return (x - hi) - lo; }
};

struct fmax_op {
  __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct dsum_op {
  __device__ double operator()(double a, double b) const { return a + b; }
};

// Reductions over a group of NT threads that own one row.  NT == 64: one
// wavefront; NT > 64: the whole workgroup (NT threads) through LDS.
template <int NT>
struct group {
  static constexpr int kWaves = NT / kWave;

  template <typename T, typename F>
  __device__ static T reduce(T v, F op) {
    v = wave_allreduce(v, op);
    if constexpr (NT == kWave) {
      return v;
    } else {
      __shared__ T red[kWaves];
      const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
      __syncthreads();
      if (lane == 0) red[wave] = v;
      __syncthreads();
      T r = red[0];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) r = op(r, red[w]);
      return r;
    }
  }

  // As reduce, for a kernel that makes each SLOT's reduction once: the slot
  // has its own LDS array, so no barrier guards earlier reads of it.
  template <int SLOT, typename T, typename F>
  __device__ static T reduce_once(T v, F op) {
    static_assert(NT == kWave || NT >= 256, "one group per workgroup");
    v = wave_allreduce(v, op);
    if constexpr (NT == kWave) {
      return v;
    } else {
      __shared__ T red[kWaves];
      const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
      if (lane == 0) red[wave] = v;
      __syncthreads();
      T r = red[0];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) r = op(r, red[w]);
      return r;
    }
  }

  // Softmax statistics of the group: each thread holds the maximum m of its
  // values and the sum s of exp(value - m); returns the group's maximum M
  // and sum S of exp(value - M).  One LDS exchange (one barrier): every
  // wave publishes its (max, sum) pair once.  Used once per kernel.
  __device__ static void softmax_stats(float m, double s, float &M, double &S) {
    static_assert(NT == kWave || NT >= 256, "one group per workgroup");
    const float mw = wave_allreduce(m, fmax_op{});
    const double sw = wave_allreduce(s * static_cast<double>(rescale(m, mw)), dsum_op{});
    if constexpr (NT == kWave) {
      M = mw;
      S = sw;
    } else {
      __shared__ float rm[kWaves];
      __shared__ double rs[kWaves];
      const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
      if (lane == 0) {
        rm[wave] = mw;
        rs[wave] = sw;
      }
      __syncthreads();
      float mg = rm[0];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) mg = fmaxf(mg, rm[w]);
      double sg = 0.0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) sg += rs[w] * static_cast<double>(rescale(rm[w], mg));
      M = mg;
      S = sg;
    }
  }
};

// Access modes of a row: scalar (any cols, any alignment), float4 with
// per-slot bounds checks, or float4 over a row that exactly fills the
// NT x V x 4 register tile (no checks, fewer registers).
enum row_mode { kScalar = 0, kVec = 1, kFull = 2 };

// Loads V float4 (vector modes) or 4V scalars of row `row` owned by thread
// `t` of an NT-thread group: element j of slot k is column
// (k*NT + t)*4 + j.  Columns >= cols read as `pad`.  STREAM: the data is read
// once (input rows), so non-temporal loads keep it out of the caches;
// gamma/beta are re-read by every row and use ordinary loads.
template <int NT, int V, int M, bool STREAM = true>
__device__ __forceinline__ void load_row(const float *__restrict__ row, int64_t cols, int t,
                                         float pad, float (&x)[V][4]) {
#pragma unroll
  for (int k = 0; k < V; ++k) {
    int64_t c = (int64_t(k) * NT + t) * 4;
    if constexpr (M != kScalar) {
      if (M == kFull || c < cols) {
        const float4 *q = reinterpret_cast<const float4 *>(row) + c / 4;
        float4 v;
        if constexpr (STREAM) {
          v.x = __builtin_nontemporal_load(&q->x);
          v.y = __builtin_nontemporal_load(&q->y);
          v.z = __builtin_nontemporal_load(&q->z);
          v.w = __builtin_nontemporal_load(&q->w);
        } else {
          v = *q;
        }
        x[k][0] = v.x;
        x[k][1] = v.y;
        x[k][2] = v.z;
        x[k][3] = v.w;
      } else {
        x[k][0] = x[k][1] = x[k][2] = x[k][3] = pad;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) x[k][j] = (c + j < cols) ? row[c + j] : pad;
    }
  }
}

template <int NT, int V, int M>
__device__ __forceinline__ void store_row(float *__restrict__ row, int64_t cols, int t,
                                          const float (&y)[V][4]) {
#pragma unroll
  for (int k = 0; k < V; ++k) {
    int64_t c = (int64_t(k) * NT + t) * 4;
    if constexpr (M != kScalar) {
      if (M == kFull || c < cols) {
        float4 *q = reinterpret_cast<float4 *>(row) + c / 4;
        __builtin_nontemporal_store(y[k][0], &q->x);
        __builtin_nontemporal_store(y[k][1], &q->y);
        __builtin_nontemporal_store(y[k][2], &q->z);
        __builtin_nontemporal_store(y[k][3], &q->w);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (c + j < cols) row[c + j] = y[k][j];
    }
  }
}

// Launch shape: NT threads per row, RPB rows per workgroup: 256 / NT rows of
// one wavefront each for NT == 64, one row per workgroup of NT threads
// otherwise.
template <int NT>
constexpr int rows_per_block() { return NT < 256 ? 256 / NT : 1; }
template <int NT>
constexpr int row_block() { return NT * rows_per_block<NT>(); }

template <int NT, int V, int M>
__global__ __launch_bounds__(row_block<NT>()) void softmax_reg_k(const float *__restrict__ in,
                                                                 float *__restrict__ out,
                                                                 int64_t rows, int64_t cols) {
  constexpr int RPB = rows_per_block<NT>();
  const int64_t r = int64_t(blockIdx.x) * RPB + threadIdx.x / NT;
  const int t = threadIdx.x % NT;
  if (NT == kWave && r >= rows) return;  // whole wavefronts exit together
  const float *src = in + r * cols;
  float x[V][4];
  // A wave-per-row softmax with 32 values per lane raises the wave's issue
  // priority while it issues its row's loads, so a newly started row's loads
  // go out ahead of the exponentials of rows already loaded (4096 x 2048:
  // 12.9 -> 10.6 us); with 4 or fewer float4 per lane (16384 x 1024,
  // 65536 x 256) and with 512-thread rows it measured about 1% slower.
  constexpr bool kLoadPrio = NT == kWave && V >= 8;
  if constexpr (kLoadPrio) __builtin_amdgcn_s_setprio(3);
  load_row<NT, V, M>(src, cols, t, -INFINITY, x);
  if constexpr (kLoadPrio) __builtin_amdgcn_s_setprio(0);
  // Each thread exponentiates against its own maximum m, so the row's
  // maximum and sum meet in one exchange: (m, s) pairs combine as
  // M = max m, S = sum s * exp(m - M).
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < V; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) m = fmaxf(m, x[k][j]);
  // A thread with no finite maximum (padding, -inf entries) exponentiates
  // against 0: its -inf entries give 0 and NaN entries stay NaN.
  const float m_eff = m == -INFINITY ? 0.0f : m;
  double s = 0.0;
#pragma unroll
  for (int k = 0; k < V; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float e = expf(x[k][j] - m_eff);
      x[k][j] = e;
      s += static_cast<double>(e);
    }
  float mr;
  double sr;
  group<NT>::softmax_stats(m, s, mr, sr);
  // One reciprocal per row, then a multiply per element.
  const float inv = 1.0f / static_cast<float>(sr);
  const float c = rescale(m, mr) * inv;
#pragma unroll
  for (int k = 0; k < V; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) x[k][j] = x[k][j] * c;
  store_row<NT, V, M>(out + r * cols, cols, t, x);
}

template <int NT, int V, int M>
__global__ __launch_bounds__(row_block<NT>()) void layer_norm_reg_k(
    const float *__restrict__ in, float *__restrict__ out, const float *__restrict__ gamma,
    const float *__restrict__ beta, int64_t rows, int64_t cols, float eps) {
  constexpr int RPB = rows_per_block<NT>();
  const int64_t r = int64_t(blockIdx.x) * RPB + threadIdx.x / NT;
  const int t = threadIdx.x % NT;
  if (NT == kWave && r >= rows) return;
  float x[V][4];
  // Raised issue priority while the row's loads go out, for workgroup rows
  // only (4096 x 8192: 46.2 -> 45.8 us, 8192 x 4096: 46.2 -> 43.3;
  // wave-per-row rows measured 5% slower with it).
  if constexpr (NT > kWave) __builtin_amdgcn_s_setprio(3);
  load_row<NT, V, M>(in + r * cols, cols, t, 0.0f, x);
  if constexpr (NT > kWave) __builtin_amdgcn_s_setprio(0);
  double s = 0.0;
#pragma unroll
  for (int k = 0; k < V; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) s += static_cast<double>(x[k][j]);
  s = group<NT>::template reduce_once<0>(s, dsum_op{});
  const mean_split mu(s / static_cast<double>(cols));
  double ss = 0.0;
#pragma unroll
  for (int k = 0; k < V; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int64_t c = (int64_t(k) * NT + t) * 4 + j;
      float d = mu.deviation(x[k][j]);
      x[k][j] = d;
      if (M == kFull || c < cols) ss += static_cast<double>(d) * static_cast<double>(d);
    }
  ss = group<NT>::template reduce_once<1>(ss, dsum_op{});
  const float var = static_cast<float>(ss / static_cast<double>(cols));
  const float inv_std = 1.0f / sqrtf(var + eps);
  float g[V][4], b[V][4];
  load_row<NT, V, M, false>(gamma, cols, t, 0.0f, g);
  load_row<NT, V, M, false>(beta, cols, t, 0.0f, b);
#pragma unroll
  for (int k = 0; k < V; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) x[k][j] = (x[k][j] * inv_std) * g[k][j] + b[k][j];
  store_row<NT, V, M>(out + r * cols, cols, t, x);
}

// Rows longer than the register path: one workgroup per row, two reads.
constexpr int kLoopBlock = 256;

__global__ __launch_bounds__(kLoopBlock) void softmax_loop_k(const float *__restrict__ in,
                                                             float *__restrict__ out,
                                                             int64_t cols) {
  const float *src = in + int64_t(blockIdx.x) * cols;
  float *dst = out + int64_t(blockIdx.x) * cols;
  // Online (max, sum) per thread, rescaling the sum when the max grows.
  float m = -INFINITY;
  double s = 0.0;
  for (int64_t c = threadIdx.x; c < cols; c += kLoopBlock) {
    float v = src[c];
    if (v > m) {
      s = s * static_cast<double>(expf(m - v)) + 1.0;
      m = v;
    } else if (v != -INFINITY) {
      // A -inf entry adds exp(-inf) = 0; skipped, so that one seen while m
      // is still -inf does not add exp(-inf - -inf) = NaN.  NaN entries
      // take this branch and make the row NaN.
      s += static_cast<double>(expf(v - m));
    }
  }
  const float gm = group<kLoopBlock>::reduce(m, fmax_op{});
  double part = (m == -INFINITY) ? 0.0 : s * static_cast<double>(expf(m - gm));
  const float sf = static_cast<float>(group<kLoopBlock>::reduce(part, dsum_op{}));
  for (int64_t c = threadIdx.x; c < cols; c += kLoopBlock) dst[c] = expf(src[c] - gm) / sf;
}

__global__ __launch_bounds__(kLoopBlock) void layer_norm_loop_k(
    const float *__restrict__ in, float *__restrict__ out, const float *__restrict__ gamma,
    const float *__restrict__ beta, int64_t cols, float eps) {
  const float *src = in + int64_t(blockIdx.x) * cols;
  float *dst = out + int64_t(blockIdx.x) * cols;
  double s = 0.0;
  for (int64_t c = threadIdx.x; c < cols; c += kLoopBlock) s += static_cast<double>(src[c]);
  s = group<kLoopBlock>::reduce(s, dsum_op{});
  const mean_split mu(s / static_cast<double>(cols));
  double ss = 0.0;
  for (int64_t c = threadIdx.x; c < cols; c += kLoopBlock) {
    float d = mu.deviation(src[c]);
    ss += static_cast<double>(d) * static_cast<double>(d);
  }
  ss = group<kLoopBlock>::reduce(ss, dsum_op{});
  const float inv_std = 1.0f / sqrtf(static_cast<float>(ss / static_cast<double>(cols)) + eps);
  for (int64_t c = threadIdx.x; c < cols; c += kLoopBlock)
    dst[c] = (mu.deviation(src[c]) * inv_std) * gamma[c] + beta[c];
}

// ---- dispatch ---------------------------------------------------------------

struct row_launch {
  int nt;      // threads per row
  int v;       // float4 slots per thread
};

// Register configuration that covers `cols`, or {0,0} for the looped
// kernels.  Rows over 4096 take 512 threads so each thread holds at most
// 8 float4 (measured on [4096, 8192]: 512 x 4 beats 256 x 8 for layer_norm,
// whose gamma/beta otherwise double the register footprint).
row_launch pick(int64_t cols) {
  if (cols <= 256) return {64, 1};
  if (cols <= 512) return {64, 2};
  if (cols <= 1024) return {64, 4};
  if (cols <= 2048) return {64, 8};
  if (cols <= 4096) return {256, 4};
  if (cols <= 8192) return {512, 4};
  if (cols <= 16384) return {512, 8};
  return {0, 0};
}

template <int NT, int V, int M>
void go_softmax(const float *in, float *out, int64_t rows, int64_t cols, hipStream_t s) {
  constexpr int RPB = rows_per_block<NT>();
  softmax_reg_k<NT, V, M><<<static_cast<unsigned>(cdiv(rows, RPB)), row_block<NT>(), 0, s>>>(
      in, out, rows, cols);
}

template <int NT, int V, int M>
void go_ln(const float *in, float *out, const float *g, const float *b, int64_t rows,
           int64_t cols, float eps, hipStream_t s) {
  constexpr int RPB = rows_per_block<NT>();
  layer_norm_reg_k<NT, V, M>
      <<<static_cast<unsigned>(cdiv(rows, RPB)), row_block<NT>(), 0, s>>>(in, out, g, b, rows,
                                                                          cols, eps);
}

#define SILGPU_ROW_DISPATCH(FN, MODE, ...)                                               \
  switch (L.nt * 100 + L.v) {                                                           \
    case 6401: FN<64, 1, MODE>(__VA_ARGS__); break;                                      \
    case 6402: FN<64, 2, MODE>(__VA_ARGS__); break;                                      \
    case 6404: FN<64, 4, MODE>(__VA_ARGS__); break;                                      \
    case 6408: FN<64, 8, MODE>(__VA_ARGS__); break;                                      \
    case 25604: FN<256, 4, MODE>(__VA_ARGS__); break;                                    \
    case 51204: FN<512, 4, MODE>(__VA_ARGS__); break;                                    \
    default: FN<512, 8, MODE>(__VA_ARGS__); break;                                       \
  }

}  // namespace
}  // namespace silgpu

using namespace silgpu;

extern "C" {

int silgpu_softmax_rows_f32(const float *d_in, float *d_out, int64_t rows, int64_t cols) {
  SILGPU_REQUIRE(rows >= 0 && cols >= 0, "silgpu_softmax_rows_f32: negative extent");
  if (rows == 0 || cols == 0) return SILGPU_OK;
  SILGPU_REQUIRE(d_in && d_out, "silgpu_softmax_rows_f32: null pointer");
  SILGPU_REQUIRE(rows <= (int64_t(1) << 31) - 1, "silgpu_softmax_rows_f32: too many rows");
  SILGPU_CTX(c);
  row_launch L = pick(cols);
  if (L.nt == 0) {
    softmax_loop_k<<<static_cast<unsigned>(rows), kLoopBlock, 0, c->stream>>>(d_in, d_out,
                                                                              cols);
    SILGPU_LAUNCH_CHECK("softmax_loop_k");
    return SILGPU_OK;
  }
  const bool vec = cols % 4 == 0 && aligned16(d_in) && aligned16(d_out);
  if (vec && cols == int64_t(L.nt) * L.v * 4) {
    SILGPU_ROW_DISPATCH(go_softmax, kFull, d_in, d_out, rows, cols, c->stream);
  } else if (vec) {
    SILGPU_ROW_DISPATCH(go_softmax, kVec, d_in, d_out, rows, cols, c->stream);
  } else {
    SILGPU_ROW_DISPATCH(go_softmax, kScalar, d_in, d_out, rows, cols, c->stream);
  }
  SILGPU_LAUNCH_CHECK("softmax_reg_k");
  return SILGPU_OK;
}

int silgpu_layer_norm_rows_f32(const float *d_in, float *d_out, const float *d_gamma,
                               const float *d_beta, int64_t rows, int64_t cols, float eps) {
  SILGPU_REQUIRE(rows >= 0 && cols >= 0, "silgpu_layer_norm_rows_f32: negative extent");
  if (rows == 0 || cols == 0) return SILGPU_OK;
  SILGPU_REQUIRE(d_in && d_out && d_gamma && d_beta,
                 "silgpu_layer_norm_rows_f32: null pointer");
  SILGPU_CTX(c);
  row_launch L = pick(cols);
  if (L.nt == 0) {
    layer_norm_loop_k<<<static_cast<unsigned>(rows), kLoopBlock, 0, c->stream>>>(
        d_in, d_out, d_gamma, d_beta, cols, eps);
    SILGPU_LAUNCH_CHECK("layer_norm_loop_k");
    return SILGPU_OK;
  }
  const bool vec = cols % 4 == 0 && aligned16(d_in) && aligned16(d_out) &&
                   aligned16(d_gamma) && aligned16(d_beta);
  if (vec && cols == int64_t(L.nt) * L.v * 4) {
    SILGPU_ROW_DISPATCH(go_ln, kFull, d_in, d_out, d_gamma, d_beta, rows, cols, eps,
                        c->stream);
  } else if (vec) {
    SILGPU_ROW_DISPATCH(go_ln, kVec, d_in, d_out, d_gamma, d_beta, rows, cols, eps,
                        c->stream);
  } else {
    SILGPU_ROW_DISPATCH(go_ln, kScalar, d_in, d_out, d_gamma, d_beta, rows, cols, eps,
                        c->stream);
  }
  SILGPU_LAUNCH_CHECK("layer_norm_reg_k");
  return SILGPU_OK;
}

}  // extern "C"
