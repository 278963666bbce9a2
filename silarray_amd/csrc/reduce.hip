// Reductions: full-array sum / min / max, sum over an axis, per-row argmax.
//
// The reference reduces with one pass that writes up to 256 per-threadgroup
// partials, a blocking host round trip, and a host finish over the partials
// (include/array.h:1535-1545; include/gpu.h:323-354).  Here one launch does
// both stages: every workgroup writes its partial to scratch, publishes it
// with an agent-scope fence and a counter increment, and the workgroup that
// arrives last reduces all partials in a fixed order.  The result never
// leaves HBM unless the caller asks, and the fixed order makes results
// deterministic run to run.
//
// All kernels are HBM-bound (4 bytes read per element).  Loads are 16-byte
// vectors, four in flight per thread.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>

#include "internal.h"

namespace silgpu {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr int kUnroll = 4;
constexpr int kMaxFullBlocks = 2048;

enum { R_SUM = 0, R_MIN = 1, R_MAX = 2 };

template <int R>
struct racc;
template <>
struct racc<R_SUM> {
  using T = double;  // fp64 accumulation: free on an HBM-bound pass
  __device__ static T init() { return 0.0; }
  __device__ static T add(T a, float x) { return a + static_cast<double>(x); }
  __device__ static T merge(T a, T b) { return a + b; }
};
template <>
struct racc<R_MIN> {
  using T = float;
  __device__ static T init() { return INFINITY; }
  __device__ static T add(T a, float x) { return fminf(a, x); }
  __device__ static T merge(T a, T b) { return fminf(a, b); }
};
template <>
struct racc<R_MAX> {
  using T = float;
  __device__ static T init() { return -INFINITY; }
  __device__ static T add(T a, float x) { return fmaxf(a, x); }
  __device__ static T merge(T a, T b) { return fmaxf(a, b); }
};

template <int R>
__device__ __forceinline__ typename racc<R>::T wave_merge(typename racc<R>::T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = racc<R>::merge(v, __shfl_xor(v, o, kWave));
  return v;
}

// Workgroup-wide merge; the result is valid in every thread.
template <int R>
__device__ __forceinline__ typename racc<R>::T block_merge(typename racc<R>::T v) {
  using T = typename racc<R>::T;
  __shared__ T red[kWaves];
  v = wave_merge<R>(v);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  __syncthreads();  // red[] may still be read by a previous call
  if (lane == 0) red[wave] = v;
  __syncthreads();
  T r = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = racc<R>::merge(r, red[w]);
  return r;
}

// Returns true in every thread of the workgroup that arrives last at
// `counter` (expected arrivals: `total`), and resets the counter for the
// next kernel on the stream.  Before calling, each workgroup has written its
// partial; the fences publish it across the XCDs' L2s and make the last
// workgroup's later reads see every partial.
__device__ __forceinline__ bool last_arrival(unsigned int *counter, unsigned int total) {
  __shared__ bool last;
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned int prev = atomicAdd(counter, 1u);
    last = (prev == total - 1);
    if (last) atomicExch(counter, 0u);
  }
  __syncthreads();
  if (last) __threadfence();
  return last;
}

// Full reduction of x[0..n).  x4 = x + head (16-byte aligned), n4 float4s
// after the `head` leading scalars; `tail` trailing scalars follow.
template <int R>
__global__ __launch_bounds__(kBlock) void reduce_full_k(
    const float *__restrict__ x, int head, const float4 *__restrict__ x4, int64_t n4,
    const float *__restrict__ tail_ptr, int tail, typename racc<R>::T *__restrict__ partial,
    unsigned int *counter, float *__restrict__ out) {
  using T = typename racc<R>::T;
  T acc = racc<R>::init();
  const int64_t step = int64_t(gridDim.x) * kBlock;
  int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  for (; i + (kUnroll - 1) * step < n4; i += kUnroll * step) {
    float4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = x4[i + u * step];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      acc = racc<R>::add(acc, v[u].x);
      acc = racc<R>::add(acc, v[u].y);
      acc = racc<R>::add(acc, v[u].z);
      acc = racc<R>::add(acc, v[u].w);
    }
  }
  for (; i < n4; i += step) {
    float4 v = x4[i];
    acc = racc<R>::add(acc, v.x);
    acc = racc<R>::add(acc, v.y);
    acc = racc<R>::add(acc, v.z);
    acc = racc<R>::add(acc, v.w);
  }
  if (blockIdx.x == 0) {
    if (threadIdx.x < head) acc = racc<R>::add(acc, x[threadIdx.x]);
    if (threadIdx.x < tail) acc = racc<R>::add(acc, tail_ptr[threadIdx.x]);
  }
  T b = block_merge<R>(acc);
  if (gridDim.x == 1) {
    if (threadIdx.x == 0) out[0] = static_cast<float>(b);
    return;
  }
  if (threadIdx.x == 0) partial[blockIdx.x] = b;
  if (!last_arrival(counter, gridDim.x)) return;
  T f = racc<R>::init();
  for (int j = threadIdx.x; j < static_cast<int>(gridDim.x); j += kBlock)
    f = racc<R>::merge(f, partial[j]);
  f = block_merge<R>(f);
  if (threadIdx.x == 0) out[0] = static_cast<float>(f);
}

template <int R>
int launch_full(const float *x, int64_t n, float *out) {
  SILGPU_REQUIRE(n >= 0, "reduce: negative n");
  SILGPU_REQUIRE(n > 0 || R == R_SUM, "reduce: min/max of an empty array");
  SILGPU_REQUIRE(out != nullptr && (n == 0 || x != nullptr), "reduce: null pointer");
  SILGPU_CTX(c);
  if (n == 0) {
    float zero = 0.0f;
    SILGPU_HIP_CHECK(hipMemcpyAsync(out, &zero, sizeof(float), hipMemcpyHostToDevice,
                                    c->stream));
    SILGPU_HIP_CHECK(hipStreamSynchronize(c->stream));
    return SILGPU_OK;
  }
  int head = static_cast<int>(((16 - (reinterpret_cast<uintptr_t>(x) & 15)) & 15) / 4);
  if (reinterpret_cast<uintptr_t>(x) & 3) head = 0;  // not even 4-aligned: scalar only
  if (head > n) head = static_cast<int>(n);
  int64_t body = n - head;
  int64_t n4 = (reinterpret_cast<uintptr_t>(x) & 3) ? 0 : body / 4;
  int64_t rest = body - n4 * 4;
  const float *tail_ptr = x + head + n4 * 4;
  int64_t g = cdiv(n4, int64_t(kBlock) * kUnroll);
  if (g < 1) g = 1;
  if (g > kMaxFullBlocks) g = kMaxFullBlocks;
  using T = typename racc<R>::T;
  reduce_full_k<R><<<static_cast<unsigned>(g), kBlock, 0, c->stream>>>(
      x, head, reinterpret_cast<const float4 *>(x + head), n4, tail_ptr, static_cast<int>(rest),
      static_cast<T *>(c->partials), c->counters, out);
  SILGPU_LAUNCH_CHECK("reduce_full_k");
  return SILGPU_OK;
}

// Scalar fallback for inputs that are not 4-byte aligned (never produced by
// the allocator; kept so every pointer is accepted).
template <int R>
__global__ __launch_bounds__(kBlock) void reduce_scalar_k(const float *__restrict__ x,
                                                          int64_t n,
                                                          typename racc<R>::T *partial,
                                                          unsigned int *counter,
                                                          float *__restrict__ out) {
  using T = typename racc<R>::T;
  T acc = racc<R>::init();
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * kBlock)
    acc = racc<R>::add(acc, x[i]);
  T b = block_merge<R>(acc);
  if (threadIdx.x == 0) partial[blockIdx.x] = b;
  if (!last_arrival(counter, gridDim.x)) return;
  T f = racc<R>::init();
  for (int j = threadIdx.x; j < static_cast<int>(gridDim.x); j += kBlock)
    f = racc<R>::merge(f, partial[j]);
  f = block_merge<R>(f);
  if (threadIdx.x == 0) out[0] = static_cast<float>(f);
}

template <int R>
int launch_reduce(const float *x, int64_t n, float *out) {
  if (n > 0 && x && (reinterpret_cast<uintptr_t>(x) & 3)) {
    SILGPU_CTX(c);
    int64_t g = cdiv(n, int64_t(kBlock) * 16);
    if (g > kMaxFullBlocks) g = kMaxFullBlocks;
    using T = typename racc<R>::T;
    reduce_scalar_k<R><<<static_cast<unsigned>(g), kBlock, 0, c->stream>>>(
        x, n, static_cast<T *>(c->partials), c->counters, out);
    SILGPU_LAUNCH_CHECK("reduce_scalar_k");
    return SILGPU_OK;
  }
  return launch_full<R>(x, n, out);
}

// ---- sum over the last axis (rows of a [rows, cols] view) -------------------
//
// grid = (chunks, rows).  Workgroup (c, r) sums columns
// [c*chunk, min(cols, (c+1)*chunk)) of row r in fp64.  With one chunk the
// workgroup writes out[r]; otherwise partials go to scratch and the last
// arrival for row r finishes in chunk order.
__global__ __launch_bounds__(kBlock) void row_sum_k(const float *__restrict__ x,
                                                    int64_t cols, int64_t chunk,
                                                    bool vec, double *__restrict__ partial,
                                                    unsigned int *counters,
                                                    float *__restrict__ out) {
  const int64_t r = blockIdx.y;
  const float *row = x + r * cols;
  const int64_t c0 = int64_t(blockIdx.x) * chunk;
  const int64_t c1 = c0 + chunk < cols ? c0 + chunk : cols;
  double acc = 0.0;
  if (vec) {  // cols % 4 == 0, row 16-byte aligned, chunk % 4 == 0
    const float4 *r4 = reinterpret_cast<const float4 *>(row);
    int64_t i = c0 / 4 + threadIdx.x, e4 = c1 / 4;
    for (; i + 3 * kBlock < e4; i += 4 * kBlock) {
      float4 v0 = r4[i], v1 = r4[i + kBlock], v2 = r4[i + 2 * kBlock], v3 = r4[i + 3 * kBlock];
      acc += (double)v0.x + (double)v0.y + (double)v0.z + (double)v0.w;
      acc += (double)v1.x + (double)v1.y + (double)v1.z + (double)v1.w;
      acc += (double)v2.x + (double)v2.y + (double)v2.z + (double)v2.w;
      acc += (double)v3.x + (double)v3.y + (double)v3.z + (double)v3.w;
    }
    for (; i < e4; i += kBlock) {
      float4 v = r4[i];
      acc += (double)v.x + (double)v.y + (double)v.z + (double)v.w;
    }
  } else {
    for (int64_t i = c0 + threadIdx.x; i < c1; i += kBlock) acc += (double)row[i];
  }
  double b = block_merge<R_SUM>(acc);
  if (gridDim.x == 1) {
    if (threadIdx.x == 0) out[r] = static_cast<float>(b);
    return;
  }
  if (threadIdx.x == 0) partial[r * gridDim.x + blockIdx.x] = b;
  if (!last_arrival(counters + r, gridDim.x)) return;
  if (threadIdx.x == 0) {
    double f = 0.0;
    for (unsigned j = 0; j < gridDim.x; ++j) f += partial[r * gridDim.x + j];
    out[r] = static_cast<float>(f);
  }
}

// Short rows: one wavefront per row, four rows per workgroup.
__global__ __launch_bounds__(kBlock) void row_sum_wave_k(const float *__restrict__ x,
                                                         int64_t rows, int64_t cols,
                                                         float *__restrict__ out) {
  const int64_t r = int64_t(blockIdx.x) * kWaves + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (r >= rows) return;
  const float *row = x + r * cols;
  double acc = 0.0;
  for (int64_t i = lane; i < cols; i += kWave) acc += (double)row[i];
  acc = wave_sum(acc);
  if (lane == 0) out[r] = static_cast<float>(acc);
}

// ---- sum over a middle axis: out[o, i] = sum_a x[o, a, i], inner > 1 -------
//
// grid = (ceil(inner / kBlock), splits, outer).  Threads walk inner
// (coalesced), each sums its share of the axis.  With splits > 1 partials
// go to scratch and the last arrival per (o, inner-tile) finishes in split
// order.
__global__ __launch_bounds__(kBlock) void axis_sum_k(const float *__restrict__ x,
                                                     int64_t axis_len, int64_t inner,
                                                     int64_t per_split,
                                                     double *__restrict__ partial,
                                                     unsigned int *counters,
                                                     float *__restrict__ out) {
  const int64_t o = blockIdx.z;
  const int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  const int64_t a0 = int64_t(blockIdx.y) * per_split;
  const int64_t a1 = a0 + per_split < axis_len ? a0 + per_split : axis_len;
  double acc = 0.0;
  if (i < inner) {
    const float *p = x + o * axis_len * inner + i;
    int64_t a = a0;
    for (; a + 3 < a1; a += 4) {
      float v0 = p[a * inner], v1 = p[(a + 1) * inner], v2 = p[(a + 2) * inner],
            v3 = p[(a + 3) * inner];
      acc += (double)v0;
      acc += (double)v1;
      acc += (double)v2;
      acc += (double)v3;
    }
    for (; a < a1; ++a) acc += (double)p[a * inner];
  }
  if (gridDim.y == 1) {
    if (i < inner) out[o * inner + i] = static_cast<float>(acc);
    return;
  }
  const int64_t tile = o * gridDim.x + blockIdx.x;
  const int64_t nsplit = gridDim.y;
  if (i < inner) partial[(tile * nsplit + blockIdx.y) * kBlock + threadIdx.x] = acc;
  if (!last_arrival(counters + tile, gridDim.y)) return;
  if (i < inner) {
    double f = 0.0;
    for (int64_t s = 0; s < nsplit; ++s) f += partial[(tile * nsplit + s) * kBlock + threadIdx.x];
    out[o * inner + i] = static_cast<float>(f);
  }
}

// ---- argmax per row ---------------------------------------------------------

struct vi {
  float v;
  int64_t i;
};

// Larger value wins; equal values keep the smaller index; NaN never wins.
__device__ __forceinline__ vi better(vi a, vi b) {
  bool take_b = (b.v > a.v) || (b.v == a.v && b.i < a.i) || (a.v != a.v && b.v == b.v);
  return take_b ? b : a;
}

__device__ __forceinline__ vi wave_best(vi x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    vi y;
    y.v = __shfl_xor(x.v, o, kWave);
    y.i = __shfl_xor(x.i, o, kWave);
    x = better(x, y);
  }
  return x;
}

__device__ __forceinline__ vi block_best(vi x) {
  __shared__ float sv[kWaves];
  __shared__ int64_t si[kWaves];
  x = wave_best(x);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) {
    sv[wave] = x.v;
    si[wave] = x.i;
  }
  __syncthreads();
  vi r{sv[0], si[0]};
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = better(r, vi{sv[w], si[w]});
  return r;
}

constexpr int64_t kNoIndex = INT64_MAX;

// grid = (chunks, rows); workgroup (c, r) scans columns of chunk c of row r.
__global__ __launch_bounds__(kBlock) void argmax_k(const float *__restrict__ x, int64_t cols,
                                                   int64_t chunk, bool vec,
                                                   vi *__restrict__ partial,
                                                   unsigned int *counters,
                                                   int32_t *__restrict__ out) {
  const int64_t r = blockIdx.y;
  const float *row = x + r * cols;
  const int64_t c0 = int64_t(blockIdx.x) * chunk;
  const int64_t c1 = c0 + chunk < cols ? c0 + chunk : cols;
  vi best{NAN, kNoIndex};
  if (vec) {
    const float4 *r4 = reinterpret_cast<const float4 *>(row);
    for (int64_t i = c0 / 4 + threadIdx.x; i < c1 / 4; i += kBlock) {
      float4 v = r4[i];
      int64_t b = i * 4;
      // Within a thread indices increase, so strict > keeps the first max.
      if (v.x > best.v || (best.v != best.v && v.x == v.x)) best = vi{v.x, b};
      if (v.y > best.v || (best.v != best.v && v.y == v.y)) best = vi{v.y, b + 1};
      if (v.z > best.v || (best.v != best.v && v.z == v.z)) best = vi{v.z, b + 2};
      if (v.w > best.v || (best.v != best.v && v.w == v.w)) best = vi{v.w, b + 3};
    }
  } else {
    for (int64_t i = c0 + threadIdx.x; i < c1; i += kBlock) {
      float v = row[i];
      if (v > best.v || (best.v != best.v && v == v)) best = vi{v, i};
    }
  }
  vi b = block_best(best);
  if (gridDim.x == 1) {
    if (threadIdx.x == 0) out[r] = static_cast<int32_t>(b.i == kNoIndex ? 0 : b.i);
    return;
  }
  if (threadIdx.x == 0) partial[r * gridDim.x + blockIdx.x] = b;
  if (!last_arrival(counters + r, gridDim.x)) return;
  vi f{NAN, kNoIndex};
  for (int64_t j = threadIdx.x; j < gridDim.x; j += kBlock)
    f = better(f, partial[r * gridDim.x + j]);
  f = block_best(f);
  if (threadIdx.x == 0) out[r] = static_cast<int32_t>(f.i == kNoIndex ? 0 : f.i);
}

// Short rows: one wavefront per row.
__global__ __launch_bounds__(kBlock) void argmax_wave_k(const float *__restrict__ x,
                                                        int64_t rows, int64_t cols,
                                                        int32_t *__restrict__ out) {
  const int64_t r = int64_t(blockIdx.x) * kWaves + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (r >= rows) return;
  const float *row = x + r * cols;
  vi best{NAN, kNoIndex};
  for (int64_t i = lane; i < cols; i += kWave) {
    float v = row[i];
    if (v > best.v || (best.v != best.v && v == v)) best = vi{v, i};
  }
  best = wave_best(best);
  if (lane == 0) out[r] = static_cast<int32_t>(best.i == kNoIndex ? 0 : best.i);
}

// Chunks per row so that rows * chunks fills the GPU, each chunk >= 4096
// elements and a multiple of 4 * kBlock.
int64_t pick_chunks(int64_t rows, int64_t cols, int64_t max_chunks) {
  int64_t target = 2048 / (rows > 0 ? rows : 1);
  if (target < 1) target = 1;
  int64_t by_size = cols / 4096;
  if (by_size < 1) by_size = 1;
  int64_t ch = target < by_size ? target : by_size;
  if (ch > max_chunks) ch = max_chunks;
  return ch;
}

}  // namespace
}  // namespace silgpu

using namespace silgpu;

extern "C" {

int silgpu_sum_f32(const float *d_in, int64_t n, float *d_out) {
  return launch_reduce<R_SUM>(d_in, n, d_out);
}
int silgpu_min_f32(const float *d_in, int64_t n, float *d_out) {
  return launch_reduce<R_MIN>(d_in, n, d_out);
}
int silgpu_max_f32(const float *d_in, int64_t n, float *d_out) {
  return launch_reduce<R_MAX>(d_in, n, d_out);
}

int silgpu_sum_axis_f32(const float *d_in, int64_t outer, int64_t axis_len, int64_t inner,
                        float *d_out) {
  SILGPU_REQUIRE(outer >= 0 && axis_len >= 0 && inner >= 0,
                 "silgpu_sum_axis_f32: negative extent");
  if (outer == 0 || inner == 0) return SILGPU_OK;
  SILGPU_REQUIRE(d_out != nullptr, "silgpu_sum_axis_f32: d_out is null");
  SILGPU_CTX(c);
  if (axis_len == 0) return silgpu_fill_u32(d_out, 0u, outer * inner);
  SILGPU_REQUIRE(d_in != nullptr, "silgpu_sum_axis_f32: d_in is null");
  if (inner == 1) {
    const int64_t rows = outer, cols = axis_len;
    if (rows > 65535 && cols > 2048) {  // grid.y limit: issue batches of rows
      for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
        int64_t nr = rows - r0 < 65535 ? rows - r0 : 65535;
        int rc = silgpu_sum_axis_f32(d_in + r0 * cols, nr, cols, 1, d_out + r0);
        if (rc != SILGPU_OK) return rc;
      }
      return SILGPU_OK;
    }
    if (cols <= 2048) {
      row_sum_wave_k<<<static_cast<unsigned>(cdiv(rows, kWaves)), kBlock, 0, c->stream>>>(
          d_in, rows, cols, d_out);
      SILGPU_LAUNCH_CHECK("row_sum_wave_k");
      return SILGPU_OK;
    }
    bool vec = cols % 4 == 0 && aligned16(d_in);
    int64_t chunks = pick_chunks(rows, cols, kCounterCount / (rows > 0 ? rows : 1));
    if (chunks > 1 && rows * chunks * int64_t(sizeof(double)) > int64_t(kPartialBytes))
      chunks = 1;
    int64_t chunk = cdiv(cdiv(cols, chunks), 4 * kBlock) * 4 * kBlock;
    chunks = cdiv(cols, chunk);
    dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(rows));
    row_sum_k<<<grid, kBlock, 0, c->stream>>>(d_in, cols, chunk, vec,
                                              static_cast<double *>(c->partials),
                                              c->counters, d_out);
    SILGPU_LAUNCH_CHECK("row_sum_k");
    return SILGPU_OK;
  }
  SILGPU_REQUIRE(outer <= 65535, "silgpu_sum_axis_f32: outer %lld exceeds the grid",
                 (long long)outer);
  int64_t tiles_x = cdiv(inner, kBlock);
  int64_t tiles = tiles_x * outer;
  int64_t splits = 1;
  if (tiles < 1024) {
    splits = 2048 / tiles;
    int64_t max_by_len = axis_len / 64;  // keep >= 64 rows per split
    if (splits > max_by_len) splits = max_by_len;
    if (splits < 1) splits = 1;
    if (splits > 65535) splits = 65535;
    while (splits > 1 &&
           tiles * splits * kBlock * int64_t(sizeof(double)) > int64_t(kPartialBytes))
      splits /= 2;
    if (tiles > kCounterCount) splits = 1;
  }
  int64_t per_split = cdiv(axis_len, splits);
  splits = cdiv(axis_len, per_split);
  dim3 grid(static_cast<unsigned>(tiles_x), static_cast<unsigned>(splits),
            static_cast<unsigned>(outer));
  axis_sum_k<<<grid, kBlock, 0, c->stream>>>(d_in, axis_len, inner, per_split,
                                             static_cast<double *>(c->partials), c->counters,
                                             d_out);
  SILGPU_LAUNCH_CHECK("axis_sum_k");
  return SILGPU_OK;
}

int silgpu_argmax_rows_f32(const float *d_in, int64_t rows, int64_t cols, int32_t *d_out) {
  SILGPU_REQUIRE(rows >= 0 && cols >= 0, "silgpu_argmax_rows_f32: negative extent");
  if (rows == 0) return SILGPU_OK;
  SILGPU_REQUIRE(d_out != nullptr, "silgpu_argmax_rows_f32: d_out is null");
  SILGPU_REQUIRE(cols <= INT32_MAX, "silgpu_argmax_rows_f32: cols %lld exceed int32",
                 (long long)cols);
  SILGPU_CTX(c);
  if (cols == 0) return silgpu_fill_u32(d_out, 0u, rows);
  SILGPU_REQUIRE(d_in != nullptr, "silgpu_argmax_rows_f32: d_in is null");
  if (cols <= 2048) {
    argmax_wave_k<<<static_cast<unsigned>(cdiv(rows, kWaves)), kBlock, 0, c->stream>>>(
        d_in, rows, cols, d_out);
    SILGPU_LAUNCH_CHECK("argmax_wave_k");
    return SILGPU_OK;
  }
  if (rows > 65535) {  // grid.y limit: issue batches of rows
    for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
      int64_t nr = rows - r0 < 65535 ? rows - r0 : 65535;
      int rc = silgpu_argmax_rows_f32(d_in + r0 * cols, nr, cols, d_out + r0);
      if (rc != SILGPU_OK) return rc;
    }
    return SILGPU_OK;
  }
  bool vec = cols % 4 == 0 && aligned16(d_in);
  int64_t chunks = pick_chunks(rows, cols, kCounterCount / rows);
  if (chunks > 1 && rows * chunks * int64_t(sizeof(vi)) > int64_t(kPartialBytes)) chunks = 1;
  int64_t chunk = cdiv(cdiv(cols, chunks), 4 * kBlock) * 4 * kBlock;
  chunks = cdiv(cols, chunk);
  dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(rows));
  argmax_k<<<grid, kBlock, 0, c->stream>>>(d_in, cols, chunk, vec,
                                           static_cast<vi *>(c->partials), c->counters, d_out);
  SILGPU_LAUNCH_CHECK("argmax_k");
  return SILGPU_OK;
}

}  // extern "C"
