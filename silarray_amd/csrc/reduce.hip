// Reductions: full-array sum / min / max, sum over an axis, per-row argmax.
//
// The reference reduces with one pass that writes up to 256 per-threadgroup
// partials, a blocking host round trip, and a host finish over the partials
// (include/array.h:1535-1545; include/gpu.h:323-354).  Here the whole
// reduction stays on the device and never synchronises with the host:
//   pass 1: each workgroup streams one contiguous chunk of the input with
//           16-byte non-temporal loads (eight in flight per thread) and
//           writes one partial to scratch;
//   pass 2: a small kernel reduces the partials in a fixed order.
// The kernel boundary orders pass 2 after pass 1; an in-kernel "last
// workgroup finishes" scheme needs agent-scope release/acquire fences
// (L2 write-back + invalidate on every XCD), which on MI355X cost far more
// than the second launch.  The fixed partial order makes every result
// deterministic run to run.
//
// All kernels are HBM-bound (4 bytes read per element).
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>

#include "internal.h"

namespace silgpu {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr int kUnroll = 8;          // 16-byte loads in flight per thread
constexpr int kFullBlocks = 2048;   // pass-1 workgroups for a full reduction
constexpr int kFinishLoads = 8;     // partials in flight per thread in pass 2

enum { R_SUM = 0, R_MIN = 1, R_MAX = 2 };

template <int R>
struct racc;
template <>
struct racc<R_SUM> {
  using T = double;  // fp64 accumulation: free on an HBM-bound pass
  __device__ static T init() { return 0.0; }
  __device__ static T add(T a, float x) { return a + static_cast<double>(x); }
  __device__ static T add4(T a, float4 v) {
    return a + (static_cast<double>(v.x) + static_cast<double>(v.y)) +
           (static_cast<double>(v.z) + static_cast<double>(v.w));
  }
  __device__ static T merge(T a, T b) { return a + b; }
};
template <>
struct racc<R_MIN> {
  using T = float;
  __device__ static T init() { return INFINITY; }
  __device__ static T add(T a, float x) { return fminf(a, x); }
  __device__ static T add4(T a, float4 v) { return fminf(fminf(a, fminf(v.x, v.y)), fminf(v.z, v.w)); }
  __device__ static T merge(T a, T b) { return fminf(a, b); }
};
template <>
struct racc<R_MAX> {
  using T = float;
  __device__ static T init() { return -INFINITY; }
  __device__ static T add(T a, float x) { return fmaxf(a, x); }
  __device__ static T add4(T a, float4 v) { return fmaxf(fmaxf(a, fmaxf(v.x, v.y)), fmaxf(v.z, v.w)); }
  __device__ static T merge(T a, T b) { return fmaxf(a, b); }
};

__device__ __forceinline__ float4 load_nt(const float4 *p) {
  float4 v;
  v.x = __builtin_nontemporal_load(&p->x);
  v.y = __builtin_nontemporal_load(&p->y);
  v.z = __builtin_nontemporal_load(&p->z);
  v.w = __builtin_nontemporal_load(&p->w);
  return v;
}

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

// Accumulates float4s [c0, c1) of x4 owned by this thread (stride kBlock).
template <int R>
__device__ __forceinline__ typename racc<R>::T stream4(const float4 *__restrict__ x4,
                                                      int64_t c0, int64_t c1,
                                                      typename racc<R>::T acc) {
  int64_t i = c0 + threadIdx.x;
  for (; i + (kUnroll - 1) * kBlock < c1; i += kUnroll * kBlock) {
    float4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = load_nt(x4 + i + u * kBlock);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc = racc<R>::add4(acc, v[u]);
  }
  for (; i < c1; i += kBlock) acc = racc<R>::add4(acc, load_nt(x4 + i));
  return acc;
}

// Pass 1 of a full reduction.  Workgroup b streams float4s
// [b*chunk4, (b+1)*chunk4) of x4; workgroup 0 also takes the `head` scalars
// before x4 and the `tail` scalars after the last float4.
template <int R>
__global__ __launch_bounds__(kBlock) void reduce_part_k(
    const float *__restrict__ head_ptr, int head, const float4 *__restrict__ x4, int64_t n4,
    int64_t chunk4, const float *__restrict__ tail_ptr, int tail,
    typename racc<R>::T *__restrict__ partial) {
  using T = typename racc<R>::T;
  const int64_t c0 = int64_t(blockIdx.x) * chunk4;
  const int64_t c1 = c0 + chunk4 < n4 ? c0 + chunk4 : n4;
  T acc = stream4<R>(x4, c0, c1, racc<R>::init());
  if (blockIdx.x == 0) {
    if (threadIdx.x < head) acc = racc<R>::add(acc, head_ptr[threadIdx.x]);
    if (threadIdx.x < tail) acc = racc<R>::add(acc, tail_ptr[threadIdx.x]);
  }
  T b = block_merge<R>(acc);
  if (threadIdx.x == 0) partial[blockIdx.x] = b;
}

// Inputs that are not 4-byte aligned (never produced by the allocator; kept
// so every pointer is accepted): scalar loads, same partial layout.
template <int R>
__global__ __launch_bounds__(kBlock) void reduce_part_scalar_k(
    const float *__restrict__ x, int64_t n, int64_t chunk,
    typename racc<R>::T *__restrict__ partial) {
  using T = typename racc<R>::T;
  const int64_t c0 = int64_t(blockIdx.x) * chunk;
  const int64_t c1 = c0 + chunk < n ? c0 + chunk : n;
  T acc = racc<R>::init();
  for (int64_t i = c0 + threadIdx.x; i < c1; i += kBlock) acc = racc<R>::add(acc, x[i]);
  T b = block_merge<R>(acc);
  if (threadIdx.x == 0) partial[blockIdx.x] = b;
}

// Pass 2: one workgroup reduces np partials in a fixed order.
template <int R>
__global__ __launch_bounds__(kBlock) void reduce_finish_k(
    const typename racc<R>::T *__restrict__ partial, int np, float *__restrict__ out) {
  using T = typename racc<R>::T;
  // Groups of kFinishLoads partials per thread are loaded together (one
  // memory latency per group rather than per partial).
  T f = racc<R>::init();
  for (int j0 = threadIdx.x; j0 < np; j0 += kFinishLoads * kBlock) {
    T v[kFinishLoads];
#pragma unroll
    for (int g = 0; g < kFinishLoads; ++g) {
      const int j = j0 + g * kBlock;
      v[g] = j < np ? partial[j] : racc<R>::init();
    }
#pragma unroll
    for (int g = 0; g < kFinishLoads; ++g) f = racc<R>::merge(f, v[g]);
  }
  f = block_merge<R>(f);
  if (threadIdx.x == 0) out[0] = static_cast<float>(f);
}

template <int R>
int launch_reduce(const float *x, int64_t n, float *out) {
  SILGPU_REQUIRE(n >= 0, "reduce: negative n");
  SILGPU_REQUIRE(n > 0 || R == R_SUM, "reduce: min/max of an empty array");
  SILGPU_REQUIRE(out != nullptr && (n == 0 || x != nullptr), "reduce: null pointer");
  SILGPU_CTX(c);
  using T = typename racc<R>::T;
  T *partial = static_cast<T *>(c->partials);
  if (n == 0) return silgpu_fill_u32(out, 0u, 1);  // sum of nothing: +0.0f
  int64_t blocks;
  if (reinterpret_cast<uintptr_t>(x) & 3) {
    blocks = cdiv(n, int64_t(kBlock) * 64);
    if (blocks > kFullBlocks) blocks = kFullBlocks;
    int64_t chunk = cdiv(n, blocks);
    blocks = cdiv(n, chunk);
    reduce_part_scalar_k<R><<<static_cast<unsigned>(blocks), kBlock, 0, c->stream>>>(
        x, n, chunk, partial);
    SILGPU_LAUNCH_CHECK("reduce_part_scalar_k");
  } else {
    int head = static_cast<int>(((16 - (reinterpret_cast<uintptr_t>(x) & 15)) & 15) / 4);
    if (head > n) head = static_cast<int>(n);
    const int64_t n4 = (n - head) / 4;
    const int tail = static_cast<int>(n - head - 4 * n4);
    // Chunks of whole kUnroll*kBlock float4 groups, at most kFullBlocks of them.
    const int64_t group = int64_t(kUnroll) * kBlock;
    int64_t chunk4 = cdiv(cdiv(n4 > 0 ? n4 : 1, kFullBlocks), group) * group;
    blocks = n4 > 0 ? cdiv(n4, chunk4) : 1;
    reduce_part_k<R><<<static_cast<unsigned>(blocks), kBlock, 0, c->stream>>>(
        x, head, reinterpret_cast<const float4 *>(x + head), n4, chunk4, x + head + 4 * n4,
        tail, partial);
    SILGPU_LAUNCH_CHECK("reduce_part_k");
  }
  reduce_finish_k<R><<<1, kBlock, 0, c->stream>>>(partial, static_cast<int>(blocks), out);
  SILGPU_LAUNCH_CHECK("reduce_finish_k");
  return SILGPU_OK;
}

// ---- sum over the last axis (rows of a [rows, cols] view) -------------------
//
// grid = (chunks, rows).  Workgroup (c, r) sums columns
// [c*chunk, min(cols, (c+1)*chunk)) of row r in fp64.  With one chunk it
// writes out[r]; otherwise it writes partial[r*chunks + c] and
// row_sum_finish_k adds each row's partials in chunk order.
__global__ __launch_bounds__(kBlock) void row_sum_k(const float *__restrict__ x, int64_t cols,
                                                    int64_t chunk, bool vec,
                                                    double *__restrict__ partial,
                                                    float *__restrict__ out) {
  const int64_t r = blockIdx.y;
  const float *row = x + r * cols;
  const int64_t c0 = int64_t(blockIdx.x) * chunk;
  const int64_t c1 = c0 + chunk < cols ? c0 + chunk : cols;
  double acc = 0.0;
  if (vec)  // cols % 4 == 0, row 16-byte aligned, chunk % 4 == 0
    acc = stream4<R_SUM>(reinterpret_cast<const float4 *>(row), c0 / 4, c1 / 4, acc);
  else
    for (int64_t i = c0 + threadIdx.x; i < c1; i += kBlock) acc += (double)row[i];
  double b = block_merge<R_SUM>(acc);
  if (threadIdx.x != 0) return;
  if (gridDim.x == 1)
    out[r] = static_cast<float>(b);
  else
    partial[r * gridDim.x + blockIdx.x] = b;
}

// One thread per row adds that row's `chunks` partials in order.
__global__ __launch_bounds__(kBlock) void row_sum_finish_k(const double *__restrict__ partial,
                                                           int64_t rows, int64_t chunks,
                                                           float *__restrict__ out) {
  const int64_t r = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (r >= rows) return;
  double f = 0.0;
#pragma unroll 8
  for (int64_t j = 0; j < chunks; ++j) f += partial[r * chunks + j];
  out[r] = static_cast<float>(f);
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
// (coalesced), each sums its share of the axis.  With splits > 1 the
// partials go to scratch as partial[(o*inner + i)*splits + s] and
// axis_sum_finish_k adds them in split order.
__global__ __launch_bounds__(kBlock) void axis_sum_k(const float *__restrict__ x,
                                                     int64_t axis_len, int64_t inner,
                                                     int64_t per_split,
                                                     double *__restrict__ partial,
                                                     float *__restrict__ out) {
  const int64_t o = blockIdx.z;
  const int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= inner) return;
  const int64_t a0 = int64_t(blockIdx.y) * per_split;
  const int64_t a1 = a0 + per_split < axis_len ? a0 + per_split : axis_len;
  const float *p = x + o * axis_len * inner + i;
  double acc = 0.0;
  int64_t a = a0;
  for (; a + 7 < a1; a += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = __builtin_nontemporal_load(p + (a + u) * inner);
#pragma unroll
    for (int u = 0; u < 8; ++u) acc += (double)v[u];
  }
  for (; a < a1; ++a) acc += (double)p[a * inner];
  if (gridDim.y == 1)
    out[o * inner + i] = static_cast<float>(acc);
  else
    partial[(o * inner + i) * gridDim.y + blockIdx.y] = acc;
}

__global__ __launch_bounds__(kBlock) void axis_sum_finish_k(const double *__restrict__ partial,
                                                            int64_t count, int64_t splits,
                                                            float *__restrict__ out) {
  const int64_t j = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (j >= count) return;
  double f = 0.0;
#pragma unroll 8
  for (int64_t s = 0; s < splits; ++s) f += partial[j * splits + s];
  out[j] = static_cast<float>(f);
}

// ---- argmax per row ---------------------------------------------------------

struct vi {
  float v;
  int32_t pad;
  int64_t i;
};

constexpr int64_t kNoIndex = INT64_MAX;

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
  vi r{sv[0], 0, si[0]};
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = better(r, vi{sv[w], 0, si[w]});
  return r;
}

// Within one thread indices only increase, so a strict > keeps the first
// maximum; NaN is replaced by any number.
__device__ __forceinline__ void scan1(vi &best, float v, int64_t i) {
  if (v > best.v || (best.v != best.v && v == v)) best = vi{v, 0, i};
}

// grid = (chunks, rows); workgroup (c, r) scans columns of chunk c of row r.
__global__ __launch_bounds__(kBlock) void argmax_k(const float *__restrict__ x, int64_t cols,
                                                   int64_t chunk, bool vec,
                                                   vi *__restrict__ partial,
                                                   int32_t *__restrict__ out) {
  const int64_t r = blockIdx.y;
  const float *row = x + r * cols;
  const int64_t c0 = int64_t(blockIdx.x) * chunk;
  const int64_t c1 = c0 + chunk < cols ? c0 + chunk : cols;
  vi best{NAN, 0, kNoIndex};
  if (vec) {
    // Compare each float4 group by its maximum (three fmaxf, which drop
    // NaN) and, only when the group improves on the best so far (a branch
    // the wavefront rarely takes once its maximum has settled), locate the
    // first lane holding that maximum.  Groups are visited in increasing
    // order and replace the best only when strictly larger, so the first
    // maximum of this thread's columns wins, as in scan1.
    const float4 *r4 = reinterpret_cast<const float4 *>(row);
    int64_t i = c0 / 4 + threadIdx.x;
    const int64_t e4 = c1 / 4;
    auto scan4 = [&](const float4 &v, int64_t g) {
      const float m = fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w));
      if (m > best.v || (best.v != best.v && m == m)) {
        const int j = v.x == m ? 0 : v.y == m ? 1 : v.z == m ? 2 : 3;
        best = vi{m, 0, g * 4 + j};
      }
    };
    for (; i + (kUnroll - 1) * kBlock < e4; i += kUnroll * kBlock) {
      float4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) v[u] = load_nt(r4 + i + u * kBlock);
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) scan4(v[u], i + u * kBlock);
    }
    for (; i < e4; i += kBlock) scan4(load_nt(r4 + i), i);
  } else {
    for (int64_t i = c0 + threadIdx.x; i < c1; i += kBlock) scan1(best, row[i], i);
  }
  vi b = block_best(best);
  if (threadIdx.x != 0) return;
  if (gridDim.x == 1)
    out[r] = static_cast<int32_t>(b.i == kNoIndex ? 0 : b.i);
  else
    partial[r * gridDim.x + blockIdx.x] = b;
}

// One workgroup per row merges that row's chunk results.
__global__ __launch_bounds__(kBlock) void argmax_finish_k(const vi *__restrict__ partial,
                                                          int64_t chunks,
                                                          int32_t *__restrict__ out) {
  const int64_t r = blockIdx.x;
  vi f{NAN, 0, kNoIndex};
  for (int64_t j0 = threadIdx.x; j0 < chunks; j0 += kFinishLoads * kBlock) {
    vi v[kFinishLoads];
#pragma unroll
    for (int g = 0; g < kFinishLoads; ++g) {
      const int64_t j = j0 + g * kBlock;
      v[g] = j < chunks ? partial[r * chunks + j] : vi{NAN, 0, kNoIndex};
    }
#pragma unroll
    for (int g = 0; g < kFinishLoads; ++g) f = better(f, v[g]);
  }
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
  vi best{NAN, 0, kNoIndex};
  for (int64_t i = lane; i < cols; i += kWave) scan1(best, row[i], i);
  best = wave_best(best);
  if (lane == 0) out[r] = static_cast<int32_t>(best.i == kNoIndex ? 0 : best.i);
}

// Chunks per row: enough workgroups (rows * chunks ~ 2048) to fill the GPU,
// each chunk >= 16384 elements and a whole number of kUnroll*kBlock float4
// groups; the partials must fit the scratch area.
int64_t chunk_len(int64_t rows, int64_t cols, size_t partial_bytes, int64_t &chunks) {
  int64_t target = 2048 / (rows > 0 ? rows : 1);
  if (target < 1) target = 1;
  int64_t by_size = cols / 16384;
  if (by_size < 1) by_size = 1;
  chunks = target < by_size ? target : by_size;
  while (chunks > 1 && rows * chunks * int64_t(partial_bytes) > int64_t(kPartialBytes)) chunks /= 2;
  const int64_t group = int64_t(kUnroll) * kBlock * 4;
  int64_t chunk = cdiv(cdiv(cols, chunks), group) * group;
  chunks = cdiv(cols, chunk);
  return chunk;
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
  double *partial = static_cast<double *>(c->partials);
  if (inner == 1) {
    const int64_t rows = outer, cols = axis_len;
    if (cols <= 2048) {
      row_sum_wave_k<<<static_cast<unsigned>(cdiv(rows, kWaves)), kBlock, 0, c->stream>>>(
          d_in, rows, cols, d_out);
      SILGPU_LAUNCH_CHECK("row_sum_wave_k");
      return SILGPU_OK;
    }
    if (rows > 65535) {  // grid.y limit: issue batches of rows
      for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
        int64_t nr = rows - r0 < 65535 ? rows - r0 : 65535;
        int rc = silgpu_sum_axis_f32(d_in + r0 * cols, nr, cols, 1, d_out + r0);
        if (rc != SILGPU_OK) return rc;
      }
      return SILGPU_OK;
    }
    const bool vec = cols % 4 == 0 && aligned16(d_in);
    int64_t chunks;
    const int64_t chunk = chunk_len(rows, cols, sizeof(double), chunks);
    dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(rows));
    row_sum_k<<<grid, kBlock, 0, c->stream>>>(d_in, cols, chunk, vec, partial, d_out);
    SILGPU_LAUNCH_CHECK("row_sum_k");
    if (chunks > 1) {
      row_sum_finish_k<<<static_cast<unsigned>(cdiv(rows, kBlock)), kBlock, 0, c->stream>>>(
          partial, rows, chunks, d_out);
      SILGPU_LAUNCH_CHECK("row_sum_finish_k");
    }
    return SILGPU_OK;
  }
  SILGPU_REQUIRE(outer <= 65535, "silgpu_sum_axis_f32: outer %lld exceeds the grid",
                 (long long)outer);
  const int64_t tiles_x = cdiv(inner, kBlock);
  const int64_t tiles = tiles_x * outer;
  int64_t splits = 1;
  if (tiles < 1024) {
    splits = 2048 / tiles;
    int64_t max_by_len = axis_len / 64;  // keep >= 64 rows per split
    if (splits > max_by_len) splits = max_by_len;
    if (splits < 1) splits = 1;
    if (splits > 65535) splits = 65535;
    while (splits > 1 &&
           outer * inner * splits * int64_t(sizeof(double)) > int64_t(kPartialBytes))
      splits /= 2;
  }
  int64_t per_split = cdiv(axis_len, splits);
  splits = cdiv(axis_len, per_split);
  dim3 grid(static_cast<unsigned>(tiles_x), static_cast<unsigned>(splits),
            static_cast<unsigned>(outer));
  axis_sum_k<<<grid, kBlock, 0, c->stream>>>(d_in, axis_len, inner, per_split, partial, d_out);
  SILGPU_LAUNCH_CHECK("axis_sum_k");
  if (splits > 1) {
    const int64_t count = outer * inner;
    axis_sum_finish_k<<<static_cast<unsigned>(cdiv(count, kBlock)), kBlock, 0, c->stream>>>(
        partial, count, splits, d_out);
    SILGPU_LAUNCH_CHECK("axis_sum_finish_k");
  }
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
  const bool vec = cols % 4 == 0 && aligned16(d_in);
  int64_t chunks;
  const int64_t chunk = chunk_len(rows, cols, sizeof(vi), chunks);
  vi *partial = static_cast<vi *>(c->partials);
  dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(rows));
  argmax_k<<<grid, kBlock, 0, c->stream>>>(d_in, cols, chunk, vec, partial, d_out);
  SILGPU_LAUNCH_CHECK("argmax_k");
  if (chunks > 1) {
    argmax_finish_k<<<static_cast<unsigned>(rows), kBlock, 0, c->stream>>>(partial, chunks,
                                                                           d_out);
    SILGPU_LAUNCH_CHECK("argmax_finish_k");
  }
  return SILGPU_OK;
}

}  // extern "C"
