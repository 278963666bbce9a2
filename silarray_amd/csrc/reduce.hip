// Reductions: full-array sum / min / max, sum over an axis, per-row argmax.
//
// The reference reduces with one pass that writes up to 256 per-threadgroup
// partials, a blocking host round trip, and a host finish over the partials
// (include/array.h:1535-1545; include/gpu.h:323-354).  Here the whole
// reduction is one launch that never synchronises with the host:
//   - each workgroup streams one contiguous chunk of the input with 16-byte
//     non-temporal loads (eight in flight per thread) and reduces it;
//   - every workgroup but the last publishes its partial in a 64-bit slot
//     (one agent-scope atomic store of the value's complement, so a slot
//     reads zero until it is written);
//   - the last workgroup, which the dispatcher starts after all the others,
//     reduces its own chunk, then reads every slot -- waiting on any that
//     still reads zero -- in a fixed order, clears them and writes the
//     result.
// Each slot is one atomic location written once, so the finisher needs no
// fence: it sees either zero or the whole value.  A release/acquire "last
// workgroup" handoff would need L2 write-back and invalidate on every XCD;
// a second launch (the earlier design) costs ~2 us of launch gap and cache
// maintenance, 5% of a 64M-element reduction.  The fixed partial order makes
// every result deterministic run to run.
//
// All kernels are HBM-bound (4 bytes read per element).
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <vector>

#include "internal.h"

namespace silgpu {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr int kUnroll = 8;          // 16-byte loads in flight per thread
constexpr int kFullBlocks = 1024;   // workgroups of a full reduction (measured best
                                    // of 256..4096 at 64M elements)
constexpr int kFinishLoads = 8;     // slots in flight per thread in the finish
enum { R_SUM = 0, R_MIN = 1, R_MAX = 2 };

template <int R>
struct racc;
template <>
struct racc<R_SUM> {
  using T = double;  // fp64 accumulation: free on an HBM-bound pass
  // A partial sum is never the all-ones pattern: a NaN from the data keeps
  // a float payload (low 29 bits zero), and arithmetic NaNs are canonical.
  __device__ static uint64_t pack(T v) { return uint64_t(__double_as_longlong(v)); }
  __device__ static T unpack(uint64_t b) { return __longlong_as_double((long long)b); }
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
  __device__ static uint64_t pack(T v) { return uint64_t(__float_as_uint(v)); }
  __device__ static T unpack(uint64_t b) { return __uint_as_float(uint32_t(b)); }
  __device__ static T init() { return INFINITY; }
  __device__ static T add(T a, float x) { return fminf(a, x); }
  __device__ static T add4(T a, float4 v) { return fminf(fminf(a, fminf(v.x, v.y)), fminf(v.z, v.w)); }
  __device__ static T merge(T a, T b) { return fminf(a, b); }
};
template <>
struct racc<R_MAX> {
  using T = float;
  __device__ static uint64_t pack(T v) { return uint64_t(__float_as_uint(v)); }
  __device__ static T unpack(uint64_t b) { return __uint_as_float(uint32_t(b)); }
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
  using T = typename racc<R>::T;
  return wave_allreduce(v, [](T a, T b) { return racc<R>::merge(a, b); });
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

// The last workgroup's finish: partial g of the G workgroups is slot g for
// g < G - 1 and `own` for g = G - 1, merged in a fixed order (thread t takes
// g = t, t + kBlock, ..., kFinishLoads of them in flight), then across the
// workgroup.
template <int R>
__device__ __forceinline__ void finish_full(typename racc<R>::T own, const slot_ctl &sc, int G,
                                            float *__restrict__ out) {
  using T = typename racc<R>::T;
  T f = racc<R>::init();
  uint64_t deadline = 0;
  for (int j0 = threadIdx.x; j0 < G; j0 += kFinishLoads * kBlock) {
    uint64_t seen[kFinishLoads];
#pragma unroll
    for (int g = 0; g < kFinishLoads; ++g) {
      const int j = j0 + g * kBlock;
      seen[g] = j < G - 1 ? slot_peek(sc.slots + j) : 0;
    }
#pragma unroll
    for (int g = 0; g < kFinishLoads; ++g) {
      const int j = j0 + g * kBlock;
      T v = racc<R>::init();
      uint64_t bits;
      if (j < G - 1) {
        if (slot_take(sc.slots + j, seen[g], deadline, sc, bits)) v = racc<R>::unpack(bits);
      } else if (j == G - 1) {
        v = own;
      }
      f = racc<R>::merge(f, v);
    }
  }
  f = block_merge<R>(f);
  if (threadIdx.x == 0) out[0] = static_cast<float>(f);
}

// A full reduction in one launch.  Workgroup b streams float4s
// [b*chunk4, (b+1)*chunk4) of x4; workgroup 0 also takes the `head` scalars
// before x4 and the `tail` scalars after the last float4.
template <int R>
__global__ __launch_bounds__(kBlock) void reduce_k(
    const float *__restrict__ head_ptr, int head, const float4 *__restrict__ x4, int64_t n4,
    int64_t chunk4, const float *__restrict__ tail_ptr, int tail, slot_ctl sc,
    float *__restrict__ out) {
  using T = typename racc<R>::T;
  const int64_t c0 = int64_t(blockIdx.x) * chunk4;
  const int64_t c1 = c0 + chunk4 < n4 ? c0 + chunk4 : n4;
  T acc = stream4<R>(x4, c0, c1, racc<R>::init());
  if (blockIdx.x == 0) {
    if (threadIdx.x < head) acc = racc<R>::add(acc, head_ptr[threadIdx.x]);
    if (threadIdx.x < tail) acc = racc<R>::add(acc, tail_ptr[threadIdx.x]);
  }
  const T b = block_merge<R>(acc);
  const int G = gridDim.x;
  if (blockIdx.x != G - 1) {
    if (threadIdx.x == 0) slot_publish(sc.slots + blockIdx.x, racc<R>::pack(b));
    return;
  }
  finish_full<R>(b, sc, G, out);
}

// Inputs that are not 4-byte aligned (never produced by the allocator; kept
// so every pointer is accepted): scalar loads, same slots and finish.
template <int R>
__global__ __launch_bounds__(kBlock) void reduce_scalar_k(const float *__restrict__ x, int64_t n,
                                                          int64_t chunk, slot_ctl sc,
                                                          float *__restrict__ out) {
  using T = typename racc<R>::T;
  const int64_t c0 = int64_t(blockIdx.x) * chunk;
  const int64_t c1 = c0 + chunk < n ? c0 + chunk : n;
  T acc = racc<R>::init();
  for (int64_t i = c0 + threadIdx.x; i < c1; i += kBlock) acc = racc<R>::add(acc, x[i]);
  const T b = block_merge<R>(acc);
  const int G = gridDim.x;
  if (blockIdx.x != G - 1) {
    if (threadIdx.x == 0) slot_publish(sc.slots + blockIdx.x, racc<R>::pack(b));
    return;
  }
  finish_full<R>(b, sc, G, out);
}

template <int R>
int launch_reduce(const float *x, int64_t n, float *out) {
  SILGPU_REQUIRE(n >= 0, "reduce: negative n");
  SILGPU_REQUIRE(n > 0 || R == R_SUM, "reduce: min/max of an empty array");
  SILGPU_REQUIRE(out != nullptr && (n == 0 || x != nullptr), "reduce: null pointer");
  SILGPU_CTX(c);
  if (int rc = check_device_failure(c, false)) return rc;
  if (n == 0) return silgpu_fill_u32(out, 0u, 1);  // sum of nothing: +0.0f
  int64_t blocks;
  static_assert(kFullBlocks <= kSlots, "a full reduction's partials need a slot each");
  if (reinterpret_cast<uintptr_t>(x) & 3) {
    blocks = cdiv(n, int64_t(kBlock) * 64);
    if (blocks > kFullBlocks) blocks = kFullBlocks;
    int64_t chunk = cdiv(n, blocks);
    blocks = cdiv(n, chunk);
    reduce_scalar_k<R><<<static_cast<unsigned>(blocks), kBlock, 0, c->stream>>>(
        x, n, chunk, slot_control(c), out);
    SILGPU_LAUNCH_CHECK("reduce_scalar_k");
  } else {
    int head = static_cast<int>(((16 - (reinterpret_cast<uintptr_t>(x) & 15)) & 15) / 4);
    if (head > n) head = static_cast<int>(n);
    const int64_t n4 = (n - head) / 4;
    const int tail = static_cast<int>(n - head - 4 * n4);
    // Chunks of whole kUnroll*kBlock float4 groups, at most kFullBlocks of them.
    const int64_t group = int64_t(kUnroll) * kBlock;
    int64_t chunk4 = cdiv(cdiv(n4 > 0 ? n4 : 1, kFullBlocks), group) * group;
    blocks = n4 > 0 ? cdiv(n4, chunk4) : 1;
    reduce_k<R><<<static_cast<unsigned>(blocks), kBlock, 0, c->stream>>>(
        x, head, reinterpret_cast<const float4 *>(x + head), n4, chunk4, x + head + 4 * n4,
        tail, slot_control(c), out);
    SILGPU_LAUNCH_CHECK("reduce_k");
  }
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

// (value, column) of a candidate maximum.  Columns fit int32 (checked at
// the entry point), so the pair is two registers and one 64-bit slot.
struct vi {
  float v;
  int32_t i;
};

constexpr int32_t kNoIndex = INT32_MAX;  // above every column index

// Larger value wins; equal values keep the smaller index; NaN never wins.
__device__ __forceinline__ vi better(vi a, vi b) {
  bool take_b = (b.v > a.v) || (b.v == a.v && b.i < a.i) || (a.v != a.v && b.v == b.v);
  return take_b ? b : a;
}

// The wave's best (value, index) in every lane, as wave_allreduce: four DPP
// steps per 16-lane row, then the rows from lanes 0, 16, 32 and 48.  A lane
// holds a NaN only as {NaN, kNoIndex}, so `better` selects by one total order
// (value, then smaller index) and the pairing does not change the result.
template <int CTRL>
__device__ __forceinline__ vi dpp_vi(vi x) {
  return vi{dpp_mov<CTRL>(x.v), __builtin_amdgcn_mov_dpp(x.i, CTRL, 0xF, 0xF, false)};
}
__device__ __forceinline__ vi wave_best(vi x) {
  x = better(x, dpp_vi<kDppQuadXor1>(x));
  x = better(x, dpp_vi<kDppQuadXor2>(x));
  x = better(x, dpp_vi<kDppHalfMirror>(x));
  x = better(x, dpp_vi<kDppRowMirror>(x));
  const auto at = [&](int l) { return vi{lane_value(x.v, l), __builtin_amdgcn_readlane(x.i, l)}; };
  return better(better(at(0), at(16)), better(at(32), at(48)));
}

__device__ __forceinline__ vi block_best(vi x) {
  __shared__ float sv[kWaves];
  __shared__ int32_t si[kWaves];
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

// Within one thread indices only increase, so a strict > keeps the first
// maximum; NaN is replaced by any number.
__device__ __forceinline__ void scan1(vi &best, float v, int64_t i) {
  if (v > best.v || (best.v != best.v && v == v)) best = vi{v, static_cast<int32_t>(i)};
}

// A (value, index) pair in one slot: the index (>= 0) in the high word, the
// value's bits in the low word.  The high word is never all ones, so no
// packed pair is.
__device__ __forceinline__ uint64_t pack_vi(vi x) {
  return (uint64_t(uint32_t(x.i)) << 32) | __float_as_uint(x.v);
}
__device__ __forceinline__ vi unpack_vi(uint64_t b) {
  return vi{__uint_as_float(uint32_t(b)), int32_t(uint32_t(b >> 32))};
}

// grid = (chunks, rows); workgroup (c, r) scans columns of chunk c of row r.
// With one chunk it writes out[r]; otherwise chunks 0..chunks-2 publish their
// (value, index) in slots r*chunks + c and the last chunk of the row, which
// the dispatcher starts after the row's other chunks, merges them in chunk
// order and writes out[r].
__global__ __launch_bounds__(kBlock) void argmax_k(const float *__restrict__ x, int64_t cols,
                                                   int64_t chunk, bool vec, slot_ctl sc,
                                                   int32_t *__restrict__ out) {
  const int64_t r = blockIdx.y;
  const float *row = x + r * cols;
  const int64_t c0 = int64_t(blockIdx.x) * chunk;
  const int64_t c1 = c0 + chunk < cols ? c0 + chunk : cols;
  vi best{NAN, kNoIndex};
  if (vec) {
    // A thread scans batches of kUnroll float4 groups (kUnroll * kBlock
    // apart).  Each batch is reduced to its maximum (fmaxf drops NaN) and
    // compared once with the best so far; a batch that is strictly larger
    // (or the first batch with a number) becomes the best and is kept in
    // registers, and the column is located in the kept batch only after the
    // scan -- the first element equal to the best, which is the first
    // maximum of the thread's columns since batches are visited in order.
    // Walking an improving batch inside the loop instead (the loop then
    // carries the column search) measured 5% slower than a plain max scan;
    // keeping the batch costs 1%.
    const float4 *r4 = reinterpret_cast<const float4 *>(row);
    int64_t i = c0 / 4 + threadIdx.x;
    const int64_t e4 = c1 / 4;
    float4 keep[kUnroll];
    int64_t keep_i = -1;
    for (; i + (kUnroll - 1) * kBlock < e4; i += kUnroll * kBlock) {
      float4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) v[u] = load_nt(r4 + i + u * kBlock);
      // All loads issued before the first use (left to itself the scheduler
      // starts the maxima after two loads and waits there).
      __builtin_amdgcn_sched_barrier(0);
      float m = fmaxf(fmaxf(v[0].x, v[0].y), fmaxf(v[0].z, v[0].w));
#pragma unroll
      for (int u = 1; u < kUnroll; ++u)
        m = fmaxf(m, fmaxf(fmaxf(v[u].x, v[u].y), fmaxf(v[u].z, v[u].w)));
      if (m > best.v || (best.v != best.v && m == m)) {
        best.v = m;
        keep_i = i;
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) keep[u] = v[u];
      }
    }
    if (keep_i >= 0) {
      // the first element of the kept batch equal to its maximum
      int64_t col = 0;
#pragma unroll
      for (int u = kUnroll - 1; u >= 0; --u) {
        const float4 w = keep[u];
        const int j = w.x == best.v ? 0 : w.y == best.v ? 1 : w.z == best.v ? 2
                    : w.w == best.v ? 3 : -1;
        if (j >= 0) col = (keep_i + int64_t(u) * kBlock) * 4 + j;
      }
      best.i = static_cast<int32_t>(col);
    }
    // the columns after the last whole batch, group by group
    for (; i < e4; i += kBlock) {
      const float4 v = load_nt(r4 + i);
      const float m = fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w));
      if (m > best.v || (best.v != best.v && m == m)) {
        const int j = v.x == m ? 0 : v.y == m ? 1 : v.z == m ? 2 : 3;
        best = vi{m, static_cast<int32_t>(i * 4 + j)};
      }
    }
  } else {
    for (int64_t i = c0 + threadIdx.x; i < c1; i += kBlock) scan1(best, row[i], i);
  }
  const vi b = block_best(best);
  const int64_t chunks = gridDim.x;
  if (chunks == 1) {
    if (threadIdx.x == 0) out[r] = b.i == kNoIndex ? 0 : b.i;
    return;
  }
  uint64_t *row_slots = sc.slots + r * chunks;
  if (blockIdx.x != chunks - 1) {
    if (threadIdx.x == 0) slot_publish(row_slots + blockIdx.x, pack_vi(b));
    return;
  }
  // The row's finish, in chunk order (thread t takes chunks t, t + kBlock, ...).
  vi f{NAN, kNoIndex};
  uint64_t deadline = 0;
  for (int64_t j0 = threadIdx.x; j0 < chunks; j0 += kFinishLoads * kBlock) {
    uint64_t seen[kFinishLoads];
#pragma unroll
    for (int g = 0; g < kFinishLoads; ++g) {
      const int64_t j = j0 + g * kBlock;
      seen[g] = j < chunks - 1 ? slot_peek(row_slots + j) : 0;
    }
#pragma unroll
    for (int g = 0; g < kFinishLoads; ++g) {
      const int64_t j = j0 + g * kBlock;
      vi v{NAN, kNoIndex};
      uint64_t bits;
      if (j < chunks - 1) {
        if (slot_take(row_slots + j, seen[g], deadline, sc, bits)) v = unpack_vi(bits);
      } else if (j == chunks - 1) {
        v = b;
      }
      f = better(f, v);
    }
  }
  f = block_best(f);
  if (threadIdx.x == 0) out[r] = f.i == kNoIndex ? 0 : f.i;
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
  for (int64_t i = lane; i < cols; i += kWave) scan1(best, row[i], i);
  best = wave_best(best);
  if (lane == 0) out[r] = best.i == kNoIndex ? 0 : best.i;
}

// Chunks per row: enough workgroups (rows * chunks ~ `total`) to fill the
// GPU, each chunk >= 16384 elements and a whole number of kUnroll*kBlock
// float4 groups; the partials must fit the scratch area (row sums) and
// rows * chunks the slots (argmax).
int64_t chunk_len(int64_t rows, int64_t cols, size_t partial_bytes, int64_t &chunks,
                  int64_t total = 2048) {
  int64_t target = total / (rows > 0 ? rows : 1);
  if (target < 1) target = 1;
  int64_t by_size = cols / 16384;
  if (by_size < 1) by_size = 1;
  chunks = target < by_size ? target : by_size;
  while (chunks > 1 && (rows * chunks * int64_t(partial_bytes) > int64_t(kPartialBytes) ||
                        rows * chunks > kSlots))
    chunks /= 2;
  const int64_t group = int64_t(kUnroll) * kBlock * 4;
  int64_t chunk = cdiv(cdiv(cols, chunks), group) * group;
  chunks = cdiv(cols, chunk);
  return chunk;
}

// Test hook for the bounded slot wait: workgroup 1 finishes over slots
// [0, nslots) that no producer of this launch writes, so every wait ends at
// its deadline; workgroup 0, when late_ticks > 0, publishes slot 0 once
// late_ticks have passed (a producer later than the finisher's deadline),
// which leaves a stale value behind for the host's clean-up to remove.
// Every wait in it is bounded by the wall clock.
__global__ __launch_bounds__(kBlock) void slot_wait_selftest_k(slot_ctl sc, int nslots,
                                                               uint64_t late_ticks,
                                                               uint32_t *__restrict__ taken) {
  if (blockIdx.x == 0) {
    if (late_ticks > 0 && threadIdx.x == 0) {
      const uint64_t until = wall_clock64() + late_ticks;
      while (wall_clock64() < until) __builtin_amdgcn_s_sleep(127);
      slot_publish(sc.slots, 0x5117ull);
    }
    return;
  }
  uint64_t deadline = 0;
  uint32_t n = 0;
  for (int j = threadIdx.x; j < nslots; j += kBlock) {
    uint64_t bits;
    if (slot_take(sc.slots + j, slot_peek(sc.slots + j), deadline, sc, bits)) ++n;
  }
  if (n) atomicAdd(taken, n);
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
  if (outer > kMaxGridBatch) {  // grid.z limit: issue batches of outer slices
    for (int64_t o0 = 0; o0 < outer; o0 += kMaxGridBatch) {
      const int64_t no = outer - o0 < kMaxGridBatch ? outer - o0 : kMaxGridBatch;
      const int rc =
          silgpu_sum_axis_f32(d_in + o0 * axis_len * inner, no, axis_len, inner, d_out + o0 * inner);
      if (rc != SILGPU_OK) return rc;
    }
    return SILGPU_OK;
  }
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
  if (int rc = check_device_failure(c, false)) return rc;
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
  const int64_t chunk = chunk_len(rows, cols, sizeof(uint64_t), chunks, kFullBlocks);
  if (chunks > 1 && rows * chunks > kSlots)
    return set_error(SILGPU_ERR_INVALID, "silgpu_argmax_rows_f32: %lld x %lld partials exceed "
                     "the %d slots", (long long)rows, (long long)chunks, kSlots);
  dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(rows));
  argmax_k<<<grid, kBlock, 0, c->stream>>>(d_in, cols, chunk, vec, slot_control(c), d_out);
  SILGPU_LAUNCH_CHECK("argmax_k");
  return SILGPU_OK;
}

int silgpu_slot_wait_selftest(int nslots, int64_t wait_us, int64_t late_us,
                              uint32_t *d_taken) {
  SILGPU_REQUIRE(nslots >= 1 && nslots <= kSlots,
                 "silgpu_slot_wait_selftest: nslots %d outside [1, %d]", nslots, kSlots);
  SILGPU_REQUIRE(wait_us >= 1 && wait_us <= 1000000,
                 "silgpu_slot_wait_selftest: wait_us %lld outside [1, 1e6]", (long long)wait_us);
  SILGPU_REQUIRE(late_us >= 0 && late_us <= 2000000,
                 "silgpu_slot_wait_selftest: late_us %lld outside [0, 2e6]", (long long)late_us);
  SILGPU_REQUIRE(d_taken != nullptr, "silgpu_slot_wait_selftest: d_taken is null");
  SILGPU_CTX(c);
  if (int rc = check_device_failure(c, false)) return rc;
  slot_ctl sc = slot_control(c);
  sc.wait_ticks = uint64_t(wait_us) * c->wall_ticks_per_us;
  slot_wait_selftest_k<<<2, kBlock, 0, c->stream>>>(sc, nslots,
                                                    uint64_t(late_us) * c->wall_ticks_per_us,
                                                    d_taken);
  SILGPU_LAUNCH_CHECK("slot_wait_selftest_k");
  return SILGPU_OK;
}

int silgpu_slots_in_use(int64_t *count) {
  SILGPU_REQUIRE(count != nullptr, "silgpu_slots_in_use: count is null");
  SILGPU_CTX(c);
  SILGPU_HIP_CHECK(hipStreamSynchronize(c->stream));
  std::vector<uint64_t> h(kSlots);
  SILGPU_HIP_CHECK(hipMemcpy(h.data(), c->slots, kSlots * sizeof(uint64_t),
                             hipMemcpyDeviceToHost));
  int64_t n = 0;
  for (uint64_t v : h) n += v != 0;
  *count = n;
  return SILGPU_OK;
}

}  // extern "C"
