// Internal declarations shared by the HIP translation units of libsilgpu.
// Device code here targets gfx950 (CDNA4) only: 64-lane wavefronts, fp32
// MFMA, 160 KiB LDS per CU.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/silgpu.h"

namespace silgpu {

// ---- error plumbing --------------------------------------------------------

// Records a message for silgpu_last_error() and returns `code`.
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Library context: device, the single stream, scratch for multi-pass
// reductions.
struct context {
  int device = -1;
  hipStream_t stream = nullptr;
  int cu_count = 0;
  int clock_khz = 0;
  // Scratch: per-workgroup partial results (floats / doubles / (value,
  // index) pairs) written by a reduction's first pass and read by its
  // second.  Launches on the one stream run in order, so every call may
  // reuse the whole area.
  void *partials = nullptr;  // kPartialBytes
  // GEMM split-K workspace: grown to the largest request seen, never shrunk.
  void *workspace = nullptr;
  size_t workspace_bytes = 0;
  // Device address of the fixed scratch array of silgpu_gemm_noalloc
  // (kNoAllocScratchBytes), looked up once at init.
  float *noalloc_scratch = nullptr;
  // One-launch reductions: kSlots 64-bit slots, zero between launches.  A
  // workgroup publishes its partial result in its slot (the bitwise
  // complement of the result's 64-bit pattern, so zero means "not written
  // yet"); the workgroup that finishes the reduction waits for the slots it
  // needs, reads them and sets them back to zero before the launch ends.
  uint64_t *slots = nullptr;
  // Failure word in pinned, coherent host memory (fail_host for the host,
  // fail_dev for kernels): a finishing workgroup that gives up waiting for a
  // slot stores kFailSlotWait there.  silgpu_sync and the reduction entry
  // points read it, report the failure and clear the slots again.
  uint32_t *fail_host = nullptr;
  uint32_t *fail_dev = nullptr;
  // Device wall-clock ticks (wall_clock64) per microsecond.
  uint64_t wall_ticks_per_us = 100;
};

constexpr int kSlots = 16384;

// How long a finishing workgroup waits for the partial results it needs
// before it gives up: far beyond any producer's running time (a 64M-element
// reduction runs for ~40 us), far below a stalled-queue watchdog.
constexpr int64_t kSlotWaitUs = 50000;

// Codes a kernel stores into the failure word.
constexpr uint32_t kFailSlotWait = 1;

// What a kernel that publishes or takes slots needs.
struct slot_ctl {
  uint64_t *slots;      // kSlots slots, zero at rest
  uint32_t *fail;       // failure word (host-mapped)
  uint64_t wait_ticks;  // wall-clock ticks a finisher waits before giving up
};

// slot_ctl of the context with the library's wait limit.
inline slot_ctl slot_control(const context *c) {
  return slot_ctl{c->slots, c->fail_dev, uint64_t(kSlotWaitUs) * c->wall_ticks_per_us};
}

// Reports (and clears) a failure recorded by a kernel, re-zeroing the slots
// after every launch issued so far.  `idle`: the stream has just been
// synchronised, so the clearing is waited for too.
int check_device_failure(context *c, bool idle);

// ---- slots: one 64-bit location per published value, zero at rest ----------
//
// A producer publishes the complement of a value's 64-bit pattern with one
// agent-scope atomic store (never zero unless the value is all ones); a
// consumer in the same launch waits until the slot reads non-zero, takes the
// value and clears the slot, so the area is zero again when the launch ends.
// Each slot is written once and read as a whole, so no fence is needed.
//
// Forward progress: a consumer only waits for producers with a lower
// workgroup index, and producers never wait.  Workgroups are dispatched in
// index order on each XCD (the eight XCDs dispatch independently), so the
// lowest-indexed waiting consumer always has every producer it waits for
// either running, finished, or queued behind workgroups that will finish
// without waiting: every wait ends once the producers have run.  The bound
// below (one deadline per consumer thread, read from the device wall clock)
// only turns a device that breaks this into a reported failure instead of a
// stalled stream.

__device__ __forceinline__ void slot_publish(uint64_t *slot, uint64_t bits) {
  __hip_atomic_store(slot, ~bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t slot_peek(uint64_t *slot) {
  return __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Completes a read started with slot_peek(): waits while the slot reads zero
// (at most until `deadline`, set at this thread's first wait and shared by
// its later ones), clears the slot and returns true with the published bits.
// After the deadline it records kFailSlotWait in the failure word, leaves
// the slot alone (the host clears every slot once the launch has ended) and
// returns false: the caller leaves that partial out and the host reports
// the result as failed.
__device__ __forceinline__ bool slot_take(uint64_t *slot, uint64_t seen, uint64_t &deadline,
                                          const slot_ctl &sc, uint64_t &bits) {
  if (seen == 0) {
    if (deadline == 0) deadline = wall_clock64() + sc.wait_ticks;
    do {
      __builtin_amdgcn_s_sleep(1);
      seen = slot_peek(slot);
    } while (seen == 0 && wall_clock64() < deadline);
    if (seen == 0) {
      __hip_atomic_store(sc.fail, kFailSlotWait, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      return false;
    }
  }
  __hip_atomic_store(slot, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  bits = ~seen;
  return true;
}
// Two floats in one slot.
__device__ __forceinline__ uint64_t pack_f2(float a, float b) {
  return (uint64_t(__float_as_uint(b)) << 32) | __float_as_uint(a);
}
__device__ __forceinline__ float2 unpack_f2(uint64_t v) {
  return make_float2(__uint_as_float(uint32_t(v)), __uint_as_float(uint32_t(v >> 32)));
}

constexpr size_t kPartialBytes = size_t(16) << 20;  // 16 MiB
// Largest y or z extent of a launch grid: batched launches (products,
// attention heads, reduction slices) beyond it are issued in pieces.
constexpr int64_t kMaxGridBatch = 65535;
// Size of the fixed scratch array behind silgpu_gemm_noalloc.
constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;  // 32 MiB

// Makes c->workspace hold at least `bytes` (synchronises the stream before
// replacing a smaller block).
int ensure_workspace(context *c, size_t bytes);

// Returns the initialised context, or nullptr after recording an error.
context *ctx();
// The context if silgpu_init has completed, else nullptr after recording an
// error; never initialises (for entry points that must not allocate).
context *ctx_if_ready();

// Checks a HIP call; on failure records the error and returns SILGPU_ERR_HIP.
#define SILGPU_HIP_CHECK(call)                                                       \
  do {                                                                               \
    hipError_t e_ = (call);                                                          \
    if (e_ != hipSuccess)                                                            \
      return ::silgpu::set_error(SILGPU_ERR_HIP, "%s failed: %s (%s:%d)", #call,     \
                                 hipGetErrorString(e_), __FILE__, __LINE__);         \
  } while (0)

// Checks the launch just issued.
#define SILGPU_LAUNCH_CHECK(name)                                                    \
  do {                                                                               \
    hipError_t e_ = hipGetLastError();                                               \
    if (e_ != hipSuccess)                                                            \
      return ::silgpu::set_error(SILGPU_ERR_HIP, "launch of %s failed: %s", name,    \
                                 hipGetErrorString(e_));                             \
  } while (0)

#define SILGPU_REQUIRE(cond, ...)                                                    \
  do {                                                                               \
    if (!(cond)) return ::silgpu::set_error(SILGPU_ERR_INVALID, __VA_ARGS__);        \
  } while (0)

#define SILGPU_CTX(c)                                                                \
  ::silgpu::context *c = ::silgpu::ctx();                                            \
  if (!c) return SILGPU_ERR_NODEVICE

// Direct convolution (conv.hip) for reductions K*K*C_in <= kConvDirectMaxK:
// NHWC in [M = N*H*W pixels][C_in], OHWI w, NHWC out, stride 1, padding K/2.
constexpr int kConvDirectMaxK = 64;
constexpr int64_t kConvDirectMaxCo = int64_t(65535) * 64;  // grid.y = ceil(C_out / 64) blocks
int conv2d_direct(const float *in, const float *w, float *out, int M, int H, int W, int cin,
                  int K, int Co, hipStream_t s);

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
__device__ __forceinline__ bool aligned16_dev(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---- device helpers ---------------------------------------------------------

constexpr int kWave = 64;

// Register-only exchanges within a wavefront (no LDS round trip).  DPP
// controls act within each row of 16 lanes: quad_perm [1,0,3,2] and [2,3,0,1]
// read lane i ^ 1 and i ^ 2, row_half_mirror lane 7 - i of each group of 8,
// row_mirror lane 15 - i of the row.
constexpr int kDppQuadXor1 = 0xB1, kDppQuadXor2 = 0x4E, kDppHalfMirror = 0x141,
              kDppRowMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp_mov(double v) {
  return __hiloint2double(__builtin_amdgcn_mov_dpp(__double2hiint(v), CTRL, 0xF, 0xF, false),
                          __builtin_amdgcn_mov_dpp(__double2loint(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_value(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ double lane_value(double v, int lane) {
  return __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(v), lane),
                          __builtin_amdgcn_readlane(__double2loint(v), lane));
}

// All-reduce over the 64 lanes of a wavefront, every lane active.  After the
// four DPP steps each lane's value covers its whole row of 16 lanes (the
// steps pair lanes across 2, 4, 8 and 16); the rows then combine in a fixed
// order from lanes 0, 16, 32 and 48 (scalar reads), so every lane returns the
// same value.
template <typename T, typename F>
__device__ __forceinline__ T wave_allreduce(T v, F op) {
  v = op(v, dpp_mov<kDppQuadXor1>(v));
  v = op(v, dpp_mov<kDppQuadXor2>(v));
  v = op(v, dpp_mov<kDppHalfMirror>(v));
  v = op(v, dpp_mov<kDppRowMirror>(v));
  return op(op(lane_value(v, 0), lane_value(v, 16)), op(lane_value(v, 32), lane_value(v, 48)));
}

// op over lanes i and i ^ 16 (ROWS = 16) or i and i ^ 32 (ROWS = 32) through
// gfx950's v_permlane16_swap / v_permlane32_swap with v as both operands: the
// two results hold, on both lanes of each pair, the pair's lower- and
// upper-half values, so both lanes compute op(lower, upper) and agree.
template <int ROWS, typename F>
__device__ __forceinline__ float pair_reduce(float v, F op) {
  static_assert(ROWS == 16 || ROWS == 32, "lane distance 16 or 32");
  const unsigned u = __float_as_uint(v);
  if constexpr (ROWS == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
}

// Reductions across the 64 lanes of a wavefront (every lane active); every
// lane returns the result.
struct add_op {
  template <typename T>
  __device__ T operator()(T a, T b) const { return a + b; }
};
__device__ __forceinline__ float wave_sum(float v) { return wave_allreduce(v, add_op{}); }
__device__ __forceinline__ double wave_sum(double v) { return wave_allreduce(v, add_op{}); }
__device__ __forceinline__ float wave_max(float v) {
  return wave_allreduce(v, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ float wave_min(float v) {
  return wave_allreduce(v, [](float a, float b) { return fminf(a, b); });
}

__device__ __forceinline__ float sigmoidf_dev(float x) { return 1.0f / (1.0f + expf(-x)); }

// 16-byte loads and stores; NT: non-temporal (streaming) accesses, for data
// touched once and too large to be served from the caches by a consumer.
// A copy on MI355X reaches 6.5 TB/s with both non-temporal against 5.95 TB/s
// with neither.
template <bool NT>
__device__ __forceinline__ float4 ld4(const float4 *p) {
  if constexpr (NT) {
    float4 v;
    v.x = __builtin_nontemporal_load(&p->x);
    v.y = __builtin_nontemporal_load(&p->y);
    v.z = __builtin_nontemporal_load(&p->z);
    v.w = __builtin_nontemporal_load(&p->w);
    return v;
  } else {
    return *p;
  }
}
template <bool NT>
__device__ __forceinline__ void st4(float4 *p, float4 v) {
  if constexpr (NT) {
    __builtin_nontemporal_store(v.x, &p->x);
    __builtin_nontemporal_store(v.y, &p->y);
    __builtin_nontemporal_store(v.z, &p->z);
    __builtin_nontemporal_store(v.w, &p->w);
  } else {
    *p = v;
  }
}

// Streaming kernels switch to non-temporal accesses from this many bytes per
// operand (half the 256 MiB Infinity Cache: smaller results are likely to
// be read again from the cache by the next kernel of a graph).
constexpr int64_t kStreamBytes = int64_t(128) << 20;

}  // namespace silgpu
