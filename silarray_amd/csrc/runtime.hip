// Context, error reporting, pooled device memory, copies and events.
//
// Stands in for the reference's gpu_context (include/gpu.h:49-260: one Metal
// queue, one lazily created command buffer, blocking flush) and its
// unified-memory buffer_pool (include/unified_memory.h:29-62).  On MI355X the
// equivalents are one HIP stream (issue order = execution order, like the
// single command buffer), hipStreamSynchronize for flush, and a size-class
// pool of hipMalloc'd HBM blocks.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstring>
#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "internal.h"

namespace silgpu {

namespace {

thread_local char g_err[512] = "";

// Scratch of silgpu_gemm_noalloc (K-split partial planes, GEMV partials): a
// fixed array in device memory, so that entry point never allocates.  In host
// code the name `scratch` is only a stand-in for the symbol; every host use
// goes through the device address hipGetSymbolAddress returns at init
// (context::noalloc_scratch).  Calls on one device share it, so calls of
// silgpu_gemm_noalloc that overlap in time on one device race.
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

std::mutex g_init_mu;
context g_ctx;
// Set with release once g_ctx is complete; ctx() reads it with acquire, so a
// thread that sees it set also sees the stream and scratch pointers.
std::atomic<bool> g_ready{false};

int init_locked() {
  if (g_ready.load(std::memory_order_relaxed)) return SILGPU_OK;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0)
    return set_error(SILGPU_ERR_NODEVICE, "no HIP device visible (%s)",
                     e == hipSuccess ? "count 0" : hipGetErrorString(e));
  SILGPU_HIP_CHECK(hipSetDevice(0));
  hipDeviceProp_t prop;
  SILGPU_HIP_CHECK(hipGetDeviceProperties(&prop, 0));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return set_error(SILGPU_ERR_UNSUPPORTED,
                     "device 0 is %s; this library is built for gfx950 only",
                     prop.gcnArchName);
  g_ctx.device = 0;
  g_ctx.cu_count = prop.multiProcessorCount;
  g_ctx.clock_khz = prop.clockRate;
  // Default priority on purpose: streams of mixed priority are avoided.
  SILGPU_HIP_CHECK(hipStreamCreateWithFlags(&g_ctx.stream, hipStreamNonBlocking));
  SILGPU_HIP_CHECK(hipMalloc(&g_ctx.partials, kPartialBytes));
  SILGPU_HIP_CHECK(hipMalloc(&g_ctx.slots, kSlots * sizeof(uint64_t)));
  SILGPU_HIP_CHECK(hipMemsetAsync(g_ctx.slots, 0, kSlots * sizeof(uint64_t), g_ctx.stream));
  // The failure word: pinned, coherent host memory, so the host reads what a
  // kernel stored without a copy (a plain load after the stream has synchronised).
  void *fw = nullptr;
  SILGPU_HIP_CHECK(hipHostMalloc(&fw, sizeof(uint32_t), hipHostMallocCoherent | hipHostMallocMapped));
  g_ctx.fail_host = static_cast<uint32_t *>(fw);
  __atomic_store_n(g_ctx.fail_host, 0u, __ATOMIC_RELEASE);
  void *fwd = nullptr;
  SILGPU_HIP_CHECK(hipHostGetDevicePointer(&fwd, fw, 0));
  g_ctx.fail_dev = static_cast<uint32_t *>(fwd);
  int wall_khz = 0;
  SILGPU_HIP_CHECK(hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, 0));
  SILGPU_REQUIRE(wall_khz >= 1000, "init: wall clock rate of %d kHz", wall_khz);
  g_ctx.wall_ticks_per_us = uint64_t(wall_khz) / 1000;
  // With device 0 current: this device's copy of the no-allocation scratch.
  void *sp = nullptr;
  SILGPU_HIP_CHECK(hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)));
  SILGPU_REQUIRE(sp != nullptr, "init: no device address for the scratch array");
  g_ctx.noalloc_scratch = static_cast<float *>(sp);
  SILGPU_HIP_CHECK(hipDeviceSynchronize());
  g_ready.store(true, std::memory_order_release);
  return SILGPU_OK;
}

// ---- size-class pool --------------------------------------------------------

// Size classes: multiples of 256 B up to 64 KiB, then four classes per power
// of two (waste <= 25%).  The reference keeps exact-byte free lists
// (include/unified_memory.h:38-51); classes let nearby sizes share blocks.
size_t size_class(size_t bytes) {
  if (bytes == 0) bytes = 1;
  if (bytes <= 65536) return (bytes + 255) & ~size_t(255);
  size_t p = size_t(1) << (63 - __builtin_clzll(bytes));  // floor pow2
  size_t step = p / 4;
  return (bytes + step - 1) / step * step;
}

struct pool {
  std::mutex mu;
  std::unordered_map<size_t, std::vector<void *>> free_lists;
  std::unordered_map<void *, size_t> live;  // ptr -> class bytes
  size_t in_use = 0;
  size_t cached = 0;
};

pool &the_pool() {
  static pool *p = new pool();  // never destroyed: blocks outlive static dtors
  return *p;
}

// Pinned host blocks (host mirrors of storages), pooled by the same size
// classes: hipHostMalloc'd memory is DMA'd directly (≈57 GB/s each way on
// this platform, against ≈32 GB/s host-to-device and ≈18 GB/s back for
// pageable memory, which the runtime stages through its own buffers).
pool &the_host_pool() {
  static pool *p = new pool();
  return *p;
}

// Device-to-device copy of n16 16-byte slots: a workgroup moves one
// contiguous 32 KiB block, each thread 8 slots strided by the workgroup
// width (all loads issued before the first store), non-temporal both ways.
// On [4096, 8192]-float buffers this shape copied at 6.3 TB/s against
// 5.3 TB/s for hipMemcpyAsync's copy kernel.
constexpr int kCopyBlock = 256;
constexpr int kCopyV = 8;

__global__ __launch_bounds__(kCopyBlock) void copy16_k(const float4 *__restrict__ src,
                                                       float4 *__restrict__ dst, int64_t n16) {
  const int64_t base = int64_t(blockIdx.x) * (kCopyBlock * kCopyV) + threadIdx.x;
  float4 v[kCopyV];
  if (int64_t(blockIdx.x + 1) * (kCopyBlock * kCopyV) <= n16) {
    // Whole blocks without per-slot checks: each store then waits only for
    // its own load.
#pragma unroll
    for (int k = 0; k < kCopyV; ++k) v[k] = ld4<true>(src + base + k * kCopyBlock);
#pragma unroll
    for (int k = 0; k < kCopyV; ++k) st4<true>(dst + base + k * kCopyBlock, v[k]);
    return;
  }
#pragma unroll
  for (int k = 0; k < kCopyV; ++k) {
    const int64_t i = base + int64_t(k) * kCopyBlock;
    if (i < n16) v[k] = ld4<true>(src + i);
  }
#pragma unroll
  for (int k = 0; k < kCopyV; ++k) {
    const int64_t i = base + int64_t(k) * kCopyBlock;
    if (i < n16) st4<true>(dst + i, v[k]);
  }
}

}  // namespace

int set_error(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_err[0] = '\0'; }

int ensure_workspace(context *c, size_t bytes) {
  if (bytes <= c->workspace_bytes) return SILGPU_OK;
  size_t grow = (bytes + (size_t(64) << 20) - 1) & ~((size_t(64) << 20) - 1);  // 64 MiB steps
  SILGPU_HIP_CHECK(hipStreamSynchronize(c->stream));
  if (c->workspace) SILGPU_HIP_CHECK(hipFree(c->workspace));
  c->workspace = nullptr;
  c->workspace_bytes = 0;
  hipError_t e = hipMalloc(&c->workspace, grow);
  if (e != hipSuccess)
    return set_error(SILGPU_ERR_NOMEM, "GEMM workspace of %zu bytes: %s", grow,
                     hipGetErrorString(e));
  c->workspace_bytes = grow;
  return SILGPU_OK;
}

context *ctx() {
  if (g_ready.load(std::memory_order_acquire)) return &g_ctx;
  std::lock_guard<std::mutex> lk(g_init_mu);
  if (init_locked() != SILGPU_OK) return nullptr;
  return &g_ctx;
}

int check_device_failure(context *c, bool idle) {
  const uint32_t f = __atomic_load_n(c->fail_host, __ATOMIC_ACQUIRE);
  if (f == 0) return SILGPU_OK;
  __atomic_store_n(c->fail_host, 0u, __ATOMIC_RELEASE);
  // Zero every slot after the launches issued so far, so a producer that
  // published after its finisher gave up leaves nothing for the next launch.
  int rc = silgpu_fill_u32(c->slots, 0u, int64_t(kSlots) * 2);
  if (rc == SILGPU_OK && idle) {
    hipError_t e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess)
      return set_error(SILGPU_ERR_HIP, "hipStreamSynchronize after a reduction failure: %s",
                       hipGetErrorString(e));
  }
  if (rc != SILGPU_OK) return rc;
  return set_error(SILGPU_ERR_HIP,
                   "a one-launch reduction (sum/min/max/argmax) gave up waiting for a "
                   "workgroup's partial result (failure code %u; the library waits up to %lld us "
                   "before giving up); that result is wrong. The slots have been cleared for "
                   "later calls.",
                   f, (long long)kSlotWaitUs);
}

context *ctx_if_ready() {
  if (g_ready.load(std::memory_order_acquire)) return &g_ctx;
  set_error(SILGPU_ERR_INVALID, "the library is not initialised: call silgpu_init() first");
  return nullptr;
}

}  // namespace silgpu

using namespace silgpu;

extern "C" {

const char *silgpu_last_error(void) { return g_err; }

int silgpu_init(void) {
  std::lock_guard<std::mutex> lk(g_init_mu);
  return init_locked();
}

int silgpu_sync(void) {
  SILGPU_CTX(c);
  SILGPU_HIP_CHECK(hipStreamSynchronize(c->stream));
  return check_device_failure(c, true);
}

int silgpu_device_info(int *cu_count, int *clock_khz, int *lds_bytes, char *arch,
                       size_t arch_len) {
  SILGPU_CTX(c);
  hipDeviceProp_t prop;
  SILGPU_HIP_CHECK(hipGetDeviceProperties(&prop, c->device));
  if (cu_count) *cu_count = prop.multiProcessorCount;
  if (clock_khz) *clock_khz = prop.clockRate;
  if (lds_bytes) *lds_bytes = static_cast<int>(prop.sharedMemPerBlock);
  if (arch && arch_len) {
    std::strncpy(arch, prop.gcnArchName, arch_len - 1);
    arch[arch_len - 1] = '\0';
  }
  return SILGPU_OK;
}

int silgpu_alloc(size_t bytes, void **d_ptr) {
  SILGPU_REQUIRE(d_ptr != nullptr, "silgpu_alloc: d_ptr is null");
  SILGPU_CTX(c);
  (void)c;
  size_t cls = size_class(bytes);
  pool &p = the_pool();
  {
    std::lock_guard<std::mutex> lk(p.mu);
    auto it = p.free_lists.find(cls);
    if (it != p.free_lists.end() && !it->second.empty()) {
      void *ptr = it->second.back();
      it->second.pop_back();
      p.live[ptr] = cls;
      p.in_use += cls;
      p.cached -= cls;
      *d_ptr = ptr;
      return SILGPU_OK;
    }
  }
  void *ptr = nullptr;
  hipError_t e = hipMalloc(&ptr, cls);
  if (e != hipSuccess) {
    // Release cached blocks and retry once before giving up.
    silgpu_pool_trim();
    e = hipMalloc(&ptr, cls);
    if (e != hipSuccess)
      return set_error(SILGPU_ERR_NOMEM, "hipMalloc(%zu) failed: %s", cls,
                       hipGetErrorString(e));
  }
  std::lock_guard<std::mutex> lk(p.mu);
  p.live[ptr] = cls;
  p.in_use += cls;
  *d_ptr = ptr;
  return SILGPU_OK;
}

int silgpu_free(void *d_ptr) {
  if (!d_ptr) return SILGPU_OK;
  pool &p = the_pool();
  std::lock_guard<std::mutex> lk(p.mu);
  auto it = p.live.find(d_ptr);
  if (it == p.live.end())
    return set_error(SILGPU_ERR_INVALID, "silgpu_free: %p was not allocated by silgpu_alloc",
                     d_ptr);
  size_t cls = it->second;
  p.live.erase(it);
  p.in_use -= cls;
  p.cached += cls;
  // Work already issued on the stream may still read this block; any later
  // user is ordered after it on the same stream, so reuse is safe.
  p.free_lists[cls].push_back(d_ptr);
  return SILGPU_OK;
}

int silgpu_pool_trim(void) {
  SILGPU_CTX(c);
  SILGPU_HIP_CHECK(hipStreamSynchronize(c->stream));
  for (pool *pp : {&the_pool(), &the_host_pool()}) {
    pool &p = *pp;
    std::lock_guard<std::mutex> lk(p.mu);
    for (auto &kv : p.free_lists) {
      for (void *ptr : kv.second) (void)(pp == &the_pool() ? hipFree(ptr) : hipHostFree(ptr));
      kv.second.clear();
    }
    p.cached = 0;
  }
  return SILGPU_OK;
}

int silgpu_pool_stats(size_t *in_use, size_t *cached) {
  pool &p = the_pool();
  std::lock_guard<std::mutex> lk(p.mu);
  if (in_use) *in_use = p.in_use;
  if (cached) *cached = p.cached;
  return SILGPU_OK;
}

int silgpu_host_alloc(size_t bytes, void **h_ptr) {
  SILGPU_REQUIRE(h_ptr != nullptr, "silgpu_host_alloc: h_ptr is null");
  SILGPU_CTX(c);
  (void)c;
  const size_t cls = size_class(bytes);
  pool &p = the_host_pool();
  {
    std::lock_guard<std::mutex> lk(p.mu);
    auto it = p.free_lists.find(cls);
    if (it != p.free_lists.end() && !it->second.empty()) {
      void *ptr = it->second.back();
      it->second.pop_back();
      p.live[ptr] = cls;
      p.in_use += cls;
      p.cached -= cls;
      *h_ptr = ptr;
      return SILGPU_OK;
    }
  }
  void *ptr = nullptr;
  hipError_t e = hipHostMalloc(&ptr, cls, hipHostMallocDefault);
  if (e != hipSuccess)
    return set_error(SILGPU_ERR_NOMEM, "hipHostMalloc(%zu) failed: %s", cls,
                     hipGetErrorString(e));
  std::lock_guard<std::mutex> lk(p.mu);
  p.live[ptr] = cls;
  p.in_use += cls;
  *h_ptr = ptr;
  return SILGPU_OK;
}

int silgpu_host_free(void *h_ptr) {
  if (!h_ptr) return SILGPU_OK;
  pool &p = the_host_pool();
  std::lock_guard<std::mutex> lk(p.mu);
  auto it = p.live.find(h_ptr);
  if (it == p.live.end())
    return set_error(SILGPU_ERR_INVALID,
                     "silgpu_host_free: %p was not allocated by silgpu_host_alloc", h_ptr);
  const size_t cls = it->second;
  p.live.erase(it);
  p.in_use -= cls;
  p.cached += cls;
  // Copies from and to these blocks complete before the copy calls return,
  // so a freed block has no transfer in flight.
  p.free_lists[cls].push_back(h_ptr);
  return SILGPU_OK;
}

int silgpu_memcpy_h2d(void *d_dst, const void *h_src, size_t bytes) {
  if (bytes == 0) return SILGPU_OK;
  SILGPU_REQUIRE(d_dst && h_src, "silgpu_memcpy_h2d: null pointer");
  SILGPU_CTX(c);
  SILGPU_HIP_CHECK(hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice, c->stream));
  // The caller may overwrite h_src as soon as this returns.
  SILGPU_HIP_CHECK(hipStreamSynchronize(c->stream));
  return SILGPU_OK;
}

int silgpu_memcpy_d2h(void *h_dst, const void *d_src, size_t bytes) {
  if (bytes == 0) return SILGPU_OK;
  SILGPU_REQUIRE(h_dst && d_src, "silgpu_memcpy_d2h: null pointer");
  SILGPU_CTX(c);
  SILGPU_HIP_CHECK(hipMemcpyAsync(h_dst, d_src, bytes, hipMemcpyDeviceToHost, c->stream));
  SILGPU_HIP_CHECK(hipStreamSynchronize(c->stream));
  return SILGPU_OK;
}

int silgpu_memcpy_d2d(void *d_dst, const void *d_src, size_t bytes) {
  if (bytes == 0) return SILGPU_OK;
  SILGPU_REQUIRE(d_dst && d_src, "silgpu_memcpy_d2d: null pointer");
  SILGPU_CTX(c);
  size_t head = 0;  // bytes moved by copy16_k
  if (aligned16(d_dst) && aligned16(d_src)) {
    const int64_t n16 = static_cast<int64_t>(bytes / 16);
    if (n16 > 0) {
      const int64_t blocks = cdiv(n16, int64_t(kCopyBlock) * kCopyV);
      SILGPU_REQUIRE(blocks <= INT32_MAX, "silgpu_memcpy_d2d: %zu bytes is too large", bytes);
      copy16_k<<<static_cast<unsigned>(blocks), kCopyBlock, 0, c->stream>>>(
          static_cast<const float4 *>(d_src), static_cast<float4 *>(d_dst), n16);
      SILGPU_LAUNCH_CHECK("copy16_k");
      head = static_cast<size_t>(n16) * 16;
    }
  }
  if (head < bytes)  // unaligned buffers, or the last bytes % 16
    SILGPU_HIP_CHECK(hipMemcpyAsync(static_cast<char *>(d_dst) + head,
                                    static_cast<const char *>(d_src) + head, bytes - head,
                                    hipMemcpyDeviceToDevice, c->stream));
  return SILGPU_OK;
}

int silgpu_event_create(void **ev) {
  SILGPU_REQUIRE(ev != nullptr, "silgpu_event_create: ev is null");
  SILGPU_CTX(c);
  (void)c;
  hipEvent_t e;
  SILGPU_HIP_CHECK(hipEventCreate(&e));
  *ev = e;
  return SILGPU_OK;
}

int silgpu_event_destroy(void *ev) {
  if (!ev) return SILGPU_OK;
  SILGPU_HIP_CHECK(hipEventDestroy(static_cast<hipEvent_t>(ev)));
  return SILGPU_OK;
}

int silgpu_event_record(void *ev) {
  SILGPU_REQUIRE(ev != nullptr, "silgpu_event_record: ev is null");
  SILGPU_CTX(c);
  SILGPU_HIP_CHECK(hipEventRecord(static_cast<hipEvent_t>(ev), c->stream));
  return SILGPU_OK;
}

int silgpu_event_elapsed_ms(void *ev_start, void *ev_end, float *ms) {
  SILGPU_REQUIRE(ev_start && ev_end && ms, "silgpu_event_elapsed_ms: null argument");
  SILGPU_HIP_CHECK(hipEventSynchronize(static_cast<hipEvent_t>(ev_end)));
  SILGPU_HIP_CHECK(hipEventElapsedTime(ms, static_cast<hipEvent_t>(ev_start),
                                       static_cast<hipEvent_t>(ev_end)));
  return SILGPU_OK;
}

int silgpu_get_stream(void **stream) {
  SILGPU_REQUIRE(stream != nullptr, "silgpu_get_stream: stream is null");
  SILGPU_CTX(c);
  *stream = c->stream;
  return SILGPU_OK;
}

}  // extern "C"
