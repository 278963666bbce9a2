#pragma once
// Device memory for sil::array on MI355X.
//
// The reference hands out unified-memory MTLBuffers whose `data` pointer the
// host reads and writes directly (include/unified_memory.h:17-79).  MI355X
// memory is discrete HBM, so a storage here owns a pooled HBM block
// (silgpu_alloc, on first device use) and, only when the host touches the
// data, a host mirror.  A small state machine keeps the two coherent:
//
//   host_read()   : download if the device copy is newer; host copy valid
//   host_write()  : as host_read(), then the device copy becomes stale
//   dev_read()    : upload if the host copy is newer
//   dev_write()   : the host copy becomes stale (kernel output)
//
// Views (slices, rows, broadcasts, transposes) share one `block` and differ
// in `off`/`len`, as in the reference.  Raw users of `data` (the reference's
// boundary tests write into storage::make()'s buffer and call gpu:: directly)
// start in the host-valid state.  Their host may rewrite `data` at any time
// without telling the storage (the reference's unified-memory contract), so
// every kernel that reads a raw storage whose host copy is valid uploads it
// again; synchronize() downloads every raw storage a kernel has written.
// Array-owned blocks are downloaded only when the host reads them
// (buffer_data, at, iteration), so synchronize() costs no copies for them.

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_set>

#include "../../include/silgpu.h"

namespace sil {

namespace detail {

inline void check(int rc, const char *what) {
  if (rc != SILGPU_OK)
    throw std::runtime_error(std::string("gpu: ") + what + ": " + silgpu_last_error());
}

// silgpu_init is idempotent and thread-safe; the flag only skips the call.
inline void ensure_init() {
  static std::atomic<bool> done{false};
  if (!done.load(std::memory_order_acquire)) {
    check(silgpu_init(), "init");
    done.store(true, std::memory_order_release);
  }
}

struct block;

// Raw blocks (storage::make) whose device copy is newer than the host
// mirror; synchronize() downloads them (reference semantics: after
// synchronize the host sees every result through `data`).
struct dirty_set {
  std::mutex mu;
  std::unordered_set<block *> blocks;
  static dirty_set &instance() {
    static auto *s = new dirty_set();
    return *s;
  }
};

struct block {
  void *dev = nullptr;   // HBM, allocated on first device use
  void *host = nullptr;  // host mirror, allocated on first host access
  size_t bytes = 0;
  // Neither valid: a fresh block whose content nobody has written yet.
  bool host_valid = false;
  bool dev_valid = false;
  // Handed out through storage::make(): the caller may read `data` directly
  // after synchronize(), so kernel writes are tracked for download.
  bool raw = false;
  bool pinned = false;  // host mirror from silgpu_host_alloc

  explicit block(size_t n) : bytes(n) {}
  block(const block &) = delete;
  block &operator=(const block &) = delete;
  ~block() {
    if (raw) {
      auto &d = dirty_set::instance();
      std::lock_guard<std::mutex> lk(d.mu);
      d.blocks.erase(this);
    }
    if (dev) silgpu_free(dev);
    if (pinned) silgpu_host_free(host);
    else std::free(host);
  }

  void *dev_ptr() {
    if (!dev) {
      ensure_init();
      check(silgpu_alloc(bytes ? bytes : 4, &dev), "alloc");
    }
    return dev;
  }

  // Mirrors of kPinnedMirrorBytes or more are pinned (pooled
  // silgpu_host_alloc), so uploads and downloads are direct DMA, and so are
  // mirrors of at most kPinnedTinyBytes: the scalar results of full
  // reductions come back in one DMA (sum of 1M floats through the array
  // API: 22.1 -> 15.4 us on MI355X) instead of a staged copy.  The sizes
  // between, and every mirror when no GPU is usable (host-only work such as
  // shape logic and int reductions runs without one), are plain pageable
  // memory (pinning every mirror gained nothing else in the MNIST and
  // transformer benchmarks, with one MNIST run 15% slower).
  static constexpr size_t kPinnedMirrorBytes = size_t(256) << 10;
  static constexpr size_t kPinnedTinyBytes = 256;
  static bool pinning_available() {
    static const bool ok = silgpu_init() == SILGPU_OK;
    return ok;
  }
  void *host_ptr() {
    if (!host) {
      const size_t n = ((bytes ? bytes : 4) + 63) / 64 * 64;
      if ((n >= kPinnedMirrorBytes || n <= kPinnedTinyBytes) && pinning_available() &&
          silgpu_host_alloc(n, &host) == SILGPU_OK) {
        pinned = true;
      } else {
        host = std::aligned_alloc(64, n);
        if (!host) throw std::bad_alloc();
      }
    }
    return host;
  }

  void host_read() {
    host_ptr();
    if (!host_valid) {
      if (dev_valid) check(silgpu_memcpy_d2h(host, dev_ptr(), bytes), "download");
      else std::memset(host, 0, bytes);  // fresh block: defined as zeros
      host_valid = true;
      unmark_dirty();
    }
  }

  void host_write() {
    host_read();
    dev_valid = false;
  }

  // A raw block's host copy may have been rewritten through `data` since the
  // last upload, so while it is valid it is uploaded for every kernel read.
  void dev_read() {
    if (!dev_valid || (raw && host_valid)) {
      if (host_valid) check(silgpu_memcpy_h2d(dev_ptr(), host, bytes), "upload");
      dev_valid = true;
    }
  }

  void dev_write() {
    dev_valid = true;
    host_valid = false;
    mark_dirty();
  }

  // A kernel writes part of the block: keep untouched bytes by making the
  // device copy current first.
  void dev_write_partial() {
    dev_read();
    dev_write();
  }

  void mark_dirty() {
    if (!raw) return;
    auto &d = dirty_set::instance();
    std::lock_guard<std::mutex> lk(d.mu);
    d.blocks.insert(this);
  }
  void unmark_dirty() {
    if (!raw) return;
    auto &d = dirty_set::instance();
    std::lock_guard<std::mutex> lk(d.mu);
    d.blocks.erase(this);
  }
};

}  // namespace detail

// A typed window onto a block: elements [off, off + len) of the block.
// Replaces the reference's storage {buf, data, mtl_buf, off, len}
// (include/unified_memory.h:17-25).  `data` is the host mirror's base
// address, valid after host_data()/storage::make; device code never reads
// it.
struct storage {
  std::shared_ptr<detail::block> buf;
  void *data = nullptr;  // host mirror base (element 0 of the block)
  size_t off = 0;        // in elements
  size_t len = 0;        // in elements

  // A new block of `bytes`, zero-filled and host-authoritative, with `data`
  // ready for host writes (the reference's boundary tests memcpy into it
  // before launching a kernel).
  static storage make(size_t bytes) {
    storage s;
    s.buf = std::make_shared<detail::block>(bytes);
    s.buf->raw = true;
    s.buf->host_read();
    s.data = s.buf->host;
    return s;
  }

  // A new block with undefined content and no host mirror yet: the form for
  // kernel outputs and for arrays whose elements are set afterwards.
  static storage make_device(size_t bytes) {
    storage s;
    s.buf = std::make_shared<detail::block>(bytes);
    return s;
  }

  explicit operator bool() const { return static_cast<bool>(buf); }

  // Device address of element `off` for element type T, made current.
  template <typename T>
  const T *dev_in() const {
    buf->dev_read();
    return static_cast<const T *>(buf->dev_ptr()) + off;
  }
  template <typename T>
  T *dev_out() {
    if (off == 0 && len * sizeof(T) >= buf->bytes) buf->dev_write();
    else buf->dev_write_partial();
    return static_cast<T *>(buf->dev_ptr()) + off;
  }

  // In-place kernels: the device copy is read and then overwritten.
  template <typename T>
  T *dev_inout() {
    buf->dev_read();
    buf->dev_write();
    return static_cast<T *>(buf->dev_ptr()) + off;
  }

  // Host address of element `off`, made current (read) or made current and
  // taken over (write).
  template <typename T>
  const T *host_in() const {
    buf->host_read();
    const_cast<storage *>(this)->data = buf->host;
    return static_cast<const T *>(buf->host) + off;
  }
  template <typename T>
  T *host_out() {
    buf->host_write();
    data = buf->host;
    return static_cast<T *>(buf->host) + off;
  }
};

}  // namespace sil
