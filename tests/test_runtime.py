"""The memory layer behind storage::make (the reference's buffer_pool,
include/unified_memory.h:27-61): the size-class device pool reuses freed
blocks, keeps them cached until silgpu_pool_trim, and reports its sizes;
pinned host blocks are pooled the same way."""

from __future__ import annotations

import ctypes as C
import gc

import numpy as np
import pytest

from gpu_util import announce, down, up

pytestmark = pytest.mark.gpu


def _stats(nat):
    used, cached = C.c_size_t(), C.c_size_t()
    nat.call("silgpu_pool_stats", C.byref(used), C.byref(cached))
    return used.value, cached.value


def _alloc(nat, nbytes, host=False):
    p = C.c_void_p()
    nat.call("silgpu_host_alloc" if host else "silgpu_alloc", C.c_size_t(nbytes), C.byref(p))
    return p.value


def test_device_pool_reuses_and_trims(native):
    announce("device pool reuse / trim")
    gc.collect()  # buffers of earlier tests return to the pool now, not mid-test
    native.call("silgpu_pool_trim")
    used0, cached0 = _stats(native)
    assert cached0 == 0
    # 3,000,000 bytes fall in the 3 MiB class (four classes per power of two
    # above 64 KiB: 2 MiB + k * 512 KiB)
    cls = 3 * 1024 * 1024
    p = _alloc(native, 3_000_000)
    assert _stats(native) == (used0 + cls, 0)
    native.call("silgpu_free", C.c_void_p(p))
    assert _stats(native) == (used0, cls)
    # a nearby size of the same class gets the cached block back
    q = _alloc(native, 3_100_000)
    assert q == p and _stats(native) == (used0 + cls, 0)
    # the reused block is an ordinary block: data written through it round-trips
    x = np.arange(3_100_000 // 4, dtype=np.float32)
    native.call("silgpu_memcpy_h2d", C.c_void_p(q), x.ctypes.data_as(C.c_void_p),
                C.c_size_t(x.nbytes))
    y = np.empty_like(x)
    native.call("silgpu_memcpy_d2h", y.ctypes.data_as(C.c_void_p), C.c_void_p(q),
                C.c_size_t(y.nbytes))
    assert np.array_equal(x, y)
    native.call("silgpu_free", C.c_void_p(q))
    # a different class does not take it
    r = _alloc(native, 5_000_000)
    assert r != q
    native.call("silgpu_free", C.c_void_p(r))
    used, cached = _stats(native)
    assert used == used0 and cached >= cls
    native.call("silgpu_pool_trim")
    assert _stats(native) == (used0, 0)
    # freeing a pointer the pool did not hand out is an error, not a crash
    with pytest.raises(native.SilGpuError):
        native.call("silgpu_free", C.c_void_p(q + 256))


def test_small_classes_and_pinned_host_pool(native):
    announce("small classes and pinned host pool")
    a = _alloc(native, 1)
    b = _alloc(native, 256)
    assert a % 256 == 0 and b % 256 == 0 and a != b
    native.call("silgpu_free", C.c_void_p(a))
    c = _alloc(native, 200)  # same 256-byte class as `a`
    assert c == a
    for p in (b, c):
        native.call("silgpu_free", C.c_void_p(p))
    h = _alloc(native, 1 << 20, host=True)
    native.call("silgpu_host_free", C.c_void_p(h))
    h2 = _alloc(native, (1 << 20) - 100, host=True)
    assert h2 == h
    # a pinned block is a valid copy source and destination
    buf = (C.c_float * 4).from_address(h2)
    buf[:] = [1.0, 2.0, 3.0, 4.0]
    d = up(native, np.zeros(4, np.float32))
    native.call("silgpu_memcpy_h2d", C.c_void_p(d.ptr), C.c_void_p(h2), C.c_size_t(16))
    assert np.array_equal(down(native, d, 4), [1.0, 2.0, 3.0, 4.0])
    native.call("silgpu_host_free", C.c_void_p(h2))
    native.call("silgpu_pool_trim")


# (bytes, source offset, destination offset): empty, below one 16-byte slot,
# one slot, a slot plus a tail, exactly one 32 KiB workgroup block, one block
# plus a partial block and a tail, 64 MiB + 3; offsets that keep both
# pointers 16-byte aligned (the streaming kernel), and ones that do not (the
# runtime's copy)
COPY_CASES = [(0, 0, 0), (7, 0, 0), (16, 0, 0), (21, 0, 0), (32768, 0, 0), (32768 + 4096 + 5, 0, 0),
              (64 * 1024 * 1024 + 3, 0, 0), (100_000, 16, 48), (100_000, 4, 0), (100_001, 0, 3)]


@pytest.mark.parametrize("nbytes,so,do", COPY_CASES)
def test_memcpy_d2d(native, nbytes, so, do):
    announce(f"memcpy_d2d {nbytes} B, offsets {so}/{do}")
    g = np.random.default_rng(nbytes + so)
    src = g.integers(0, 256, nbytes + so, dtype=np.uint8)
    s = native.DeviceBuffer(max(nbytes + so, 1))
    d = native.DeviceBuffer(nbytes + do + 64)
    if nbytes + so:
        s.upload(src)
    guard = np.full(nbytes + do + 64, 0xA5, np.uint8)
    d.upload(guard)
    native.call("silgpu_memcpy_d2d", C.c_void_p(d.at(do)), C.c_void_p(s.at(so)), C.c_size_t(nbytes))
    out = d.download(nbytes + do + 64, np.uint8)
    assert np.array_equal(out[do:do + nbytes], src[so:so + nbytes])
    # nothing outside the destination range is touched
    assert np.all(out[:do] == 0xA5) and np.all(out[do + nbytes:] == 0xA5)
