"""The bounded wait of the one-launch reductions (sum, min, max, argmax).

Their finishing workgroup waits on the device for the partial results the
other workgroups publish in 64-bit slots; the reference finishes on the host
and never waits on the device (include/gpu.h:331-354, include/array.h:1535-1545).
A finisher gives up at a wall-clock deadline, records the failure in a
host-mapped word, and the next silgpu_sync (or reduction call) returns
SILGPU_ERR_HIP and clears the slots.  These tests force the give-up from the
host through silgpu_slot_wait_selftest (a finisher over slots that no
workgroup of its launch writes, with a short deadline), so every kernel still
ends on its own: no wait here is unbounded."""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from gpu_util import announce, down, empty, up

pytestmark = pytest.mark.gpu


def _in_use(nat) -> int:
    n = C.c_int64(-1)
    nat.call("silgpu_slots_in_use", C.byref(n))
    return n.value


def _taken(nat, buf) -> int:
    return int(down(nat, buf, (1,), np.uint32)[0])


def _sum_ok(nat, seed):
    """A 1M-element sum (a full one-launch reduction through the slots) is
    right after the failure path has run."""
    x = np.random.default_rng(seed).uniform(-1, 1, 1 << 20).astype(np.float32)
    dx, out = up(nat, x), empty(nat, 1)
    nat.sum_f32(dx, x.size, out)
    got = float(down(nat, out, (1,))[0])
    ref = float(np.sum(x.astype(np.float64)))
    assert abs(got - ref) <= 1e-5 * np.sum(np.abs(x.astype(np.float64))), (got, ref)


def test_finisher_receives_a_producer_within_its_deadline(native):
    announce("slot wait: producer at 1 ms, deadline 200 ms")
    assert _in_use(native) == 0
    taken = up(native, np.zeros(1, np.uint32))
    native.call("silgpu_slot_wait_selftest", 1, 200_000, 1_000, native.vp(taken))
    native.sync()  # no failure: the slot arrived in time
    assert _taken(native, taken) == 1
    assert _in_use(native) == 0  # the finisher cleared the slot it took


def test_finisher_gives_up_and_the_sync_reports_it(native):
    announce("slot wait: 100 slots nobody writes, deadline 2 ms")
    assert _in_use(native) == 0
    taken = up(native, np.zeros(1, np.uint32))
    native.call("silgpu_slot_wait_selftest", 100, 2_000, 0, native.vp(taken))
    rc = native.raw("silgpu_sync")()
    assert rc == native.ERR_HIP, rc
    assert "gave up" in native.last_error()
    assert _taken(native, taken) == 0
    assert _in_use(native) == 0
    native.sync()  # reported once: the next sync is clean
    _sum_ok(native, 1)


def test_late_producer_leaves_nothing_behind(native):
    announce("slot wait: producer at 10 ms, deadline 2 ms")
    taken = up(native, np.zeros(1, np.uint32))
    native.call("silgpu_slot_wait_selftest", 1, 2_000, 10_000, native.vp(taken))
    rc = native.raw("silgpu_sync")()
    assert rc == native.ERR_HIP and "gave up" in native.last_error()
    assert _taken(native, taken) == 0
    # the producer published after the finisher gave up; the host cleared it
    assert _in_use(native) == 0
    _sum_ok(native, 2)
    # argmax over one long row: its finisher takes many slots
    x = np.random.default_rng(3).uniform(-1, 1, (1, 1 << 22)).astype(np.float32)
    x[0, 1_234_567] = 2.0
    out = empty(native, 1, np.int32)
    native.argmax_rows_f32(up(native, x), 1, x.shape[1], out)
    assert int(down(native, out, (1,), np.int32)[0]) == 1_234_567


def test_reduction_call_reports_a_pending_failure(native):
    announce("slot wait: failure reported by the next sum call")
    taken = up(native, np.zeros(1, np.uint32))
    e0, e1 = native.Event(), native.Event()
    e0.record()
    native.call("silgpu_slot_wait_selftest", 8, 2_000, 0, native.vp(taken))
    e1.record()
    e0.elapsed_ms(e1)  # waits for the launch without consuming the failure
    x = up(native, np.ones(4096, np.float32))
    out = empty(native, 1)
    rc = native.raw("silgpu_sum_f32")(x.ptr, 4096, out.ptr)
    assert rc == native.ERR_HIP and "gave up" in native.last_error()
    native.sync()
    assert _in_use(native) == 0
    native.sum_f32(x, 4096, out)  # and the call after it runs
    assert float(down(native, out, (1,))[0]) == 4096.0
