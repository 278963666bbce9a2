"""Helpers for GPU parity tests: upload/download through the C ABI and the
tolerance checks the tests state."""

import math
import sys

import numpy as np


def announce(name: str) -> None:
    """Names the case before its GPU step, so a crash can be attributed."""
    sys.stdout.write(f"[gpu-case] {name}\n")
    sys.stdout.flush()


def up(nat, a):
    return nat.DeviceBuffer.from_array(np.ascontiguousarray(a))


def empty(nat, n, dtype=np.float32):
    return nat.DeviceBuffer(max(int(n) * np.dtype(dtype).itemsize, 4))


def down(nat, buf, shape, dtype=np.float32):
    nat.sync()
    return buf.download(shape, dtype)


def gemm_tolerance_ok(C, C64, Cabs, K):
    """SGEMM/GEMV bar: normwise ||C - C64||_F / ||C64||_F <= 1e-5 sqrt(K) and
    per element |c - c64| <= 1e-5 sqrt(K) sum_k |a_ik b_kj| (+ 1e-30)."""
    tol = 1e-5 * math.sqrt(max(K, 1))
    diff = np.abs(C.astype(np.float64) - C64)
    nrm = np.linalg.norm(C64)
    normwise = np.linalg.norm(diff) / nrm if nrm > 0 else np.linalg.norm(diff)
    elem_ok = np.all(diff <= tol * Cabs + 1e-30)
    return normwise <= tol and elem_ok, normwise, float(np.max(diff / (Cabs + 1e-30)))


def sigmoid_bound(C64, Cabs, K):
    """Reference and per-element bound (in gemm_tolerance_ok's units) after a
    sigmoid epilogue.  sigmoid is 1/4-Lipschitz, so the pre-activation bound
    carries over as Cabs / 4; the fp32 sigmoid itself (exp, add, divide)
    adds up to about 3 ulp of its result y, allowed as 4 * 2^-24 * y.
    Without that term a short K (K = 2: a bar below 1 ulp of y) would hold
    the sigmoid to more than fp32 can give."""
    y = 1 / (1 + np.exp(-C64))
    tol = 1e-5 * math.sqrt(max(K, 1))
    return y, Cabs / 4 + 4 * 2.0 ** -24 * y / tol


def ulp_diff(a, b):
    """Distance in float32 ulps (same-sign finite values)."""
    ai = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(ai - bi)
