"""silgpu_gemm_noalloc: the GEMM entry point that allocates nothing (its
K-split planes and GEMV partials live in a fixed device array looked up at
init) against silgpu_gemm, the entry point it is a variant of.

Bar: bit-identical to silgpu_gemm where both run the same plan (the partial
planes fit the array); where the array narrows the K split, within the SGEMM
tolerance of the fp64 oracle (per element 1e-5 sqrt(K) sum|a b|, normwise
1e-5 sqrt(K)).  Calls run back to back, each later one smaller than the one
before, so leftovers of a larger call would show.
"""

from __future__ import annotations

import math
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from conftest import rng
from gpu_util import announce, down, empty, gemm_tolerance_ok, up

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


def _pair(native, M, N, K, epi, seed, bias=True):
    g = rng(seed)
    A = g.normal(0, 0.02, (M, K)).astype(np.float32)
    B = g.normal(0, 0.02, (K, N)).astype(np.float32)
    b = g.normal(0, 0.02, N).astype(np.float32)
    dA, dB, db = up(native, A), up(native, B), up(native, b)
    c_ref, c_na = empty(native, M * N), empty(native, M * N)
    kw = dict(epi=epi, bias=db if bias else None, bias_len=N if bias else 0)
    native.gemm(0, 0, M, N, K, dA, K, dB, N, c_ref, N, **kw)
    native.gemm(0, 0, M, N, K, dA, K, dB, N, c_na, N, noalloc=True, **kw)
    return A, B, b, down(native, c_ref, (M, N)), down(native, c_na, (M, N))


def test_noalloc_matches_gemm_on_consecutive_calls(native):
    # linear_sigmoid 256x4096x4096 (K split in four: 16 MiB of planes), then
    # the smaller M = 32 product (ten splits), then a vector product
    for (M, N, K, epi, seed) in [(256, 4096, 4096, native.EPI_BIAS_SIGMOID, 1),
                                 (32, 768, 4096, native.EPI_BIAS, 2),
                                 (1, 4096, 4096, native.EPI_NONE, 3),
                                 (1, 1000, 333, native.EPI_BIAS, 4)]:
        announce(f"gemm_noalloc {M}x{N}x{K} epi={epi}")
        *_, c_ref, c_na = _pair(native, M, N, K, epi, seed, bias=epi != native.EPI_NONE)
        assert np.array_equal(c_na, c_ref), (M, N, K, float(np.max(np.abs(c_na - c_ref))))


def test_noalloc_narrows_a_split_that_does_not_fit(native, oracle):
    # 2048 x 2048 x 32768: a few large tiles and a deep K, so the planner
    # splits K; planes of 16 MiB each, more than two of which do not fit.
    M = N = 2048
    K = 32768
    announce(f"gemm_noalloc {M}x{N}x{K}")
    g = rng(5)
    A = g.uniform(-1, 1, (M, K)).astype(np.float32)
    B = g.uniform(-1, 1, (K, N)).astype(np.float32)
    dA, dB = up(native, A), up(native, B)
    c_ref, c_na = empty(native, M * N), empty(native, M * N)
    native.gemm(0, 0, M, N, K, dA, K, dB, N, c_ref, N)
    native.gemm(0, 0, M, N, K, dA, K, dB, N, c_na, N, noalloc=True)
    Cr, Cn = down(native, c_ref, (M, N)), down(native, c_na, (M, N))
    rows = g.integers(0, M, 2048)
    cols = g.integers(0, N, 2048)
    ref, refabs = oracle.sgemm_sampled_f64(A, B, rows, cols)
    tol = 1e-5 * math.sqrt(K)
    for C in (Cr, Cn):
        diff = np.abs(C[rows, cols] - ref)
        assert np.all(diff <= tol * refabs), float(np.max(diff / refabs))
        assert np.linalg.norm(diff) / np.linalg.norm(ref) <= tol
    # then a smaller product through the same array: bit-identical again
    announce("gemm_noalloc 96x160x200 after the large call")
    A2, B2, b2, c_ref2, c_na2 = _pair(native, 96, 160, 200, native.EPI_BIAS_RELU, 6)
    assert np.array_equal(c_na2, c_ref2)
    C64, Cabs = oracle.sgemm_f64(A2, B2, with_abs=True)
    ok, nw, el = gemm_tolerance_ok(c_na2, np.maximum(C64 + b2, 0.0), Cabs + np.abs(b2), 200)
    assert ok, (nw, el)


def test_noalloc_before_init_is_an_error():
    """In a fresh process that has not called silgpu_init, the entry point
    returns SILGPU_ERR_INVALID and allocates nothing."""
    announce("gemm_noalloc before init (subprocess)")
    code = (
        "import sys, ctypes as C\n"
        f"sys.path.insert(0, {str(ROOT)!r})\n"
        "from silarray_amd import _native as nat\n"
        "d = nat.GemmDesc()\n"
        "d.M = d.N = d.K = 4\n"
        "d.lda = d.ldb = d.ldc = 4\n"
        "d.batch_outer = d.batch_inner = 1\n"
        "d.A = d.B = d.C = 4096\n"
        "rc = nat.raw('silgpu_gemm_noalloc')(C.byref(d))\n"
        "print(rc, nat.last_error())\n"
    )
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                          timeout=120)
    assert proc.returncode == 0, proc.stderr
    rc, msg = proc.stdout.strip().split(" ", 1)
    assert int(rc) == -1 and "silgpu_init" in msg, proc.stdout
