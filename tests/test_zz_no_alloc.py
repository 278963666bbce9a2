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
    # 2048 x 2048 x 32764: K % 16 != 0 keeps the product off the LDS-direct
    # kernel, and the planner picks 256 x 256 tiles with four K splits: four
    # 16 MiB partial planes, of which the 32 MiB array holds two.
    M = N = 2048
    K = 32764
    plane = M * N * 4
    fixed = 32 << 20
    announce(f"gemm_noalloc {M}x{N}x{K}")
    g = rng(5)
    A = g.uniform(-1, 1, (M, K)).astype(np.float32)
    B = g.uniform(-1, 1, (K, N)).astype(np.float32)
    dA, dB = up(native, A), up(native, B)
    c_ref, c_na, c_forced = empty(native, M * N), empty(native, M * N), empty(native, M * N)
    native.gemm(0, 0, M, N, K, dA, K, dB, N, c_ref, N)
    plan_ref = native.last_plan()
    native.gemm(0, 0, M, N, K, dA, K, dB, N, c_na, N, noalloc=True)
    plan_na = native.last_plan()
    assert len(plan_ref) == 1 and len(plan_na) == 1, (plan_ref, plan_na)
    (tile, s_ref, _), (tile_na, s_na, _) = plan_ref[0], plan_na[0]
    assert tile == tile_na, (plan_ref, plan_na)
    assert s_ref * plane > fixed, plan_ref             # the planned split does not fit
    assert 2 <= s_na < s_ref and s_na * plane <= fixed, plan_na  # the widest that fits
    assert (s_na + 1) * plane > fixed, plan_na
    # the narrowed product is the forced plan with that split, bit for bit
    native.sgemm_tuned(0, 0, M, N, K, dA, K, 0, dB, N, 0, c_forced, N, 0, tile=tile, splits=s_na)
    assert native.last_plan() == plan_na
    Cr, Cn, Cf = (down(native, c, (M, N)) for c in (c_ref, c_na, c_forced))
    assert np.array_equal(Cn, Cf)
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


def test_noalloc_allocates_no_device_memory():
    """In a fresh process: after silgpu_init and the operands' allocation,
    the no-allocation entry point runs a split-K product, the narrowed deep
    product, a small-M product and a vector product without changing the
    device's free memory (hipMemGetInfo); the same products through
    silgpu_gemm then grow the split-K workspace, which the same measurement
    sees."""
    announce("gemm_noalloc free device memory (subprocess)")
    code = (
        "import sys, ctypes as C\n"
        f"sys.path.insert(0, {str(ROOT)!r})\n"
        "import numpy as np\n"
        "from silarray_amd import _native as nat\n"
        "nat.init()\n"
        "hip = C.CDLL('libamdhip64.so')\n"
        "def free():\n"
        "    nat.sync()\n"
        "    f, t = C.c_size_t(), C.c_size_t()\n"
        "    assert hip.hipMemGetInfo(C.byref(f), C.byref(t)) == 0\n"
        "    return f.value\n"
        "g = np.random.default_rng(7)\n"
        "shapes = [(256, 4096, 4096), (2048, 2048, 32764), (32, 768, 4096), (1, 4096, 4096)]\n"
        "ops = []\n"
        "for M, N, K in shapes:\n"
        "    A = nat.DeviceBuffer.from_array(g.normal(0, 0.02, (M, K)).astype(np.float32))\n"
        "    B = nat.DeviceBuffer.from_array(g.normal(0, 0.02, (K, N)).astype(np.float32))\n"
        "    ops.append((M, N, K, A, B, nat.DeviceBuffer(M * N * 4)))\n"
        "def run(noalloc):\n"
        "    for M, N, K, A, B, Cm in ops:\n"
        "        nat.gemm(0, 0, M, N, K, A, K, B, N, Cm, N, noalloc=noalloc)\n"
        "# one small launch first: the runtime loads the code object on first use\n"
        "nat.gemm(0, 0, 64, 64, 64, ops[0][3], 4096, ops[0][4], 4096, ops[0][5], 4096,"
        " noalloc=True)\n"
        "f0 = free()\n"
        "run(True)\n"
        "run(True)\n"
        "f1 = free()\n"
        "run(False)\n"
        "f2 = free()\n"
        "print(f0, f1, f2)\n"
    )
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                          timeout=300)
    assert proc.returncode == 0, proc.stderr[-2000:]
    f0, f1, f2 = map(int, proc.stdout.split()[-3:])
    assert f1 == f0, (f0, f1)          # the no-allocation calls took nothing
    assert f2 < f1, (f1, f2)           # the allocating entry point's workspace shows


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
