"""Every BASELINE.json configuration at its stated size, against the oracle.

  C1  SGEMM 1024^3 through the C++ sil::array::dot (bench_graph dot-dump),
      against the fp64 oracle (the reference's config,
      bench/micro/bench_sgemm.cpp:34).
  C3  full-tensor sum / min / max over 67,108,864 uniform[-1, 1] floats with
      a unique planted maximum (argmax at that size is in
      test_gpu_kernels.py).
  C4  SGEMM 4096^3 (2048^3 and 8192^3 are in test_gpu_kernels.py) and the
      20-node affine chain on 67,108,864 floats, both through the C ABI's
      fused program and through sil::eval (bench_graph chain-dump),
      bit-exact against the oracle's sequential fma chain.
  C5  the encoder block B4 S512 d768 H12 F3072 is the last case of
      test_graph_bench.py's encoder parametrisation.

Bars: SGEMM per element |c - c64| <= 1e-5 sqrt(K) sum|a b| and normwise
1e-5 sqrt(K); sums relative 1e-5 of the fp64 sum; min / max and the affine
chain bit-exact.
"""

from __future__ import annotations

import math
import subprocess
from pathlib import Path

import numpy as np
import pytest

from conftest import rng
from gpu_util import announce, down, empty, gemm_tolerance_ok, up

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
BENCH = ROOT / "silarray_amd" / "bench" / "bench_graph"
N64M = 64 * 1024 * 1024


def _bench() -> Path:
    if not BENCH.exists():
        pytest.fail(f"{BENCH} is not built (run __graft_entry__.build())")
    return BENCH


def test_c1_dot_1024_through_array_api(oracle, tmp_path):
    announce("C1 sil::array::dot 1024^3")
    proc = subprocess.run([str(_bench()), "dot-dump", "1024", "1024", "1024", str(tmp_path)],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stderr
    A = np.fromfile(tmp_path / "A.bin", np.float32).reshape(1024, 1024)
    B = np.fromfile(tmp_path / "B.bin", np.float32).reshape(1024, 1024)
    C = np.fromfile(tmp_path / "C.bin", np.float32).reshape(1024, 1024)
    assert np.all(np.abs(A) <= 1.0) and A.std() > 0.5  # uniform[-1, 1)
    C64, Cabs = oracle.sgemm_f64(A, B, with_abs=True)
    ok, nw, el = gemm_tolerance_ok(C, C64, Cabs, 1024)
    assert ok, (nw, el)


@pytest.fixture(scope="module")
def x64m():
    g = rng(2601)
    x = g.uniform(-1, 1, N64M).astype(np.float32)
    x[(N64M * 7) // 9 + 1] = 2.0  # unique planted maximum, not 4- or chunk-aligned
    return x


def test_c3_sum_min_max_64m(native, oracle, x64m):
    announce("C3 sum/min/max n=67108864")
    dx, do = up(native, x64m), empty(native, 1)
    native.sum_f32(dx, N64M, do)
    s, s64 = float(down(native, do, 1)[0]), oracle.sum_f64(x64m)
    # the sum cancels heavily (|sum| ~ 5e3 against sum|x| ~ 3e7); the fp32
    # result must still be within 1e-5 of the exact value
    assert abs(s - s64) <= 1e-5 * abs(s64), (s, s64)
    native.min_f32(dx, N64M, do)
    assert down(native, do, 1)[0] == oracle.fmin(x64m)
    native.max_f32(dx, N64M, do)
    assert down(native, do, 1)[0] == oracle.fmax(x64m) == np.float32(2.0)
    # the same buffer twice more: a call leaves nothing behind that the next
    # call could read
    native.sum_f32(dx, N64M, do)
    assert float(down(native, do, 1)[0]) == s
    native.argmax_rows_f32(dx, 1, N64M, do)
    assert int(down(native, do, 1, np.int32)[0]) == (N64M * 7) // 9 + 1


def test_c4_sgemm_4096_sampled(native, oracle):
    S = 4096
    announce(f"C4 sgemm {S}^3 sampled")
    g = rng(1400 + S)
    A = g.uniform(-1, 1, (S, S)).astype(np.float32)
    B = g.uniform(-1, 1, (S, S)).astype(np.float32)
    dA, dB, dC = up(native, A), up(native, B), empty(native, S * S)
    native.sgemm(0, 0, S, S, S, dA, S, 0, dB, S, 0, dC, S, 0)
    Cg = down(native, dC, (S, S))
    rows = g.integers(0, S, 4096)
    cols = g.integers(0, S, 4096)
    rows[:4] = [0, S - 1, 0, S - 1]
    cols[:4] = [0, S - 1, S - 1, 0]
    ref, refabs = oracle.sgemm_sampled_f64(A, B, rows, cols)
    tol = 1e-5 * math.sqrt(S)
    diff = np.abs(Cg[rows, cols] - ref)
    assert np.all(diff <= tol * refabs), float(np.max(diff / refabs))
    assert np.linalg.norm(diff) / np.linalg.norm(ref) <= tol
    # every tile row and column of C against fp64: the full last row and
    # column exercise the grid's edges
    C64, Cabs = oracle.sgemm_f64(A[-1:], B, with_abs=True)
    ok, nw, el = gemm_tolerance_ok(Cg[-1:], C64, Cabs, S)
    assert ok, ("last row", nw, el)
    C64, Cabs = oracle.sgemm_f64(A, B[:, -1:], with_abs=True)
    ok, nw, el = gemm_tolerance_ok(Cg[:, -1:], C64, Cabs, S)
    assert ok, ("last column", nw, el)


def test_c4_affine_chain_64m_program(native, oracle, x64m):
    announce("C4 20-op affine chain n=67108864 (C ABI program)")
    g = rng(2602)
    sc = g.uniform(0.9, 1.1, 20).astype(np.float32)
    of = g.uniform(-0.1, 0.1, 20).astype(np.float32)
    dx, do = up(native, x64m), empty(native, N64M)
    instrs = [(native.PI_LOAD, 0, 0, 0, 0.0, 0.0)] + \
             [(native.PI_FMAI, 0, 0, 0, float(a), float(b)) for a, b in zip(sc, of)]
    prog = native.make_program((N64M,), [(dx, (1,))], instrs)
    native.program_f32(prog, do)
    assert np.array_equal(down(native, do, N64M), oracle.affine_chain(x64m, sc, of))


def test_c4_affine_chain_64m_through_eval(oracle, tmp_path):
    """bench_graph's chain: y = y * (1 + 0.001 i) + 0.01 i for i < 10 on the
    array API, one sil::eval.  Each scalar node folds as the reference's
    try_affine_reduce folds it (include/array.h:1888-1940): x * s ->
    fma(x, s, 0 * s), x + o -> fma(x, 1, 0 + o); the oracle applies the same
    20 fmas in order."""
    announce("C4 20-op affine chain n=67108864 (sil::eval)")
    proc = subprocess.run([str(_bench()), "chain-dump", str(N64M), str(tmp_path)],
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr
    x = np.fromfile(tmp_path / "x.bin", np.float32)
    y = np.fromfile(tmp_path / "y.bin", np.float32)
    assert x.size == N64M and y.size == N64M
    scales, offsets = [], []
    for i in range(10):
        s = np.float32(1.0) + np.float32(0.001) * np.float32(i)
        o = np.float32(0.01) * np.float32(i)
        scales += [s, np.float32(1.0)]
        offsets += [np.float32(0.0) * s, np.float32(0.0) + o]
    ref = oracle.affine_chain(x, np.array(scales, np.float32), np.array(offsets, np.float32))
    assert np.array_equal(y, ref)
