"""Seeded random products through every GEMM entry point against the oracle.

Each case draws an entry point (silgpu_sgemm, silgpu_sgemm_tuned with a forced
tile and K split, silgpu_gemm, silgpu_gemm_noalloc), a shape from one of the
routes (LDS-direct multiples, ragged, small M, vector products, N = 1),
transposes, padded leading dimensions, operands offset off 16-byte alignment,
one- or two-level batches, every epilogue with the bias taken modulo a random
length, the scalar affine node and the residual.  C and its row padding start
as NaN and 64 NaN canaries follow C: every element of C must be written, and
nothing past its N columns or its end.  Bar: gemm_tolerance_ok (sigmoid_bound
after a sigmoid).  Reference: include/array.h:1360-1416, 1462-1472 (dot,
batched_dot, linear, linear_sigmoid), bias[col % bias_len] as in
include/gpu_kernels.metal:620-678.
"""

import math

import numpy as np
import pytest

from conftest import rng
from gpu_util import announce, down, gemm_tolerance_ok, sigmoid_bound, up

pytestmark = pytest.mark.gpu

CANARY = 64
N_CASES = 120


def _shape(g):
    k = int(g.integers(0, 6))
    if k == 0:    # LDS-direct multiples
        return int(64 * g.integers(1, 17)), int(64 * g.integers(1, 17)), int(16 * g.integers(1, 100))
    if k == 1:    # ragged, log-uniform
        return tuple(int(x) + 1 for x in np.exp(g.uniform(0, math.log(1200), 3)).astype(int))
    if k == 2:    # small M
        return int(g.integers(1, 33)), int(g.integers(1, 3000)), int(g.integers(1, 3000))
    if k == 3:    # vector times matrix
        return 1, int(g.integers(1, 4000)), int(g.integers(1, 4000))
    if k == 4:    # matrix times vector
        return int(g.integers(1, 2000)), 1, int(g.integers(1, 2000))
    return int(256 * g.integers(1, 5)), int(128 * g.integers(1, 9)), int(16 * g.integers(1, 160))


def _case(i):
    g = rng(31000 + i)
    mode = str(g.choice(["sgemm", "tuned", "gemm", "noalloc"]))
    M, N, K = _shape(g)
    while M * N * K > 2e8:
        M, N = max(1, M // 2), max(1, N // 2)
    c = dict(mode=mode, M=M, N=N, K=K, ta=int(g.integers(0, 2)), tb=int(g.integers(0, 2)),
             pad_a=int(g.integers(0, 8)), pad_b=int(g.integers(0, 8)),
             pad_c=int(g.choice([0, 0, 3])), off_a=int(g.choice([0, 0, 1, 3])),
             off_b=int(g.choice([0, 0, 2])), bo=1, bi=1)
    if mode in ("sgemm", "tuned"):
        c["bi"] = int(g.choice([1, 1, 2, 3]))
    elif mode == "gemm":
        c["bo"], c["bi"] = int(g.choice([1, 2])), int(g.choice([1, 2]))
    c["epi"] = int(g.choice([0, 1, 2, 3, 4]))
    c["bias_len"] = (int(g.choice([N, 1, int(g.integers(1, N + 1))]))
                     if c["epi"] in (1, 2, 4) else 0)
    c["scale"] = ((float(np.float32(g.uniform(-2, 2))), float(np.float32(g.uniform(-1, 1))))
                  if mode in ("gemm", "noalloc") and g.random() < 0.3 else None)
    c["resid"] = mode in ("gemm", "noalloc") and c["bo"] * c["bi"] == 1 and g.random() < 0.4
    c["ldr"] = N + int(g.choice([0, 1]))
    c["tile"], c["splits"] = int(g.integers(1, 11)), int(g.choice([1, 2, 3, 4, 7, 16]))
    c["seed"] = 32000 + i
    return c


@pytest.mark.parametrize("i", range(N_CASES))
def test_gemm_random_entry_points(native, oracle, i):
    c = _case(i)
    M, N, K, ta, tb = c["M"], c["N"], c["K"], c["ta"], c["tb"]
    announce("gemm random " + " ".join(f"{k}={v}" for k, v in c.items()))
    g = rng(c["seed"])
    ra, ca = (K, M) if ta else (M, K)
    rb, cb = (N, K) if tb else (K, N)
    lda, ldb, ldc = ca + c["pad_a"], cb + c["pad_b"], N + c["pad_c"]
    bo, bi = c["bo"], c["bi"]
    nb = bo * bi
    sA, sB, sC = ra * lda, rb * ldb, M * ldc
    A = g.uniform(-1, 1, c["off_a"] + nb * sA).astype(np.float32)
    B = g.uniform(-1, 1, c["off_b"] + nb * sB).astype(np.float32)
    bias_len = c["bias_len"]
    bias = g.normal(0, 1, max(bias_len, 1)).astype(np.float32)
    R = g.normal(0, 1, M * c["ldr"]).astype(np.float32)
    dA, dB = up(native, A), up(native, B)
    dC = up(native, np.full(nb * sC + CANARY, np.nan, np.float32))
    dbias = up(native, bias) if bias_len else None
    dR = up(native, R) if c["resid"] else None
    pA, pB = dA.ptr + 4 * c["off_a"], dB.ptr + 4 * c["off_b"]
    epi = c["epi"]
    if c["mode"] == "sgemm":
        native.sgemm(ta, tb, M, N, K, pA, lda, sA, pB, ldb, sB, dC, ldc, sC, bi, dbias,
                     bias_len, epi)
    elif c["mode"] == "tuned":
        native.sgemm_tuned(ta, tb, M, N, K, pA, lda, sA, pB, ldb, sB, dC, ldc, sC, bi, dbias,
                           bias_len, epi, tile=c["tile"], splits=c["splits"])
    else:
        native.gemm(ta, tb, M, N, K, pA, lda, pB, ldb, dC, ldc, batch_outer=bo,
                    batch_inner=bi, strides_a=(sA * bi, sA), strides_b=(sB * bi, sB),
                    strides_c=(sC * bi, sC), epi=epi, scale=c["scale"], bias=dbias,
                    bias_len=bias_len, residual=dR, ldr=c["ldr"] if c["resid"] else 0,
                    noalloc=c["mode"] == "noalloc")
    Cg = down(native, dC, (nb * sC + CANARY,))
    assert np.all(np.isnan(Cg[nb * sC:])), "canary after C overwritten"
    for b in range(nb):
        Ab = A[c["off_a"] + b * sA: c["off_a"] + (b + 1) * sA].reshape(ra, lda)[:, :ca]
        Bb = B[c["off_b"] + b * sB: c["off_b"] + (b + 1) * sB].reshape(rb, ldb)[:, :cb]
        C64, Cabs = oracle.sgemm_f64(np.ascontiguousarray(Ab), np.ascontiguousarray(Bb),
                                     ta=bool(ta), tb=bool(tb), with_abs=True)
        if c["scale"] is not None:
            s, o = c["scale"]
            C64, Cabs = C64 * s + o, Cabs * abs(s) + abs(o)
        if bias_len:
            bv = bias[np.arange(N) % bias_len].astype(np.float64)
            C64, Cabs = C64 + bv, Cabs + np.abs(bv)
        if epi == 2:
            C64, Cabs = sigmoid_bound(C64, Cabs, K)
        if epi in (3, 4):
            C64 = np.maximum(C64, 0)
        if c["resid"]:
            Rm = R.reshape(M, c["ldr"])[:, :N].astype(np.float64)
            C64, Cabs = C64 + Rm, Cabs + np.abs(Rm)
        Cb = Cg[b * sC: (b + 1) * sC].reshape(M, ldc)
        assert np.all(np.isnan(Cb[:, N:])), f"batch {b}: C row padding overwritten"
        got = Cb[:, :N]
        assert np.all(np.isfinite(got)), f"batch {b}: unwritten or non-finite elements"
        ok, nw, el = gemm_tolerance_ok(got, C64, Cabs, K)
        assert ok, (b, nw, el)
