"""Seeded random cases of the non-GEMM kernels against the oracle.

Each case draws one kernel and a shape around its dispatch thresholds, with
unaligned pointers, -inf and NaN entries and ties where the kernel has a rule
for them, and checks it with the bar its own tests state:
  softmax (include/array.h:1677-1709): relative 1e-5 per element, NaN rows
    (a row of -inf only) matching the float64 reference's NaN;
  layer_norm (include/cpu.h:352-373): 1e-5 * max(1, |y|), rows offset from
    zero so the mean is large against the spread;
  sum (relative 1e-5 plus 6e-8 of sum |x|) and bit-exact min / max
    (include/array.h:1523-1552, 1600-1658);
  sum(axis) over every axis of 1-3-D arrays (include/array.h:1554-1583);
  argmax rows, bit-exact, first index of the maximum, NaN never wins
    (include/array.h:1711-1750);
  strided binary ops with broadcast axes, bit-exact (include/array.h:2478-2612);
  fused attention (2e-5 sqrt(max(D, Sk)) max|V|) and conv2d (the GEMM bar with
    K = k*k*C_in).
Writes past the end of every output (NaN canaries) fail the case.
"""

import math

import numpy as np
import pytest

from conftest import rng
from gpu_util import announce, gemm_tolerance_ok

pytestmark = pytest.mark.gpu

N_CASES = 120
KINDS = ("softmax", "layer_norm", "reduce", "sum_axis", "argmax", "binary", "attention", "conv2d")


def _logu(g, lo, hi):
    return int(np.exp(g.uniform(math.log(lo), math.log(hi + 1))))


def _cols(g):
    if g.random() < 0.4:
        return int(max(1, g.choice([256, 512, 1024, 2048, 4096, 8192, 16384]) + g.integers(-3, 4)))
    return _logu(g, 1, 40000)


def _with_offset(native, x, off):
    """x flattened behind `off` leading floats: (buffer, device pointer of x)."""
    buf = np.concatenate([np.zeros(off, np.float32), x.ravel()]).astype(np.float32)
    d = native.DeviceBuffer.from_array(buf)
    return d, d.ptr + 4 * off


def _canary_buffer(native, n, dtype=np.float32):
    fill = np.full(n + 16, np.nan, np.float32) if dtype == np.float32 else np.full(n + 16, -7, dtype)
    return native.DeviceBuffer.from_array(fill)


def _softmax(native, oracle, g):
    R, C = _logu(g, 1, 2000), _cols(g)
    while R * C > 8e6:
        R = max(1, R // 2)
    x = g.normal(0, float(g.choice([0.1, 3, 30])), (R, C)).astype(np.float32)
    if C > 1 and g.random() < 0.5:
        rows = g.integers(0, R, max(1, R // 8))
        x[rows, g.integers(0, C, rows.size)] = -np.inf
    if R > 1 and g.random() < 0.2:
        x[R // 2, :] = -np.inf
    off = int(g.choice([0, 1, 2]))
    dx, px = _with_offset(native, x, off)
    do = _canary_buffer(native, R * C)
    announce(f"random softmax {R}x{C} off={off}")
    native.softmax_rows_f32(px, do, R, C)
    out = do.download((R * C + 16,), np.float32)
    assert np.all(np.isnan(out[R * C:])), "wrote past the end"
    o = out[:R * C].reshape(R, C).astype(np.float64)
    with np.errstate(invalid="ignore"):
        ref = oracle.softmax_rows_f64(x)
    assert np.array_equal(np.isnan(o), np.isnan(ref))
    o, ref = np.nan_to_num(o), np.nan_to_num(ref)
    assert np.all(np.abs(o - ref) <= 1e-5 * ref + 1e-30)


def _layer_norm(native, oracle, g):
    R, C = _logu(g, 1, 2000), _cols(g)
    while R * C > 8e6:
        R = max(1, R // 2)
    x = (g.normal(0, float(g.choice([0.1, 3, 30])), (R, C)) + g.normal(0, 50)).astype(np.float32)
    gamma = g.uniform(0.5, 1.5, C).astype(np.float32)
    beta = g.uniform(-1, 1, C).astype(np.float32)
    off = int(g.choice([0, 1]))
    dx, px = _with_offset(native, x, off)
    dg, db = native.DeviceBuffer.from_array(gamma), native.DeviceBuffer.from_array(beta)
    do = _canary_buffer(native, R * C)
    announce(f"random layer_norm {R}x{C} off={off}")
    native.layer_norm_rows_f32(px, do, dg, db, R, C, 1e-5)
    out = do.download((R * C + 16,), np.float32)
    assert np.all(np.isnan(out[R * C:])), "wrote past the end"
    o = out[:R * C].reshape(R, C).astype(np.float64)
    ref = oracle.layer_norm_f64(x, gamma, beta, 1e-5)
    assert np.all(np.abs(o - ref) <= 1e-5 * np.maximum(1.0, np.abs(ref)))


def _reduce(native, oracle, g):
    n = _logu(g, 1, 20_000_000)
    off = int(g.integers(0, 4))
    x = (g.uniform(-1, 1, n) * (10.0 ** g.integers(-3, 4))).astype(np.float32)
    dx, px = _with_offset(native, x, off)
    do = native.DeviceBuffer.from_array(np.zeros(4, np.float32))
    announce(f"random sum/min/max n={n} off={off}")
    native.sum_f32(px, n, do)
    s = float(do.download((1,), np.float32)[0])
    native.min_f32(px, n, do)
    mn = do.download((1,), np.float32)[0]
    native.max_f32(px, n, do)
    mx = do.download((1,), np.float32)[0]
    s64 = oracle.sum_f64(x)
    assert abs(s - s64) <= 1e-5 * abs(s64) + 6e-8 * float(np.sum(np.abs(x.astype(np.float64))))
    assert mn == oracle.fmin(x) and mx == oracle.fmax(x)


def _sum_axis(native, oracle, g):
    nd = int(g.integers(1, 4))
    shape = [_logu(g, 1, 300) for _ in range(nd)]
    shape[int(g.integers(0, nd))] = _logu(g, 1, 100000)
    while np.prod(shape) > 8e6:
        i = int(np.argmax(shape))
        shape[i] = max(1, shape[i] // 2)
    ax = int(g.integers(0, nd))
    x = g.normal(0, 3, shape).astype(np.float32)
    outer, inner = int(np.prod(shape[:ax])), int(np.prod(shape[ax + 1:]))
    dx, do = native.DeviceBuffer.from_array(x), _canary_buffer(native, outer * inner)
    announce(f"random sum_axis {shape} axis={ax}")
    native.sum_axis_f32(dx, outer, shape[ax], inner, do)
    got = do.download((outer * inner + 16,), np.float32)
    assert np.all(np.isnan(got[outer * inner:])), "wrote past the end"
    got = got[:outer * inner].astype(np.float64)
    ref = oracle.sum_axis_f64(x, ax).ravel()
    absref = oracle.sum_axis_f64(np.abs(x), ax).ravel()
    assert np.all(np.abs(got - ref) <= 1e-5 * np.abs(ref) + 6e-8 * absref + 1e-30)


def _argmax(native, oracle, g):
    rows, cols = _logu(g, 1, 2000), _logu(g, 1, 2_000_000)
    while rows * cols > 8e6:
        rows = max(1, rows // 2)
    x = g.uniform(-1, 1, (rows, cols)).astype(np.float32)
    kind = int(g.integers(0, 4))
    if kind == 1:
        x[np.arange(rows), g.integers(0, cols, rows)] = 2.0
        x[np.arange(rows), g.integers(0, cols, rows)] = 2.0
    elif kind == 2:
        x[g.random((rows, cols)) < 0.01] = np.nan
    elif kind == 3:
        x = (np.round(x * 4) / 4).astype(np.float32)
    off = int(g.integers(0, 4))
    dx, px = _with_offset(native, x, off)
    do = _canary_buffer(native, rows, np.int32)
    announce(f"random argmax {rows}x{cols} kind={kind} off={off}")
    native.argmax_rows_f32(px, rows, cols, do)
    got = do.download((rows + 16,), np.int32)
    assert np.all(got[rows:] == -7), "wrote past the end"
    assert np.array_equal(got[:rows], oracle.argmax_rows(x))


def _binary(native, oracle, g):
    nd = int(g.integers(1, 5))
    shape = [_logu(g, 1, 200) for _ in range(nd)]
    while np.prod(shape) > 4e6:
        i = int(np.argmax(shape))
        shape[i] = max(1, shape[i] // 2)
    op = int(g.integers(0, 4))  # add, sub, mul, div: correctly rounded, so bit-exact

    def operand():
        bshape = [s if g.random() < 0.6 else 1 for s in shape]
        a = g.uniform(0.5, 2, bshape).astype(np.float32)
        return a, [0 if bshape[d] == 1 else int(np.prod(bshape[d + 1:])) for d in range(nd)]
    a, sa = operand()
    b, sb = operand()
    n = int(np.prod(shape))
    da, db, do = native.DeviceBuffer.from_array(a), native.DeviceBuffer.from_array(b), \
        _canary_buffer(native, n)
    announce(f"random binary op={op} {shape} sa={sa} sb={sb}")
    native.binary_strided_f32(op, shape, da, sa, db, sb, do)
    got = do.download((n + 16,), np.float32)
    assert np.all(np.isnan(got[n:])), "wrote past the end"
    ref = oracle.binary_strided_f32(op, shape, a.ravel(), sa, b.ravel(), sb)
    assert np.array_equal(got[:n], np.asarray(ref, np.float32).ravel())


def _attention(native, oracle, g):
    B, H = int(g.integers(1, 4)), int(g.integers(1, 5))
    Sq, Sk = _logu(g, 1, 600), _logu(g, 1, 600)
    D = int(g.choice([16, 32, 64, 128]))
    merged = bool(g.integers(0, 2))
    scale = float(np.float32(1.0 / np.sqrt(D)))

    def make(S):
        if merged:
            buf = g.normal(0, 1, (B, S, H, D)).astype(np.float32)
            return buf, buf.transpose(0, 2, 1, 3), H * D, (S * H * D, D)
        buf = g.normal(0, 1, (B, H, S, D)).astype(np.float32)
        return buf, buf, D, (H * S * D, S * D)
    qb, Qv, ldq, sq = make(Sq)
    kb, Kv, ldk, sk = make(Sk)
    vb, Vv, ldv, sv = make(Sk)
    dQ, dK, dV = (native.DeviceBuffer.from_array(t) for t in (qb, kb, vb))
    dO = _canary_buffer(native, qb.size)
    announce(f"random attention B={B} H={H} Sq={Sq} Sk={Sk} D={D} merged={merged}")
    native.attention(Sq, Sk, D, scale, dQ, ldq, dK, ldk, dV, ldv, dO, ldq, B, H, sq, sk, sv, sq)
    out = dO.download((qb.size + 16,), np.float32)
    assert np.all(np.isnan(out[qb.size:])), "wrote past the end"
    o = out[:qb.size].reshape(qb.shape)
    Ov = o.transpose(0, 2, 1, 3) if merged else o
    S = np.einsum("...qd,...kd->...qk", Qv.astype(np.float64), Kv.astype(np.float64)) * scale
    P = np.exp(S - S.max(axis=-1, keepdims=True))
    ref = (P / P.sum(axis=-1, keepdims=True)) @ Vv.astype(np.float64)
    err = np.abs(Ov.astype(np.float64) - ref).max()
    assert np.isfinite(Ov).all() and err <= 2e-5 * np.sqrt(max(D, Sk)) * np.abs(Vv).max()


def _conv2d(native, oracle, g):
    N, H, W = int(g.integers(1, 4)), _logu(g, 1, 40), _logu(g, 1, 40)
    Ci, K, Co = _logu(g, 1, 96), int(g.choice([1, 2, 3, 3, 4, 5, 7])), _logu(g, 1, 200)
    x = g.normal(0, 1, (N, H, W, Ci)).astype(np.float32)
    w = g.normal(0, 1, (Co, K, K, Ci)).astype(np.float32)
    n = N * H * W * Co
    dx, dw, do = native.DeviceBuffer.from_array(x), native.DeviceBuffer.from_array(w), \
        _canary_buffer(native, n)
    announce(f"random conv2d N={N} H={H} W={W} C_in={Ci} K={K} C_out={Co}")
    native.conv2d(dx, dw, do, N, H, W, Ci, K, Co)
    out = do.download((n + 16,), np.float32)
    assert np.all(np.isnan(out[n:])), "wrote past the end"
    ref = oracle.conv2d_f64(x, w).reshape(-1, Co)
    refabs = oracle.conv2d_f64(np.abs(x), np.abs(w)).reshape(-1, Co)
    ok, nw, el = gemm_tolerance_ok(out[:n].reshape(-1, Co), ref, refabs, K * K * Ci)
    assert ok, (nw, el)


CASES = {"softmax": _softmax, "layer_norm": _layer_norm, "reduce": _reduce,
         "sum_axis": _sum_axis, "argmax": _argmax, "binary": _binary, "attention": _attention,
         "conv2d": _conv2d}


@pytest.mark.parametrize("i", range(N_CASES))
def test_ops_random(native, oracle, i):
    g = rng(41000 + i)
    CASES[KINDS[i % len(KINDS)]](native, oracle, g)
