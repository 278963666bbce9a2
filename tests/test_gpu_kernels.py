"""GPU parity of every C ABI entry point against the CPU oracle.

Bars (stated per test): bit-exact for integer/index results, min/max,
add/sub/mul/div, affine and fused affine chains; <= a few float32 ulps for
functions built on exp/pow (the GPU's and glibc's expf/powf differ by up to
1-2 ulp); relative 1e-5 for softmax, layer_norm and sums; SGEMM/GEMV
normwise 1e-5*sqrt(K) plus a per-element bound 1e-5*sqrt(K)*sum|a||b|.
"""

import math

import numpy as np
import pytest

from conftest import rng
from gpu_util import announce, down, empty, gemm_tolerance_ok, sigmoid_bound, ulp_diff, up

pytestmark = pytest.mark.gpu

ADD, SUB, MUL, DIV, POW = range(5)


# ---- elementwise --------------------------------------------------------------

@pytest.mark.parametrize("op", [ADD, SUB, MUL, DIV])
@pytest.mark.parametrize("n,a_len,b_len", [(4096, 4096, 4096), (4099, 4099, 4099),
                                           (4096, 4096, 1), (4096, 1, 4096),
                                           (4096, 4096, 256), (4096, 512, 4096),
                                           (1000, 1000, 7), (13, 1, 1)])
def test_binary_f32_exact(native, oracle, op, n, a_len, b_len):
    announce(f"binary_f32 op={op} n={n} a_len={a_len} b_len={b_len}")
    g = rng(100 + op)
    a = g.uniform(-2, 2, a_len).astype(np.float32)
    b = g.uniform(0.25, 2, b_len).astype(np.float32) * np.where(g.random(b_len) < 0.5, -1, 1).astype(np.float32)
    da, db, do = up(native, a), up(native, b), empty(native, n)
    native.binary_f32(op, da, a_len, db, b_len, do, n)
    out = down(native, do, n)
    ref = oracle.binary_mod_f32(op, a, b, n)
    assert np.array_equal(out, ref)


def test_binary_f32_pow_ulps(native, oracle):
    announce("binary_f32 pow")
    g = rng(7)
    a = g.uniform(0.1, 3, 5000).astype(np.float32)
    b = g.uniform(-3, 3, 5000).astype(np.float32)
    da, db, do = up(native, a), up(native, b), empty(native, 5000)
    native.binary_f32(POW, da, 5000, db, 5000, do, 5000)
    out = down(native, do, 5000)
    assert np.max(ulp_diff(out, oracle.binary_mod_f32(POW, a, b, 5000))) <= 2


def test_binary_reference_goldens(native, ref_vectors):
    announce("binary goldens")
    v = ref_vectors["vector_arith"]
    a, b = np.array(v["a"], np.float32), np.array(v["b"], np.float32)
    da, db, do = up(native, a), up(native, b), empty(native, 16)
    for op, key in [(ADD, "add"), (SUB, "sub"), (MUL, "mul"), (DIV, "div")]:
        native.binary_f32(op, da, 16, db, 16, do, 16)
        assert np.max(np.abs(down(native, do, 16) - v[key])) <= v["tol_abs"], key
    m = ref_vectors["msl_add"]
    da, db, do = up(native, np.float32(m["bcast_a"])), up(native, np.float32(m["bcast_b"])), empty(native, 4)
    native.binary_f32(ADD, da, 4, db, 1, do, 4)
    assert np.array_equal(down(native, do, 4), m["bcast_out"])
    ia, ib, io = up(native, np.int32(m["int_a"])), up(native, np.int32(m["int_b"])), empty(native, 4, np.int32)
    native.binary_i32(ADD, ia, 4, ib, 4, io, 4)
    assert np.array_equal(down(native, io, 4, np.int32), m["int_out"])


@pytest.mark.parametrize("op", [ADD, SUB, MUL, DIV, POW])
def test_binary_i32_exact(native, oracle, op):
    announce(f"binary_i32 op={op}")
    g = rng(200 + op)
    n = 3001
    a = g.integers(-50, 50, n).astype(np.int32)
    b = g.integers(1, 6, 97).astype(np.int32) if op != SUB else g.integers(-9, 9, 97).astype(np.int32)
    if op == POW:
        a = g.integers(-6, 6, n).astype(np.int32)
        b = g.integers(0, 5, 97).astype(np.int32)
    da, db, do = up(native, a), up(native, b), empty(native, n, np.int32)
    native.binary_i32(op, da, n, db, 97, do, n)
    assert np.array_equal(down(native, do, n, np.int32), oracle.binary_mod_i32(op, a, b, n))


@pytest.mark.parametrize("shape,sa_shape,sb_shape", [
    ((2, 2, 3), (2, 2, 3), (2, 1, 3)),     # middle-axis broadcast
    ((3, 3), (3, 1), (1, 3)),              # two-sided
    ((4, 5, 6, 7), (4, 1, 6, 1), (1, 5, 1, 7)),
    ((64, 300), (64, 300), (300,)),
])
def test_binary_strided(native, oracle, shape, sa_shape, sb_shape):
    announce(f"binary_strided {shape}")
    g = rng(300)
    a = g.uniform(-1, 1, sa_shape).astype(np.float32)
    b = g.uniform(-1, 1, sb_shape).astype(np.float32)
    ab = np.broadcast_to(a, shape)
    bb = np.broadcast_to(b.reshape((1,) * (len(shape) - b.ndim) + b.shape), shape)
    sa = [s // 4 for s in ab.strides]
    sb = [s // 4 for s in bb.strides]
    da, db, do = up(native, a), up(native, b), empty(native, int(np.prod(shape)))
    native.binary_strided_f32(MUL, shape, da, sa, db, sb, do)
    out = down(native, do, shape)
    assert np.array_equal(out, oracle.binary_strided_f32(MUL, shape, a, sa, b, sb))
    assert np.array_equal(out, ab * bb)


@pytest.mark.parametrize("n", [1, 5, 4096, 100003])
def test_unary(native, oracle, n):
    announce(f"unary n={n}")
    x = rng(400).normal(0, 4, n).astype(np.float32)
    dx, do = up(native, x), empty(native, n)
    native.unary_f32(native.SIGMOID, dx, do, n)
    assert np.max(ulp_diff(down(native, do, n), oracle.sigmoid(x))) <= 4
    native.unary_f32(native.RELU, dx, do, n)
    assert np.array_equal(down(native, do, n), oracle.relu(x))


def test_unary_goldens(native, ref_vectors):
    announce("unary goldens")
    s = ref_vectors["sigmoid"]
    dx, do = up(native, np.float32(s["x"])), empty(native, 5)
    native.unary_f32(native.SIGMOID, dx, do, 5)
    out = down(native, do, 5)
    assert np.max(np.abs(out[:3] - s["expected_first3"])) <= s["tol_abs"]
    assert out[3] > s["x3_gt"] and out[4] < s["x4_lt"]


def test_bias_sigmoid_and_backward(native, oracle):
    announce("bias_sigmoid / sigmoid_backward")
    g = rng(500)
    d = g.normal(0, 1, (33, 70)).astype(np.float32)
    b = g.normal(0, 1, 70).astype(np.float32)
    dd, db = up(native, d), up(native, b)
    native.bias_sigmoid_f32(dd, db, d.size, 70)
    assert np.max(ulp_diff(down(native, dd, d.shape), oracle.bias_sigmoid(d, b))) <= 4
    dout = g.normal(0, 1, 999).astype(np.float32)
    x = g.normal(0, 2, 999).astype(np.float32)
    ddo, dxx, do = up(native, dout), up(native, x), empty(native, 999)
    native.sigmoid_backward_f32(ddo, dxx, do, 999)
    ref = oracle.sigmoid_backward(dout, x)
    assert np.max(np.abs(down(native, do, 999) - ref) / (np.abs(ref) + 1e-30)) < 2e-6


@pytest.mark.parametrize("n", [4096, 4097, 3])
def test_affine_exact(native, oracle, n):
    announce(f"affine n={n}")
    x = rng(600).uniform(-1, 1, n).astype(np.float32)
    dx, do = up(native, x), empty(native, n)
    native.affine_f32(dx, do, n, 1.7, -0.3)
    assert np.array_equal(down(native, do, n), oracle.affine(x, 1.7, -0.3))


# ---- fused program ----------------------------------------------------------------

@pytest.mark.parametrize("n", [1 << 20, 1001])
def test_program_affine_chain_exact(native, oracle, n):
    announce(f"program chain n={n}")
    g = rng(700)
    x = g.uniform(-1, 1, n).astype(np.float32)
    sc = g.uniform(0.9, 1.1, 20).astype(np.float32)
    of = g.uniform(-0.1, 0.1, 20).astype(np.float32)
    dx, do = up(native, x), empty(native, n)
    instrs = [(native.PI_LOAD, 0, 0, 0, 0.0, 0.0)] + \
             [(native.PI_FMAI, 0, 0, 0, float(a), float(b)) for a, b in zip(sc, of)]
    prog = native.make_program((n,), [(dx, (1,))], instrs)
    native.program_f32(prog, do)
    assert np.array_equal(down(native, do, n), oracle.affine_chain(x, sc, of))


def test_program_general_graph(native, oracle):
    """relu(x*w + b) - sigmoid(y) / 3 with b broadcast over rows, y full."""
    announce("program general")
    g = rng(710)
    R, Cc = 37, 129
    x = g.normal(0, 1, (R, Cc)).astype(np.float32)
    y = g.normal(0, 1, (R, Cc)).astype(np.float32)
    b = g.normal(0, 1, Cc).astype(np.float32)
    dx, dy, dbb, do = up(native, x), up(native, y), up(native, b), empty(native, R * Cc)
    P = native
    instrs = [(P.PI_LOAD, 0, 0), (P.PI_MULI, 0, 0, 0, 0.75), (P.PI_LOAD, 1, 2),
              (P.PI_ADD, 0, 0, 1), (P.PI_RELU, 0, 0), (P.PI_LOAD, 2, 1), (P.PI_SIGMOID, 2, 2),
              (P.PI_CONST, 3, 0, 0, 3.0), (P.PI_DIV, 2, 2, 3), (P.PI_SUB, 0, 0, 2)]
    prog = P.make_program((R, Cc), [(dx, (Cc, 1)), (dy, (Cc, 1)), (dbb, (0, 1))], instrs)
    P.program_f32(prog, do)
    out = down(native, do, (R, Cc))
    t = oracle.relu(oracle.binary_mod_f32(ADD, oracle.binary_mod_f32(MUL, x.ravel(), [0.75], x.size),
                                          b, x.size))
    s = oracle.binary_mod_f32(DIV, oracle.sigmoid(y.ravel()), [3.0], y.size)
    ref = oracle.binary_mod_f32(SUB, t, s, x.size).reshape(R, Cc)
    # Every op but sigmoid is correctly rounded on both sides, and the GPU's
    # expf may differ from glibc's by 1-2 ulp.  The final subtraction can
    # cancel, so the bound is 4 ulp of the operands' magnitude, not of the
    # result.
    scale = (np.abs(t) + np.abs(s)).reshape(R, Cc)
    assert np.all(np.abs(out - ref) <= 4 * np.finfo(np.float32).eps * scale + 1e-30)


# How the program kernel reads each input: contiguous (16-byte aligned or
# not), a block repeated along the leading axes (period a multiple of 4 or
# not, aligned or not), general strides, a scalar.  (shape, [(base offset in
# elements, strides)], buffer lengths): out = (in0 * in1 + in2) - in0, which is
# correctly rounded in fp32 on both sides.
PROGRAM_MODE_CASES = [
    ("contig aligned, ragged", (2048 * 3 + 5,), [(0, (1,)), (0, (1,)), (0, (1,))]),
    ("contig unaligned", (4099,), [(1, (1,)), (3, (1,)), (0, (1,))]),
    ("row period 512", (33, 512), [(0, (512, 1)), (0, (0, 1)), (0, (512, 1))]),
    ("row period 129", (37, 129), [(0, (129, 1)), (0, (0, 1)), (1, (0, 1))]),
    ("row period unaligned", (20, 64), [(0, (64, 1)), (1, (0, 1)), (0, (0, 0))]),
    ("matrix period", (3, 17, 24), [(0, (408, 24, 1)), (0, (0, 24, 1)), (0, (0, 0, 1))]),
    ("transposed", (31, 45), [(0, (1, 31)), (0, (45, 1)), (2, (0, 1))]),
    ("column broadcast", (40, 36), [(0, (36, 1)), (0, (1, 0)), (0, (0, 0))]),
]


def _strided_view(buf_flat, base, strides, shape):
    idx = np.zeros(shape, np.int64) + base
    for d, st in enumerate(strides):
        sh = [1] * len(shape)
        sh[d] = shape[d]
        idx = idx + (np.arange(shape[d]) * st).reshape(sh)
    return buf_flat[idx]


@pytest.mark.parametrize("name,shape,ins", PROGRAM_MODE_CASES, ids=[c[0] for c in PROGRAM_MODE_CASES])
def test_program_input_modes(native, name, shape, ins):
    announce(f"program input modes: {name} {shape}")
    g = rng(720)
    P = native
    bufs, vals = [], []
    for base, strides in ins:
        span = base + 1 + sum((e - 1) * st for e, st in zip(shape, strides))
        h = g.normal(0, 1, span + 3).astype(np.float32)
        bufs.append((up(native, h), base, strides))
        vals.append(_strided_view(h, base, strides, shape))
    n = int(np.prod(shape))
    do = empty(native, n)
    instrs = [(P.PI_LOAD, 0, 0), (P.PI_LOAD, 1, 1), (P.PI_MUL, 2, 0, 1), (P.PI_LOAD, 3, 2),
              (P.PI_ADD, 2, 2, 3), (P.PI_SUB, 2, 2, 0)]
    prog = P.make_program(shape, [(b.ptr + 4 * base, st) for b, base, st in bufs], instrs,
                          out_reg=2)
    P.program_f32(prog, do)
    a, b, c = vals
    ref = ((a * b) + c) - a
    assert np.array_equal(down(native, do, shape), ref.astype(np.float32))


# A program that is one binary operation on two loaded inputs runs on the
# binary kernels: (shape, (base, strides) of the left and right inputs,
# register order of the loads).
PROGRAM_BINARY_CASES = [
    ((4096,), (0, (1,)), (0, (1,)), False),
    ((4099,), (0, (1,)), (0, (1,)), True),
    ((64, 64), (0, (64, 1)), (0, (0, 0)), False),
    ((64, 64), (0, (0, 0)), (0, (64, 1)), True),
    ((16, 256), (0, (256, 1)), (0, (0, 1)), False),
    ((16, 256), (0, (0, 1)), (0, (256, 1)), False),
    ((30, 129), (0, (129, 1)), (0, (0, 1)), False),
    ((4096,), (1, (1,)), (0, (1,)), False),
]


@pytest.mark.parametrize("op", [ADD, SUB, MUL, DIV])
@pytest.mark.parametrize("shape,lhs,rhs,swap", PROGRAM_BINARY_CASES)
def test_program_single_binary_op(native, oracle, op, shape, lhs, rhs, swap):
    announce(f"program binary op={op} {shape} {lhs} {rhs} swap={swap}")
    g = rng(740 + op)
    P = native
    vals, ptrs = [], []
    for base, strides in (lhs, rhs):
        span = base + 1 + sum((e - 1) * st for e, st in zip(shape, strides))
        h = g.uniform(0.25, 2, span + 3).astype(np.float32) * np.where(
            g.random(span + 3) < 0.5, -1, 1).astype(np.float32)
        buf = up(native, h)
        ptrs.append((buf, base, strides))
        vals.append(_strided_view(h, base, strides, shape))
    n = int(np.prod(shape))
    do = empty(native, n)
    pi = {ADD: P.PI_ADD, SUB: P.PI_SUB, MUL: P.PI_MUL, DIV: P.PI_DIV}[op]
    # registers: left in r3, right in r1; the loads in either order
    loads = [(P.PI_LOAD, 3, 0), (P.PI_LOAD, 1, 1)]
    if swap:
        loads.reverse()
    prog = P.make_program(shape, [(b.ptr + 4 * base, st) for b, base, st in ptrs],
                          loads + [(pi, 5, 3, 1)], out_reg=5)
    P.program_f32(prog, do)
    a, b = (v.ravel() for v in vals)
    assert np.array_equal(down(native, do, n), oracle.binary_mod_f32(op, a, b, n))


def test_program_period_beyond_32bit_index(native):
    """More than 2^32 output elements: the repeated-block offset takes 64-bit
    arithmetic.  out[r, c] = row[c] * 2 + s over a [4294980, 1000] output
    (16 GiB), checked on slices at both ends and across element 2^32."""
    announce("program over 2^32 elements")
    P = native
    rows = (1 << 32) // 1000 + 13
    n = rows * 1000
    row = rng(730).normal(0, 1, 1000).astype(np.float32)
    drow, ds = up(native, row), up(native, np.array([0.25], np.float32))
    out = native.DeviceBuffer(4 * n)
    try:
        instrs = [(P.PI_LOAD, 0, 0), (P.PI_MULI, 0, 0, 0, 2.0), (P.PI_LOAD, 1, 1),
                  (P.PI_ADD, 0, 0, 1)]
        prog = P.make_program((rows, 1000), [(drow, (0, 1)), (ds, (0, 0))], instrs)
        P.program_f32(prog, out)
        expect = np.tile(row * np.float32(2.0) + np.float32(0.25), 3)
        for start in (0, (1 << 32) // 1000 * 1000 - 1000, n - 3000):
            got = out.download(3000, offset_bytes=4 * start)
            assert np.array_equal(got, expect), start
    finally:
        out.free()
        native.call("silgpu_pool_trim")


# ---- reductions ------------------------------------------------------------------

# Sizes of whole 4096-float load groups (25,165,824) and ones that end a
# few floats into a group (8,388,612, 20,480,012, and 20,480,013 unaligned).
@pytest.mark.parametrize("n,offset", [(1, 0), (7, 0), (1000, 1), (65536, 0), (1 << 22, 3),
                                      (12345679, 2), (25165824, 0), (8388612, 0),
                                      (20480012, 0), (20480013, 1)])
def test_sum_min_max(native, oracle, n, offset):
    announce(f"sum/min/max n={n} offset={offset}")
    g = rng(800 + n % 97)
    x = g.uniform(-1, 1, n + offset).astype(np.float32)
    dx, do = up(native, x), empty(native, 1)
    view = dx.ptr + 4 * offset
    native.sum_f32(view, n, do)
    s = float(down(native, do, 1)[0])
    s64 = oracle.sum_f64(x[offset:])
    assert abs(s - s64) <= 1e-5 * abs(s64) + 1e-6, (s, s64)
    native.min_f32(view, n, do)
    assert down(native, do, 1)[0] == oracle.fmin(x[offset:])
    native.max_f32(view, n, do)
    assert down(native, do, 1)[0] == oracle.fmax(x[offset:])


def test_sum_empty_and_min_empty(native):
    announce("sum empty")
    do = empty(native, 1)
    native.sum_f32(do, 0, do)
    assert down(native, do, 1)[0] == 0.0
    with pytest.raises(native.SilGpuError):
        native.min_f32(do, 0, do)


def test_reduction_goldens(native, ref_vectors):
    announce("reduction goldens")
    ag = ref_vectors["aggregates"]
    t = np.array(ag["t_3_2_3"], np.float32)
    dt, do = up(native, t), empty(native, 16)
    native.sum_f32(dt, t.size, do)
    assert down(native, do, 1)[0] == ag["sum"]
    for ax in range(3):
        outer = int(np.prod(t.shape[:ax]))
        inner = int(np.prod(t.shape[ax + 1:]))
        native.sum_axis_f32(dt, outer, t.shape[ax], inner, do)
        got = down(native, do, outer * inner)
        assert np.array_equal(got, np.ravel(ag[f"sum{ax}"])), ax
    ones = up(native, np.ones((256, 128), np.float32))
    native.sum_f32(ones, 256 * 128, do)
    assert down(native, do, 1)[0] == ag["ones_256x128_sum"]
    native.sum_axis_f32(ones, 1, 256, 128, do)
    assert down(native, do, 1)[0] == ag["ones_256x128_sum0_first"]


@pytest.mark.parametrize("shape,axis", [((4096, 8192), 1), ((4096, 8192), 0), ((3, 100000), 1),
                                        ((100, 3), 1), ((7, 300, 9), 1), ((5, 4, 3, 2), 2),
                                        ((1, 5000000), 1), ((20000, 4), 0), ((70000, 2), 1)])
def test_sum_axis(native, oracle, shape, axis):
    announce(f"sum_axis {shape} axis={axis}")
    x = rng(900).normal(0, 3, shape).astype(np.float32)
    outer = int(np.prod(shape[:axis]))
    inner = int(np.prod(shape[axis + 1:]))
    dx, do = up(native, x), empty(native, outer * inner)
    native.sum_axis_f32(dx, outer, shape[axis], inner, do)
    got = down(native, do, outer * inner).astype(np.float64)
    ref = oracle.sum_axis_f64(x, axis).ravel()
    absref = oracle.sum_axis_f64(np.abs(x), axis).ravel()
    # relative 1e-5 of the exact sum, with the fp32 output rounding (2^-24 of
    # the magnitude) as a floor for sums that cancel to near zero
    assert np.all(np.abs(got - ref) <= 1e-5 * np.abs(ref) + 6e-8 * absref + 1e-30)


@pytest.mark.parametrize("rows,cols", [(2, 3), (4096, 256), (1024, 2048), (1, 67108864),
                                       (64, 100003), (3, 1 << 20), (70000, 5)])
def test_argmax_rows(native, oracle, rows, cols):
    announce(f"argmax {rows}x{cols}")
    g = rng(1000 + rows)
    x = g.uniform(-1, 1, (rows, cols)).astype(np.float32)
    # a unique planted maximum not aligned to 4 or to a workgroup chunk, and ties
    x[:, (cols * 7) // 9] = 2.0
    if cols > 10:
        x[rows // 2, 3] = 2.0  # tie with the later column: first index must win
    dx, do = up(native, x), empty(native, rows, np.int32)
    native.argmax_rows_f32(dx, rows, cols, do)
    assert np.array_equal(down(native, do, rows, np.int32), oracle.argmax_rows(x))


def test_argmax_long_row_rules(native, oracle):
    """Rows long enough for the split float4 kernel: the maximum shares a
    float4 group with NaN and with a tie, equal maxima sit in different
    chunks, signed zeros tie, a row is all NaN, and one row is all negative
    with NaNs."""
    announce("argmax long-row rules")
    cols = (1 << 20) + 8
    g = rng(4242)
    x = g.uniform(-1, 1, (6, cols)).astype(np.float32)
    base = 4 * 100003                       # start of a float4 group
    x[0, base:base + 4] = [np.nan, 7.0, 9.0, 9.0]   # first 9 (lane 2) wins
    x[1, 17] = 5.0
    x[1, cols - 3] = 5.0                    # tie in another chunk: 17 wins
    x[2, :] = 0.0
    x[2, 5] = -0.0                          # all equal: index 0
    x[3, :] = np.nan                        # no number: index 0
    x[4, :] = -np.abs(x[4, :]) - 1.0
    x[4, ::7] = np.nan
    x[4, 999_999] = -0.5                    # the largest of a negative row
    x[5, 3 * (cols // 4) + 1: 3 * (cols // 4) + 3] = [3.0, 3.0]  # tie within a group
    dx, do = up(native, x), empty(native, 6, np.int32)
    native.argmax_rows_f32(dx, 6, cols, do)
    got = down(native, do, 6, np.int32)
    ref = oracle.argmax_rows(x)
    assert list(ref) == [base + 2, 17, 0, 0, 999_999, 3 * (cols // 4) + 1]
    assert np.array_equal(got, ref)


def test_argmax_golden_nan_negative(native, oracle, ref_vectors):
    announce("argmax goldens")
    a = np.array(ref_vectors["argmax"]["x"], np.float32)
    dx, do = up(native, a), empty(native, 2, np.int32)
    native.argmax_rows_f32(dx, 2, 3, do)
    assert list(down(native, do, 2, np.int32)) == ref_vectors["argmax"]["out"]
    z = np.array([[np.nan, 1.0, 3.0, np.nan, -1.0, 3.0], [-5, -4, -3, -2, -1, -9]], np.float32)
    dz, do = up(native, z), empty(native, 2, np.int32)
    native.argmax_rows_f32(dz, 2, 6, do)
    assert list(down(native, do, 2, np.int32)) == list(oracle.argmax_rows(z)) == [2, 4]


def test_wave_exchange_lane_patterns(native, oracle):
    """Rows whose deciding values sit in single lanes of different 16-lane
    rows of a wavefront (and of different wavefronts for 512-thread rows), so
    the in-register exchanges must carry them across rows and waves.  In the
    one-wavefront argmax, column c is scanned by lane c % 64; in the row ops,
    thread t holds columns 4(k NT + t) .. + 3."""
    announce("wave exchange lane patterns")
    cols = 256
    x = np.full((7, cols), -1.0, np.float32)
    x[0, [48, 32, 16, 64]] = 5.0            # lanes 48, 32, 16, 0: first index (16)
    x[1, [127, 66, 250]] = 5.0              # lanes 63, 2, 58: 66
    x[2, :] = np.nan                        # no number: index 0
    x[3, 0:16] = np.nan
    x[3, 175] = 0.5                         # lane 47 past a row of NaN lanes
    x[4, 99] = -0.0                         # lane 35
    x[4, 20] = 0.0                          # lane 20: equal to -0, first index wins
    x[5, :] = -np.inf
    x[5, 61] = -3e38                        # the only number, lane 61
    x[6, :] = np.nan
    x[6, 200] = -np.inf                     # lane 8: -inf beats no number
    dx, do = up(native, x), empty(native, 7, np.int32)
    native.argmax_rows_f32(dx, 7, cols, do)
    ref = oracle.argmax_rows(x)
    assert list(ref) == [16, 66, 0, 175, 20, 61, 200]
    assert np.array_equal(down(native, do, 7, np.int32), ref)

    # softmax / layer_norm: one-wavefront rows (256 columns: thread t holds
    # 4t .. 4t + 3) and 512-thread rows (8192 columns, 8 wavefronts)
    for rows, cols, spots in [(3, 256, [(201, 2.0), (13, 1.0)]),
                              (3, 8192, [(4 * (2 * 512 + 357) + 1, 2.0), (13, 1.0),
                                         (4 * (3 * 512 + 511) + 3, 0.5)])]:
        y = np.full((rows, cols), -np.inf, np.float32)
        for c, v in spots:
            y[0, c] = v                       # finite values in two or three lanes only
        y[1] = rng(77).normal(0, 1, cols)
        y[1, cols - 1] = 30.0                 # the last lane's value dominates
        y[2] = rng(78).normal(0, 3, cols)
        dy, do = up(native, y), empty(native, rows * cols)
        native.softmax_rows_f32(dy, do, rows, cols)
        out = down(native, do, (rows, cols)).astype(np.float64)
        sref = oracle.softmax_rows_f64(y)
        assert np.all(np.abs(out - sref) <= 1e-5 * sref + 1e-30), cols
        z = np.zeros((rows, cols), np.float32)
        for c, v in spots:
            z[0, c] = 100.0 * v                # outliers in single lanes
        z[1], z[2] = y[1], y[2]
        gamma = np.ones(cols, np.float32)
        beta = np.zeros(cols, np.float32)
        dz, dg, db = up(native, z), up(native, gamma), up(native, beta)
        native.layer_norm_rows_f32(dz, do, dg, db, rows, cols, 1e-5)
        out = down(native, do, (rows, cols)).astype(np.float64)
        lref = oracle.layer_norm_f64(z, gamma, beta, 1e-5)
        assert np.all(np.abs(out - lref) <= 1e-5 * np.maximum(1.0, np.abs(lref))), cols


# ---- row ops ----------------------------------------------------------------------

# Every register configuration in its three modes: rows that exactly fill the
# tile (256, 512, 1024, 2048, 4096, 8192, 16384), float4 rows with a ragged
# end (768, 1000, 3000, 6000, 12000), scalar rows (3, 1001, 4097, 6001,
# 9999), the looped kernel (40000), and row counts that leave a partial
# workgroup.
ROW_SHAPES = [(2, 3), (64, 32), (7, 256), (300, 512), (5, 1024), (50, 2048), (9, 4096),
              (4096, 8192), (3, 16384), (2048, 768), (100, 1000), (33, 3000), (11, 6000),
              (6, 12000), (9, 1001), (7, 4097), (5, 6001), (4, 9999), (5, 40000), (1, 1)]


@pytest.mark.parametrize("rows,cols", ROW_SHAPES)
def test_softmax_rows(native, oracle, rows, cols):
    announce(f"softmax {rows}x{cols}")
    x = rng(1100 + cols).normal(0, 3, (rows, cols)).astype(np.float32)
    dx, do = up(native, x), empty(native, rows * cols)
    native.softmax_rows_f32(dx, do, rows, cols)
    out = down(native, do, (rows, cols)).astype(np.float64)
    ref = oracle.softmax_rows_f64(x)
    # relative 1e-5 per element (entries below 1e-30 compared absolutely)
    assert np.all(np.abs(out - ref) <= 1e-5 * ref + 1e-30)


@pytest.mark.parametrize("rows,cols", [(5, 20000), (3, 16387), (4, 8192), (6, 1000), (7, 2)])
def test_softmax_neg_inf_entries(native, oracle, rows, cols):
    """-inf entries (masked scores) add exp(-inf) = 0 to their row, also when
    they are the first values a thread of the looped kernel (rows over 16384)
    reads; a row of -inf only is NaN, as exp(-inf - max) is in float64."""
    announce(f"softmax -inf entries {rows}x{cols}")
    x = rng(1150 + cols).normal(0, 3, (rows, cols)).astype(np.float32)
    x[0, : min(cols - 1, 300): 3] = -np.inf   # the first value of every third thread
    x[1, -1] = -np.inf
    x[2, :] = -np.inf
    if rows > 3:
        x[3, 1:] = -np.inf                  # one finite entry: probability 1
    dx, do = up(native, x), empty(native, rows * cols)
    native.softmax_rows_f32(dx, do, rows, cols)
    out = down(native, do, (rows, cols)).astype(np.float64)
    with np.errstate(invalid="ignore"):
        ref = oracle.softmax_rows_f64(x)
    assert np.all(np.isnan(out[2])) and np.all(np.isnan(ref[2]))
    keep = [r for r in range(rows) if r != 2]
    assert np.all(np.abs(out[keep] - ref[keep]) <= 1e-5 * ref[keep] + 1e-30)


def test_softmax_golden(native, ref_vectors):
    announce("softmax golden")
    s = ref_vectors["softmax"]
    dx, do = up(native, np.float32([s["x"]])), empty(native, 3)
    native.softmax_rows_f32(dx, do, 1, 3)
    assert np.max(np.abs(down(native, do, 3) - s["expected"])) <= s["tol_abs"]


@pytest.mark.parametrize("rows,cols", ROW_SHAPES + [(3, 50000)])
def test_layer_norm_rows(native, oracle, rows, cols):
    announce(f"layer_norm {rows}x{cols}")
    g = rng(1200 + cols)
    x = g.normal(0, 3, (rows, cols)).astype(np.float32)
    if rows * cols <= 1 << 20:
        gamma = g.uniform(0.5, 1.5, cols).astype(np.float32)
        beta = g.uniform(-1, 1, cols).astype(np.float32)
    else:
        gamma = np.ones(cols, np.float32)
        beta = np.zeros(cols, np.float32)
    dx, dg, db, do = up(native, x), up(native, gamma), up(native, beta), empty(native, rows * cols)
    native.layer_norm_rows_f32(dx, do, dg, db, rows, cols, 1e-5)
    out = down(native, do, (rows, cols)).astype(np.float64)
    ref = oracle.layer_norm_f64(x, gamma, beta, 1e-5)
    # |y - y64| <= 1e-5 * max(1, |y64|): relative 1e-5 at the unit scale the
    # normalisation produces
    assert np.all(np.abs(out - ref) <= 1e-5 * np.maximum(1.0, np.abs(ref)))


@pytest.mark.parametrize("rows,cols", [(64, 8192), (17, 768), (33, 3000), (5, 1001), (3, 50000)])
def test_layer_norm_outlier_and_constant_rows(native, oracle, rows, cols):
    """A first value 100 sigma out, and a constant row (variance exactly 0,
    so the output is beta), match the float64 two-pass statistics."""
    announce(f"layer_norm outlier first value {rows}x{cols}")
    x = rng(1300 + cols).normal(0, 3, (rows, cols)).astype(np.float32)
    x[:, 0] = 300.0
    x[1, 0] = -300.0
    x[2, :] = 1.25
    gamma = np.ones(cols, np.float32)
    beta = np.linspace(-1, 1, cols).astype(np.float32)
    dx, dg, db, do = up(native, x), up(native, gamma), up(native, beta), empty(native, rows * cols)
    native.layer_norm_rows_f32(dx, do, dg, db, rows, cols, 1e-5)
    out = down(native, do, (rows, cols)).astype(np.float64)
    ref = oracle.layer_norm_f64(x, gamma, beta, 1e-5)
    assert np.all(np.abs(out - ref) <= 1e-5 * np.maximum(1.0, np.abs(ref)))
    assert np.array_equal(out[2], beta.astype(np.float64))


@pytest.mark.parametrize("rows,cols", [(64, 2), (33, 5), (17, 768), (9, 8192), (3, 50000)])
def test_layer_norm_large_mean(native, oracle, rows, cols):
    """Rows whose spread is small against their mean (1000 +- 0.01, -300 +-
    0.001, 1e5 +- 0.5): each deviation is taken from the fp64 mean, so the
    output keeps the relative 1e-5 bar; subtracting the float-rounded mean
    would err by up to half an ulp of the mean (3e-5 at 1000) in every
    deviation."""
    announce(f"layer_norm large mean {rows}x{cols}")
    g = rng(1400 + cols)
    x = np.empty((rows, cols), np.float32)
    for r in range(rows):
        mean, spread = [(1000.0, 0.01), (-300.0, 1e-3), (1e5, 0.5)][r % 3]
        x[r] = (mean + g.normal(0, spread, cols)).astype(np.float32)
    gamma = g.uniform(0.5, 1.5, cols).astype(np.float32)
    beta = g.uniform(-1, 1, cols).astype(np.float32)
    dx, dg, db, do = up(native, x), up(native, gamma), up(native, beta), empty(native, rows * cols)
    native.layer_norm_rows_f32(dx, do, dg, db, rows, cols, 1e-5)
    out = down(native, do, (rows, cols)).astype(np.float64)
    ref = oracle.layer_norm_f64(x, gamma, beta, 1e-5)
    assert np.all(np.abs(out - ref) <= 1e-5 * np.maximum(1.0, np.abs(ref)))


def test_layer_norm_golden(native, ref_vectors):
    announce("layer_norm golden")
    ln = ref_vectors["layer_norm"]
    x = np.array(ln["x"], np.float32)
    dx, do = up(native, x), empty(native, 6)
    native.layer_norm_rows_f32(dx, do, up(native, np.float32(ln["gamma"])),
                               up(native, np.float32(ln["beta"])), 2, 3, 1e-5)
    assert np.max(np.abs(down(native, do, (2, 3))[0] - ln["row0"])) <= ln["tol_abs"]


# ---- GEMM / GEMV ------------------------------------------------------------------

def _gemm_case(native, oracle, M, N, K, ta=False, tb=False, epi=0, bias_len=0, seed=0,
               dist="uniform"):
    g = rng(seed + 7 * M + 3 * N + K)
    if dist == "uniform":
        A = g.uniform(-1, 1, (K, M) if ta else (M, K)).astype(np.float32)
        B = g.uniform(-1, 1, (N, K) if tb else (K, N)).astype(np.float32)
    else:
        A = g.normal(0, 0.02, (K, M) if ta else (M, K)).astype(np.float32)
        B = g.normal(0, 0.02, (N, K) if tb else (K, N)).astype(np.float32)
    dA, dB, dC = up(native, A), up(native, B), empty(native, M * N)
    bias = g.normal(0, 1, max(bias_len, 1)).astype(np.float32)
    dbias = up(native, bias) if bias_len else None
    native.sgemm(ta, tb, M, N, K, dA, A.shape[1], 0, dB, B.shape[1], 0, dC, N, 0, 1,
                 dbias, bias_len, epi)
    Cg = down(native, dC, (M, N))
    C64, Cabs = oracle.sgemm_f64(A, B, ta=ta, tb=tb, with_abs=True)
    if epi in (native.EPI_BIAS, native.EPI_BIAS_SIGMOID, native.EPI_BIAS_RELU):
        bb = bias[np.arange(N) % bias_len].astype(np.float64)
        C64 = C64 + bb
        Cabs = Cabs + np.abs(bb)
    if epi == native.EPI_BIAS_SIGMOID:
        C64, Cabs = sigmoid_bound(C64, Cabs, K)
    if epi in (native.EPI_RELU, native.EPI_BIAS_RELU):
        C64 = np.maximum(C64, 0)
    return Cg, C64, Cabs


ROUTING_SHAPES = [(1, 16, 3), (15, 16, 16), (16, 16, 16), (17, 50, 17), (32, 768, 4096),
                  (33, 65, 15), (63, 64, 784), (64, 64, 64), (96, 4096, 8), (97, 1, 17),
                  (100, 768, 784), (128, 128, 16), (256, 512, 130), (1, 4096, 4096),
                  (64, 1, 300), (3, 5, 1),
                  # small products the plan splits 8 or 16 ways along K
                  (256, 512, 2048), (128, 768, 2048), (64, 2048, 768), (256, 512, 256)]


@pytest.mark.parametrize("M,N,K", ROUTING_SHAPES)
def test_sgemm_routing_shapes(native, oracle, M, N, K):
    announce(f"sgemm NN {M}x{N}x{K}")
    Cg, C64, Cabs = _gemm_case(native, oracle, M, N, K)
    ok, nw, el = gemm_tolerance_ok(Cg, C64, Cabs, K)
    assert ok, (nw, el)


@pytest.mark.parametrize("ta,tb", [(0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(4, 3, 2), (17, 33, 65), (128, 256, 64), (200, 130, 70),
                                   (1, 300, 200), (300, 1, 200)])
def test_sgemm_transposed(native, oracle, ta, tb, M, N, K):
    announce(f"sgemm ta={ta} tb={tb} {M}x{N}x{K}")
    Cg, C64, Cabs = _gemm_case(native, oracle, M, N, K, ta=ta, tb=tb)
    ok, nw, el = gemm_tolerance_ok(Cg, C64, Cabs, K)
    assert ok, (nw, el)


@pytest.mark.parametrize("epi,bias_len", [(1, 96), (2, 96), (3, 0), (4, 96), (1, 32)])
@pytest.mark.parametrize("M,N,K", [(100, 96, 48), (256, 384, 256), (1, 96, 64)])
def test_sgemm_epilogues(native, oracle, epi, bias_len, M, N, K):
    announce(f"sgemm epi={epi} {M}x{N}x{K}")
    Cg, C64, Cabs = _gemm_case(native, oracle, M, N, K, epi=epi, bias_len=bias_len)
    ok, nw, el = gemm_tolerance_ok(Cg, C64, Cabs, K)
    assert ok, (nw, el)


def test_sgemm_reference_goldens(native, ref_vectors):
    announce("sgemm goldens")
    d = ref_vectors["dot"]
    a = np.float32(d["mm_a_3x4_iota1"])
    b = np.float32(d["mm_b_4x2_iota1"])
    dA, dB, dC = up(native, a), up(native, b), empty(native, 6)
    native.sgemm(0, 0, 3, 2, 4, dA, 4, 0, dB, 2, 0, dC, 2, 0)
    assert np.array_equal(down(native, dC, (3, 2)), d["mm_out"])
    lin = ref_vectors["linear"]
    dX, dW, dbias, dO = (up(native, np.float32(lin["x"])), up(native, np.float32(lin["W"])),
                         up(native, np.float32(lin["b"])), empty(native, 4))
    native.sgemm(0, 0, 2, 2, 3, dX, 3, 0, dW, 2, 0, dO, 2, 0, 1, dbias, 2, native.EPI_BIAS)
    assert np.array_equal(down(native, dO, (2, 2)), lin["out"])
    e = ref_vectors["dot_example"]
    dx, dW, dy = up(native, np.float32(e["x"])), up(native, np.float32(e["W"])), empty(native, 2)
    native.sgemm(0, 0, 1, 2, 3, dx, 3, 0, dW, 2, 0, dy, 2, 0)
    assert np.array_equal(down(native, dy, 2), e["y"])
    t = ref_vectors["dot_transposed"]
    dd, dW2, dxo = up(native, np.ones((4, 2), np.float32)), up(native, np.full((3, 2), 0.5, np.float32)), empty(native, 12)
    native.sgemm(0, 1, 4, 3, 2, dd, 2, 0, dW2, 2, 0, dxo, 3, 0)
    assert np.allclose(down(native, dxo, (4, 3)), t["dx"]["value"], rtol=t["eps_rel"])


def test_sgemm_batched(native, oracle):
    announce("sgemm batched 48x512x64x512")
    g = rng(1300)
    Bt, M, N, K = 48, 512, 512, 64
    A = g.normal(0, 1, (Bt, M, K)).astype(np.float32)
    B = g.normal(0, 1, (Bt, K, N)).astype(np.float32)
    dA, dB, dC = up(native, A), up(native, B), empty(native, Bt * M * N)
    native.sgemm(0, 0, M, N, K, dA, K, M * K, dB, N, K * N, dC, N, M * N, Bt)
    Cg = down(native, dC, (Bt, M, N))
    for b in (0, 17, 47):
        C64, Cabs = oracle.sgemm_f64(A[b], B[b], with_abs=True)
        ok, nw, el = gemm_tolerance_ok(Cg[b], C64, Cabs, K)
        assert ok, (b, nw, el)


@pytest.mark.parametrize("S", [2048, 8192])
def test_sgemm_large_sampled(native, oracle, S):
    """Full-size square SGEMM (configs 4): fp64 dot products at 4096 sampled
    entries plus the closed form ones * ones = K on a second run."""
    announce(f"sgemm {S}^3 sampled")
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
    del A, B
    ones = up(native, np.ones((S, S), np.float32))
    native.sgemm(0, 0, S, S, S, ones, S, 0, ones, S, 0, dC, S, 0)
    assert np.all(down(native, dC, (S, S)) == S)


def test_gemv_config(native, oracle):
    """configs[1](a): 1x4096 . 4096x4096, N(0, 0.02)."""
    announce("gemv 1x4096x4096")
    g = rng(1500)
    x = g.normal(0, 0.02, 4096).astype(np.float32)
    B = g.normal(0, 0.02, (4096, 4096)).astype(np.float32)
    dx, dB, dy = up(native, x), up(native, B), empty(native, 4096)
    native.sgemv(dx, dB, 4096, dy, 4096, 4096)
    y = down(native, dy, 4096)
    C64, Cabs = oracle.sgemm_f64(x[None, :], B, with_abs=True)
    ok, nw, el = gemm_tolerance_ok(y[None, :], C64, Cabs, 4096)
    assert ok, (nw, el)
    # the sgemm entry routes M == 1 to the same kernel
    dy2 = empty(native, 4096)
    native.sgemm(0, 0, 1, 4096, 4096, dx, 4096, 0, dB, 4096, 0, dy2, 4096, 0)
    assert np.array_equal(down(native, dy2, 4096), y)


# Float4 finish with 64 splits (4096 x 4096), 91 splits over two load
# groups (1024 x 3000), 32 splits (8192 x 2048) and one split (100 x 5);
# scalar paths for N % 4 != 0.
@pytest.mark.parametrize("N,K,ldb", [(4093, 1000, 4093), (100, 5, 128), (4096, 4096, 4100),
                                     (1024, 3000, 1024), (8192, 2048, 8192), (1, 1, 1)])
def test_gemv_ragged(native, oracle, N, K, ldb):
    announce(f"gemv N={N} K={K} ldb={ldb}")
    g = rng(1600 + N)
    x = g.normal(0, 1, K).astype(np.float32)
    Bfull = g.normal(0, 1, (K, ldb)).astype(np.float32)
    dx, dB, dy = up(native, x), up(native, Bfull), empty(native, N)
    native.sgemv(dx, dB, ldb, dy, N, K)
    y = down(native, dy, N)
    C64, Cabs = oracle.sgemm_f64(x[None, :], Bfull[:, :N], with_abs=True)
    ok, nw, el = gemm_tolerance_ok(y[None, :], C64, Cabs, K)
    assert ok, (nw, el)


@pytest.mark.parametrize("entry", ["sgemv", "gemm", "gemm_noalloc"])
def test_gemv_wider_than_the_partials(native, oracle, entry):
    """1 x 3 . 3 x 8,388,620: more columns than one partial row of the
    scratch area holds (4M floats for silgpu_sgemv / silgpu_gemm, 8M for the
    fixed array of silgpu_gemm_noalloc), so the product runs in column
    pieces of whole 256-column tiles; the last piece is ragged."""
    N, K = 8_388_620, 3
    announce(f"gemv wide N={N} K={K} via {entry}")
    g = rng(1650)
    x = g.normal(0, 1, K).astype(np.float32)
    B = g.normal(0, 1, (K, N)).astype(np.float32)
    dx, dB = up(native, x), up(native, B)
    dy = up(native, np.full(N + 16, np.nan, np.float32))
    if entry == "sgemv":
        native.sgemv(dx, dB, N, dy, N, K)
    else:
        native.gemm(0, 0, 1, N, K, dx, K, dB, N, dy, N, noalloc=entry == "gemm_noalloc")
    y = down(native, dy, N + 16)
    assert np.all(np.isnan(y[N:]))
    C64, Cabs = oracle.sgemm_f64(x[None, :], B, with_abs=True)
    ok, nw, el = gemm_tolerance_ok(y[None, :N], C64, Cabs, K)
    assert ok, (nw, el)


def test_linear_sigmoid_config(native, oracle):
    """configs[1](c): sigmoid(X . W + b), X 256x4096, W 4096x4096, N(0, 0.02)."""
    announce("linear_sigmoid 256x4096x4096")
    Cg, C64, Cabs = _gemm_case(native, oracle, 256, 4096, 4096, epi=native.EPI_BIAS_SIGMOID,
                               bias_len=4096, dist="normal")
    ok, nw, el = gemm_tolerance_ok(Cg, C64, Cabs, 4096)
    assert ok, (nw, el)


@pytest.mark.parametrize("K", [1, 2, 3])
def test_linear_sigmoid_short_k(native, oracle, K):
    """K of 1-3 (B transposed, bias taken modulo 173): the propagated product
    bound is then below one ulp of the sigmoid's output, so the bar rests on
    the allowance for the fp32 sigmoid itself (sigmoid_bound)."""
    M, N, bias_len = 1268, 279, 173
    announce(f"linear_sigmoid {M}x{N}x{K} tb bias_len={bias_len}")
    g = rng(900 + K)
    A = g.uniform(-1, 1, (M, K)).astype(np.float32)
    B = g.uniform(-1, 1, (N, K)).astype(np.float32)
    bias = g.normal(0, 1, bias_len).astype(np.float32)
    dA, dB, dC, db = up(native, A), up(native, B), empty(native, M * N), up(native, bias)
    native.sgemm(0, 1, M, N, K, dA, K, 0, dB, K, 0, dC, N, 0, 1, db, bias_len,
                 native.EPI_BIAS_SIGMOID)
    Cg = down(native, dC, (M, N))
    C64, Cabs = oracle.sgemm_f64(A, B, tb=True, with_abs=True)
    bb = bias[np.arange(N) % bias_len].astype(np.float64)
    C64, Cabs = sigmoid_bound(C64 + bb, Cabs + np.abs(bb), K)
    ok, nw, el = gemm_tolerance_ok(Cg, C64, Cabs, K)
    assert ok, (nw, el)


def test_small_batch_config(native, oracle):
    """configs[1](b): 32x4096 . 4096x768."""
    announce("sgemm 32x768x4096")
    Cg, C64, Cabs = _gemm_case(native, oracle, 32, 768, 4096, dist="normal")
    ok, nw, el = gemm_tolerance_ok(Cg, C64, Cabs, 4096)
    assert ok, (nw, el)


@pytest.mark.parametrize("tile", [1, 2, 3, 4, 5, 6, 7, 8, 9, 10])
@pytest.mark.parametrize("splits", [1, 3, 8])
@pytest.mark.parametrize("M,N,K,ta,tb,epi", [(33, 70, 200, 0, 0, 0), (128, 256, 512, 0, 0, 2),
                                             (100, 130, 1000, 1, 0, 1), (64, 96, 777, 0, 1, 4),
                                             (512, 256, 320, 0, 0, 1), (256, 512, 272, 1, 1, 3)])
def test_sgemm_tuned_configs(native, oracle, tile, splits, M, N, K, ta, tb, epi):
    """Every forced tile configuration and K split against the oracle."""
    announce(f"sgemm_tuned tile={tile} splits={splits} {M}x{N}x{K} ta={ta} tb={tb} epi={epi}")
    g = rng(1700 + M + N + K)
    A = g.uniform(-1, 1, (K, M) if ta else (M, K)).astype(np.float32)
    B = g.uniform(-1, 1, (N, K) if tb else (K, N)).astype(np.float32)
    bias_len = N if epi in (1, 2, 4) else 0
    bias = g.normal(0, 1, max(bias_len, 1)).astype(np.float32)
    dA, dB, dC = up(native, A), up(native, B), empty(native, M * N)
    dbias = up(native, bias) if bias_len else None
    native.sgemm_tuned(ta, tb, M, N, K, dA, A.shape[1], 0, dB, B.shape[1], 0, dC, N, 0, 1,
                       dbias, bias_len, epi, tile=tile, splits=splits)
    Cg = down(native, dC, (M, N))
    C64, Cabs = oracle.sgemm_f64(A, B, ta=ta, tb=tb, with_abs=True)
    if bias_len:
        C64, Cabs = C64 + bias, Cabs + np.abs(bias)
    if epi == 2:
        C64, Cabs = sigmoid_bound(C64, Cabs, K)
    if epi in (3, 4):
        C64 = np.maximum(C64, 0)
    ok, nw, el = gemm_tolerance_ok(Cg, C64, Cabs, K)
    assert ok, (nw, el)


SKINNY_CASES = [
    # M, N, K, tb, lda_pad, ldb_pad, ldc_pad, epi
    (32, 768, 4096, 0, 0, 0, 0, 0), (32, 768, 4096, 1, 0, 0, 0, 2), (2, 4096, 768, 0, 0, 0, 0, 1),
    (31, 130, 100, 0, 1, 0, 3, 4), (5, 7, 15, 0, 0, 0, 0, 0), (16, 64, 1, 0, 0, 0, 0, 3),
    (17, 96, 333, 1, 0, 1, 0, 1), (32, 100, 200, 1, 2, 2, 1, 2), (3, 260, 1000, 0, 0, 2, 4, 0),
    (32, 4096, 64, 0, 0, 0, 0, 1), (8, 36, 4100, 1, 3, 0, 0, 0),
    # wide and deep: the automatic plan takes 64-column groups (N odd: back to 32)
    (8, 4096, 4096, 0, 0, 0, 0, 0), (4, 4097, 4096, 0, 0, 0, 0, 0), (16, 4096, 4096, 1, 0, 0, 0, 1),
    # the boundary of that rule: N = 3072 and narrow N with very deep K keep
    # 32-column groups
    (16, 3072, 4096, 0, 0, 0, 0, 0), (32, 768, 32768, 0, 0, 0, 0, 1),
]


@pytest.mark.parametrize("tile,splits", [(6, 0), (6, 1), (6, 5), (6, 64), (7, 3), (8, 2),
                                         (8, 17)])
@pytest.mark.parametrize("M,N,K,tb,lpa,lpb,lpc,epi", SKINNY_CASES)
def test_sgemm_small_m(native, oracle, tile, splits, M, N, K, tb, lpa, lpb, lpc, epi):
    """The small-M kernel (M <= 32) through silgpu_sgemm_tuned with forced
    column-group widths and K splits (0 = the library's choice): padded lda /
    ldb (unaligned rows take the scalar loads), ldc > N, both B layouts, every
    epilogue, K not a multiple of the 16-deep chunk."""
    announce(f"sgemm small-M tile={tile} splits={splits} {M}x{N}x{K} tb={tb} "
             f"pads=({lpa},{lpb},{lpc}) epi={epi}")
    g = rng(4100 + M + 3 * N + K + tb)
    lda, ldb, ldc = K + lpa, (K if tb else N) + lpb, N + lpc
    A = g.uniform(-1, 1, (M, lda)).astype(np.float32)
    B = g.uniform(-1, 1, ((N if tb else K), ldb)).astype(np.float32)
    bias_len = N if epi in (1, 2, 4) else 0
    bias = g.normal(0, 1, max(bias_len, 1)).astype(np.float32)
    dA, dB, dC = up(native, A), up(native, B), empty(native, M * ldc)
    dbias = up(native, bias) if bias_len else None
    if splits == 0:
        native.sgemm(0, tb, M, N, K, dA, lda, 0, dB, ldb, 0, dC, ldc, 0, 1, dbias, bias_len,
                     epi)
    else:
        native.sgemm_tuned(0, tb, M, N, K, dA, lda, 0, dB, ldb, 0, dC, ldc, 0, 1, dbias,
                           bias_len, epi, tile=tile, splits=splits)
    Cg = down(native, dC, (M, ldc))[:, :N]
    Bv = B[:, :K] if tb else B[:, :N]
    C64, Cabs = oracle.sgemm_f64(A[:, :K], Bv, tb=bool(tb), with_abs=True)
    if bias_len:
        C64, Cabs = C64 + bias, Cabs + np.abs(bias)
    if epi == 2:
        C64, Cabs = sigmoid_bound(C64, Cabs, K)
    if epi in (3, 4):
        C64 = np.maximum(C64, 0)
    ok, nw, el = gemm_tolerance_ok(Cg, C64, Cabs, max(K, 1))
    assert ok, (nw, el)


# ---- silgpu_gemm: two-level batch, fused scale / residual ----------------------------

# Shapes whose unsplit tiles fill whole rounds of the 256 CUs plus part of
# another: the plan runs the last tile rows as a second product split along
# K (2048x2304x768: 256 rows in 3 splits; 2176x4096x768 on 128x128 tiles:
# 128 rows in 6 splits; 1152x4096x512: 128 rows in 4 splits).
@pytest.mark.parametrize("M,N,K", [(2048, 2304, 768), (2176, 4096, 768), (1152, 4096, 512)])
def test_sgemm_peeled_tail(native, oracle, M, N, K):
    announce(f"sgemm peeled tail {M}x{N}x{K}")
    g = rng(2600 + M)
    A = g.uniform(-1, 1, (M, K)).astype(np.float32)
    B = g.uniform(-1, 1, (K, N)).astype(np.float32)
    bias = g.normal(0, 1, N).astype(np.float32)
    dA, dB, db, dC = up(native, A), up(native, B), up(native, bias), empty(native, M * N)
    native.sgemm(0, 0, M, N, K, dA, K, 0, dB, N, 0, dC, N, 0, 1, db, N, native.EPI_BIAS)
    Cg = down(native, dC, (M, N))
    # every row of the last 256 (head/tail boundary and tail), random elsewhere
    rows = np.concatenate([np.repeat(np.arange(M - 256, M), 8), g.integers(0, M, 2048)])
    cols = g.integers(0, N, rows.size)
    ref, refabs = oracle.sgemm_sampled_f64(A, B, rows, cols)
    ref = ref + bias[cols]
    refabs = refabs + np.abs(bias[cols])
    tol = 1e-5 * math.sqrt(K)
    diff = np.abs(Cg[rows, cols] - ref)
    assert np.all(diff <= tol * refabs), float(np.max(diff / refabs))


def test_gemm_two_level_batch_head_split(native, oracle):
    """Q K^T for every (batch, head) of a [B*S, 3*H*dh] qkv array in one launch:
    A and B are strided head views (outer stride per batch, inner per head)."""
    announce("gemm two-level batch")
    B_, S, H, dh = 3, 40, 4, 16
    D = H * dh
    g = rng(2100)
    qkv = g.normal(0, 1, (B_ * S, 3 * D)).astype(np.float32)
    dq, dc = up(native, qkv), empty(native, B_ * H * S * S)
    base = native.vp(dq).value
    native.gemm(0, 1, S, S, dh, base, 3 * D, base + 4 * D, 3 * D, dc, S,
                batch_outer=B_, batch_inner=H, strides_a=(S * 3 * D, dh),
                strides_b=(S * 3 * D, dh), strides_c=(H * S * S, S * S))
    got = down(native, dc, (B_, H, S, S))
    q = qkv.reshape(B_, S, 3, H, dh)[:, :, 0].transpose(0, 2, 1, 3).astype(np.float64)
    k = qkv.reshape(B_, S, 3, H, dh)[:, :, 1].transpose(0, 2, 1, 3).astype(np.float64)
    ref = q @ k.transpose(0, 1, 3, 2)
    refabs = np.abs(q) @ np.abs(k.transpose(0, 1, 3, 2))
    assert np.all(np.abs(got - ref) <= 1e-5 * math.sqrt(dh) * refabs + 1e-30)


@pytest.mark.parametrize("M,N,K", [(100, 130, 200), (256, 256, 4096), (1, 300, 257),
                                   (512, 512, 96), (2048, 2304, 768), (2048, 3072, 768),
                                   (4096, 4096, 512), (1500, 513, 120)])
def test_gemm_fused_epilogue_bit_exact(native, oracle, M, N, K):
    """scale -> bias -> relu -> residual fused into the product equals the
    same fp32 steps run as separate kernels (affine fma, bias add, relu,
    residual add), bit for bit, on every GEMM path (MFMA tiles, split K,
    GEMV for M == 1, a peeled split tail; unsplit LDS-direct 128 x 64 and
    256 x 128 tiles and a ragged register-staged product, whose epilogues
    load bias and residual ahead of the stores)."""
    announce(f"gemm fused epilogue {M}x{N}x{K}")
    g = rng(2200 + M + K)
    A = g.uniform(-1, 1, (M, K)).astype(np.float32)
    B = g.uniform(-1, 1, (K, N)).astype(np.float32)
    bias = g.normal(0, 1, N).astype(np.float32)
    ldr = N + 3
    R = g.normal(0, 1, (M, ldr)).astype(np.float32)
    s = np.float32(0.125 + 1.0 / 3.0)
    off = np.float32(0.0) * s
    dA, dB, db, dR = up(native, A), up(native, B), up(native, bias), up(native, R)
    fused, plain = empty(native, M * N), empty(native, M * N)
    native.gemm(0, 0, M, N, K, dA, K, dB, N, fused, N, epi=native.EPI_BIAS_RELU,
                scale=(float(s), float(off)), bias=db, bias_len=N, residual=dR, ldr=ldr)
    native.sgemm(0, 0, M, N, K, dA, K, 0, dB, N, 0, plain, N, 0)
    t1, t2, t3 = empty(native, M * N), empty(native, M * N), empty(native, M * N)
    native.affine_f32(plain, t1, M * N, float(s), float(off))
    native.binary_f32(ADD, t1, M * N, db, N, t2, M * N)
    native.unary_f32(native.RELU, t2, t3, M * N)
    Rc = up(native, np.ascontiguousarray(R[:, :N]))
    out = empty(native, M * N)
    native.binary_f32(ADD, t3, M * N, Rc, M * N, out, M * N)
    assert np.array_equal(down(native, fused, (M, N)), down(native, out, (M, N)))


def test_gemm_desc_validation(native):
    announce("gemm descriptor validation")
    dA, dC = empty(native, 64), empty(native, 64)
    with pytest.raises(native.SilGpuError, match="residual"):
        native.gemm(0, 0, 4, 4, 4, dA, 4, dA, 4, dC, 4, batch_outer=2, batch_inner=1,
                    residual=dA, ldr=4)
    with pytest.raises(native.SilGpuError, match="ldc"):
        native.gemm(0, 0, 4, 8, 4, dA, 4, dA, 8, dC, 4)


@pytest.mark.parametrize("K,splits", [(80, 1), (96, 1), (96, 3), (80, 3)])
@pytest.mark.parametrize("tile", [5, 1, 4])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_lds_direct_batched(native, oracle, ta, tb, tile, K, splits):
    """Full 256 x 256 (tile 5), 128 x 128 (tile 1) and 128 x 64 (tile 4)
    tiles take the LDS-direct kernel: batched, strided (padded leading
    dimensions), every transpose, bias + relu epilogue.  The 256 and 128 x 64
    tiles run K tiles of 32 when K % 32 == 0 (K = 96) and of 16 otherwise
    (K = 80); splits = 3 adds the split-K partial pass (K ranges 32 + 32 + 32
    and 32 + 32 + 16; split K runs unbatched)."""
    announce(f"sgemm lds-direct batched tile={tile} ta={ta} tb={tb} K={K} splits={splits}")
    M, N, batch = 256, 512, (3 if splits == 1 else 1)
    g = rng(2300 + 2 * ta + tb)
    lda = (M if ta else K) + 4
    ldb = (K if tb else N) + 8
    rows_a, rows_b = (K if ta else M), (N if tb else K)
    A = g.uniform(-1, 1, (batch, rows_a, lda)).astype(np.float32)
    B = g.uniform(-1, 1, (batch, rows_b, ldb)).astype(np.float32)
    bias = g.normal(0, 1, N).astype(np.float32)
    dA, dB, db, dC = up(native, A), up(native, B), up(native, bias), empty(native, batch * M * N)
    native.sgemm_tuned(ta, tb, M, N, K, dA, lda, rows_a * lda, dB, ldb, rows_b * ldb, dC, N,
                       M * N, batch, db, N, native.EPI_BIAS_RELU, tile=tile, splits=splits)
    Cg = down(native, dC, (batch, M, N))
    for z in range(batch):
        a = A[z][:, :M] if ta else A[z][:, :K]
        b = B[z][:, :K] if tb else B[z][:, :N]
        C64, Cabs = oracle.sgemm_f64(np.ascontiguousarray(a), np.ascontiguousarray(b), ta=ta,
                                     tb=tb, with_abs=True)
        ref = np.maximum(C64 + bias, 0)
        ok, nw, el = gemm_tolerance_ok(Cg[z], ref, Cabs + np.abs(bias), K)
        assert ok, (z, nw, el)


K_GROUP_CASES = [(9, 64, 64, 64, 1, 1), (9, 256, 512, 1024, 1, 1), (9, 192, 128, 320, 3, 1),
                 (9, 128, 192, 4096, 8, 1), (9, 128, 256, 192, 1, 3), (10, 128, 128, 128, 1, 1),
                 (10, 256, 512, 3072, 1, 1), (10, 192, 128, 640, 2, 1), (10, 128, 192, 4096, 8, 1),
                 (10, 128, 256, 384, 1, 3)]


@pytest.mark.parametrize("tile,M,N,K,splits,batch", K_GROUP_CASES)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_k_groups(native, oracle, ta, tb, tile, M, N, K, splits, batch):
    """Tiles 9 and 10: 64 x 64 tiles on the LDS-direct kernel with each
    workgroup's K range split between two (9) or four (10) wave groups and
    added through LDS.  Padded leading dimensions, every transpose, bias +
    relu, K splits on top (K ranges of whole 64s or 128s: 320 = 128 + 128 +
    64, 640 = 384 + 256) and batches; the plan record shows the kernel ran,
    and the padding columns of C stay unwritten."""
    announce(f"sgemm k-groups tile={tile} ta={ta} tb={tb} {M}x{N}x{K} splits={splits} "
             f"batch={batch}")
    g = rng(2400 + 2 * ta + tb + K)
    lda = (M if ta else K) + 4
    ldb = (K if tb else N) + 8
    ldc = N + 4
    rows_a, rows_b = (K if ta else M), (N if tb else K)
    A = g.uniform(-1, 1, (batch, rows_a, lda)).astype(np.float32)
    B = g.uniform(-1, 1, (batch, rows_b, ldb)).astype(np.float32)
    bias = g.normal(0, 1, N).astype(np.float32)
    canary = np.full((batch, M, ldc), 7.25, np.float32)
    dA, dB, db, dC = up(native, A), up(native, B), up(native, bias), up(native, canary)
    native.sgemm_tuned(ta, tb, M, N, K, dA, lda, rows_a * lda, dB, ldb, rows_b * ldb, dC, ldc,
                       M * ldc, batch, db, N, native.EPI_BIAS_RELU, tile=tile, splits=splits)
    plan = native.last_plan()
    assert plan and plan[0][0] == tile, plan
    Cg = down(native, dC, (batch, M, ldc))
    assert np.all(Cg[:, :, N:] == 7.25)
    for z in range(batch):
        a = A[z][:, :M] if ta else A[z][:, :K]
        b = B[z][:, :K] if tb else B[z][:, :N]
        C64, Cabs = oracle.sgemm_f64(np.ascontiguousarray(a), np.ascontiguousarray(b), ta=ta,
                                     tb=tb, with_abs=True)
        ref = np.maximum(C64 + bias, 0)
        ok, nw, el = gemm_tolerance_ok(Cg[z][:, :N], ref, Cabs + np.abs(bias), K)
        assert ok, (z, nw, el)


@pytest.mark.parametrize("M,N,K,tile,splits", [(1024, 1024, 1024, 9, 1), (256, 2048, 512, 9, 2),
                                               (128, 2048, 768, 9, 4), (256, 4096, 4096, 10, 1)])
def test_k_groups_planner_pick_with_residual(native, oracle, M, N, K, tile, splits):
    """Products whose 64 x 64 tiles (times a few K splits) fill the CUs once
    run tile 9 (tile 10 where K >= 3072 needs no split) by the planner's own
    choice, through silgpu_gemm with bias and residual, and through
    silgpu_gemm_noalloc bit for bit the same."""
    announce(f"k-groups planner pick {M}x{N}x{K}")
    g = rng(2500 + M + K)
    A = g.normal(0, 1, (M, K)).astype(np.float32)
    B = g.normal(0, 1, (K, N)).astype(np.float32)
    b = g.normal(0, 1, N).astype(np.float32)
    R = g.normal(0, 1, (M, N)).astype(np.float32)
    dA, dB, db, dR = up(native, A), up(native, B), up(native, b), up(native, R)
    dC, dCn = empty(native, M * N), empty(native, M * N)
    native.gemm(0, 0, M, N, K, dA, K, dB, N, dC, N, epi=native.EPI_BIAS, bias=db, bias_len=N,
                residual=dR, ldr=N)
    assert native.last_plan() == [(tile, splits, M)], native.last_plan()
    native.gemm(0, 0, M, N, K, dA, K, dB, N, dCn, N, epi=native.EPI_BIAS, bias=db, bias_len=N,
                residual=dR, ldr=N, noalloc=True)
    assert native.last_plan() == [(tile, splits, M)], native.last_plan()
    C, Cn = down(native, dC, (M, N)), down(native, dCn, (M, N))
    assert np.array_equal(C, Cn)
    C64, Cabs = oracle.sgemm_f64(A, B, with_abs=True)
    ok, nw, el = gemm_tolerance_ok(C, C64 + b + R, Cabs + np.abs(b) + np.abs(R), K)
    assert ok, (nw, el)


@pytest.mark.parametrize("batch,M,N,K,tile", [(8, 256, 256, 4096, 10), (16, 128, 128, 1024, 9),
                                              (48, 64, 64, 512, 9), (3, 64, 192, 3200, 10),
                                              (3, 1024, 1024, 512, 9), (9, 256, 1024, 256, 9),
                                              (7, 512, 1024, 256, 4)])
def test_k_groups_planner_pick_batched(native, oracle, batch, M, N, K, tile):
    """Batched products whose 64 x 64 tiles fill at most one round of the CUs
    run the K-group tile by the planner's own choice (four groups for K >=
    3072), and so do those whose 128 x 64 tiles would leave a last round at
    most half full (384 and 288 tiles here, not 448), through silgpu_gemm
    with a two-level batch and bias."""
    announce(f"k-groups batched planner pick {batch} x {M}x{N}x{K}")
    g = rng(2600 + batch + K)
    A = g.normal(0, 1, (batch, M, K)).astype(np.float32)
    B = g.normal(0, 1, (batch, K, N)).astype(np.float32)
    b = g.normal(0, 1, N).astype(np.float32)
    dA, dB, db, dC = up(native, A), up(native, B), up(native, b), empty(native, batch * M * N)
    bo, bi = (batch // 2, 2) if batch % 2 == 0 else (batch, 1)
    native.gemm(0, 0, M, N, K, dA, K, dB, N, dC, N, batch_outer=bo, batch_inner=bi,
                strides_a=(bi * M * K, M * K), strides_b=(bi * K * N, K * N),
                strides_c=(bi * M * N, M * N), epi=native.EPI_BIAS, bias=db, bias_len=N)
    assert native.last_plan() == [(tile, 1, M)], native.last_plan()
    C = down(native, dC, (batch, M, N))
    for z in range(batch):
        C64, Cabs = oracle.sgemm_f64(A[z], B[z], with_abs=True)
        ok, nw, el = gemm_tolerance_ok(C[z], C64 + b, Cabs + np.abs(b), K)
        assert ok, (z, nw, el)


# ---- fused attention ----------------------------------------------------------------

def _attention_f64(Q, K, V, scale):
    """softmax(scale * Q K^T) V per leading index, in float64 (the unfused
    reference graph: product, scalar scale, row softmax, product)."""
    S = np.einsum("...qd,...kd->...qk", Q.astype(np.float64), K.astype(np.float64)) * scale
    S -= S.max(axis=-1, keepdims=True)
    P = np.exp(S)
    P /= P.sum(axis=-1, keepdims=True)
    return P @ V.astype(np.float64)


# B, H, Sq, Sk, D, layout ("merged": [B, S, H, D] buffers as attention heads
# split out of a [B*S, H*D] array; "heads": contiguous [B, H, S, D])
ATTN_CASES = [(1, 1, 64, 64, 64, "heads"), (2, 3, 37, 100, 64, "merged"),
              (1, 2, 130, 1, 32, "heads"), (1, 1, 5, 200, 16, "merged"),
              (2, 2, 64, 77, 128, "merged"), (4, 12, 512, 512, 64, "merged"),
              (3, 1, 200, 64, 32, "heads"), (2, 2, 33, 70, 32, "unaligned")]


@pytest.mark.parametrize("B,H,Sq,Sk,D,layout", ATTN_CASES)
def test_attention_fused(native, B, H, Sq, Sk, D, layout):
    """silgpu_attention_f32 against float64 on seeded N(0, 1) inputs: every
    output is a convex combination of V rows, so the error is measured
    against max|V|; tolerance 2e-5 * sqrt(max(D, Sk))."""
    announce(f"attention B={B} H={H} Sq={Sq} Sk={Sk} D={D} {layout}")
    g = rng(5100 + B * H + Sq + Sk + D)
    scale = float(np.float32(1.0 / np.sqrt(D)))

    def make(S):
        if layout == "unaligned":  # rows of D + 1 floats, buffer offset by one float
            buf = g.normal(0, 1, (B, H, S, D + 1)).astype(np.float32)
            return buf, buf[..., :D], D + 1, (H * S * (D + 1), S * (D + 1))
        if layout == "merged":
            buf = g.normal(0, 1, (B, S, H, D)).astype(np.float32)
            view = buf.transpose(0, 2, 1, 3)  # [B, H, S, D]
            return buf, view, H * D, (S * H * D, D)
        buf = g.normal(0, 1, (B, H, S, D)).astype(np.float32)
        return buf, buf, D, (H * S * D, S * D)

    qb, Qv, ldq, sq = make(Sq)
    kb, Kv, ldk, sk = make(Sk)
    vb, Vv, ldv, sv = make(Sk)
    ob = np.full(qb.shape, np.nan, np.float32)
    dQ, dK, dV, dO = up(native, qb), up(native, kb), up(native, vb), up(native, ob)
    off = (1, 1, 1, 0) if layout == "unaligned" else (0, 0, 0, 0)
    if off[0]:  # Q, K, V start one float into their buffers (rows D + 1 wide)
        qb, kb, vb = (np.concatenate([[0.0], x.ravel()]).astype(np.float32) for x in (qb, kb, vb))
        dQ, dK, dV = up(native, qb), up(native, kb), up(native, vb)
    native.attention(Sq, Sk, D, scale, dQ, ldq, dK, ldk, dV, ldv, dO, ldq, B, H, sq, sk, sv, sq,
                     offsets=off)
    out = down(native, dO, ob.shape)
    Ov = out.transpose(0, 2, 1, 3) if layout == "merged" else out
    if layout == "unaligned":
        Ov = Ov[..., :D]
    ref = _attention_f64(Qv, Kv, Vv, scale)
    err = np.abs(Ov.astype(np.float64) - ref).max()
    tol = 2e-5 * np.sqrt(max(D, Sk)) * np.abs(Vv).max()
    assert np.isfinite(Ov).all() and err <= tol, (err, tol)


def test_attention_large_scores(native):
    """Scores of several hundred (q, k ~ N(0, 8)): the online softmax's
    running-max subtraction keeps every exponent finite and the rows close to
    one-hot; the float64 bar widens by the scores' rounding, |s| * 2^-24."""
    announce("attention large scores")
    B, H, S, D = 1, 3, 97, 64
    g = rng(5300)
    Q = (g.normal(0, 8, (B, H, S, D))).astype(np.float32)
    K = (g.normal(0, 8, (B, H, S, D))).astype(np.float32)
    V = g.normal(0, 1, (B, H, S, D)).astype(np.float32)
    scale = float(np.float32(1.0 / np.sqrt(D)))
    dQ, dK, dV, dO = up(native, Q), up(native, K), up(native, V), empty(native, Q.size)
    st = (H * S * D, S * D)
    native.attention(S, S, D, scale, dQ, D, dK, D, dV, D, dO, D, B, H, st, st, st, st)
    out = down(native, dO, Q.shape)
    ref = _attention_f64(Q, K, V, scale)
    smax = np.abs(np.einsum("bhqd,bhkd->bhqk", Q.astype(np.float64), K.astype(np.float64))).max() * scale
    err = np.abs(out.astype(np.float64) - ref).max()
    tol = (2e-5 * np.sqrt(S) + 4 * smax * 2.0 ** -24) * np.abs(V).max()
    assert np.isfinite(out).all() and err <= tol, (err, tol, smax)


def test_attention_no_keys_gives_zero(native):
    announce("attention Sk=0")
    ob = np.full((2, 16, 32), np.nan, np.float32)
    dO = up(native, ob)
    native.attention(16, 0, 32, 1.0, None, 32, None, 32, None, 32, dO, 32, 1, 2, (0, 0),
                     (0, 0), (0, 0), (0, 16 * 32))
    assert np.all(down(native, dO, ob.shape) == 0)


# ---- batches beyond one launch's grid (65535 in y and z) --------------------------

@pytest.mark.parametrize("outer,inner", [(1, 70000), (3, 30000), (2, 65536)])
def test_gemm_batch_beyond_the_grid(native, oracle, outer, inner):
    """A batched product of more than 65535 matrices runs in several launches:
    whole outer indices per launch while the inner batch fits, else pieces of
    each outer index's inner batch (a batched_dot over a long leading axis)."""
    announce(f"gemm batch {outer}x{inner}")
    M, N, K = 3, 5, 7
    g = rng(7700 + outer)
    A = g.uniform(-1, 1, (outer, inner, M, K)).astype(np.float32)
    B = g.uniform(-1, 1, (outer, inner, K, N)).astype(np.float32)
    dA, dB = up(native, A), up(native, B)
    dC = up(native, np.full(outer * inner * M * N + 16, np.nan, np.float32))
    native.gemm(0, 0, M, N, K, dA, K, dB, N, dC, N, batch_outer=outer, batch_inner=inner,
                strides_a=(inner * M * K, M * K), strides_b=(inner * K * N, K * N),
                strides_c=(inner * M * N, M * N))
    out = down(native, dC, (outer * inner * M * N + 16,))
    assert np.all(np.isnan(out[outer * inner * M * N:]))
    C = out[:outer * inner * M * N].reshape(outer, inner, M, N).astype(np.float64)
    ref = np.matmul(A.astype(np.float64), B.astype(np.float64))
    refabs = np.matmul(np.abs(A.astype(np.float64)), np.abs(B.astype(np.float64)))
    assert np.all(np.abs(C - ref) <= 1e-5 * np.sqrt(K) * refabs + 1e-30)


def test_attention_batch_beyond_the_grid(native):
    """70000 (batch, head) pairs: several launches of at most 65535."""
    announce("attention batch 2x35000")
    Bo, Bi, S, D = 2, 35000, 3, 16
    g = rng(7800)
    Q, K, V = (g.normal(0, 1, (Bo, Bi, S, D)).astype(np.float32) for _ in range(3))
    dQ, dK, dV = up(native, Q), up(native, K), up(native, V)
    dO = up(native, np.full(Q.size, np.nan, np.float32))
    st = (Bi * S * D, S * D)
    native.attention(S, S, D, 0.25, dQ, D, dK, D, dV, D, dO, D, Bo, Bi, st, st, st, st)
    out = down(native, dO, Q.shape).astype(np.float64)
    ref = _attention_f64(Q, K, V, 0.25)
    assert np.isfinite(out).all()
    assert np.abs(out - ref).max() <= 2e-5 * np.sqrt(max(D, S)) * np.abs(V).max()


def test_sum_axis_outer_beyond_the_grid(native, oracle):
    """sum over the middle axis of [70000, 5, 3]: outer slices in batches."""
    announce("sum_axis [70000, 5, 3] axis 1")
    x = rng(7900).normal(0, 3, (70000, 5, 3)).astype(np.float32)
    dx, do = up(native, x), empty(native, 70000 * 3)
    native.sum_axis_f32(dx, 70000, 5, 3, do)
    got = down(native, do, 70000 * 3).astype(np.float64)
    ref = oracle.sum_axis_f64(x, 1).ravel()
    absref = oracle.sum_axis_f64(np.abs(x), 1).ravel()
    assert np.all(np.abs(got - ref) <= 1e-5 * np.abs(ref) + 6e-8 * absref + 1e-30)


# ---- conv2d (implicit GEMM) ---------------------------------------------------------

# N, H, W, C_in, K, C_out, by the kernel the entry point picks:
#  direct (K*K*C_in <= 64): C_out below, at and above one 32-channel block,
#    C_out % 4 != 0, 1x1 and even kernels;
#  LDS-direct implicit GEMM (C_in % 16 == 0, M % 128 == 0, C_out % 64 ==
#    0): BK 16 (C_in = 16, 48) and 32, K = 1, 2, 3, 5;
#  register-staged implicit GEMM: float4 (C_in % 4 == 0) and scalar gathers,
#    ragged tiles on both GEMM axes, C_out <= 32 and above;
# the reference benchmark's three layers (bench/micro/bench_nn_ops.cpp:
# 193-195) at full size; and shapes whose 128 x 64 tiles fill three rounds of
# 256 CUs plus a thin last round, which runs as a second launch (split along
# K into 9 pieces with BK 32 and 16, or unsplit); between one and two tiles
# per CU with K*K*C_in >= 1024 (the deep layer; BK 16 with K = 4, C_in = 80)
# the K range is first split in two; (16, 28, 28, 48, 3, 256) stays unsplit (BK 16,
# an odd number of K tiles).
CONV_CASES = [(1, 8, 8, 3, 3, 16), (1, 5, 6, 4, 1, 5), (2, 9, 5, 6, 2, 40), (3, 4, 4, 1, 3, 1),
              (1, 5, 7, 2, 3, 37), (2, 6, 6, 64, 1, 33),
              (2, 8, 8, 16, 3, 64), (1, 16, 16, 48, 3, 128), (1, 8, 16, 32, 5, 64),
              (1, 8, 16, 32, 2, 64), (1, 16, 8, 128, 1, 128),
              (2, 7, 9, 16, 3, 32), (1, 6, 6, 8, 5, 12), (1, 13, 11, 20, 3, 70),
              (1, 3, 3, 2, 7, 3), (2, 8, 8, 16, 3, 60),
              (1, 224, 224, 3, 3, 32), (16, 56, 56, 64, 3, 128), (16, 28, 28, 128, 3, 256),
              (16, 56, 56, 48, 3, 128), (1, 116, 256, 32, 3, 256), (16, 28, 28, 80, 4, 256),
              (16, 28, 28, 48, 3, 256),
              # direct path (K*K*C_in <= 64): every step count, 1/2/4 channel
              # blocks, two channel-block rows, ragged pixel tiles across images
              (2, 7, 5, 2, 2, 20), (1, 9, 11, 4, 3, 24), (2, 5, 5, 1, 5, 70), (3, 5, 3, 3, 3, 17),
              (4, 12, 10, 1, 1, 3), (2, 33, 17, 7, 3, 64), (1, 1, 9, 2, 3, 5), (2, 6, 1, 2, 5, 4)]


@pytest.mark.parametrize("N,H,W,Ci,K,Co", CONV_CASES)
def test_conv2d(native, oracle, N, H, W, Ci, K, Co):
    """silgpu_conv2d_f32 against the float64 restatement, GEMM bar with the
    reduction length K*K*C_in: normwise and per element against the
    convolution of |x| with |w|."""
    announce(f"conv2d N={N} H={H} W={W} C_in={Ci} K={K} C_out={Co}")
    g = rng(1900 + H * Ci + K)
    x = g.normal(0, 1, (N, H, W, Ci)).astype(np.float32)
    w = g.normal(0, 1, (Co, K, K, Ci)).astype(np.float32)
    dx, dw, do = up(native, x), up(native, w), empty(native, N * H * W * Co)
    native.conv2d(dx, dw, do, N, H, W, Ci, K, Co)
    out = down(native, do, (N * H * W, Co))
    ref = oracle.conv2d_f64(x, w).reshape(-1, Co)
    refabs = oracle.conv2d_f64(np.abs(x), np.abs(w)).reshape(-1, Co)
    ok, nw, el = gemm_tolerance_ok(out, ref, refabs, K * K * Ci)
    assert ok, (nw, el)


def test_conv2d_ones_closed_form(native):
    """Ones in, ones weights: each output is C_in times the taps that fall
    inside the image (corner, edge and interior counts of a 3x3 kernel)."""
    announce("conv2d ones")
    N, H, W, Ci, K, Co = 2, 6, 5, 16, 3, 8
    do = empty(native, N * H * W * Co)
    native.conv2d(up(native, np.ones((N, H, W, Ci), np.float32)),
                  up(native, np.ones((Co, K, K, Ci), np.float32)), do, N, H, W, Ci, K, Co)
    out = down(native, do, (N, H, W, Co))
    rows = np.array([2] + [3] * (H - 2) + [2])
    cols = np.array([2] + [3] * (W - 2) + [2])
    ref = (Ci * rows[:, None] * cols[None, :]).astype(np.float32)
    assert np.array_equal(out, np.broadcast_to(ref[None, :, :, None], out.shape))


def test_conv2d_empty_reduction_writes_zeros(native):
    announce("conv2d C_in=0")
    do = up(native, np.full(2 * 3 * 3 * 4, np.nan, np.float32))
    native.conv2d(None, None, do, 2, 3, 3, 0, 3, 4)
    assert np.all(down(native, do, 72) == 0)


def _random_gemm_cases(n=60, seed=2026):
    """Seeded shapes across every route: the LDS-direct tiles (M, N multiples
    of 64/128/256, K a multiple of 16), the register-staged tiles (any
    shape), small-M products, GEMV; random transposes, leading dimensions
    padded by 0-7 floats, operands offset by 0-3 floats (so some lose 16-byte
    alignment), and batches of 1-3."""
    g = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        kind = i % 4
        if kind == 0:    # LDS-direct eligible
            M = int(g.choice([128, 256, 384, 512, 768, 1024]))
            N = int(g.choice([64, 128, 256, 384, 512]))
            K = int(16 * g.integers(1, 64))
        elif kind == 1:  # ragged
            M, N, K = (int(x) for x in g.integers(1, 700, 3))
        elif kind == 2:  # small M
            M, N, K = int(g.integers(1, 33)), int(g.integers(64, 2048)), int(g.integers(64, 3000))
        else:            # products near GEMV
            M, N, K = int(g.choice([1, 2])), int(g.integers(1, 4096)), int(g.integers(1, 4096))
        ta, tb = bool(g.integers(0, 2)), bool(g.integers(0, 2))
        pad_a, pad_b = int(g.integers(0, 8)), int(g.integers(0, 8))
        off_a, off_b = int(g.choice([0, 0, 1, 3])), int(g.choice([0, 0, 2]))
        batch = int(g.choice([1, 1, 2, 3]))
        cases.append((M, N, K, ta, tb, pad_a, pad_b, off_a, off_b, batch))
    return cases


@pytest.mark.parametrize("M,N,K,ta,tb,pad_a,pad_b,off_a,off_b,batch", _random_gemm_cases())
def test_sgemm_random_shapes(native, oracle, M, N, K, ta, tb, pad_a, pad_b, off_a, off_b, batch):
    announce(f"sgemm random {M}x{N}x{K} ta={ta} tb={tb} pads={pad_a},{pad_b} "
             f"offs={off_a},{off_b} batch={batch}")
    g = rng(M * 7 + N * 3 + K + batch)
    ra, ca = (K, M) if ta else (M, K)
    rb, cb = (N, K) if tb else (K, N)
    lda, ldb = ca + pad_a, cb + pad_b
    sA, sB = ra * lda, rb * ldb
    A = g.uniform(-1, 1, off_a + batch * sA).astype(np.float32)
    B = g.uniform(-1, 1, off_b + batch * sB).astype(np.float32)
    dA, dB, dC = up(native, A), up(native, B), empty(native, batch * M * N)
    native.sgemm(ta, tb, M, N, K, dA.ptr + 4 * off_a, lda, sA, dB.ptr + 4 * off_b, ldb, sB, dC, N,
                 M * N, batch)
    Cg = down(native, dC, (batch, M, N))
    for b in range(batch):
        Ab = A[off_a + b * sA: off_a + (b + 1) * sA].reshape(ra, lda)[:, :ca]
        Bb = B[off_b + b * sB: off_b + (b + 1) * sB].reshape(rb, ldb)[:, :cb]
        C64, Cabs = oracle.sgemm_f64(np.ascontiguousarray(Ab), np.ascontiguousarray(Bb), ta=ta,
                                     tb=tb, with_abs=True)
        ok, nw, el = gemm_tolerance_ok(Cg[b], C64, Cabs, K)
        assert ok, (b, nw, el)


def _random_programs(n=40, seed=77):
    """Seeded elementwise programs: 2-D or 3-D outputs, 1-4 inputs, each read
    contiguous, as a scalar, as a repeated row or matrix block, as a column
    broadcast or transposed, and 3-10 instructions of the correctly rounded
    ops (so the result is bit-exact against numpy float32)."""
    g = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        nd = int(g.integers(2, 4))
        shape = tuple(int(x) for x in g.integers(1, 70, nd))
        if g.random() < 0.3:
            shape = shape[:-1] + (int(g.choice([64, 128, 512])),)
        ins = []
        for _k in range(int(g.integers(1, 5))):
            kind = g.choice(["contig", "scalar", "row", "col", "trans"])
            ins.append((str(kind), int(g.choice([0, 0, 1, 2]))))
        prog = []
        regs = []  # registers holding a value
        for k in range(len(ins)):
            prog.append(("load", k, k))
            regs.append(k)
        for _i in range(int(g.integers(1, 7))):
            op = str(g.choice(["add", "sub", "mul", "div", "addi", "muli", "rsubi", "rdivi", "relu"]))
            a, b = int(g.choice(regs)), int(g.choice(regs))
            dst = int(g.integers(0, 8))
            prog.append((op, dst, a, b, float(np.float32(g.uniform(0.5, 2.0)))))
            if dst not in regs:
                regs.append(dst)
        out = prog[-1][1]
        cases.append((shape, ins, prog, out))
    return cases


def _input_view(kind, shape, g):
    """(host buffer, strides, numpy view of the output shape) for one input."""
    nd = len(shape)
    if kind == "scalar":
        h = g.uniform(0.5, 2, 4).astype(np.float32)
        return h, (0,) * nd, lambda base: np.broadcast_to(h[base], shape)
    if kind == "row":   # the last axis repeated over the leading ones
        L = shape[-1]
        h = g.uniform(0.5, 2, L + 4).astype(np.float32)
        return h, (0,) * (nd - 1) + (1,), lambda base: np.broadcast_to(h[base:base + L], shape)
    if kind == "col":   # the first axis, broadcast along the others
        L = shape[0]
        h = g.uniform(0.5, 2, L + 4).astype(np.float32)
        return h, (1,) + (0,) * (nd - 1), lambda base: np.broadcast_to(
            h[base:base + L].reshape((L,) + (1,) * (nd - 1)), shape)
    n = int(np.prod(shape))
    h = g.uniform(0.5, 2, n + 4).astype(np.float32)
    if kind == "contig":
        st = tuple(int(np.prod(shape[d + 1:])) for d in range(nd))
        return h, st, lambda base: h[base:base + n].reshape(shape)
    # trans: column-major storage
    st = tuple(int(np.prod(shape[:d])) for d in range(nd))
    return h, st, lambda base: h[base:base + n].reshape(shape[::-1]).transpose(
        tuple(range(nd))[::-1])


@pytest.mark.parametrize("case", range(40))
def test_program_random(native, case):
    shape, ins, prog, out_reg = _random_programs()[case]
    announce(f"program random {case}: shape {shape}, inputs {ins}, {len(prog)} instructions")
    g = rng(900 + case)
    P = native
    inputs, views, keep = [], [], []
    for kind, base in ins:
        h, st, view = _input_view(kind, shape, g)
        d = up(native, h)
        keep.append(d)
        inputs.append((d.ptr + 4 * base, st))
        views.append(view(base).astype(np.float32))
    code = {"add": P.PI_ADD, "sub": P.PI_SUB, "mul": P.PI_MUL, "div": P.PI_DIV,
            "addi": P.PI_ADDI, "muli": P.PI_MULI, "rsubi": P.PI_RSUBI, "rdivi": P.PI_RDIVI,
            "relu": P.PI_RELU}
    instrs, regs = [], {}
    with np.errstate(all="ignore"):
        for ins_ in prog:
            if ins_[0] == "load":
                instrs.append((P.PI_LOAD, ins_[1], ins_[2]))
                regs[ins_[1]] = views[ins_[2]]
                continue
            op, dst, a, b, imm = ins_
            instrs.append((code[op], dst, a, b, imm))
            x, y, c = regs[a], regs[b], np.float32(imm)
            regs[dst] = {"add": lambda: x + y, "sub": lambda: x - y, "mul": lambda: x * y,
                         "div": lambda: x / y, "addi": lambda: x + c, "muli": lambda: x * c,
                         "rsubi": lambda: c - x, "rdivi": lambda: c / x,
                         "relu": lambda: np.maximum(x, np.float32(0))}[op]().astype(np.float32)
    n = int(np.prod(shape))
    do = empty(native, n)
    P.program_f32(P.make_program(shape, inputs, instrs, out_reg=out_reg), do)
    got = down(native, do, shape)
    ref = np.broadcast_to(regs[out_reg], shape)
    assert np.array_equal(got, ref, equal_nan=True)
