"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Every oracle function is checked against at least one of: the reference's own
golden vectors (test/test_array.cpp, transcribed in tests/golden), a closed
form, an invariant, or an independent implementation (numpy float64,
math.fsum, scipy) on inputs chosen so that a dropped term, a wrong sign or a
transposed operand fails.  CPU only.
"""

import math

import numpy as np
import pytest
from scipy import special

from conftest import rng

ADD, SUB, MUL, DIV, POW = range(5)


# ---- GEMM ------------------------------------------------------------------

def test_sgemm_reference_goldens(oracle, ref_vectors):
    d = ref_vectors["dot"]
    a = np.array(d["mm_a_3x4_iota1"], np.float32)
    b = np.array(d["mm_b_4x2_iota1"], np.float32)
    assert np.array_equal(oracle.sgemm_f64(a, b), np.array(d["mm_out"]))
    # v . m, m . v, v . v as 1xK / Kx1 products (include/array.h:2700-2728)
    v = np.array(d["vm_a"], np.float32)[None, :]
    assert np.array_equal(oracle.sgemm_f64(v, b)[0], d["vm_out"])
    mv = np.array(d["mv_a_2x4_iota1"], np.float32)
    col = np.array(d["mv_b"], np.float32)[:, None]
    assert np.array_equal(oracle.sgemm_f64(mv, col)[:, 0], d["mv_out"])
    vv = oracle.sgemm_f64(np.array(d["vv_a"], np.float32)[None, :],
                          np.array(d["vv_b"], np.float32)[:, None])
    assert vv[0, 0] == d["vv_out"]
    e = ref_vectors["dot_example"]
    y = oracle.sgemm_f64(np.array(e["x"], np.float32)[None, :], np.array(e["W"], np.float32))
    assert np.array_equal(y[0], e["y"])


def test_sgemm_transposed_goldens(oracle, ref_vectors):
    t = ref_vectors["dot_transposed"]
    dout = np.ones(t["dx"]["dout_shape"], np.float32)
    W = np.full(t["dx"]["W_shape"], t["dx"]["W_value"], np.float32)
    dx = oracle.sgemm_f64(dout, W, tb=True)  # dout . W^T, W stored [3][2]
    assert dx.shape == (4, 3) and np.allclose(dx, t["dx"]["value"], rtol=t["eps_rel"])
    x = np.ones(t["dW"]["x_shape"], np.float32)
    dW = oracle.sgemm_f64(x, np.ones(t["dW"]["dout_shape"], np.float32), ta=True)
    assert dW.shape == (3, 2) and np.allclose(dW, t["dW"]["value"], rtol=t["eps_rel"])


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_brute_force_vs_numpy(oracle, ta, tb):
    g = rng(11 + 2 * ta + tb)
    M, N, K = 17, 23, 31
    A = g.uniform(-1, 1, (K, M) if ta else (M, K)).astype(np.float32)
    B = g.uniform(-1, 1, (N, K) if tb else (K, N)).astype(np.float32)
    Ad = A.astype(np.float64).T if ta else A.astype(np.float64)
    Bd = B.astype(np.float64).T if tb else B.astype(np.float64)
    C, Cabs = oracle.sgemm_f64(A, B, ta=ta, tb=tb, with_abs=True)
    np.testing.assert_allclose(C, Ad @ Bd, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(Cabs, np.abs(Ad) @ np.abs(Bd), rtol=1e-12, atol=1e-12)
    rows = g.integers(0, M, 50)
    cols = g.integers(0, N, 50)
    s, sa = oracle.sgemm_sampled_f64(A, B, rows, cols, ta=ta, tb=tb)
    np.testing.assert_array_equal(s, C[rows, cols])
    np.testing.assert_array_equal(sa, Cabs[rows, cols])


def test_sgemm_closed_form_ones(oracle):
    K = 777
    C = oracle.sgemm_f64(np.ones((5, K), np.float32), np.ones((K, 3), np.float32))
    assert np.all(C == K)


def test_openblas_baseline_matches_f64(oracle):
    import openblas
    g = rng(3)
    M, N, K = 64, 48, 256
    A = g.uniform(-1, 1, (M, K)).astype(np.float32)
    B = g.uniform(-1, 1, (K, N)).astype(np.float32)
    C = openblas.sgemm(A, B)
    ref = oracle.sgemm_f64(A, B)
    assert np.linalg.norm(C - ref) / np.linalg.norm(ref) <= 1e-5 * math.sqrt(K)


def test_gemv_oracle(oracle):
    g = rng(5)
    x = g.normal(0, 0.02, 300).astype(np.float32)
    B = g.normal(0, 0.02, (300, 70)).astype(np.float32)
    y = oracle.gemv_f32(x, B)
    ref = x.astype(np.float64) @ B.astype(np.float64)
    assert np.max(np.abs(y - ref)) <= 1e-5 * math.sqrt(300) * np.max(np.abs(x[:, None] * B).sum(0))


# ---- elementwise -------------------------------------------------------------

def test_binary_reference_goldens(oracle, ref_vectors):
    v = ref_vectors["vector_arith"]
    a, b = np.array(v["a"], np.float32), np.array(v["b"], np.float32)
    for op, key in [(ADD, "add"), (SUB, "sub"), (MUL, "mul"), (DIV, "div")]:
        out = oracle.binary_mod_f32(op, a, b, 16)
        assert np.max(np.abs(out - np.array(v[key]))) <= v["tol_abs"], key
    p = ref_vectors["pow"]
    fa, fb = np.array(p["a"], np.float32), np.array(p["b"], np.float32)
    assert np.allclose(oracle.binary_mod_f32(POW, fa, fb, 3), p["a_pow_b"], atol=1e-3)
    assert np.allclose(oracle.binary_mod_f32(POW, fb, fa, 3), p["b_pow_a"], atol=1e-3)
    assert np.array_equal(oracle.binary_mod_i32(POW, p["a"], p["b"], 3), p["a_pow_b"])
    assert np.array_equal(oracle.binary_mod_i32(POW, p["b"], p["a"], 3), p["b_pow_a"])
    m = ref_vectors["msl_add"]
    assert np.array_equal(oracle.binary_mod_f32(ADD, m["float_a"], m["float_b"], 4), m["float_out"])
    assert np.array_equal(oracle.binary_mod_i32(ADD, m["int_a"], m["int_b"], 4), m["int_out"])
    assert np.array_equal(oracle.binary_mod_f32(ADD, m["bcast_a"], m["bcast_b"], 4), m["bcast_out"])
    im = ref_vectors["int_matrix_arith"]
    a2 = np.array(im["a"]).ravel()
    for op, key in [(ADD, "add"), (SUB, "sub"), (MUL, "mul"), (DIV, "div")]:
        assert np.array_equal(oracle.binary_mod_i32(op, a2, a2, 12), np.ravel(im[key])), key


def test_scalar_ops_goldens(oracle, ref_vectors):
    s = ref_vectors["scalar_arith"]
    a = np.array(s["a"], np.float32).ravel()
    one, two = np.float32([1.0]), np.float32([2.0])
    assert np.array_equal(oracle.binary_mod_f32(ADD, a, one, 4), np.ravel(s["a_plus_1"]))
    assert np.array_equal(oracle.binary_mod_f32(SUB, a, one, 4), np.ravel(s["a_minus_1"]))
    assert np.array_equal(oracle.binary_mod_f32(MUL, a, two, 4), np.ravel(s["a_times_2"]))
    assert np.array_equal(oracle.binary_mod_f32(DIV, a, two, 4), np.ravel(s["a_div_2"]))
    assert np.array_equal(oracle.binary_mod_f32(SUB, one, a, 4), np.ravel(s["one_minus_a"]))
    assert np.array_equal(oracle.binary_mod_f32(DIV, two, a, 4),
                          np.ravel(s["two_div_a"]).astype(np.float32))


def test_binary_mod_semantics_vs_numpy(oracle):
    g = rng(7)
    a = g.uniform(-2, 2, 24).astype(np.float32)
    b = g.uniform(0.5, 2, 5).astype(np.float32)
    n = 60
    ia, ib = np.arange(n) % 24, np.arange(n) % 5
    for op, f in [(ADD, np.add), (SUB, np.subtract), (MUL, np.multiply), (DIV, np.divide)]:
        assert np.array_equal(oracle.binary_mod_f32(op, a, b, n), f(a[ia], b[ib]))
    # integer semantics: C truncation for division
    assert list(oracle.binary_mod_i32(DIV, [-7, 7], [2, -2], 2)) == [-3, -3]
    assert oracle.binary_mod_i32(POW, [2], [10], 1)[0] == 1024


def test_strided_broadcast_goldens(oracle, ref_vectors):
    bi = ref_vectors["broadcast_int"]
    a223 = np.array(bi["a_2_2_3"], np.float32)
    b23 = np.array(bi["b_2_3"], np.float32)
    out = oracle.binary_strided_f32(ADD, (2, 2, 3), a223, (6, 3, 1), b23, (0, 3, 1))
    assert np.array_equal(out, bi["a_2_2_3_plus_b_2_3"])
    b3 = np.array(bi["b_3"], np.float32)
    out = oracle.binary_strided_f32(ADD, (2, 2, 3), a223, (6, 3, 1), b3, (0, 0, 1))
    assert np.array_equal(out, bi["a_2_2_3_plus_b_3"])
    ts = ref_vectors["broadcast_two_sided"]
    out = oracle.binary_strided_f32(ADD, (3, 3), np.ravel(ts["a_3_1"]), (1, 0),
                                    np.ravel(ts["b_1_3"]), (0, 1))
    assert np.array_equal(out, ts["out"])


def test_strided_middle_axis_vs_numpy(oracle):
    g = rng(9)
    a = g.uniform(-1, 1, (2, 3, 4)).astype(np.float32)
    b = g.uniform(-1, 1, (2, 1, 4)).astype(np.float32)
    out = oracle.binary_strided_f32(MUL, (2, 3, 4), a, (12, 4, 1), b, (4, 0, 1))
    assert np.array_equal(out, a * b)


def test_unary_goldens(oracle, ref_vectors):
    s = ref_vectors["sigmoid"]
    out = oracle.sigmoid(s["x"])
    assert np.max(np.abs(out[:3] - s["expected_first3"])) <= s["tol_abs"]
    assert out[3] > s["x3_gt"] and out[4] < s["x4_lt"]
    r = ref_vectors["relu"]
    assert np.array_equal(oracle.relu(r["x"]), r["out"])


def test_sigmoid_vs_f64(oracle):
    x = rng(13).normal(0, 4, 4096).astype(np.float32)
    ref = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(oracle.sigmoid(x) - ref) / ref) < 1e-6


def test_sigmoid_bound_admits_fp32_sigmoid(oracle):
    """The GPU tests' bar after a sigmoid epilogue (gpu_util.sigmoid_bound)
    admits an fp32 sigmoid of an exact pre-activation at K = 1, where only
    its allowance for the sigmoid's own rounding is left, and still rejects
    a dropped bias of 0.02."""
    from gpu_util import gemm_tolerance_ok, sigmoid_bound
    x = rng(29).uniform(-12, 12, 100000).astype(np.float32)
    y64, bound = sigmoid_bound(x.astype(np.float64), np.zeros(x.size), 1)
    assert gemm_tolerance_ok(oracle.sigmoid(x), y64, bound, 1)[0]
    y64b, bound_b = sigmoid_bound(x.astype(np.float64) + 0.02, np.full(x.size, 0.02), 1)
    assert not gemm_tolerance_ok(oracle.sigmoid(x), y64b, bound_b, 1)[0]


def test_bias_sigmoid_and_backward(oracle):
    g = rng(17)
    d = g.normal(0, 1, (6, 10)).astype(np.float32)
    b = g.normal(0, 1, 10).astype(np.float32)
    out = oracle.bias_sigmoid(d, b)
    ref = 1 / (1 + np.exp(-(d.astype(np.float64) + b)))
    assert np.max(np.abs(out - ref)) < 1e-6
    dout = g.normal(0, 1, 60).astype(np.float32)
    x = g.normal(0, 2, 60).astype(np.float32)
    s = 1 / (1 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(oracle.sigmoid_backward(dout, x) - dout * s * (1 - s))) < 1e-6


def test_affine_and_chain(oracle):
    g = rng(19)
    x = g.uniform(-1, 1, 1000).astype(np.float32)
    out = oracle.affine(x, 1.5, -0.25)
    ref = (x.astype(np.float64) * 1.5 - 0.25).astype(np.float32)  # exact product, one rounding
    assert np.array_equal(out, ref)
    # chain of x*2 twenty times = x * 2^20 exactly
    assert np.array_equal(oracle.affine_chain(x, [2.0] * 20, [0.0] * 20), x * np.float32(2 ** 20))
    # chain equals step-by-step affine
    sc = g.uniform(0.5, 1.5, 20).astype(np.float32)
    of = g.uniform(-1, 1, 20).astype(np.float32)
    y = x.copy()
    for a, b in zip(sc, of):
        y = oracle.affine(y, a, b)
    assert np.array_equal(oracle.affine_chain(x, sc, of), y)


# ---- reductions -------------------------------------------------------------------

def test_reduction_goldens(oracle, ref_vectors):
    ag = ref_vectors["aggregates"]
    t = np.array(ag["t_3_2_3"], np.float32)
    assert oracle.sum_f64(t) == ag["sum"]
    assert oracle.fmin(t) == ag["min"] and oracle.fmax(t) == ag["max"]
    assert oracle.sum_f64(t) / t.size == ag["mean"]
    for ax in range(3):
        assert np.array_equal(oracle.sum_axis_f64(t, ax), ag[f"sum{ax}"])
        assert np.array_equal(oracle.sum_axis_f64(t, ax) / t.shape[ax], ag[f"mean{ax}"])
    assert abs(oracle.sum_ref(ag["f_sum_in"]) - ag["f_sum"]) <= ag["f_sum_tol_abs"]
    assert oracle.sum_f64(np.ones(10000, np.float32)) == ag["ones_10000_sum"]
    assert oracle.sum_axis_f64(np.ones((256, 128), np.float32), 0)[0] == ag["ones_256x128_sum0_first"]


def test_sum_exact_vs_fsum(oracle):
    x = rng(23).uniform(-1, 1, 100000).astype(np.float32)
    assert abs(oracle.sum_f64(x) - math.fsum(x.astype(np.float64))) < 1e-9
    n = 4096
    assert oracle.sum_f64(np.arange(n, dtype=np.float32)) == n * (n - 1) / 2


def test_sum_axis_vs_numpy(oracle):
    x = rng(29).normal(0, 1, (3, 5, 7)).astype(np.float32)
    for ax in range(3):
        np.testing.assert_allclose(oracle.sum_axis_f64(x, ax), x.astype(np.float64).sum(ax),
                                   rtol=1e-12, atol=1e-12)


def test_sum_axis_ref_order_and_goldens(oracle, ref_vectors):
    """The float path: the reference's goldens (integer-valued, exact in
    float), an explicit float32 loop in axis order on a small tensor, and
    the fp64 sum within the float accumulation bound on a large row."""
    ag = ref_vectors["aggregates"]
    t = np.array(ag["t_3_2_3"], np.float32)
    for ax in range(3):
        assert np.array_equal(oracle.sum_axis_ref(t, ax), np.array(ag[f"sum{ax}"], np.float32))
    x = rng(37).normal(0, 1, (4, 6, 5)).astype(np.float32)
    for ax in range(3):
        moved = np.moveaxis(x, ax, 0)
        acc = np.zeros(moved.shape[1:], np.float32)
        for a in range(moved.shape[0]):
            acc = (acc + moved[a]).astype(np.float32)
        assert np.array_equal(oracle.sum_axis_ref(x, ax), acc), ax
    big = rng(38).uniform(-1, 1, (2, 100000)).astype(np.float32)
    got = oracle.sum_axis_ref(big, 1).astype(np.float64)
    exact = oracle.sum_axis_f64(big, 1)
    bound = 100000 * np.finfo(np.float32).eps * np.abs(big).astype(np.float64).sum(1)
    assert np.all(np.abs(got - exact) <= bound)
    assert np.any(got != exact.astype(np.float32))  # it is float accumulation


def test_min_max_vs_numpy(oracle):
    x = rng(31).normal(0, 1, 5001).astype(np.float32)
    assert oracle.fmin(x) == x.min() and oracle.fmax(x) == x.max()


def test_argmax_goldens_and_rules(oracle, ref_vectors):
    a = ref_vectors["argmax"]
    assert list(oracle.argmax_rows(a["x"])) == a["out"]
    # ties: first index wins
    x = np.array([[1, 5, 5, 2], [7, 7, 7, 7]], np.float32)
    assert list(oracle.argmax_rows(x)) == [1, 0]
    # planted unique maximum
    y = rng(37).uniform(-1, 1, (3, 1000)).astype(np.float32)
    y[0, 777], y[1, 0], y[2, 999] = 2.0, 2.0, 2.0
    assert list(oracle.argmax_rows(y)) == [777, 0, 999]
    # NaN never wins
    z = np.array([[np.nan, 1.0, 3.0, np.nan]], np.float32)
    assert oracle.argmax_rows(z)[0] == 2
    # brute force vs numpy (numpy also returns the first maximum)
    w = rng(41).integers(-5, 5, (50, 40)).astype(np.float32)
    assert np.array_equal(oracle.argmax_rows(w), np.argmax(w, axis=1))


def test_argmax_cpu_reference_quirk(oracle):
    # include/array.h:1734 starts from numeric_limits<float>::min() (> 0):
    # an all-negative row returns 0 there; the true argmax is reported here.
    x = np.array([[-3.0, -1.0, -2.0]], np.float32)
    assert oracle.argmax_rows_cpu_ref(x)[0] == 0
    assert oracle.argmax_rows(x)[0] == 1


# ---- row ops ----------------------------------------------------------------------

def test_softmax_goldens(oracle, ref_vectors):
    s = ref_vectors["softmax"]
    x = np.array([s["x"]], np.float32)
    for out in (oracle.softmax_rows_f64(x), oracle.softmax_rows_ref(x)):
        assert np.max(np.abs(out[0] - s["expected"])) <= s["tol_abs"]
    m = np.array(s["int_rows"], np.float32)
    assert np.allclose(oracle.softmax_rows_f64(m).sum(1), 1.0, atol=1e-12)


def test_softmax_vs_scipy_and_invariants(oracle):
    x = rng(43).normal(0, 3, (16, 300)).astype(np.float32)
    f64 = oracle.softmax_rows_f64(x)
    np.testing.assert_allclose(f64, special.softmax(x.astype(np.float64), axis=1), rtol=1e-12)
    np.testing.assert_allclose(f64.sum(1), 1.0, rtol=1e-12)
    # shift invariance
    np.testing.assert_allclose(oracle.softmax_rows_f64(x + np.float32(8.0)), f64, rtol=1e-5)
    ref = oracle.softmax_rows_ref(x)
    assert np.max(np.abs(ref - f64) / f64) < 1e-5


def test_layer_norm_goldens(oracle, ref_vectors):
    ln = ref_vectors["layer_norm"]
    x = np.array(ln["x"], np.float32)
    for fn in (oracle.layer_norm_f64, oracle.layer_norm_ref):
        out = fn(x, ln["gamma"], ln["beta"])
        assert np.max(np.abs(out[0] - ln["row0"])) <= ln["tol_abs"]
        out2 = fn(x, ln["gamma2"], ln["beta2"])
        assert abs(out2[0, 1] - ln["out2_01"]) <= ln["tol_abs"]


def test_layer_norm_vs_numpy_and_invariants(oracle):
    g = rng(47)
    x = g.normal(0, 3, (8, 500)).astype(np.float32)
    gamma = g.uniform(0.5, 1.5, 500).astype(np.float32)
    beta = g.uniform(-1, 1, 500).astype(np.float32)
    xd = x.astype(np.float64)
    mu = xd.mean(1, keepdims=True)
    var = ((xd - mu) ** 2).mean(1, keepdims=True)
    ref = (xd - mu) / np.sqrt(var + 1e-5) * gamma + beta
    f64 = oracle.layer_norm_f64(x, gamma, beta)
    np.testing.assert_allclose(f64, ref, rtol=1e-12, atol=1e-12)
    unit = oracle.layer_norm_f64(x, np.ones(500, np.float32), np.zeros(500, np.float32))
    assert np.max(np.abs(unit.mean(1))) < 1e-12
    np.testing.assert_allclose(unit.var(1), (var / (var + 1e-5)).ravel(), rtol=1e-10)
    r = oracle.layer_norm_ref(x, gamma, beta)
    assert np.max(np.abs(r - f64)) / np.max(np.abs(f64)) < 1e-5


# ---- conv2d -------------------------------------------------------------------------

def _conv2d_loops(x, w):
    """Six nested loops straight from the definition (tiny inputs only)."""
    N, H, W, Ci = x.shape
    Co, K, _, _ = w.shape
    p = K // 2
    out = np.zeros((N, H, W, Co))
    for n in range(N):
        for oh in range(H):
            for ow in range(W):
                for co in range(Co):
                    acc = 0.0
                    for kh in range(K):
                        for kw in range(K):
                            ih, iw = oh + kh - p, ow + kw - p
                            if 0 <= ih < H and 0 <= iw < W:
                                for ci in range(Ci):
                                    acc += float(x[n, ih, iw, ci]) * float(w[co, kh, kw, ci])
                    out[n, oh, ow, co] = acc
    return out


@pytest.mark.parametrize("shape", [(1, 4, 5, 3, 3, 2), (2, 3, 3, 2, 1, 3), (1, 5, 4, 2, 2, 2),
                                   (1, 6, 6, 1, 5, 1)])
def test_conv2d_oracle_matches_loops(oracle, shape):
    N, H, W, Ci, K, Co = shape
    g = np.random.default_rng(77)
    x = g.normal(size=(N, H, W, Ci))
    w = g.normal(size=(Co, K, K, Ci))
    assert np.allclose(oracle.conv2d_f64(x, w), _conv2d_loops(x, w), rtol=1e-12, atol=1e-12)


def test_conv2d_oracle_closed_forms(oracle):
    # ones input and weights: C_in times the number of taps inside the image
    x = np.ones((1, 3, 3, 2))
    w = np.ones((1, 3, 3, 2))
    out = oracle.conv2d_f64(x, w)[0, :, :, 0]
    assert np.array_equal(out, [[8, 12, 8], [12, 18, 12], [8, 12, 8]])
    # a 1x1 kernel is the product of the pixels with the weight's transpose
    g = np.random.default_rng(3)
    x = g.normal(size=(2, 4, 5, 6))
    w = g.normal(size=(7, 1, 1, 6))
    ref = (x.reshape(-1, 6) @ w.reshape(7, 6).T).reshape(2, 4, 5, 7)
    assert np.allclose(oracle.conv2d_f64(x, w), ref, rtol=1e-12)


def test_conv2d_oracle_single_channel_is_correlation(oracle):
    """One channel in and out with an odd kernel: scipy's 2-D correlation
    with zero fill and output the size of the input."""
    from scipy.signal import correlate2d
    g = np.random.default_rng(5)
    for K in (1, 3, 5):
        x = g.normal(size=(9, 7))
        w = g.normal(size=(K, K))
        ref = correlate2d(x, w, mode="same", boundary="fill", fillvalue=0)
        out = oracle.conv2d_f64(x[None, :, :, None], w[None, :, :, None])[0, :, :, 0]
        assert np.allclose(out, ref, rtol=1e-12, atol=1e-12), K
