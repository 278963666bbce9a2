"""numpy-facing wrappers of liboracle.so (oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The product never imports it.
"""

from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# oracle/cpubase.py loads this file a second time with LIB_OVERRIDE set to one
# of the -O3 builds of the same C source (the CPU baseline).
LIB_PATH = Path(globals().get("LIB_OVERRIDE", HERE / "liboracle.so"))


def build() -> Path:
    subprocess.run(["make", "-s", "-B", "-C", str(HERE), "liboracle.so"], check=True)
    return LIB_PATH


if not LIB_PATH.exists() and "LIB_OVERRIDE" not in globals():
    build()

_lib = C.CDLL(str(LIB_PATH))
_vp, _i64, _f, _i = C.c_void_p, C.c_int64, C.c_float, C.c_int

_SIGS = {
    "oracle_sgemm_f64": (None, [_i, _i, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _vp]),
    "oracle_sgemm_sampled_f64": (None, [_i, _i, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64,
                                        _vp, _vp]),
    "oracle_binary_mod_f32": (None, [_i, _vp, _i64, _vp, _i64, _vp, _i64]),
    "oracle_binary_mod_i32": (None, [_i, _vp, _i64, _vp, _i64, _vp, _i64]),
    "oracle_binary_strided_f32": (None, [_i, _i, _vp, _vp, _vp, _vp, _vp, _vp]),
    "oracle_sigmoid": (None, [_vp, _vp, _i64]),
    "oracle_relu": (None, [_vp, _vp, _i64]),
    "oracle_bias_sigmoid": (None, [_vp, _vp, _i64, _i64]),
    "oracle_sigmoid_backward": (None, [_vp, _vp, _vp, _i64]),
    "oracle_affine": (None, [_vp, _vp, _i64, _f, _f]),
    "oracle_affine_chain": (None, [_vp, _vp, _i64, _vp, _vp, _i]),
    "oracle_sum_f64": (C.c_double, [_vp, _i64]),
    "oracle_sum_ref": (C.c_float, [_vp, _i64]),
    "oracle_min": (C.c_float, [_vp, _i64]),
    "oracle_max": (C.c_float, [_vp, _i64]),
    "oracle_sum_axis_f64": (None, [_vp, _i64, _i64, _i64, _vp]),
    "oracle_sum_axis_ref": (None, [_vp, _i64, _i64, _i64, _vp]),
    "oracle_argmax_rows": (None, [_vp, _i64, _i64, _vp]),
    "oracle_argmax_rows_cpu_ref": (None, [_vp, _i64, _i64, _vp]),
    "oracle_softmax_rows_f64": (None, [_vp, _i64, _i64, _vp]),
    "oracle_softmax_rows_ref": (None, [_vp, _i64, _i64, _vp]),
    "oracle_layer_norm_f64": (None, [_vp, _vp, _vp, _i64, _i64, _f, _vp]),
    "oracle_layer_norm_ref": (None, [_vp, _vp, _vp, _i64, _i64, _f, _vp]),
    "oracle_gemv_f32": (None, [_vp, _vp, _i64, _i64, _vp]),
}
for _n, (_r, _a) in _SIGS.items():
    _fn = getattr(_lib, _n)
    _fn.restype = _r
    _fn.argtypes = _a


def _p(a: np.ndarray) -> C.c_void_p:
    return a.ctypes.data_as(_vp)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def sgemm_f64(A, B, ta=False, tb=False, with_abs=False):
    """op(A) @ op(B) in float64 from float32 inputs (2-D, row-major)."""
    A, B = _f32(A), _f32(B)
    M = A.shape[1] if ta else A.shape[0]
    K = A.shape[0] if ta else A.shape[1]
    N = B.shape[0] if tb else B.shape[1]
    assert (B.shape[1] if tb else B.shape[0]) == K
    Cm = np.empty((M, N), np.float64)
    Ca = np.empty((M, N), np.float64) if with_abs else None
    _lib.oracle_sgemm_f64(int(ta), int(tb), M, N, K, _p(A), A.shape[1], _p(B), B.shape[1],
                          _p(Cm), _p(Ca) if with_abs else None)
    return (Cm, Ca) if with_abs else Cm


def sgemm_sampled_f64(A, B, rows, cols, ta=False, tb=False):
    A, B = _f32(A), _f32(B)
    K = A.shape[0] if ta else A.shape[1]
    rows = np.ascontiguousarray(rows, np.int64)
    cols = np.ascontiguousarray(cols, np.int64)
    out = np.empty(len(rows), np.float64)
    outabs = np.empty(len(rows), np.float64)
    _lib.oracle_sgemm_sampled_f64(int(ta), int(tb), K, _p(A), A.shape[1], _p(B), B.shape[1],
                                  _p(rows), _p(cols), len(rows), _p(out), _p(outabs))
    return out, outabs


def binary_mod_f32(op, a, b, n):
    a, b = _f32(a), _f32(b)
    out = np.empty(n, np.float32)
    _lib.oracle_binary_mod_f32(op, _p(a), a.size, _p(b), b.size, _p(out), n)
    return out


def binary_mod_i32(op, a, b, n):
    a = np.ascontiguousarray(a, np.int32)
    b = np.ascontiguousarray(b, np.int32)
    out = np.empty(n, np.int32)
    _lib.oracle_binary_mod_i32(op, _p(a), a.size, _p(b), b.size, _p(out), n)
    return out


def binary_strided_f32(op, shape, a, sa, b, sb):
    a, b = _f32(a), _f32(b)
    nd = len(shape)
    sh = np.asarray(shape, np.int64)
    sa_ = np.asarray(sa, np.int64)
    sb_ = np.asarray(sb, np.int64)
    out = np.empty(int(np.prod(shape)) if nd else 1, np.float32)
    _lib.oracle_binary_strided_f32(op, nd, _p(sh), _p(a), _p(sa_), _p(b), _p(sb_), _p(out))
    return out.reshape(shape)


def sigmoid(x):
    x = _f32(x)
    out = np.empty_like(x)
    _lib.oracle_sigmoid(_p(x), _p(out), x.size)
    return out


def relu(x):
    x = _f32(x)
    out = np.empty_like(x)
    _lib.oracle_relu(_p(x), _p(out), x.size)
    return out


def bias_sigmoid(data, bias):
    data = _f32(data).copy()
    bias = _f32(bias)
    _lib.oracle_bias_sigmoid(_p(data), _p(bias), data.size, bias.size)
    return data


def sigmoid_backward(dout, x):
    dout, x = _f32(dout), _f32(x)
    out = np.empty_like(x)
    _lib.oracle_sigmoid_backward(_p(dout), _p(x), _p(out), x.size)
    return out


def affine(x, scale, offset):
    x = _f32(x)
    out = np.empty_like(x)
    _lib.oracle_affine(_p(x), _p(out), x.size, scale, offset)
    return out


def affine_into(x, out, scale, offset):
    """out[i] = fmaf(x[i], scale, offset) into an existing array."""
    assert x.dtype == np.float32 and out.dtype == np.float32 and x.size == out.size
    assert x.flags.c_contiguous and out.flags.c_contiguous
    _lib.oracle_affine(_p(x), _p(out), x.size, scale, offset)


def affine_chain(x, scales, offsets):
    x = _f32(x)
    s = _f32(scales)
    o = _f32(offsets)
    out = np.empty_like(x)
    _lib.oracle_affine_chain(_p(x), _p(out), x.size, _p(s), _p(o), len(s))
    return out


def sum_f64(x) -> float:
    x = _f32(x)
    return _lib.oracle_sum_f64(_p(x), x.size)


def sum_ref(x) -> float:
    x = _f32(x)
    return _lib.oracle_sum_ref(_p(x), x.size)


def fmin(x) -> float:
    x = _f32(x)
    return _lib.oracle_min(_p(x), x.size)


def fmax(x) -> float:
    x = _f32(x)
    return _lib.oracle_max(_p(x), x.size)


def sum_axis_f64(x, axis):
    x = _f32(x)
    shape = x.shape
    outer = int(np.prod(shape[:axis])) if axis > 0 else 1
    inner = int(np.prod(shape[axis + 1:])) if axis + 1 < len(shape) else 1
    out = np.empty(outer * inner, np.float64)
    _lib.oracle_sum_axis_f64(_p(x), outer, shape[axis], inner, _p(out))
    return out.reshape(shape[:axis] + shape[axis + 1:])


def sum_axis_ref(x, axis):
    x = _f32(x)
    shape = x.shape
    outer = int(np.prod(shape[:axis])) if axis > 0 else 1
    inner = int(np.prod(shape[axis + 1:])) if axis + 1 < len(shape) else 1
    out = np.empty(outer * inner, np.float32)
    _lib.oracle_sum_axis_ref(_p(x), outer, shape[axis], inner, _p(out))
    return out.reshape(shape[:axis] + shape[axis + 1:])


def argmax_rows(x):
    x = _f32(x)
    out = np.empty(x.shape[0], np.int32)
    _lib.oracle_argmax_rows(_p(x), x.shape[0], x.shape[1], _p(out))
    return out


def argmax_rows_cpu_ref(x):
    x = _f32(x)
    out = np.empty(x.shape[0], np.int32)
    _lib.oracle_argmax_rows_cpu_ref(_p(x), x.shape[0], x.shape[1], _p(out))
    return out


def softmax_rows_f64(x):
    x = _f32(x)
    out = np.empty(x.shape, np.float64)
    _lib.oracle_softmax_rows_f64(_p(x), x.shape[0], x.shape[1], _p(out))
    return out


def softmax_rows_ref(x):
    x = _f32(x)
    out = np.empty(x.shape, np.float32)
    _lib.oracle_softmax_rows_ref(_p(x), x.shape[0], x.shape[1], _p(out))
    return out


def layer_norm_f64(x, gamma, beta, eps=1e-5):
    x, g, b = _f32(x), _f32(gamma), _f32(beta)
    out = np.empty(x.shape, np.float64)
    _lib.oracle_layer_norm_f64(_p(x), _p(g), _p(b), x.shape[0], x.shape[1], eps, _p(out))
    return out


def layer_norm_ref(x, gamma, beta, eps=1e-5):
    x, g, b = _f32(x), _f32(gamma), _f32(beta)
    out = np.empty(x.shape, np.float32)
    _lib.oracle_layer_norm_ref(_p(x), _p(g), _p(b), x.shape[0], x.shape[1], eps, _p(out))
    return out


def gemv_f32(x, B):
    x, B = _f32(x), _f32(B)
    y = np.empty(B.shape[1], np.float32)
    _lib.oracle_gemv_f32(_p(x), _p(B), B.shape[1], B.shape[0], _p(y))
    return y


def conv2d_f64(x, w):
    """2-D convolution in float64: NHWC x [N, H, W, C_in], OHWI w [C_out, K,
    K, C_in], stride 1, zero padding K // 2, output [N, H, W, C_out] --
    out[n, oh, ow, co] = sum over kh, kw, ci of x[n, oh + kh - K//2,
    ow + kw - K//2, ci] * w[co, kh, kw, ci].  Follows the reference's
    implicit-GEMM conv (include/gpu.h:1247-1257: pad = K / 2, H_out = H,
    W_out = W; include/gpu_kernels.metal:1536-1545 and the (kh, kw, ci)
    order of the K dimension), array::conv2d's shapes
    (include/array.h:1508-1517, 2259-2273) and the OHWI weight the
    reference's benchmark builds (bench/micro/bench_nn_ops.cpp:204-205)."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    N, H, W, Ci = x.shape
    Co, K, K2, Ci2 = w.shape
    assert K == K2 and Ci == Ci2
    p = K // 2
    xp = np.zeros((N, H + K - 1, W + K - 1, Ci))
    xp[:, p:p + H, p:p + W, :] = x
    out = np.zeros((N, H, W, Co))
    for kh in range(K):
        for kw in range(K):
            out += xp[:, kh:kh + H, kw:kw + W, :] @ w[:, kh, kw, :].T
    return out
