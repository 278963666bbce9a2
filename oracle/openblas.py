"""cblas_sgemm from OpenBLAS, the x86 stand-in for the reference's Accelerate
call (include/cpu.h:239-264: cblas_sgemm(RowMajor, NoTrans, NoTrans, M, N, K,
1, A, K, B, N, 0, C, N)).

TEST INFRASTRUCTURE ONLY: used by tests/ and the cpu_baseline leg of bench.py.
Uses the system libopenblas if present, else the OpenBLAS 0.3.29 (ILP64)
bundled with numpy (symbol scipy_cblas_sgemm64_).
"""

from __future__ import annotations

import ctypes as C
import ctypes.util
import glob
import os

import numpy as np

CblasRowMajor, CblasNoTrans, CblasTrans = 101, 111, 112


def _load():
    path = ctypes.util.find_library("openblas")
    if path:
        lib = C.CDLL(path)
        if hasattr(lib, "cblas_sgemm"):
            return lib, lib.cblas_sgemm, C.c_int, getattr(lib, "openblas_set_num_threads", None), path
    npdir = os.path.dirname(np.__file__)
    cands = glob.glob(os.path.join(npdir, "..", "numpy.libs", "libscipy_openblas64_*.so"))
    cands += glob.glob(os.path.join(npdir, ".libs", "libscipy_openblas64_*.so"))
    if not cands:
        raise ImportError("no OpenBLAS library found")
    lib = C.CDLL(cands[0])
    return (lib, lib.scipy_cblas_sgemm64_, C.c_int64,
            getattr(lib, "scipy_openblas_set_num_threads64_", None), cands[0])


_lib, _sgemm, _blasint, _set_threads, LIB_PATH = _load()
_sgemm.restype = None
_sgemm.argtypes = [C.c_int, C.c_int, C.c_int, _blasint, _blasint, _blasint, C.c_float,
                   C.c_void_p, _blasint, C.c_void_p, _blasint, C.c_float, C.c_void_p,
                   _blasint]
if _set_threads is not None:
    _set_threads.restype = None
    _set_threads.argtypes = [C.c_int]


def set_threads(n: int) -> None:
    if _set_threads is not None:
        _set_threads(int(n))


def sgemm(A: np.ndarray, B: np.ndarray, out: np.ndarray | None = None) -> np.ndarray:
    """C = A @ B (row-major float32, NoTrans/NoTrans), via cblas_sgemm."""
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    if out is None:
        out = np.empty((M, N), np.float32)
    _sgemm(CblasRowMajor, CblasNoTrans, CblasNoTrans, M, N, K, 1.0, A.ctypes.data, K,
           B.ctypes.data, N, 0.0, out.ctypes.data, N)
    return out
