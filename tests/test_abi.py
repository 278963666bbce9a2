"""C ABI checks that need no GPU: the library loads, exports exactly what
include/silgpu.h declares, and rejects bad arguments with a status code and a
message before touching the device."""

import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "silgpu.h"
LIB = ROOT / "silarray_amd" / "libsilgpu.so"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(silgpu_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    for required in ["silgpu_init", "silgpu_sync", "silgpu_alloc", "silgpu_free",
                     "silgpu_sgemm", "silgpu_sgemv", "silgpu_softmax_rows_f32",
                     "silgpu_layer_norm_rows_f32", "silgpu_sum_f32", "silgpu_argmax_rows_f32",
                     "silgpu_binary_f32", "silgpu_program_f32"]:
        assert required in names


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (silgpu_[a-z0-9_]+)", out))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing


def test_binding_covers_header():
    from silarray_amd import _native as nat
    assert sorted(nat.EXPORTED) == declared_functions()


def test_library_is_gfx950_only():
    # Offload bundle entry ids are embedded as text in the fat binary.
    data = LIB.read_bytes()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa-[-a-z0-9:+]*", data))
    assert targets and all(t.endswith(b"gfx950") for t in targets), targets


@pytest.fixture(scope="module")
def lib():
    from silarray_amd import _native as nat
    return nat


def test_validation_errors_without_device(lib):
    f = lib.raw
    v = C.c_void_p
    # negative extents / bad leading dimensions are rejected before any device use
    rc = f("silgpu_sgemm")(0, 0, -1, 4, 4, v(16), 4, 0, v(16), 4, 0, v(16), 4, 0, 1, None, 0, 0)
    assert rc == lib.ERR_INVALID and "negative" in lib.last_error()
    rc = f("silgpu_sgemm")(0, 0, 4, 4, 8, v(16), 4, 0, v(16), 4, 0, v(16), 4, 0, 1, None, 0, 0)
    assert rc == lib.ERR_INVALID and "lda" in lib.last_error()
    rc = f("silgpu_sgemm")(0, 0, 4, 4, 4, v(16), 4, 0, v(16), 4, 0, v(16), 4, 0, 1, None, 0, 1)
    assert rc == lib.ERR_INVALID and "bias" in lib.last_error()
    rc = f("silgpu_sgemm")(0, 0, 4, 4, 4, v(16), 4, 0, v(16), 4, 0, v(16), 4, 0, 1, None, 0, 9)
    assert rc == lib.ERR_INVALID and "epilogue" in lib.last_error()
    rc = f("silgpu_softmax_rows_f32")(v(16), v(16), -2, 8)
    assert rc == lib.ERR_INVALID
    rc = f("silgpu_unary_f32")(0, None, None, 10)
    assert rc == lib.ERR_INVALID and "null" in lib.last_error()
    rc = f("silgpu_binary_f32")(0, v(16), 0, v(16), 1, v(16), 5)
    assert rc == lib.ERR_INVALID
    rc = f("silgpu_binary_strided_f32")(0, 9, None, None, None, None, None, None)
    assert rc == lib.ERR_INVALID and "ndim" in lib.last_error()
    # empty work is a no-op success
    assert f("silgpu_sgemm")(0, 0, 0, 4, 4, None, 4, 0, None, 4, 0, None, 4, 0, 1, None, 0, 0) == 0
    assert f("silgpu_softmax_rows_f32")(None, None, 0, 8) == 0


def test_attention_validation(lib):
    d = lib.AttnDesc()
    d.Sq, d.Sk, d.D, d.batch_outer, d.batch_inner, d.scale = 8, 8, 48, 1, 1, 1.0
    d.Q = d.K = d.V = d.O = 16
    d.ldq = d.ldk = d.ldv = d.ldo = 64
    rc = lib.raw("silgpu_attention_f32")(C.byref(d))
    assert rc == lib.ERR_INVALID and "head dim" in lib.last_error()
    d.D, d.ldq = 64, 60
    rc = lib.raw("silgpu_attention_f32")(C.byref(d))
    assert rc == lib.ERR_INVALID and "row stride" in lib.last_error()
    d.ldq = 64
    d.Sq = -1
    rc = lib.raw("silgpu_attention_f32")(C.byref(d))
    assert rc == lib.ERR_INVALID and "negative" in lib.last_error()
    d.Sq = 0  # empty work is a no-op success
    assert lib.raw("silgpu_attention_f32")(C.byref(d)) == 0


def test_conv2d_validation(lib):
    f = lib.raw("silgpu_conv2d_f32")
    assert f(None, None, None, 1, 4, 4, 3, 0, 8) == lib.ERR_INVALID
    assert "kernel size" in lib.last_error()
    assert f(None, None, None, 1, -4, 4, 3, 3, 8) == lib.ERR_INVALID
    assert f(None, None, None, 1 << 40, 1 << 40, 4, 3, 3, 8) == lib.ERR_INVALID
    assert "overflows" in lib.last_error()
    assert f(None, None, None, 1 << 20, 1 << 12, 1, 3, 3, 8) == lib.ERR_INVALID
    assert "int32" in lib.last_error()
    assert f(None, None, None, 0, 4, 4, 3, 3, 8) == 0  # no output pixels: no-op


def test_program_validation(lib):
    p = lib.make_program((4,), [(16, (1,))], [(lib.PI_LOAD, 0, 3, 0, 0.0, 0.0)])
    rc = lib.raw("silgpu_program_f32")(C.byref(p), C.c_void_p(16))
    assert rc == lib.ERR_INVALID and "input" in lib.last_error()
    p = lib.make_program((4,), [(16, (1,))], [(lib.PI_LOAD, 9, 0, 0, 0.0, 0.0)])
    rc = lib.raw("silgpu_program_f32")(C.byref(p), C.c_void_p(16))
    assert rc == lib.ERR_INVALID


def test_init_reports_missing_device(lib):
    import os
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present")
    rc = lib.raw("silgpu_init")()
    assert rc == lib.ERR_NODEVICE
    assert "no HIP device" in lib.last_error()
