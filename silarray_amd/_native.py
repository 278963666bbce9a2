"""ctypes binding of libsilgpu.so, the C ABI declared in include/silgpu.h.

This is the path tests and bench.py use to call the HIP kernels.  There is no
fallback: if libsilgpu.so is missing or fails to load, importing this module
raises, and every call that returns a non-zero status raises SilGpuError with
the library's own message.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

_PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("SILGPU_LIB", _PKG / "libsilgpu.so"))

# Status codes (include/silgpu.h)
OK = 0
ERR_INVALID = -1
ERR_HIP = -2
ERR_NOMEM = -3
ERR_UNSUPPORTED = -4
ERR_NODEVICE = -5

ADD, SUB, MUL, DIV, POW = range(5)
SIGMOID, RELU = 0, 1
EPI_NONE, EPI_BIAS, EPI_BIAS_SIGMOID, EPI_RELU, EPI_BIAS_RELU = range(5)

# Program opcodes
(PI_LOAD, PI_CONST, PI_ADD, PI_SUB, PI_MUL, PI_DIV, PI_POW, PI_ADDI, PI_MULI, PI_RSUBI,
 PI_RDIVI, PI_SIGMOID, PI_RELU, PI_FMAI, PI_SIGBWD) = range(15)
PROG_MAX_INPUTS, PROG_MAX_INSTRS, PROG_MAX_REGS, PROG_MAX_DIMS = 8, 64, 8, 6


class SilGpuError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"silgpu error {code}: {msg}")
        self.code = code


if not LIB_PATH.exists():
    raise ImportError(
        f"{LIB_PATH} not found: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
    )

_lib = C.CDLL(str(LIB_PATH))

_i64 = C.c_int64
_vp = C.c_void_p
_f = C.c_float
_i = C.c_int


class ProgInstr(C.Structure):
    _fields_ = [("op", C.c_int32), ("dst", C.c_int32), ("a", C.c_int32), ("b", C.c_int32),
                ("imm", C.c_float), ("imm2", C.c_float)]


class ProgInput(C.Structure):
    _fields_ = [("ptr", C.c_void_p), ("strides", C.c_int64 * PROG_MAX_DIMS)]


class Program(C.Structure):
    _fields_ = [("n_inputs", C.c_int32), ("n_instrs", C.c_int32), ("ndim", C.c_int32),
                ("out_reg", C.c_int32), ("shape", C.c_int64 * PROG_MAX_DIMS),
                ("inputs", ProgInput * PROG_MAX_INPUTS),
                ("instrs", ProgInstr * PROG_MAX_INSTRS)]


class GemmDesc(C.Structure):
    """silgpu_gemm_desc (include/silgpu.h)."""
    _fields_ = [("trans_a", C.c_int32), ("trans_b", C.c_int32),
                ("M", C.c_int64), ("N", C.c_int64), ("K", C.c_int64),
                ("A", C.c_void_p), ("lda", C.c_int64),
                ("B", C.c_void_p), ("ldb", C.c_int64),
                ("C", C.c_void_p), ("ldc", C.c_int64),
                ("batch_outer", C.c_int64), ("batch_inner", C.c_int64),
                ("stride_a_outer", C.c_int64), ("stride_a_inner", C.c_int64),
                ("stride_b_outer", C.c_int64), ("stride_b_inner", C.c_int64),
                ("stride_c_outer", C.c_int64), ("stride_c_inner", C.c_int64),
                ("epilogue", C.c_int32), ("use_scale", C.c_int32),
                ("scale", C.c_float), ("scale_offset", C.c_float),
                ("bias", C.c_void_p), ("bias_len", C.c_int64),
                ("residual", C.c_void_p), ("ldr", C.c_int64)]


class AttnDesc(C.Structure):
    """silgpu_attn_desc (include/silgpu.h)."""
    _fields_ = [("Sq", C.c_int64), ("Sk", C.c_int64), ("D", C.c_int64),
                ("batch_outer", C.c_int64), ("batch_inner", C.c_int64), ("scale", C.c_float),
                ("Q", C.c_void_p), ("ldq", C.c_int64),
                ("stride_q_outer", C.c_int64), ("stride_q_inner", C.c_int64),
                ("K", C.c_void_p), ("ldk", C.c_int64),
                ("stride_k_outer", C.c_int64), ("stride_k_inner", C.c_int64),
                ("V", C.c_void_p), ("ldv", C.c_int64),
                ("stride_v_outer", C.c_int64), ("stride_v_inner", C.c_int64),
                ("O", C.c_void_p), ("ldo", C.c_int64),
                ("stride_o_outer", C.c_int64), ("stride_o_inner", C.c_int64)]


_SIGS = {
    "silgpu_last_error": (C.c_char_p, []),
    "silgpu_init": (_i, []),
    "silgpu_sync": (_i, []),
    "silgpu_device_info": (_i, [C.POINTER(_i), C.POINTER(_i), C.POINTER(_i), C.c_char_p,
                                C.c_size_t]),
    "silgpu_alloc": (_i, [C.c_size_t, C.POINTER(_vp)]),
    "silgpu_free": (_i, [_vp]),
    "silgpu_pool_trim": (_i, []),
    "silgpu_pool_stats": (_i, [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    "silgpu_host_alloc": (_i, [C.c_size_t, C.POINTER(_vp)]),
    "silgpu_host_free": (_i, [_vp]),
    "silgpu_memcpy_h2d": (_i, [_vp, _vp, C.c_size_t]),
    "silgpu_memcpy_d2h": (_i, [_vp, _vp, C.c_size_t]),
    "silgpu_memcpy_d2d": (_i, [_vp, _vp, C.c_size_t]),
    "silgpu_fill_u32": (_i, [_vp, C.c_uint32, _i64]),
    "silgpu_binary_f32": (_i, [_i, _vp, _i64, _vp, _i64, _vp, _i64]),
    "silgpu_binary_i32": (_i, [_i, _vp, _i64, _vp, _i64, _vp, _i64]),
    "silgpu_binary_strided_f32": (_i, [_i, _i, C.POINTER(_i64), _vp, C.POINTER(_i64), _vp,
                                       C.POINTER(_i64), _vp]),
    "silgpu_unary_f32": (_i, [_i, _vp, _vp, _i64]),
    "silgpu_sigmoid_backward_f32": (_i, [_vp, _vp, _vp, _i64]),
    "silgpu_bias_sigmoid_f32": (_i, [_vp, _vp, _i64, _i64]),
    "silgpu_affine_f32": (_i, [_vp, _vp, _i64, _f, _f]),
    "silgpu_program_f32": (_i, [C.POINTER(Program), _vp]),
    "silgpu_sum_f32": (_i, [_vp, _i64, _vp]),
    "silgpu_min_f32": (_i, [_vp, _i64, _vp]),
    "silgpu_max_f32": (_i, [_vp, _i64, _vp]),
    "silgpu_sum_axis_f32": (_i, [_vp, _i64, _i64, _i64, _vp]),
    "silgpu_argmax_rows_f32": (_i, [_vp, _i64, _i64, _vp]),
    "silgpu_slot_wait_selftest": (_i, [_i, _i64, _i64, _vp]),
    "silgpu_slots_in_use": (_i, [C.POINTER(_i64)]),
    "silgpu_softmax_rows_f32": (_i, [_vp, _vp, _i64, _i64]),
    "silgpu_layer_norm_rows_f32": (_i, [_vp, _vp, _vp, _vp, _i64, _i64, _f]),
    "silgpu_sgemm": (_i, [_i, _i, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp,
                          _i64, _i64, _i64, _vp, _i64, _i]),
    "silgpu_sgemm_tuned": (_i, [_i, _i, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64,
                                _vp, _i64, _i64, _i64, _vp, _i64, _i, _i, _i]),
    "silgpu_gemm": (_i, [C.POINTER(GemmDesc)]),
    "silgpu_gemm_noalloc": (_i, [C.POINTER(GemmDesc)]),
    "silgpu_gemm_last_plan": (_i, [C.POINTER(_i), C.POINTER(_i), C.POINTER(_i),
                                   C.POINTER(_i)]),
    "silgpu_sgemv": (_i, [_vp, _vp, _i64, _vp, _i64, _i64]),
    "silgpu_attention_f32": (_i, [C.POINTER(AttnDesc)]),
    "silgpu_conv2d_f32": (_i, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64]),
    "silgpu_event_create": (_i, [C.POINTER(_vp)]),
    "silgpu_event_destroy": (_i, [_vp]),
    "silgpu_event_record": (_i, [_vp]),
    "silgpu_event_elapsed_ms": (_i, [_vp, _vp, C.POINTER(_f)]),
    "silgpu_get_stream": (_i, [C.POINTER(_vp)]),
}

for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(_lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args

EXPORTED = tuple(_SIGS)


def last_error() -> str:
    return (_lib.silgpu_last_error() or b"").decode()


def check(rc: int) -> None:
    if rc != OK:
        raise SilGpuError(rc, last_error())


def call(name: str, *args) -> None:
    check(getattr(_lib, name)(*args))


def raw(name: str):
    """The bare ctypes function (returns the status code instead of raising)."""
    return getattr(_lib, name)


def init() -> None:
    call("silgpu_init")


def sync() -> None:
    call("silgpu_sync")


def device_info() -> dict:
    cu, clk, lds = _i(), _i(), _i()
    arch = C.create_string_buffer(64)
    call("silgpu_device_info", C.byref(cu), C.byref(clk), C.byref(lds), arch, 64)
    return {"cu_count": cu.value, "clock_khz": clk.value, "lds_bytes": lds.value,
            "arch": arch.value.decode()}


class DeviceBuffer:
    """A block of HBM from the library's pool, with numpy upload/download."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = _vp()
        call("silgpu_alloc", C.c_size_t(self.nbytes), C.byref(p))
        self.ptr = p.value
        self._freed = False

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(max(a.nbytes, 4))
        buf.upload(a)
        return buf

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        call("silgpu_memcpy_h2d", _vp(self.ptr), a.ctypes.data_as(_vp), C.c_size_t(a.nbytes))

    def download(self, shape, dtype=np.float32, offset_bytes: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert offset_bytes + out.nbytes <= self.nbytes
        call("silgpu_memcpy_d2h", out.ctypes.data_as(_vp), _vp(self.ptr + offset_bytes),
             C.c_size_t(out.nbytes))
        return out

    def at(self, offset_bytes: int) -> int:
        return self.ptr + offset_bytes

    def free(self) -> None:
        if not self._freed:
            call("silgpu_free", _vp(self.ptr))
            self._freed = True

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        p = _vp()
        call("silgpu_event_create", C.byref(p))
        self.ptr = p.value

    def record(self) -> None:
        call("silgpu_event_record", _vp(self.ptr))

    def elapsed_ms(self, end: "Event") -> float:
        ms = _f()
        call("silgpu_event_elapsed_ms", _vp(self.ptr), _vp(end.ptr), C.byref(ms))
        return ms.value

    def __del__(self):
        try:
            _lib.silgpu_event_destroy(_vp(self.ptr))
        except Exception:
            pass


def vp(x) -> C.c_void_p:
    """A device pointer argument from a DeviceBuffer or an int address."""
    if isinstance(x, DeviceBuffer):
        return _vp(x.ptr)
    return _vp(x)


# ---- thin typed wrappers ------------------------------------------------------

def binary_f32(op, a, a_len, b, b_len, out, n):
    call("silgpu_binary_f32", op, vp(a), a_len, vp(b), b_len, vp(out), n)


def binary_i32(op, a, a_len, b, b_len, out, n):
    call("silgpu_binary_i32", op, vp(a), a_len, vp(b), b_len, vp(out), n)


def binary_strided_f32(op, shape, a, sa, b, sb, out):
    nd = len(shape)
    arr = _i64 * max(nd, 1)
    call("silgpu_binary_strided_f32", op, nd, arr(*shape), vp(a), arr(*sa), vp(b), arr(*sb),
         vp(out))


def unary_f32(op, x, out, n):
    call("silgpu_unary_f32", op, vp(x), vp(out), n)


def sigmoid_backward_f32(dout, x, out, n):
    call("silgpu_sigmoid_backward_f32", vp(dout), vp(x), vp(out), n)


def bias_sigmoid_f32(data, bias, n, cols):
    call("silgpu_bias_sigmoid_f32", vp(data), vp(bias), n, cols)


def affine_f32(x, out, n, scale, offset):
    call("silgpu_affine_f32", vp(x), vp(out), n, _f(scale), _f(offset))


def sum_f32(x, n, out):
    call("silgpu_sum_f32", vp(x), n, vp(out))


def min_f32(x, n, out):
    call("silgpu_min_f32", vp(x), n, vp(out))


def max_f32(x, n, out):
    call("silgpu_max_f32", vp(x), n, vp(out))


def sum_axis_f32(x, outer, axis_len, inner, out):
    call("silgpu_sum_axis_f32", vp(x), outer, axis_len, inner, vp(out))


def argmax_rows_f32(x, rows, cols, out):
    call("silgpu_argmax_rows_f32", vp(x), rows, cols, vp(out))


def softmax_rows_f32(x, out, rows, cols):
    call("silgpu_softmax_rows_f32", vp(x), vp(out), rows, cols)


def layer_norm_rows_f32(x, out, gamma, beta, rows, cols, eps):
    call("silgpu_layer_norm_rows_f32", vp(x), vp(out), vp(gamma), vp(beta), rows, cols,
         _f(eps))


def sgemm(ta, tb, M, N, K, A, lda, sA, B, ldb, sB, Cm, ldc, sC, batch=1, bias=None,
          bias_len=0, epi=EPI_NONE):
    call("silgpu_sgemm", int(ta), int(tb), M, N, K, vp(A), lda, sA, vp(B), ldb, sB, vp(Cm),
         ldc, sC, batch, vp(bias) if bias is not None else _vp(None), bias_len, epi)


TILE_128x128, TILE_64x64, TILE_32x128, TILE_128x64, TILE_256x256 = 1, 2, 3, 4, 5
TILE_64x64_K2, TILE_64x64_K4 = 9, 10


def sgemm_tuned(ta, tb, M, N, K, A, lda, sA, B, ldb, sB, Cm, ldc, sC, batch=1, bias=None,
                bias_len=0, epi=EPI_NONE, tile=TILE_128x128, splits=1):
    call("silgpu_sgemm_tuned", int(ta), int(tb), M, N, K, vp(A), lda, sA, vp(B), ldb, sB,
         vp(Cm), ldc, sC, batch, vp(bias) if bias is not None else _vp(None), bias_len, epi,
         tile, splits)


def gemm(ta, tb, M, N, K, A, lda, B, ldb, Cm, ldc, batch_outer=1, batch_inner=1,
         strides_a=(0, 0), strides_b=(0, 0), strides_c=(0, 0), epi=EPI_NONE, scale=None,
         bias=None, bias_len=0, residual=None, ldr=0, noalloc=False):
    """silgpu_gemm (silgpu_gemm_noalloc with noalloc=True); strides_x =
    (outer, inner); scale = (scale, offset) or None."""
    d = GemmDesc()
    d.trans_a, d.trans_b, d.M, d.N, d.K = int(ta), int(tb), M, N, K
    d.A, d.lda, d.B, d.ldb, d.C, d.ldc = vp(A).value, lda, vp(B).value, ldb, vp(Cm).value, ldc
    d.batch_outer, d.batch_inner = batch_outer, batch_inner
    d.stride_a_outer, d.stride_a_inner = strides_a
    d.stride_b_outer, d.stride_b_inner = strides_b
    d.stride_c_outer, d.stride_c_inner = strides_c
    d.epilogue = epi
    if scale is not None:
        d.use_scale, d.scale, d.scale_offset = 1, scale[0], scale[1]
    d.bias = vp(bias).value if bias is not None else None
    d.bias_len = bias_len
    d.residual = vp(residual).value if residual is not None else None
    d.ldr = ldr
    call("silgpu_gemm_noalloc" if noalloc else "silgpu_gemm", C.byref(d))


def last_plan() -> list[tuple[int, int, int]]:
    """(tile, K splits, rows of C) of each product the last GEMM call on this
    thread launched (silgpu_gemm_last_plan)."""
    n = _i()
    tiles, splits, rows = (_i * 2)(), (_i * 2)(), (_i * 2)()
    call("silgpu_gemm_last_plan", C.byref(n), tiles, splits, rows)
    return [(tiles[i], splits[i], rows[i]) for i in range(n.value)]


def attention(Sq, Sk, D, scale, Q, ldq, K, ldk, V, ldv, O, ldo, batch_outer=1, batch_inner=1,
              strides_q=(0, 0), strides_k=(0, 0), strides_v=(0, 0), strides_o=(0, 0),
              offsets=(0, 0, 0, 0)):
    """silgpu_attention_f32; strides_x = (outer, inner) in elements; offsets
    = element offsets of Q, K, V, O into their buffers."""
    d = AttnDesc()
    d.Sq, d.Sk, d.D, d.scale = Sq, Sk, D, scale
    d.batch_outer, d.batch_inner = batch_outer, batch_inner
    for name, buf, ld, st, off in (("Q", Q, ldq, strides_q, offsets[0]),
                                   ("K", K, ldk, strides_k, offsets[1]),
                                   ("V", V, ldv, strides_v, offsets[2]),
                                   ("O", O, ldo, strides_o, offsets[3])):
        p = vp(buf).value
        setattr(d, name, (p + 4 * off) if p is not None else None)
        setattr(d, "ld" + name.lower(), ld)
        setattr(d, f"stride_{name.lower()}_outer", st[0])
        setattr(d, f"stride_{name.lower()}_inner", st[1])
    call("silgpu_attention_f32", C.byref(d))


def conv2d(x, w, out, N, H, W, C_in, K, C_out):
    """silgpu_conv2d_f32: NHWC x, OHWI w, NHWC out; stride 1, padding K // 2."""
    call("silgpu_conv2d_f32", vp(x), vp(w), vp(out), N, H, W, C_in, K, C_out)


def sgemv(x, B, ldb, y, N, K):
    call("silgpu_sgemv", vp(x), vp(B), ldb, vp(y), N, K)


def program_f32(prog: Program, out):
    call("silgpu_program_f32", C.byref(prog), vp(out))


def make_program(shape, inputs, instrs, out_reg=0) -> Program:
    """inputs: list of (DeviceBuffer|int, strides); instrs: list of
    (op, dst, a, b, imm, imm2) tuples."""
    p = Program()
    p.ndim = len(shape)
    for d, s in enumerate(shape):
        p.shape[d] = s
    p.n_inputs = len(inputs)
    for i, (buf, strides) in enumerate(inputs):
        p.inputs[i].ptr = buf.ptr if isinstance(buf, DeviceBuffer) else buf
        for d, s in enumerate(strides):
            p.inputs[i].strides[d] = s
    p.n_instrs = len(instrs)
    for k, ins in enumerate(instrs):
        op, dst, a, b, imm, imm2 = tuple(ins) + (0, 0, 0, 0.0, 0.0)[len(ins) - 1:] \
            if len(ins) < 6 else tuple(ins)
        p.instrs[k].op, p.instrs[k].dst, p.instrs[k].a, p.instrs[k].b = op, dst, a, b
        p.instrs[k].imm, p.instrs[k].imm2 = imm, imm2
    p.out_reg = out_reg
    return p
