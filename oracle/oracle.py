"""ctypes binding of the CPU restatement (oracle/build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker / CPU baseline.  The product
library never loads it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "liboracle.so")


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


if not os.path.exists(LIB_PATH):
    build()
lib = C.CDLL(LIB_PATH)

_sz, _i, _f = C.c_size_t, C.c_int, C.c_float
_fp = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)
_i8p = C.POINTER(C.c_int8)
_i32p = C.POINTER(C.c_int32)


def _decl(name, restype, *args):
    fn = getattr(lib, name)
    fn.restype = restype
    fn.argtypes = list(args)


_decl("orc_f16_to_f32", _f, C.c_uint16)
_decl("orc_f32_to_f16", C.c_uint16, _f)
_decl("orc_dot_q8_block_scalar", _f, _fp, _i8p, _f)
_decl("orc_dot_q4_block_scalar", _f, _fp, _u8p, _f)
_decl("orc_dot_q8_block", _f, _fp, _i8p, _f)
_decl("orc_dot_q4_block", _f, _fp, _u8p, _f)
_decl("orc_dot_q8_block_lanes", _f, _fp, _i8p, _f)
_decl("orc_dot_q4_block_lanes", _f, _fp, _u8p, _f)
_decl("orc_dot_q4q8_block", C.c_int32, _u8p, _i8p)
_decl("orc_dot_q4_1_q8_block", None, _u8p, _i8p, _i32p, _i32p)
_decl("orc_quantize_row_q8_0", None, _fp, _sz, _u8p, _fp)
for _n in ("q8", "q4", "q4_native", "q4_1", "q4_1_native", "q4_cols", "q4k", "q6k"):
    _decl(f"orc_matmul_f32_{_n}", _i, _fp, _u8p, _sz, _sz, _sz, _sz, _fp, _i)
_decl("orc_matmul_f32_f32", _i, _fp, _fp, _sz, _sz, _sz, _fp, _i)
_decl("orc_q4_0_q8_0_block_dots", _i, _fp, _u8p, _sz, _sz, _sz, _sz, _i32p)
for _n in ("q4_0", "q4_1", "q8_0"):
    _decl(f"orc_to_f32_{_n}", _i, _u8p, _sz, _sz, _fp)
_decl("orc_dequantize_q4k", _i, _u8p, _sz, _sz, _fp)
_decl("orc_dequantize_q6k", _i, _u8p, _sz, _sz, _fp)
for _n in ("q4_1_legacy", "q5_0", "q5_1", "q8_1", "q5k", "q8k", "q3k", "q2k"):
    _decl(f"orc_dequantize_{_n}", _i, _u8p, _sz, _sz, _fp)
_decl("orc_rope_tables", None, _i, _i, _f, _fp, _fp)
_decl("orc_rms_norm_row", None, _fp, _fp, _sz, _f, _fp)


class OracleError(Exception):
    def __init__(self, code):
        self.code = code
        super().__init__(f"oracle status {code}")


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(_fp)


def _u8(a):
    a = np.ascontiguousarray(a, dtype=np.uint8)
    return a, a.ctypes.data_as(_u8p)


def _i8(a):
    a = np.ascontiguousarray(a, dtype=np.int8)
    return a, a.ctypes.data_as(_i8p)


def f16_to_f32(bits: int) -> float:
    return float(lib.orc_f16_to_f32(int(bits)))


def f32_to_f16(v: float) -> int:
    return int(lib.orc_f32_to_f16(float(v)))


def dot_q8_block(x, q, scale, variant=""):
    x, xp = _f32(x)
    q, qp = _i8(q)
    return float(getattr(lib, f"orc_dot_q8_block{variant}")(xp, qp, scale))


def dot_q4_block(x, packed, scale, variant=""):
    x, xp = _f32(x)
    p, pp = _u8(packed)
    return float(getattr(lib, f"orc_dot_q4_block{variant}")(xp, pp, scale))


def dot_q4q8_block(packed, q8) -> int:
    p, pp = _u8(packed)
    q, qp = _i8(q8)
    return int(lib.orc_dot_q4q8_block(pp, qp))


def dot_q4_1_q8_block(packed, q8):
    p, pp = _u8(packed)
    q, qp = _i8(q8)
    d, s = C.c_int32(), C.c_int32()
    lib.orc_dot_q4_1_q8_block(pp, qp, C.byref(d), C.byref(s))
    return d.value, s.value


def quantize_row_q8_0(x):
    x, xp = _f32(x)
    nb = x.size // 32
    out = np.zeros(nb * 34, dtype=np.uint8)
    sc = np.zeros(nb, dtype=np.float32)
    lib.orc_quantize_row_q8_0(xp, x.size, out.ctypes.data_as(_u8p), sc.ctypes.data_as(_fp))
    return out, sc


def matmul(kind, x, w, m, k, n, threads=1):
    """kind in q8, q4, q4_native, q4_1, q4_1_native, q4_cols, q4k, q6k."""
    x, xp = _f32(x)
    w, wp = _u8(w)
    y = np.zeros(m * n, dtype=np.float32)
    rc = getattr(lib, f"orc_matmul_f32_{kind}")(xp, wp, w.size, m, k, n, y.ctypes.data_as(_fp), threads)
    if rc:
        raise OracleError(rc)
    return y


def matmul_f32_f32(x, w, m, k, n, threads=1):
    x, xp = _f32(x)
    w, wp = _f32(w)
    y = np.zeros(m * n, dtype=np.float32)
    lib.orc_matmul_f32_f32(xp, wp, m, k, n, y.ctypes.data_as(_fp), threads)
    return y


def block_dots(x, w, m, k, n):
    x, xp = _f32(x)
    w, wp = _u8(w)
    part = np.zeros(m * n * (k // 32), dtype=np.int32)
    rc = lib.orc_q4_0_q8_0_block_dots(xp, wp, w.size, m, k, n, part.ctypes.data_as(_i32p))
    if rc:
        raise OracleError(rc)
    return part.reshape(m, n, k // 32)


def to_f32(kind, w, n_elements):
    w, wp = _u8(w)
    out = np.zeros(n_elements, dtype=np.float32)
    fn = {"q4_0": lib.orc_to_f32_q4_0, "q4_1": lib.orc_to_f32_q4_1, "q8_0": lib.orc_to_f32_q8_0,
          "q4k": lib.orc_dequantize_q4k, "q6k": lib.orc_dequantize_q6k,
          "q4_1_legacy": lib.orc_dequantize_q4_1_legacy, "q5_0": lib.orc_dequantize_q5_0,
          "q5_1": lib.orc_dequantize_q5_1, "q8_1": lib.orc_dequantize_q8_1, "q5k": lib.orc_dequantize_q5k,
          "q8k": lib.orc_dequantize_q8k, "q3k": lib.orc_dequantize_q3k, "q2k": lib.orc_dequantize_q2k}[kind]
    rc = fn(wp, w.size, n_elements, out.ctypes.data_as(_fp))
    if rc:
        raise OracleError(rc)
    return out


def rope_tables(head_dim, max_seq, theta):
    half = head_dim // 2
    c = np.zeros(max_seq * half, np.float32)
    s = np.zeros(max_seq * half, np.float32)
    lib.orc_rope_tables(head_dim, max_seq, theta, c.ctypes.data_as(_fp), s.ctypes.data_as(_fp))
    return c.reshape(max_seq, half), s.reshape(max_seq, half)


def rms_norm(x, gamma, eps):
    """Tensor::rms_norm over the last axis of x (rows restated one at a time)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    g, gp = _f32(gamma)
    rows = x.reshape(-1, x.shape[-1])
    out = np.zeros_like(rows)
    for r in range(rows.shape[0]):
        row = np.ascontiguousarray(rows[r])
        o = np.zeros(row.size, np.float32)
        lib.orc_rms_norm_row(row.ctypes.data_as(_fp), gp, row.size, eps, o.ctypes.data_as(_fp))
        out[r] = o
    return out.reshape(x.shape)
