"""ctypes binding of librdlquant.so (include/rdl_quant.h).

The host-pointer functions mirror the rustml_quant facade
(rustml/quant/main/src/saf/mod.rs:1-4): same names, same argument meaning,
and a QuantError raised where the reference returns Err(QuantError::...)
(rustml/quant/main/src/api/error.rs:1-18).  The device functions take raw
device pointers (ints), e.g. torch.Tensor.data_ptr(), and a hipStream_t as int.

The library is required: importing this module raises ImportError when
librdlquant.so has not been built.  There is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "librdlquant.so")
HEADER_PATH = os.path.join(os.path.dirname(PKG_DIR), "include", "rdl_quant.h")

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"{LIB_PATH} is missing: build it with `make -C rust-deeplearning_amd` "
        "or __graft_entry__.build()"
    )

def _preload_hip_runtime():
    """Make librdlquant bind to the HIP runtime torch uses, if torch is installed.

    torch ships its own libamdhip64.so (SONAME libamdhip64.so.7).  Loading it by
    path first makes the library's libamdhip64.so.7 dependency resolve to that
    same object, whether torch is imported before or after this module, so a
    process never holds two HIP runtimes (which cannot share the device).
    """
    import importlib.util

    spec = importlib.util.find_spec("torch")
    if spec is None or spec.origin is None:
        return None
    path = os.path.join(os.path.dirname(spec.origin), "lib", "libamdhip64.so")
    if os.path.exists(path):
        return C.CDLL(path, mode=C.RTLD_GLOBAL)
    return None


_hip_runtime = _preload_hip_runtime()
lib = C.CDLL(LIB_PATH)

# ---- constants (include/rdl_quant.h) --------------------------------------
OK = 0
ERR_DTYPE_MISMATCH = 1
ERR_SHAPE_MISMATCH = 2
ERR_BLOCK_ALIGNMENT = 3
ERR_INVALID_DATA = 4
ERR_NULL_POINTER = 5
ERR_HIP = 6
ERR_NO_DEVICE = 7
ERR_UNSUPPORTED = 8

DTYPE_Q4_0 = 2
DTYPE_Q4_1 = 3
DTYPE_Q8_0 = 8
DTYPE_Q4_K = 12
DTYPE_Q6_K = 14

MODE_FLOAT = 0
MODE_NATIVE = 1

BLOCK = {DTYPE_Q4_0: (32, 18), DTYPE_Q4_1: (32, 20), DTYPE_Q8_0: (32, 34), DTYPE_Q4_K: (256, 144),
         DTYPE_Q6_K: (256, 210)}

_sz = C.c_size_t
_p = C.c_void_p
_i32 = C.c_int32
_fp = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)
_i32p = C.POINTER(C.c_int32)


def _decl(name, restype, *argtypes):
    f = getattr(lib, name)
    f.restype = restype
    f.argtypes = list(argtypes)
    return f


_decl("rdl_status_string", C.c_char_p, _i32)
_decl("rdl_last_error", C.c_char_p)
SHAPE_MAX_DIMS = 4  # RDL_SHAPE_MAX_DIMS
_decl("rdl_last_shape_mismatch", _i32, C.POINTER(_sz), C.POINTER(_sz), C.POINTER(_sz), C.POINTER(_sz))
_decl("rdl_version", C.c_char_p)
_decl("rdl_device_count", _i32)
_decl("rdl_time_next_launch", _i32, _p, _p)
COMBINE_AUTO, COMBINE_COHERENT = 0, 1
_decl("rdl_set_gemm_combine", _i32, _i32)
_decl("rdl_get_gemm_combine", _i32, C.POINTER(_i32), C.POINTER(_i32))
for _n in ("q8", "q4", "q4_native", "q4_1", "q4_1_native", "q4_k", "q6_k"):
    _decl(f"rdl_matmul_f32_{_n}", _i32, _fp, _sz, _u8p, _sz, _sz, _sz, _sz, _fp, _sz)
_decl("rdl_quantize_row_q8_0", _i32, _fp, _sz, _u8p, _sz, _fp, _sz)
_decl("rdl_q4_0_q8_0_block_dots", _i32, _fp, _sz, _u8p, _sz, _sz, _sz, _sz, _i32p, _sz)
_decl("rdl_weight_upload", _i32, _u8p, _sz, _i32, _sz, _sz, C.POINTER(_p))
_decl("rdl_weight_wrap_device", _i32, _p, _sz, _i32, _sz, _sz, C.POINTER(_p))
_decl("rdl_weight_free", _i32, _p)
_decl("rdl_linear_forward_dev", _i32, _p, _p, _sz, _p, _i32, _p)
_decl("rdl_linear_forward_dev_noalloc", _i32, _p, _p, _sz, _p, _i32, _p)
_decl("rdl_release_stream_work", _i32, _p)
_decl("rdl_linear_forward_bias_dev", _i32, _p, _p, _sz, _p, _p, _i32, _p)
NOALLOC_SCRATCH_BYTES = 16 << 20  # RDL_NOALLOC_SCRATCH_BYTES
_decl("rdl_activation_record_bytes", _sz, _sz, _sz, _i32)
_decl("rdl_prepare_activations_dev", _i32, _p, _sz, _sz, _i32, _p, _p)
_decl("rdl_linear_prepared_dev", _i32, _p, _p, _sz, _p, _i32, _p)
_decl("rdl_quantize_row_q8_0_dev", _i32, _p, _sz, _p, _p, _p)
_decl("rdl_dequantize_rows_dev", _i32, _p, _p, _sz, _p, _p)
_decl("rdl_q4_0_q8_0_block_dots_dev", _i32, _p, _p, _p, _p)
_decl("rdl_linear_fused_dev", _i32, _p, _p, _sz, _sz, _p, _i32, _p, C.c_float, _i32, _p)
_decl("rdl_stream_read_dev", _i32, _p, _sz, _p, _sz, _p)

PROLOGUE_NONE, PROLOGUE_RMSNORM, PROLOGUE_SWIGLU = 0, 1, 2
EPILOGUE_STORE, EPILOGUE_RESIDUAL, EPILOGUE_SWIGLU = 0, 1, 2


# ---- errors (QuantError, rustml/quant/main/src/api/error.rs:1-18) ---------
class QuantError(Exception):
    def __init__(self, status: int, message: str):
        self.status = status
        super().__init__(f"{lib.rdl_status_string(status).decode()}: {message}")


class DTypeMismatch(QuantError):
    pass


class ShapeMismatch(QuantError):
    """QuantError::ShapeMismatch { expected, actual } (error.rs:9-10): the two
    extents come across the ABI through rdl_last_shape_mismatch."""

    def __init__(self, status: int, message: str, expected=(), actual=()):
        super().__init__(status, message)
        self.expected = list(expected)
        self.actual = list(actual)


class BlockAlignment(QuantError):
    pass


class InvalidData(QuantError):
    pass


class DeviceError(QuantError):
    """HIP runtime failure, missing gfx950 device or an unsupported shape."""


_ERRORS = {
    ERR_DTYPE_MISMATCH: DTypeMismatch,
    ERR_SHAPE_MISMATCH: ShapeMismatch,
    ERR_BLOCK_ALIGNMENT: BlockAlignment,
    ERR_INVALID_DATA: InvalidData,
}


def last_shape_mismatch():
    """(expected, actual) extents of this thread's last RDL_ERR_SHAPE_MISMATCH, or None."""
    e, a = (_sz * SHAPE_MAX_DIMS)(), (_sz * SHAPE_MAX_DIMS)()
    ne, na = _sz(), _sz()
    if lib.rdl_last_shape_mismatch(e, C.byref(ne), a, C.byref(na)) != OK:
        return None
    return [int(v) for v in e[:ne.value]], [int(v) for v in a[:na.value]]


def check(status: int) -> None:
    if status != OK:
        msg = lib.rdl_last_error().decode()
        if status == ERR_SHAPE_MISMATCH:
            detail = last_shape_mismatch()
            raise ShapeMismatch(status, msg, *(detail or ((), ())))
        raise _ERRORS.get(status, DeviceError)(status, msg)


def set_gemm_combine(mode: int) -> None:
    """K-slice combine of the 5-64-row GEMMs: COMBINE_AUTO (XCD-local where
    the probed placement holds) or COMBINE_COHERENT (testing switch)."""
    check(lib.rdl_set_gemm_combine(mode))


def gemm_combine():
    """(mode, local): the switch, and whether the current device's next split
    GEMM takes the XCD-local combine."""
    mode, local = _i32(), _i32()
    check(lib.rdl_get_gemm_combine(C.byref(mode), C.byref(local)))
    return int(mode.value), bool(local.value)


def release_stream_work(stream) -> None:
    """rdl_release_stream_work: free the work memory kept for `stream` (a
    hipStream_t handle) on the current device, after waiting for it."""
    check(lib.rdl_release_stream_work(stream))


def device_count() -> int:
    return int(lib.rdl_device_count())


def version() -> str:
    return lib.rdl_version().decode()


def time_next_launch(start_event, stop_event):
    """Kernel-boundary timing of this thread's next product-kernel launch
    (hipEvent_t handles, e.g. torch.cuda.Event(enable_timing=True).cuda_event)."""
    check(lib.rdl_time_next_launch(start_event, stop_event))


def stream_read_dev(buf_ptr: int, nbytes: int, out_ptr: int, out_len: int, stream) -> None:
    """One plain streaming read of nbytes at buf_ptr (measurement aid): each
    of the 2 x CUs workgroups XOR-folds its share into out[workgroup]."""
    check(lib.rdl_stream_read_dev(buf_ptr, nbytes, out_ptr, out_len, stream))


# ---- host drop-ins (rustml_quant) -----------------------------------------
def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(_fp), a.size


def _u8(a):
    a = np.ascontiguousarray(a, dtype=np.uint8)
    return a, a.ctypes.data_as(_u8p), a.size


def _matmul(fn, input_data, weight_bytes, m, in_features, out_features):
    x, xp, xn = _f32(input_data)
    w, wp, wn = _u8(weight_bytes)
    y = np.zeros(m * out_features, dtype=np.float32)
    check(fn(xp, xn, wp, wn, m, in_features, out_features, y.ctypes.data_as(_fp), y.size))
    return y


def matmul_f32_q8(input_data, weight_bytes, m, in_features, out_features):
    """quantize.rs:201-260 (returns the flattened [m, out_features] output)."""
    return _matmul(lib.rdl_matmul_f32_q8, input_data, weight_bytes, m, in_features, out_features)


def matmul_f32_q4(input_data, weight_bytes, m, in_features, out_features):
    """quantize.rs:265-320."""
    return _matmul(lib.rdl_matmul_f32_q4, input_data, weight_bytes, m, in_features, out_features)


def matmul_f32_q4_native(input_data, weight_bytes, m, in_features, out_features):
    """quantize.rs:326-394."""
    return _matmul(
        lib.rdl_matmul_f32_q4_native, input_data, weight_bytes, m, in_features, out_features
    )


def matmul_f32_q4_1(input_data, weight_bytes, m, in_features, out_features):
    """quantize.rs:429-495."""
    return _matmul(lib.rdl_matmul_f32_q4_1, input_data, weight_bytes, m, in_features, out_features)


def matmul_f32_q4_1_native(input_data, weight_bytes, m, in_features, out_features):
    """quantize.rs:501-572."""
    return _matmul(
        lib.rdl_matmul_f32_q4_1_native, input_data, weight_bytes, m, in_features, out_features
    )


def matmul_f32_q4_k(input_data, weight_bytes, m, in_features, out_features):
    """Extension: the reference's dequantize_q4k + F32 Linear, from resident super-blocks."""
    return _matmul(lib.rdl_matmul_f32_q4_k, input_data, weight_bytes, m, in_features, out_features)


def matmul_f32_q6_k(input_data, weight_bytes, m, in_features, out_features):
    """Q6_K product straight from the 210-byte super-blocks (the reference
    dequantizes them at load, rustml/gguf/main/src/core/parser.rs:510-547,
    and runs the F32 Linear)."""
    return _matmul(lib.rdl_matmul_f32_q6_k, input_data, weight_bytes, m, in_features, out_features)


def quantize_row_q8_0(input_data):
    """quantize.rs:164-193; returns (q8 block bytes, f32 scales)."""
    x, xp, xn = _f32(input_data)
    nb = xn // 32
    out = np.zeros(nb * 34, dtype=np.uint8)
    sc = np.zeros(nb, dtype=np.float32)
    check(
        lib.rdl_quantize_row_q8_0(xp, xn, out.ctypes.data_as(_u8p), out.size, sc.ctypes.data_as(_fp), sc.size)
    )
    return out, sc


def q4_0_q8_0_block_dots(input_data, weight_bytes, m, in_features, out_features):
    """int32 block partials of matmul_f32_q4_native, shape [m, out_features, in_features/32]."""
    x, xp, xn = _f32(input_data)
    w, wp, wn = _u8(weight_bytes)
    nb = in_features // 32
    part = np.zeros(m * out_features * nb, dtype=np.int32)
    check(
        lib.rdl_q4_0_q8_0_block_dots(
            xp, xn, wp, wn, m, in_features, out_features, part.ctypes.data_as(_i32p), part.size
        )
    )
    return part.reshape(m, out_features, nb)


# ---- device-resident weights ----------------------------------------------
class Weight:
    """A GGUF-layout weight matrix [out_features, in_features] resident in HBM."""

    def __init__(self, handle, dtype, out_features, in_features, keepalive=None):
        self.handle = handle
        self.dtype = dtype
        self.out_features = out_features
        self.in_features = in_features
        self._keepalive = keepalive

    @classmethod
    def upload(cls, weight_bytes, dtype, out_features, in_features):
        w, wp, wn = _u8(weight_bytes)
        h = _p()
        check(lib.rdl_weight_upload(wp, wn, dtype, out_features, in_features, C.byref(h)))
        return cls(h, dtype, out_features, in_features)

    @classmethod
    def wrap_device(cls, dev_ptr, nbytes, dtype, out_features, in_features, keepalive=None):
        h = _p()
        check(lib.rdl_weight_wrap_device(dev_ptr, nbytes, dtype, out_features, in_features, C.byref(h)))
        return cls(h, dtype, out_features, in_features, keepalive)

    def free(self):
        if self.handle:
            check(lib.rdl_weight_free(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def forward_fused_dev(self, x_ptr, x_stride, m, y_ptr, prologue=0, gamma_ptr=0, eps=0.0, epilogue=0,
                          stream=0):
        """rdl_linear_fused_dev: Q4_0, m <= 4; RMSNorm / SwiGLU prologue; store / residual /
        SwiGLU-pair epilogue."""
        check(lib.rdl_linear_fused_dev(self.handle, x_ptr, x_stride, m, y_ptr, prologue, gamma_ptr or None, eps,
                                       int(epilogue), stream))

    def forward_dev(self, x_ptr, m, y_ptr, mode=MODE_FLOAT, stream=0):
        check(lib.rdl_linear_forward_dev(self.handle, x_ptr, m, y_ptr, mode, stream))

    def forward_bias_dev(self, x_ptr, m, bias_ptr, y_ptr, mode=MODE_FLOAT, stream=0):
        """rdl_linear_forward_bias_dev: forward_dev plus Linear's optional
        bias (bias_ptr: out_features device floats, or 0 for none)."""
        check(lib.rdl_linear_forward_bias_dev(self.handle, x_ptr, m, bias_ptr or None, y_ptr, mode, stream))

    def forward_dev_noalloc(self, x_ptr, m, y_ptr, mode=MODE_FLOAT, stream=0):
        """rdl_linear_forward_dev_noalloc: the same product with no device
        allocation (a static per-GPU scratch array; overlapping calls race)."""
        check(lib.rdl_linear_forward_dev_noalloc(self.handle, x_ptr, m, y_ptr, mode, stream))

    def forward_prepared_dev(self, rec_ptr, m, y_ptr, mode=MODE_FLOAT, stream=0):
        check(lib.rdl_linear_prepared_dev(self.handle, rec_ptr, m, y_ptr, mode, stream))

    def dequantize_rows_dev(self, rows_ptr, n_rows, out_ptr, stream=0):
        check(lib.rdl_dequantize_rows_dev(self.handle, rows_ptr, n_rows, out_ptr, stream))

    def block_dots_dev(self, x_ptr, part_ptr, stream=0):
        check(lib.rdl_q4_0_q8_0_block_dots_dev(self.handle, x_ptr, part_ptr, stream))


def activation_record_bytes(m, k, mode=MODE_FLOAT):
    return int(lib.rdl_activation_record_bytes(m, k, mode))


def prepare_activations_dev(x_ptr, m, k, mode, rec_ptr, stream=0):
    check(lib.rdl_prepare_activations_dev(x_ptr, m, k, mode, rec_ptr, stream))


def quantize_row_q8_0_dev(x_ptr, n, out_ptr, scales_ptr, stream=0):
    check(lib.rdl_quantize_row_q8_0_dev(x_ptr, n, out_ptr, scales_ptr, stream))


def declared_symbols():
    """Every function name the headers in include/ declare."""
    import glob

    names = set()
    for path in sorted(glob.glob(os.path.join(os.path.dirname(HEADER_PATH), "*.h"))):
        text = re.sub(r"/\*.*?\*/", "", open(path).read(), flags=re.S)
        names.update(re.findall(r"\b(rdl_[a-z0-9_]+)\s*\(", text))
    return sorted(names)
