"""ctypes binding of the GGUF reader in librdlquant.so (include/rdl_gguf.h).

GGUFFile mirrors rustml's GGUFFile (rustml/gguf/main/src/core/parser.rs):
parse_header(path) / parse_bytes(data), version, metadata, tensor_infos,
data_offset, to_model_config() and load_tensors(), with GgufError subclasses
raised where the reference returns Err(GgufError::...)
(rustml/gguf/main/src/api/error.rs:5-21).  The parsing is native: the file is
memory-mapped by the library, tensor data are zero-copy views of the mapping
(tensor_data) or go straight to device memory (upload_tensor).
"""
from __future__ import annotations

import ctypes as C
import struct
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import _ERRORS, QuantError, _decl, _i32, _p, _sz, check, lib
from .gguf_writer import (ARRAY, BOOL, F32, F64, GGML_BLOCK, I8, I16, I32, I64, STRING, U8, U16, U32,
                          U64)

ERR_GGUF_IO = 9
ERR_GGUF_INVALID_FORMAT = 10
ERR_GGUF_UNSUPPORTED_TYPE = 11
ERR_GGUF_MISSING_METADATA = 12
ERR_NOT_FOUND = 13


class GgufError(QuantError):
    pass


class GgufIoError(GgufError):
    """GgufError::Io: file errors, unexpected end of file, invalid UTF-8."""


class InvalidFormat(GgufError):
    pass


class UnsupportedType(GgufError):
    pass


class MissingMetadata(GgufError):
    pass


class NotFound(GgufError, KeyError):
    pass


_ERRORS.update({ERR_GGUF_IO: GgufIoError, ERR_GGUF_INVALID_FORMAT: InvalidFormat,
                ERR_GGUF_UNSUPPORTED_TYPE: UnsupportedType, ERR_GGUF_MISSING_METADATA: MissingMetadata,
                ERR_NOT_FOUND: NotFound})

GGML_TYPE_NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0", 9: "Q8_1",
                   10: "Q2K", 11: "Q3K", 12: "Q4K", 13: "Q5K", 14: "Q6K", 15: "Q8K"}


class _Value(C.Structure):
    _fields_ = [("type", C.c_int32), ("elem_type", C.c_int32), ("count", C.c_uint64), ("raw", C.c_void_p),
                ("raw_len", C.c_uint64)]


class _TensorInfo(C.Structure):
    _fields_ = [("name", C.c_void_p), ("name_len", C.c_uint64), ("n_dims", C.c_uint32),
                ("dims", C.POINTER(C.c_uint64)),
                ("ggml_type", C.c_int32), ("offset", C.c_uint64), ("n_bytes", C.c_uint64)]


class _ModelConfig(C.Structure):
    _fields_ = [("architecture", C.c_char * 64)] + \
               [(n, C.c_uint32) for n in ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads",
                                          "vocab_size")] + \
               [("norm_eps", C.c_float), ("max_seq_len", C.c_uint32), ("rope_theta", C.c_float),
                ("bos_token_id", C.c_int64), ("eos_token_id", C.c_int64), ("head_dim", C.c_uint32),
                ("sliding_window", C.c_uint32)] + \
               [(n, C.c_int32) for n in ("has_n_kv_heads", "has_head_dim", "has_sliding_window",
                                         "has_chat_template")]


_PV = C.POINTER(_Value)
_decl("rdl_gguf_open", _i32, C.c_char_p, C.POINTER(_p))
_decl("rdl_gguf_open_bytes", _i32, _p, _sz, C.POINTER(_p))
_decl("rdl_gguf_close", _i32, _p)
_decl("rdl_gguf_version", _i32, _p, C.POINTER(C.c_uint32))
_decl("rdl_gguf_data_offset", _i32, _p, C.POINTER(C.c_uint64))
_decl("rdl_gguf_file_size", _i32, _p, C.POINTER(C.c_uint64))
_decl("rdl_gguf_tensor_count", _i32, _p, C.POINTER(_sz))
_decl("rdl_gguf_metadata_count", _i32, _p, C.POINTER(_sz))
_decl("rdl_gguf_metadata_at", _i32, _p, _sz, C.POINTER(C.c_void_p), C.POINTER(_sz), _PV)
_decl("rdl_gguf_metadata_find", _i32, _p, C.c_char_p, _PV)
_decl("rdl_gguf_array_element", _i32, _p, _PV, C.c_uint64, _PV)
_decl("rdl_gguf_get_u32", _i32, _p, C.c_char_p, C.POINTER(C.c_uint32))
_decl("rdl_gguf_get_f32", _i32, _p, C.c_char_p, C.POINTER(C.c_float))
_decl("rdl_gguf_get_string", _i32, _p, C.c_char_p, C.POINTER(C.c_void_p), C.POINTER(_sz))
_decl("rdl_gguf_tensor_info_at", _i32, _p, _sz, C.POINTER(_TensorInfo))
_decl("rdl_gguf_find_tensor", _i32, _p, C.c_char_p, C.POINTER(_sz))
_decl("rdl_gguf_tensor_data", _i32, _p, _sz, C.POINTER(C.c_void_p), C.POINTER(C.c_uint64))
_decl("rdl_gguf_upload_tensor", _i32, _p, _sz, _p, C.c_uint64, _p)
_decl("rdl_gguf_model_config_get", _i32, _p, C.POINTER(_ModelConfig))
_decl("rdl_gguf_upload_tensor_f32", _i32, _p, _sz, _p, C.c_uint64, _p)
_decl("rdl_dequantize_gguf_dev", _i32, _i32, _p, _sz, _sz, _p, _p)

_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", U64: "<Q", I64: "<q",
        F64: "<d"}


@dataclass
class GGUFValue:
    """A metadata value (types.rs:80-95): its GGUF type id and Python value
    (int, float, bool, str, or a list of GGUFValue for arrays)."""
    type: int
    value: object

    def as_u32(self) -> Optional[int]:
        """types.rs:98-105: U32, I32 and U64 (truncating casts)."""
        if self.type in (U32, I32, U64):
            return int(self.value) & 0xFFFFFFFF
        return None

    def as_f32(self) -> Optional[float]:
        """types.rs:107-113: F32 or F64 rounded to f32."""
        if self.type in (F32, F64):
            return float(np.float32(self.value))
        return None

    def as_string(self) -> Optional[str]:
        return self.value if self.type == STRING else None


@dataclass
class GGUFTensorInfo:
    """types.rs:123-130, plus the byte size load_tensors reads."""
    name: str
    dimensions: list
    ggml_type: int
    offset: int
    n_bytes: int


@dataclass
class GgufModelConfig:
    """types.rs:165-186; optional fields are None when the file lacks them."""
    architecture: str
    dim: int
    hidden_dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: Optional[int]
    vocab_size: int
    norm_eps: float
    max_seq_len: int
    rope_theta: float
    bos_token_id: Optional[int]
    eos_token_id: Optional[int]
    chat_template: Optional[str]
    head_dim: Optional[int]
    sliding_window: Optional[int]


@dataclass
class LoadedTensor:
    """types.rs:150-155 without the copy: `data` is a read-only uint8 view of
    the mapping; shape is the reversed GGUF dims (parser.rs:317)."""
    data: np.ndarray
    shape: list
    ggml_type: int


class GGUFFile:
    def __init__(self, handle, keepalive=None):
        self._h = handle
        self._keep = keepalive
        v = C.c_uint32()
        check(lib.rdl_gguf_version(self._h, C.byref(v)))
        self.version = int(v.value)
        o = C.c_uint64()
        check(lib.rdl_gguf_data_offset(self._h, C.byref(o)))
        self.data_offset = int(o.value)
        self._metadata = None
        self._infos = None

    @classmethod
    def parse_header(cls, path) -> "GGUFFile":
        """parser.rs:143-148 (the file is mapped, not read)."""
        h = _p()
        check(lib.rdl_gguf_open(str(path).encode(), C.byref(h)))
        return cls(h)

    @classmethod
    def parse_bytes(cls, data) -> "GGUFFile":
        """parser.rs:151-211 over an in-memory buffer (kept alive by the handle)."""
        buf = np.frombuffer(bytes(data), dtype=np.uint8)
        h = _p()
        check(lib.rdl_gguf_open_bytes(buf.ctypes.data if buf.size else None, buf.size, C.byref(h)))
        return cls(h, keepalive=buf)

    def close(self):
        if getattr(self, "_h", None):
            lib.rdl_gguf_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def handle(self):
        return self._h

    @property
    def file_size(self) -> int:
        n = C.c_uint64()
        check(lib.rdl_gguf_file_size(self._h, C.byref(n)))
        return int(n.value)

    # ---- metadata ---------------------------------------------------------
    def _decode(self, v: _Value) -> GGUFValue:
        if v.type in _FMT:
            return GGUFValue(v.type, struct.unpack(_FMT[v.type], C.string_at(v.raw, v.raw_len))[0])
        if v.type == BOOL:
            return GGUFValue(BOOL, C.string_at(v.raw, 1)[0] != 0)
        if v.type == STRING:
            return GGUFValue(STRING, C.string_at(v.raw, v.raw_len).decode() if v.raw_len else "")
        elems = []
        if v.count and v.elem_type in _FMT:
            a = np.frombuffer(C.string_at(v.raw, v.raw_len), dtype=np.dtype(_FMT[v.elem_type]))
            elems = [GGUFValue(v.elem_type, x.item()) for x in a]
        else:
            e = _Value()
            for i in range(v.count):
                check(lib.rdl_gguf_array_element(self._h, C.byref(v), i, C.byref(e)))
                elems.append(self._decode(e))
        return GGUFValue(ARRAY, elems)

    @property
    def metadata(self) -> dict:
        """key -> GGUFValue (a repeated key keeps its last value)."""
        if self._metadata is None:
            n = _sz()
            check(lib.rdl_gguf_metadata_count(self._h, C.byref(n)))
            out = {}
            key, klen, v = C.c_void_p(), _sz(), _Value()
            for i in range(n.value):
                check(lib.rdl_gguf_metadata_at(self._h, i, C.byref(key), C.byref(klen), C.byref(v)))
                out[C.string_at(key, klen.value).decode()] = self._decode(v)
            self._metadata = out
        return self._metadata

    def metadata_find(self, key) -> GGUFValue:
        """The value of one key (NotFound "Key not found: <key>" if absent)."""
        v = _Value()
        check(lib.rdl_gguf_metadata_find(self._h, key.encode(), C.byref(v)))
        return self._decode(v)

    def get_u32(self, key) -> int:
        v = C.c_uint32()
        check(lib.rdl_gguf_get_u32(self._h, key.encode(), C.byref(v)))
        return int(v.value)

    def get_f32(self, key) -> float:
        v = C.c_float()
        check(lib.rdl_gguf_get_f32(self._h, key.encode(), C.byref(v)))
        return float(v.value)

    def get_string(self, key) -> str:
        p, n = C.c_void_p(), _sz()
        check(lib.rdl_gguf_get_string(self._h, key.encode(), C.byref(p), C.byref(n)))
        return C.string_at(p, n.value).decode() if n.value else ""

    # ---- tensors ------------------------------------------------------------
    @property
    def tensor_infos(self) -> list:
        if self._infos is None:
            n = _sz()
            check(lib.rdl_gguf_tensor_count(self._h, C.byref(n)))
            ti = _TensorInfo()
            out = []
            for i in range(n.value):
                check(lib.rdl_gguf_tensor_info_at(self._h, i, C.byref(ti)))
                out.append(GGUFTensorInfo(C.string_at(ti.name, ti.name_len).decode(),
                                          [int(ti.dims[d]) for d in range(ti.n_dims)],
                                          int(ti.ggml_type), int(ti.offset), int(ti.n_bytes)))
            self._infos = out
        return self._infos

    def find_tensor(self, name) -> int:
        i = _sz()
        check(lib.rdl_gguf_find_tensor(self._h, name.encode(), C.byref(i)))
        return int(i.value)

    def _index(self, tensor) -> int:
        return self.find_tensor(tensor) if isinstance(tensor, str) else int(tensor)

    def tensor_data(self, tensor) -> np.ndarray:
        """Read-only uint8 view of a tensor's bytes in the mapping (valid while
        this file is open); the bound check of load_tensors (parser.rs:306-312)."""
        p, n = C.c_void_p(), C.c_uint64()
        check(lib.rdl_gguf_tensor_data(self._h, self._index(tensor), C.byref(p), C.byref(n)))
        if n.value == 0:
            return np.empty(0, np.uint8)
        buf = (C.c_uint8 * int(n.value)).from_address(p.value)
        buf.owner = self  # the view keeps the mapping open
        a = np.frombuffer(buf, dtype=np.uint8)
        a.flags.writeable = False
        return a

    def upload_tensor(self, tensor, dst_ptr: int, dst_len: int, stream: int = 0) -> None:
        """A tensor's raw bytes into device memory at dst_ptr (synchronous)."""
        check(lib.rdl_gguf_upload_tensor(self._h, self._index(tensor), dst_ptr, dst_len, stream))

    def upload_tensor_f32(self, tensor, dst_ptr: int, dst_len: int, stream: int = 0) -> None:
        """load_tensors' F32 expansion of one tensor on the device (K-quants,
        Q4_1, Q5_*, Q8_1 as parser.rs:371-776; F16, Q4_0, Q8_0 as Tensor::to_f32)
        into dst_ptr (dst_len floats, 16-byte aligned); synchronous."""
        check(lib.rdl_gguf_upload_tensor_f32(self._h, self._index(tensor), dst_ptr, dst_len, stream))

    def load_tensors(self) -> dict:
        """name -> LoadedTensor over views of the mapping (raw GGUF bytes for
        every type; the reference's load-time dequantization of K-quants and
        Q5/Q8_1 is left to the device kernels)."""
        out = {}
        for i, ti in enumerate(self.tensor_infos):
            out[ti.name] = LoadedTensor(self.tensor_data(i), list(reversed(ti.dimensions)), ti.ggml_type)
        return out

    # ---- config ------------------------------------------------------------
    def to_model_config(self) -> GgufModelConfig:
        c = _ModelConfig()
        check(lib.rdl_gguf_model_config_get(self._h, C.byref(c)))
        chat = None
        if c.has_chat_template:
            chat = self.get_string("tokenizer.chat_template")
        return GgufModelConfig(
            architecture=c.architecture.decode(), dim=c.dim, hidden_dim=c.hidden_dim, n_layers=c.n_layers,
            n_heads=c.n_heads, n_kv_heads=c.n_kv_heads if c.has_n_kv_heads else None,
            vocab_size=c.vocab_size, norm_eps=float(c.norm_eps), max_seq_len=c.max_seq_len,
            rope_theta=float(c.rope_theta),
            bos_token_id=None if c.bos_token_id < 0 else int(c.bos_token_id),
            eos_token_id=None if c.eos_token_id < 0 else int(c.eos_token_id), chat_template=chat,
            head_dim=c.head_dim if c.has_head_dim else None,
            sliding_window=c.sliding_window if c.has_sliding_window else None)


def ggml_block(ggml_type: int):
    """(block_size, block_bytes) of a GGML type (types.rs:49-77)."""
    return GGML_BLOCK[ggml_type]


def dequantize_gguf_dev(ggml_type: int, src_ptr: int, src_len: int, n_elements: int, dst_ptr: int,
                        stream: int = 0) -> None:
    """n_elements of GGML type ggml_type (GGUF blocks at src_ptr, device) to f32
    at dst_ptr, bit-exact with the reference's load-time dequantization."""
    check(lib.rdl_dequantize_gguf_dev(ggml_type, src_ptr, src_len, n_elements, dst_ptr, stream))
