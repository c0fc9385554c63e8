"""GGUF v3 writer: synthetic model files for the loader's tests and benchmark.

GgufBuilder has the methods of the byte builder in rustml's GGUF tests
(rustml/gguf/tests/cli.rs:12-104: add_string / add_u32 / add_f32 / add_bool /
add_u32_array / add_tensor, build) and produces the same bytes for the same
calls.  On top of that it can carry tensor data (add_tensor_data): offsets are
then assigned 32-byte aligned, the data section starts at the next multiple
of 32 after the tensor infos (the alignment GGUFFile::parse_bytes assumes,
rustml/gguf/main/src/core/parser.rs:202), and `write` streams the file
tensor by tensor, so a multi-GB model never sits in memory whole.

llama_builder lays out a Llama-architecture file with the tensor names of
gguf_llama_weight_map (rustml/gguf/main/src/core/weight_map.rs:26-73) and the
metadata keys GGUFFile::to_model_config reads (parser.rs:214-289).

Pure Python + numpy; does not load librdlquant.
"""
from __future__ import annotations

import struct

import numpy as np

GGUF_MAGIC = b"GGUF"
ALIGN = 32

# metadata value type ids (parser.rs:110-130)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
           U64: "<Q", I64: "<q", F64: "<d"}

# GGML tensor type ids and (block_size, block_bytes) (rustml/gguf/main/src/api/types.rs:4-78)
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q4_1 = 0, 1, 2, 3
GGML_Q5_0, GGML_Q5_1, GGML_Q8_0, GGML_Q8_1 = 6, 7, 8, 9
GGML_Q2_K, GGML_Q3_K, GGML_Q4_K, GGML_Q5_K, GGML_Q6_K, GGML_Q8_K = 10, 11, 12, 13, 14, 15
GGML_BLOCK = {
    GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_Q4_0: (32, 18), GGML_Q4_1: (32, 20), GGML_Q5_0: (32, 22),
    GGML_Q5_1: (32, 24), GGML_Q8_0: (32, 34), GGML_Q8_1: (32, 40), GGML_Q2_K: (256, 84),
    GGML_Q3_K: (256, 110), GGML_Q4_K: (256, 144), GGML_Q5_K: (256, 176), GGML_Q6_K: (256, 210),
    GGML_Q8_K: (256, 292),
}


def tensor_nbytes(dims, ggml_type) -> int:
    """Byte size load_tensors reads for a tensor (parser.rs:298-304)."""
    n = 1
    for d in dims:
        n *= int(d)
    bs, bb = GGML_BLOCK[ggml_type]
    return (n // bs if bs > 1 else n) * bb


def _string(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def encode_value(type_id: int, value) -> bytes:
    """The bytes read_value reads for `value` of GGUF type `type_id` (without the type id).
    Arrays: value = (elem_type, [elements])."""
    if type_id in _SCALAR:
        if type_id == BOOL:
            value = 1 if value else 0
        return struct.pack(_SCALAR[type_id], value)
    if type_id == STRING:
        return _string(value)
    if type_id == ARRAY:
        et, elems = value
        out = [struct.pack("<IQ", et, len(elems))]
        if et in _SCALAR and et != BOOL:
            out.append(np.asarray(elems, dtype=np.dtype(_SCALAR[et])).tobytes())
        else:
            out.extend(encode_value(et, e) for e in elems)
        return b"".join(out)
    raise ValueError(f"unknown GGUF value type {type_id}")


class GgufBuilder:
    def __init__(self, version: int = 3):
        self.version = version
        self.metadata = []  # (key, type_id, encoded value)
        self.tensors = []   # (name, dims, ggml_type, offset)
        self._data = []     # (tensor index, nbytes, bytes-like or callable)
        self._next = 0      # next free data offset

    # ---- metadata (cli.rs:25-64) ------------------------------------------
    def add_value(self, key: str, type_id: int, value) -> "GgufBuilder":
        self.metadata.append((key, type_id, encode_value(type_id, value)))
        return self

    def add_raw(self, key, type_id: int, payload: bytes) -> "GgufBuilder":
        """A metadata entry with an arbitrary payload (for malformed-file tests)."""
        self.metadata.append((key, type_id, bytes(payload)))
        return self

    def add_string(self, key, value):
        return self.add_value(key, STRING, value)

    def add_u32(self, key, value):
        return self.add_value(key, U32, value)

    def add_i32(self, key, value):
        return self.add_value(key, I32, value)

    def add_u64(self, key, value):
        return self.add_value(key, U64, value)

    def add_f32(self, key, value):
        return self.add_value(key, F32, value)

    def add_f64(self, key, value):
        return self.add_value(key, F64, value)

    def add_bool(self, key, value):
        return self.add_value(key, BOOL, value)

    def add_u32_array(self, key, values):
        return self.add_value(key, ARRAY, (U32, list(values)))

    def add_string_array(self, key, values):
        return self.add_value(key, ARRAY, (STRING, list(values)))

    # ---- tensors (cli.rs:66-70) -------------------------------------------
    def add_tensor(self, name, dims, ggml_type, offset) -> "GgufBuilder":
        """A tensor info only, at a caller-chosen data offset (no data written)."""
        self.tensors.append((name, [int(d) for d in dims], int(ggml_type), int(offset)))
        return self

    def add_tensor_data(self, name, dims, ggml_type, data) -> "GgufBuilder":
        """A tensor info plus its bytes (bytes-like, numpy array, or a callable
        returning one, called once by build / write); offset 32-byte aligned."""
        nbytes = tensor_nbytes(dims, ggml_type)
        off = (self._next + ALIGN - 1) // ALIGN * ALIGN
        self.add_tensor(name, dims, ggml_type, off)
        self._data.append((len(self.tensors) - 1, nbytes, data))
        self._next = off + nbytes
        return self

    def header(self) -> bytes:
        """Magic, version, counts, metadata and tensor infos (cli.rs:72-103)."""
        out = [GGUF_MAGIC, struct.pack("<IQQ", self.version, len(self.tensors), len(self.metadata))]
        for key, type_id, payload in self.metadata:
            out += [_string(key), struct.pack("<I", type_id), payload]
        for name, dims, ggml_type, offset in self.tensors:
            out += [_string(name), struct.pack("<I", len(dims)), struct.pack(f"<{len(dims)}Q", *dims),
                    struct.pack("<IQ", ggml_type, offset)]
        return b"".join(out)

    def _chunks(self):
        head = self.header()
        yield head
        if not self._data:
            return
        pos = 0
        data_start = (len(head) + ALIGN - 1) // ALIGN * ALIGN
        yield b"\0" * (data_start - len(head))
        for idx, nbytes, data in self._data:
            off = self.tensors[idx][3]
            yield b"\0" * (off - pos)
            blob = data() if callable(data) else data
            mv = memoryview(np.ascontiguousarray(blob) if isinstance(blob, np.ndarray) else blob).cast("B")
            if mv.nbytes != nbytes:
                raise ValueError(f"tensor {self.tensors[idx][0]}: {mv.nbytes} bytes, dims need {nbytes}")
            yield mv
            pos = off + nbytes

    def build(self) -> bytes:
        return b"".join(bytes(c) for c in self._chunks())

    def write(self, path) -> int:
        """Writes the file; returns its size."""
        n = 0
        with open(path, "wb") as f:
            for c in self._chunks():
                f.write(c)
                n += len(c) if isinstance(c, bytes) else c.nbytes
        return n


# ---- Llama files ------------------------------------------------------------
LLAMA_MODEL_TENSORS = ("token_embd.weight", "output_norm.weight", "output.weight")
LLAMA_LAYER_TENSORS = ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm", "ffn_gate",
                       "ffn_up", "ffn_down")


def llama_tensor_shapes(cfg, types=None):
    """GGUF name -> (dims innermost first, ggml type) for a Llama model of
    `cfg` (rdlquant.llama.LlamaConfig fields), in llama.cpp's file order:
    matrices Q4_0 unless `types` ({GGUF name: GGML type}) says otherwise,
    the output matrix in cfg.output_dtype."""
    d, q, kv, f, v = cfg.dim, cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim, cfg.ffn_dim, cfg.vocab
    out = {"token_embd.weight": ([d, v], GGML_Q4_0)}
    for i in range(cfg.n_layers):
        p = f"blk.{i}."
        out[p + "attn_norm.weight"] = ([d], GGML_F32)
        out[p + "attn_q.weight"] = ([d, q], GGML_Q4_0)
        out[p + "attn_k.weight"] = ([d, kv], GGML_Q4_0)
        out[p + "attn_v.weight"] = ([d, kv], GGML_Q4_0)
        out[p + "attn_output.weight"] = ([q, d], GGML_Q4_0)
        out[p + "ffn_norm.weight"] = ([d], GGML_F32)
        out[p + "ffn_gate.weight"] = ([d, f], GGML_Q4_0)
        out[p + "ffn_up.weight"] = ([d, f], GGML_Q4_0)
        out[p + "ffn_down.weight"] = ([f, d], GGML_Q4_0)
    out["output_norm.weight"] = ([d], GGML_F32)
    out["output.weight"] = ([d, v], getattr(cfg, "output_dtype", GGML_Q4_0) or GGML_Q4_0)
    for name, t in (types or {}).items():
        out[name] = (out[name][0], t)
    return out


def llama_builder(cfg, tensor_data, arch="llama", context_length=None, extra_metadata=None,
                  skip=(), types=None):
    """A GgufBuilder of a Llama model: metadata from `cfg`, tensors in
    llama_tensor_shapes order (types: {GGUF name: GGML type}) with bytes from
    tensor_data(name) (bytes-like or a callable); names in `skip` are left
    out."""
    b = GgufBuilder()
    b.add_string("general.architecture", arch)
    b.add_string("general.name", "synthetic")
    b.add_u32(f"{arch}.embedding_length", cfg.dim)
    b.add_u32(f"{arch}.feed_forward_length", cfg.ffn_dim)
    b.add_u32(f"{arch}.block_count", cfg.n_layers)
    b.add_u32(f"{arch}.attention.head_count", cfg.n_heads)
    b.add_u32(f"{arch}.attention.head_count_kv", cfg.n_kv_heads)
    b.add_u32(f"{arch}.context_length", cfg.max_seq if context_length is None else context_length)
    b.add_f32(f"{arch}.attention.layer_norm_rms_epsilon", cfg.norm_eps)
    b.add_f32(f"{arch}.rope.freq_base", cfg.rope_theta)
    b.add_u32(f"{arch}.vocab_size", cfg.vocab)
    b.add_u32("tokenizer.ggml.bos_token_id", 1)
    b.add_u32("tokenizer.ggml.eos_token_id", 2)
    for k, (t, v) in (extra_metadata or {}).items():
        b.add_value(k, t, v)
    for name, (dims, t) in llama_tensor_shapes(cfg, types).items():
        if name not in skip:
            b.add_tensor_data(name, dims, t, tensor_data(name))
    return b
