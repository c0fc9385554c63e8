"""CPU restatement of rustml's GGUF parser, for the native reader's parity tests.

TEST INFRASTRUCTURE ONLY (imported by tests/): it checks librdlquant's
rdl_gguf_* reader and is never called by the product.

Follows, step by step, in pure Python:
  Cursor reads, read_string, read_value  rustml/gguf/main/src/core/parser.rs:14-131
  GGUFFile::parse_bytes                  rustml/gguf/main/src/core/parser.rs:151-211
  GGUFFile::to_model_config              rustml/gguf/main/src/core/parser.rs:214-289
  load_tensors' sizes and bound check    rustml/gguf/main/src/core/parser.rs:292-312
  GGMLType::from_u32 / block geometry    rustml/gguf/main/src/api/types.rs:23-77
  GGUFValue::as_u32 / as_f32 / as_string rustml/gguf/main/src/api/types.rs:97-121
  gguf_llama_weight_map                  rustml/gguf/main/src/core/weight_map.rs:26-73

Errors are raised as OracleError(kind, message) with kind one of the
GgufError variants ("Io", "InvalidFormat", "UnsupportedType",
"MissingMetadata").  Parity is pinned by the reference's own tests
(parser.rs:768-794 unit tests, the cli.rs builder fixture and its expected
values) and, beyond them, by brute force: every prefix of a file must fail
with the reference's end-of-file error, every byte position of a type id
is exercised by the randomized files of the tests.
"""
from __future__ import annotations

import struct

import numpy as np


class OracleError(Exception):
    def __init__(self, kind, message):
        self.kind = kind
        self.message = message
        super().__init__(f"{kind}: {message}")


def _eof():
    return OracleError("Io", "Unexpected end of GGUF file")


# GGMLType::from_u32 + block_size / block_bytes (types.rs:23-77)
GGML = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 9: (32, 40),
        10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 292)}


class Cursor:
    """parser.rs:14-131, one method per reference method."""

    def __init__(self, data: bytes):
        self.data = data
        self.pos = 0

    def remaining(self):
        return len(self.data) - self.pos

    def _take(self, n, fmt):
        if self.remaining() < n:
            raise _eof()
        v = struct.unpack_from(fmt, self.data, self.pos)[0]
        self.pos += n
        return v

    def read_u8(self): return self._take(1, "<B")
    def read_i8(self): return self._take(1, "<b")
    def read_u16(self): return self._take(2, "<H")
    def read_i16(self): return self._take(2, "<h")
    def read_u32(self): return self._take(4, "<I")
    def read_i32(self): return self._take(4, "<i")
    def read_u64(self): return self._take(8, "<Q")
    def read_i64(self): return self._take(8, "<q")
    def read_f32(self): return self._take(4, "<f")
    def read_f64(self): return self._take(8, "<d")

    def read_bool(self):
        return self.read_u8() != 0

    def read_string(self):
        n = self.read_u64()
        if self.remaining() < n:
            raise _eof()
        raw = self.data[self.pos:self.pos + n]
        try:
            s = raw.decode("utf-8", errors="strict")
        except UnicodeDecodeError:
            # the strict decoder rejects overlong forms, surrogates and code
            # points above U+10FFFF, as String::from_utf8 does
            raise OracleError("Io", "stream did not contain valid UTF-8")
        self.pos += n
        return s

    def read_bytes(self, n):
        if self.remaining() < n:
            raise _eof()
        b = self.data[self.pos:self.pos + n]
        self.pos += n
        return b

    def read_value(self, type_id):
        """-> (type_id, value); arrays -> (9, [(t, v), ...])."""
        r = {0: self.read_u8, 1: self.read_i8, 2: self.read_u16, 3: self.read_i16, 4: self.read_u32,
             5: self.read_i32, 6: self.read_f32, 7: self.read_bool, 8: self.read_string, 10: self.read_u64,
             11: self.read_i64, 12: self.read_f64}
        if type_id in r:
            return (type_id, r[type_id]())
        if type_id == 9:
            elem_type = self.read_u32()
            count = self.read_u64()
            return (9, [self.read_value(elem_type) for _ in range(count)])
        raise OracleError("UnsupportedType", f"Unknown GGUF value type: {type_id}")


class GGUFFile:
    def __init__(self, version, metadata, tensor_infos, data_offset):
        self.version = version
        self.metadata = metadata          # key -> (type_id, value)
        self.tensor_infos = tensor_infos  # [(name, dims, ggml_type, offset)]
        self.data_offset = data_offset


def parse_bytes(data: bytes) -> GGUFFile:
    """parser.rs:151-211."""
    cur = Cursor(bytes(data))
    magic = cur.read_bytes(4)
    if magic != b"GGUF":
        raise OracleError("InvalidFormat", f"Invalid GGUF magic: expected [71, 71, 85, 70], got {list(magic)}")
    version = cur.read_u32()
    if version < 2 or version > 3:
        raise OracleError("InvalidFormat", f"Unsupported GGUF version: {version}")
    tensor_count = cur.read_u64()
    metadata_count = cur.read_u64()
    metadata = {}
    for _ in range(metadata_count):
        key = cur.read_string()
        value_type = cur.read_u32()
        metadata[key] = cur.read_value(value_type)
    infos = []
    for _ in range(tensor_count):
        name = cur.read_string()
        n_dims = cur.read_u32()
        dims = [cur.read_u64() for _ in range(n_dims)]
        t = cur.read_u32()
        if t not in GGML:
            raise OracleError("UnsupportedType", f"GGML type: {t}")
        offset = cur.read_u64()
        infos.append((name, dims, t, offset))
    return GGUFFile(version, metadata, infos, (cur.pos + 31) & ~31)


def tensor_nbytes(dims, ggml_type):
    """load_tensors' byte size (parser.rs:298-304)."""
    n = 1
    for d in dims:
        n *= d
    bs, bb = GGML[ggml_type]
    return (n // bs if bs > 1 else n) * bb


def tensor_bytes(f: GGUFFile, data: bytes, index: int) -> bytes:
    """The slice load_tensors takes for tensor `index`, with its bound check (parser.rs:306-314)."""
    name, dims, t, offset = f.tensor_infos[index]
    size = tensor_nbytes(dims, t)
    start = f.data_offset + offset
    if start + size > len(data):
        raise OracleError("Io", f"Tensor '{name}' data exceeds file bounds")
    return bytes(data[start:start + size])


def as_u32(v):
    """types.rs:98-105."""
    if v is None:
        return None
    t, x = v
    if t in (4, 5, 10):
        return x & 0xFFFFFFFF
    return None


def as_f32(v):
    """types.rs:107-113 (F64 rounded to f32)."""
    if v is None:
        return None
    t, x = v
    if t == 6:
        return x
    if t == 12:
        with np.errstate(over="ignore"):
            return float(np.float64(x).astype(np.float32))  # `as f32`: nearest, +-inf beyond range
    return None


def as_string(v):
    if v is None or v[0] != 8:
        return None
    return v[1]


def to_model_config(f: GGUFFile) -> dict:
    """parser.rs:214-289 -> a dict with GgufModelConfig's fields."""
    md = f.metadata
    a = as_string(md.get("general.architecture"))
    arch = "llama" if a is None else a

    def get_u32(key):
        v = as_u32(md.get(key))
        if v is None:
            raise OracleError("MissingMetadata", key)
        return v

    def get_u32_opt(key):
        return as_u32(md.get(key))

    def get_f32_opt(key):
        return as_f32(md.get(key))

    dim = get_u32(f"{arch}.embedding_length")
    n_heads = get_u32(f"{arch}.attention.head_count")
    n_layers = get_u32(f"{arch}.block_count")
    vocab = get_u32_opt(f"{arch}.vocab_size")
    if vocab is None:
        vocab = get_u32_opt("tokenizer.ggml.tokens_count")
    if vocab is None:
        tv = md.get("tokenizer.ggml.tokens")
        vocab = len(tv[1]) if tv is not None and tv[0] == 9 else 32000
    hidden = get_u32_opt(f"{arch}.feed_forward_length")
    if hidden is None:
        hidden = (dim * 4) & 0xFFFFFFFF
    n_kv = get_u32_opt(f"{arch}.attention.head_count_kv")
    max_seq = get_u32_opt(f"{arch}.context_length")
    eps = get_f32_opt(f"{arch}.attention.layer_norm_rms_epsilon")
    theta = get_f32_opt(f"{arch}.rope.freq_base")
    return dict(
        architecture=arch, dim=dim, hidden_dim=hidden, n_layers=n_layers, n_heads=n_heads, n_kv_heads=n_kv,
        vocab_size=vocab, norm_eps=float(np.float32(1e-5)) if eps is None else eps,
        max_seq_len=2048 if max_seq is None else max_seq, rope_theta=10000.0 if theta is None else theta,
        bos_token_id=get_u32_opt("tokenizer.ggml.bos_token_id"),
        eos_token_id=get_u32_opt("tokenizer.ggml.eos_token_id"),
        chat_template=as_string(md.get("tokenizer.chat_template")),
        head_dim=get_u32_opt(f"{arch}.attention.key_length"),
        sliding_window=get_u32_opt(f"{arch}.attention.sliding_window"))


def llama_weight_map(n_layers: int) -> dict:
    """gguf_llama_weight_map (weight_map.rs:26-73): GGUF name -> internal name."""
    m = {"token_embd.weight": "token_embedding.weight", "output_norm.weight": "norm.weight",
         "output.weight": "output.weight"}
    for i in range(n_layers):
        m.update({
            f"blk.{i}.attn_q.weight": f"layers.{i}.attention.q_proj.weight",
            f"blk.{i}.attn_k.weight": f"layers.{i}.attention.k_proj.weight",
            f"blk.{i}.attn_v.weight": f"layers.{i}.attention.v_proj.weight",
            f"blk.{i}.attn_output.weight": f"layers.{i}.attention.out_proj.weight",
            f"blk.{i}.attn_norm.weight": f"layers.{i}.attention_norm.weight",
            f"blk.{i}.ffn_norm.weight": f"layers.{i}.ffn_norm.weight",
            f"blk.{i}.ffn_up.weight": f"layers.{i}.feed_forward.up_proj.weight",
            f"blk.{i}.ffn_down.weight": f"layers.{i}.feed_forward.down_proj.weight",
            f"blk.{i}.ffn_gate.weight": f"layers.{i}.feed_forward.gate_proj.weight",
        })
    return m
