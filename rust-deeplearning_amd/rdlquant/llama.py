"""ctypes binding of the device decoder in librdlquant.so (include/rdl_llama.h).

LlamaModel mirrors the rustml decode path for Q4_0 Llama-style models:
forward_with_cache (LlmModel::forward_with_cache_pass + KVCache::advance,
rustml/nlp/main/src/core/model.rs:890-937), prefill / decode_step
(Generator, rustml/nlp/main/src/core/generator.rs:212-240) and greedy
generation with sampling::argmax (rustml/nlp/main/src/core/sampling.rs:8-18).
Everything runs on the GPU; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _decl, _i32, _p, _sz, check, lib

TOKEN_EMBEDDING, ATTN_NORM, WQ, WK, WV, WO, FFN_NORM, W_GATE, W_UP, W_DOWN, FINAL_NORM, OUTPUT = range(12)
SLOTS = 12


class _Config(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("dim", "n_layers", "n_heads", "n_kv_heads", "head_dim", "ffn_dim",
                                           "vocab", "max_seq")] + \
               [("norm_eps", C.c_float), ("rope_theta", C.c_float), ("kv_f16", C.c_int32),
                ("max_batch", C.c_int32), ("output_dtype", C.c_int32)]


_decl("rdl_llama_create", _i32, C.POINTER(_Config), C.POINTER(_p))
_decl("rdl_llama_create_typed", _i32, C.POINTER(_Config), C.POINTER(C.c_int32), C.POINTER(_p))
_decl("rdl_llama_free", _i32, _p)
_decl("rdl_llama_set_weight", _i32, _p, _i32, _i32, _p, _sz)
_decl("rdl_llama_init_random", _i32, _p, C.c_uint64)
_decl("rdl_llama_reset", _i32, _p)
_decl("rdl_llama_position", _i32, _p, C.POINTER(_sz))
_decl("rdl_llama_forward", _i32, _p, C.POINTER(C.c_int32), _sz, C.POINTER(C.c_float), _sz)
_decl("rdl_llama_generate_greedy", _i32, _p, C.POINTER(C.c_int32), _sz, _sz, C.POINTER(C.c_int32))
_decl("rdl_llama_last_timing", _i32, _p, C.POINTER(C.c_float), C.POINTER(C.c_float))
_decl("rdl_llama_rope_tables", _i32, _p, C.POINTER(C.c_float), C.POINTER(C.c_float), _sz)
_decl("rdl_llama_get_config", _i32, _p, C.POINTER(_Config))
_decl("rdl_llama_kv_pages", _i32, _p, C.POINTER(_sz), C.POINTER(_sz))
_decl("rdl_llama_set_kv_page_table", _i32, _p, C.POINTER(C.c_int32), _sz)
_decl("rdl_llama_set_fused_attention", _i32, _p, _i32)


class _PathCounts(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("fused_decode", "prefill_mfma", "prefill_rows", "attention", "fused_down")]


_decl("rdl_llama_get_path_counts", _i32, _p, C.POINTER(_PathCounts))
_decl("rdl_llama_set_native_q4", _i32, _p, _i32, _i32)


class _GgufOptions(C.Structure):
    _fields_ = [("max_seq", C.c_int32), ("max_batch", C.c_int32), ("kv_f16", C.c_int32)]


_decl("rdl_llama_load_gguf", _i32, _p, C.POINTER(_GgufOptions), C.POINTER(_p))


@dataclass
class LlamaConfig:
    """The ModelConfig fields of the Llama path (rustml/nlp/main/src/api/types.rs:186)."""
    dim: int = 4096
    n_layers: int = 32
    n_heads: int = 32
    n_kv_heads: int = 8
    head_dim: int = 128
    ffn_dim: int = 14336
    vocab: int = 32000
    max_seq: int = 2048
    norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    kv_f16: bool = True
    max_batch: int = 128
    output_dtype: int = 2  # GGML type of the output matrix (Q4_0; also Q8_0, Q4_1, Q4_K, Q6_K)

    def _c(self):
        return _Config(self.dim, self.n_layers, self.n_heads, self.n_kv_heads, self.head_dim, self.ffn_dim,
                       self.vocab, self.max_seq, self.norm_eps, self.rope_theta, int(self.kv_f16),
                       self.max_batch, self.output_dtype)


def _i32_array(tokens):
    return np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).reshape(-1))


class LlamaModel:
    """Q4_0 Llama-style decoder resident on the current GPU."""

    def __init__(self, config: LlamaConfig, types=None):
        """types: None (every matrix Q4_0, the output in config.output_dtype) or
        {(slot, layer): GGML type id} for the matrices that are not Q4_0
        (rdl_llama_create_typed; model-level slots use layer 0)."""
        self.config = config
        h = _p()
        cfg = config._c()
        if types:
            t = np.zeros(config.n_layers * SLOTS, dtype=np.int32)
            for (slot, layer), v in types.items():
                t[layer * SLOTS + slot] = v
            check(lib.rdl_llama_create_typed(C.byref(cfg), t.ctypes.data_as(C.POINTER(C.c_int32)), C.byref(h)))
        else:
            check(lib.rdl_llama_create(C.byref(cfg), C.byref(h)))
        self._h = h

    @classmethod
    def from_gguf(cls, gguf, max_seq: int = 0, max_batch: int = 32, kv_f16: bool = True) -> "LlamaModel":
        """LlmModel::from_pretrained over a GGUF file (a path or an open
        rdlquant.gguf.GGUFFile): config from the metadata, tensors through the
        Llama weight map, bytes from the file mapping straight to HBM
        (include/rdl_llama.h: rdl_llama_load_gguf).  max_seq 0: the file's
        context_length."""
        from .gguf import GGUFFile

        f = gguf if isinstance(gguf, GGUFFile) else GGUFFile.parse_header(gguf)
        opt = _GgufOptions(max_seq, max_batch, int(kv_f16))
        h = _p()
        check(lib.rdl_llama_load_gguf(f.handle, C.byref(opt), C.byref(h)))
        c = _Config()
        status = lib.rdl_llama_get_config(h, C.byref(c))
        if status != 0:
            lib.rdl_llama_free(h)
            check(status)
        self = cls.__new__(cls)
        self._h = h
        self.config = LlamaConfig(c.dim, c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim, c.ffn_dim, c.vocab,
                                  c.max_seq, float(c.norm_eps), float(c.rope_theta), bool(c.kv_f16),
                                  c.max_batch, c.output_dtype)
        return self

    def close(self):
        if getattr(self, "_h", None) and lib is not None:  # lib is None at interpreter shutdown
            lib.rdl_llama_free(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def set_weight(self, slot: int, layer: int, data: np.ndarray) -> None:
        """GGUF block bytes (uint8) for matrices and the embedding (Q4_0; the
        output matrix in config.output_dtype), f32 for norms."""
        a = np.ascontiguousarray(data)
        check(lib.rdl_llama_set_weight(self._h, slot, layer, a.ctypes.data, a.nbytes))

    def init_random(self, seed: int) -> None:
        check(lib.rdl_llama_init_random(self._h, C.c_uint64(seed & (2**64 - 1))))

    def reset(self) -> None:
        check(lib.rdl_llama_reset(self._h))

    @property
    def position(self) -> int:
        out = _sz()
        check(lib.rdl_llama_position(self._h, C.byref(out)))
        return int(out.value)

    def set_fused_attention(self, level=1) -> None:
        """Decode steps of fused layers: 1 (default, or True) q/k/v
        projection, attention and o projection in one launch; 2 that launch
        led by the previous layer's down projection; 0 (or False) q/k/v,
        attention and o as three launches."""
        level = 1 if level is True else 0 if level is False else int(level)
        check(lib.rdl_llama_set_fused_attention(self._h, level))

    def set_native_q4_matmul(self, enabled: bool, layer: int = -1) -> None:
        """TransformerBlock::set_native_q4_matmul on one layer (layer=-1: all):
        its Q4_0 / Q4_1 Linears take the native (Q8_0 activations, int32 block
        dots) path."""
        check(lib.rdl_llama_set_native_q4(self._h, layer, int(bool(enabled))))

    def path_counts(self) -> dict:
        """Attention launches enqueued so far, by kernel (host-side counts; a
        captured decode graph counts once, at capture): fused_decode (of
        which fused_down were led by the previous layer's down projection),
        prefill_mfma, prefill_rows, attention."""
        c = _PathCounts()
        check(lib.rdl_llama_get_path_counts(self._h, C.byref(c)))
        return {n: int(getattr(c, n)) for n, _ in _PathCounts._fields_}

    def kv_pages(self):
        """(positions per page, number of pages) of the paged KV cache."""
        ps, n = _sz(), _sz()
        check(lib.rdl_llama_kv_pages(self._h, C.byref(ps), C.byref(n)))
        return int(ps.value), int(n.value)

    def set_kv_page_table(self, table) -> None:
        """table[logical page] = physical page (a permutation); empty cache only."""
        t = _i32_array(table)
        check(lib.rdl_llama_set_kv_page_table(self._h, t.ctypes.data_as(C.POINTER(C.c_int32)), t.size))

    def forward_with_cache(self, tokens) -> np.ndarray:
        """Logits of the last of `tokens` (vocab floats); the cache advances by len(tokens)."""
        t = _i32_array(tokens)
        logits = np.empty(self.config.vocab, dtype=np.float32)
        check(lib.rdl_llama_forward(self._h, t.ctypes.data_as(C.POINTER(C.c_int32)), t.size,
                                    logits.ctypes.data_as(C.POINTER(C.c_float)), logits.size))
        return logits

    def prefill(self, tokens) -> np.ndarray:
        return self.forward_with_cache(tokens)

    def decode_step(self, token: int) -> np.ndarray:
        return self.forward_with_cache([token])

    def generate_greedy(self, prompt, n_gen: int) -> np.ndarray:
        """n_gen argmax tokens after the prompt (prefill + n_gen - 1 graph-replayed steps)."""
        p = _i32_array(prompt)
        out = np.empty(n_gen, dtype=np.int32)
        check(lib.rdl_llama_generate_greedy(self._h, p.ctypes.data_as(C.POINTER(C.c_int32)), p.size, n_gen,
                                            out.ctypes.data_as(C.POINTER(C.c_int32))))
        return out

    def last_timing(self):
        """(prefill_ms, decode_ms) of the last generate_greedy call, device time."""
        a, b = C.c_float(), C.c_float()
        check(lib.rdl_llama_last_timing(self._h, C.byref(a), C.byref(b)))
        return float(a.value), float(b.value)

    def rope_tables(self):
        n = self.config.max_seq * (self.config.head_dim // 2)
        c = np.empty(n, np.float32)
        s = np.empty(n, np.float32)
        check(lib.rdl_llama_rope_tables(self._h, c.ctypes.data_as(C.POINTER(C.c_float)),
                                        s.ctypes.data_as(C.POINTER(C.c_float)), n))
        return c.reshape(self.config.max_seq, -1), s.reshape(self.config.max_seq, -1)
