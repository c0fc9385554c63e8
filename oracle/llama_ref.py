"""CPU restatement of the rustml Q4_0 Llama decode path, for the GPU decoder's
parity tests.

TEST INFRASTRUCTURE ONLY (imported by tests/): it checks librdlquant's
rdl_llama_* path and is never called by the product.

Follows, in f32:
  LlmModel::forward_with_cache_pass      rustml/nlp/main/src/core/model.rs:890-937
  TransformerBlock::forward_with_cache   rustml/nn/main/src/core/transformer_block.rs:321-355
  MultiHeadAttention::forward_with_cache rustml/nn/main/src/core/attention.rs:353-449
  FeedForward::forward (SwiGLU)          rustml/nn/main/src/core/feed_forward.rs:138-150
  RoPEFreqs::apply (scalar form)         rustml/nn/main/src/core/rope.rs:134-200
  Tensor::softmax (last dim)             rustml/core/main/src/core/tensor/ops.rs:582-628
  Tensor::silu                           rustml/core/main/src/core/tensor/ops.rs:441-446
  Embedding::forward over to_f32 rows    rustml/nn/main/src/core/embedding.rs:50-76
  sampling::argmax                       rustml/nlp/main/src/core/sampling.rs:8-18
The Q4_0 Linears and the embedding dequantization call the C restatement
(oracle/rdl_oracle.c: matmul_f32_q4, to_f32), RMSNorm its AVX2-order row
(orc_rms_norm_row) and the RoPE tables orc_rope_tables.  The f32 matmuls of
attention (faer in the reference) and the softmax sum use numpy's order: their
summation order is not pinned, only f32 accuracy.
"""
from __future__ import annotations

import numpy as np

from . import oracle as orc


def rope_apply(t, cos, sin, start):
    """RoPEFreqs::apply (rope.rs:134-200), half-split pairs (i, i + D/2):
    t [heads, S, D] at positions start .. start + S - 1;
    out[i] = x[i] cos - x[i + D/2] sin, out[i + D/2] = x[i] sin + x[i + D/2] cos
    (rope.rs:189-190) with cos / sin rows of RoPEFreqs::new (rope.rs:93-108)."""
    half = t.shape[-1] // 2
    s = t.shape[1]
    cs = cos[start:start + s][None]
    sn = sin[start:start + s][None]
    x1, x2 = t[..., :half], t[..., half:]
    return np.concatenate([x1 * cs - x2 * sn, x1 * sn + x2 * cs], axis=-1).astype(np.float32)


def attention(q, kc, vc, start):
    """Grouped-query attention of MultiHeadAttention::forward_with_cache
    (attention.rs:401-446): q [n_heads, S, D] (rows at positions start ..
    start + S - 1), kc / vc [n_kv, T, D] the cached keys and values 0 .. T-1.
    Query head h reads KV head h // (n_heads / n_kv) (repeat_kv, ops.rs:955-995,
    attention.rs:408-410); scores q.k / sqrt(D) (attention.rs:414-416), the
    causal mask keeps keys <= start + i (Tensor::causal_mask, attention.rs:424-433),
    max-subtracted softmax (ops.rs:582-628), then p . V.  Returns [n_heads, S, D]."""
    nh, s, hd = q.shape
    n_rep = nh // kc.shape[0]
    scale = np.float32(np.sqrt(np.float32(hd)))
    ctx = np.zeros((nh, s, hd), np.float32)
    for h in range(nh):
        kh, vh = kc[h // n_rep], vc[h // n_rep]
        sc = (q[h] @ kh.T).astype(np.float32) / scale
        if s > 1:  # causal mask (Tensor::causal_mask(seq_len, total_len))
            for i in range(s):
                sc[i, start + i + 1:] = -np.inf
        mx = sc.max(axis=1, keepdims=True)
        e = np.exp(sc - mx).astype(np.float32)
        p = (e / e.sum(axis=1, keepdims=True, dtype=np.float32)).astype(np.float32)
        ctx[h] = (p @ vh).astype(np.float32)
    return ctx


def swiglu(gate, up):
    """FeedForward::forward's SwiGLU (feed_forward.rs:146-148): silu(gate) * up
    with silu(g) = g * (1 / (1 + exp(-g))) (Tensor::silu, ops.rs:441-446)."""
    sig = (np.float32(1.0) / (np.float32(1.0) + np.exp(-gate))).astype(np.float32)
    return ((gate * sig) * up).astype(np.float32)


class LlamaRef:
    def __init__(self, cfg, weights, threads=8, kv_f16=False):
        """cfg: rdlquant.llama.LlamaConfig; weights: dict slot -> array (model
        slots) or (slot, layer) -> array, as given to LlamaModel.set_weight.
        kv_f16: K and V rows (after RoPE) are stored rounded to f16 (round to
        nearest, ties to even), as a half-precision cache holds them; the
        attention then reads those values in f32.  Off: f32 rows, as KVCache
        (kv_cache.rs:23-114)."""
        self.c = cfg
        self.w = weights
        self.threads = threads
        self.kv_f16 = kv_f16
        c = cfg
        self.cos, self.sin = orc.rope_tables(c.head_dim, c.max_seq, c.rope_theta)
        self.kv = [[np.zeros((c.n_kv_heads, c.max_seq, c.head_dim), np.float32) for _ in range(2)]
                   for _ in range(c.n_layers)]
        self.pos = 0

    def _linear(self, key, x, n, k):
        m = x.shape[0]
        # a matrix may be another GGUF type (weights["kinds"][key]: an oracle
        # matmul kind; "output_kind" for the output matrix); the reference
        # runs K-quants as F32 after load-time dequantization, which the
        # oracle's q4k / q6k kinds restate
        kinds = self.w.get("kinds", {})
        kind = kinds.get(key, self.w.get("output_kind", "q4") if key == "output" else "q4")
        return orc.matmul(kind, x, self.w[key], m, k, n, threads=self.threads).reshape(m, n)

    def forward_with_cache(self, tokens):
        """Last row's logits; the cache advances by len(tokens)."""
        c = self.c
        tokens = np.asarray(tokens, np.int64).reshape(-1)
        s = tokens.size
        emb = self.w["emb_f32"]
        x = emb[tokens].astype(np.float32)  # [S, dim]
        start = self.pos
        hd, nh, nkv = c.head_dim, c.n_heads, c.n_kv_heads
        for layer in range(c.n_layers):
            xn = orc.rms_norm(x, self.w[("attn_norm", layer)], c.norm_eps)
            q = self._linear(("wq", layer), xn, nh * hd, c.dim)
            k = self._linear(("wk", layer), xn, nkv * hd, c.dim)
            v = self._linear(("wv", layer), xn, nkv * hd, c.dim)
            q = q.reshape(s, nh, hd).transpose(1, 0, 2)
            k = k.reshape(s, nkv, hd).transpose(1, 0, 2)
            v = v.reshape(s, nkv, hd).transpose(1, 0, 2)
            q = rope_apply(q, self.cos, self.sin, start)
            k = rope_apply(k, self.cos, self.sin, start)
            kc, vc = self.kv[layer]
            if self.kv_f16:
                k = k.astype(np.float16).astype(np.float32)
                v = v.astype(np.float16).astype(np.float32)
            kc[:, start:start + s] = k
            vc[:, start:start + s] = v
            ctx = attention(q, kc[:, :start + s], vc[:, :start + s], start)
            ctx = ctx.transpose(1, 0, 2).reshape(s, nh * hd)
            attn = self._linear(("wo", layer), ctx, c.dim, nh * hd)
            x = (attn + x).astype(np.float32)
            xn = orc.rms_norm(x, self.w[("ffn_norm", layer)], c.norm_eps)
            gate = self._linear(("w_gate", layer), xn, c.ffn_dim, c.dim)
            up = self._linear(("w_up", layer), xn, c.ffn_dim, c.dim)
            h = swiglu(gate, up)
            down = self._linear(("w_down", layer), h, c.dim, c.ffn_dim)
            x = (x + down).astype(np.float32)
        xl = orc.rms_norm(x[-1:], self.w["final_norm"], c.norm_eps)
        logits = self._linear("output", xl, c.vocab, c.dim).reshape(-1)
        self.pos += s
        return logits


def argmax(logits):
    """sampling::argmax: first maximum wins; NaN never wins; 0 for an all-NaN row."""
    best, val = 0, -np.inf
    for i, v in enumerate(np.asarray(logits, np.float32)):
        if v > val:
            val, best = v, i
    return best
