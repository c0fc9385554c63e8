"""Seeded tiny Llama-style models for the decoder tests (CPU oracle and GPU)."""
import numpy as np

from rdlquant import synth


def tiny_config(**kw):
    from rdlquant.llama import LlamaConfig
    base = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=320,
                max_seq=64, norm_eps=1e-5, rope_theta=10000.0, kv_f16=False, max_batch=16)
    base.update(kw)
    return LlamaConfig(**base)


KIND = {2: "q4", 3: "q4_1", 8: "q8", 12: "q4k", 14: "q6k"}  # GGML type -> oracle matmul kind
DEQ = {2: "q4_0", 3: "q4_1", 8: "q8_0", 12: "q4k", 14: "q6k"}  # GGML type -> oracle to_f32 kind


def centered_q4_0_weights(n, k, seed, d_sigma=0.02):
    """Q4_0 blocks whose codes are uniform in 1..15, so q - 8 has mean 0.
    BASELINE's codes (uniform in 0..15) give every weight a mean of -d/2;
    stacked over layers that common mode swamps the residual stream and the
    logits barely depend on the tokens or the attention.  Centered codes
    keep a decoder sensitive to what its attention does."""
    r = np.random.default_rng(seed)
    nb = k // 32
    q = r.integers(1, 16, size=(n, nb, 32), dtype=np.uint8)
    d = synth.f16_bits(np.abs(r.normal(0.0, d_sigma, size=(n, nb))) / 8.0)
    out = np.empty((n, nb, 18), dtype=np.uint8)
    out[..., 0:2] = d[..., None].view(np.uint8).reshape(n, nb, 2)
    out[..., 2:] = synth.pack_q4_nibbles(q)
    return out.reshape(-1)


def tiny_weights(cfg, seed=1234, types=None, centered=False):
    """(gpu_slots, oracle_weights): the same seeded bytes for both sides.
    types: {(slot, layer): GGML type} for matrices that are not Q4_0;
    centered: Q4_0 matrices with zero-mean codes (centered_q4_0_weights)."""
    from rdlquant import llama as L
    from oracle import oracle as orc
    rng = np.random.default_rng(seed)
    q, kv = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    types = types or {}
    slots, ref = [], {"kinds": {}}
    s = seed

    def mat(slot, layer, n, k):
        nonlocal s
        s += 1
        t = types.get((slot, layer), 2)
        if centered and t == 2:
            return centered_q4_0_weights(n, k, s)
        return synth.weights(t, n, k, s)

    def norm():
        return (1.0 + 0.1 * rng.standard_normal(cfg.dim)).astype(np.float32)

    emb = mat(L.TOKEN_EMBEDDING, 0, cfg.vocab, cfg.dim)
    slots.append((L.TOKEN_EMBEDDING, 0, emb))
    et = types.get((L.TOKEN_EMBEDDING, 0), 2)
    ref["emb_f32"] = orc.to_f32(DEQ[et], emb, cfg.vocab * cfg.dim).reshape(cfg.vocab, cfg.dim)
    for layer in range(cfg.n_layers):
        for slot, name, arr in ((L.ATTN_NORM, "attn_norm", norm()), (L.WQ, "wq", mat(L.WQ, layer, q, cfg.dim)),
                                (L.WK, "wk", mat(L.WK, layer, kv, cfg.dim)),
                                (L.WV, "wv", mat(L.WV, layer, kv, cfg.dim)),
                                (L.WO, "wo", mat(L.WO, layer, cfg.dim, q)), (L.FFN_NORM, "ffn_norm", norm()),
                                (L.W_GATE, "w_gate", mat(L.W_GATE, layer, cfg.ffn_dim, cfg.dim)),
                                (L.W_UP, "w_up", mat(L.W_UP, layer, cfg.ffn_dim, cfg.dim)),
                                (L.W_DOWN, "w_down", mat(L.W_DOWN, layer, cfg.dim, cfg.ffn_dim))):
            slots.append((slot, layer, arr))
            ref[(name, layer)] = arr
            if (slot, layer) in types:
                ref["kinds"][(name, layer)] = KIND[types[(slot, layer)]]
    s += 1
    ot = types.get((L.OUTPUT, 0), cfg.output_dtype)
    out = synth.weights(ot, cfg.vocab, cfg.dim, s)
    fin = norm()
    slots += [(L.FINAL_NORM, 0, fin), (L.OUTPUT, 0, out)]
    ref["final_norm"], ref["output"] = fin, out
    ref["output_kind"] = KIND[ot]
    return slots, ref


def gguf_types(types):
    """{(slot, layer): GGML type} -> {GGUF tensor name: GGML type}."""
    return {gguf_name(sl, la): t for (sl, la), t in (types or {}).items()}


def gguf_name(slot, layer):
    """The GGUF tensor name of a decoder slot (gguf_llama_weight_map,
    rustml/gguf/main/src/core/weight_map.rs:26-73)."""
    from rdlquant import llama as L
    model = {L.TOKEN_EMBEDDING: "token_embd.weight", L.FINAL_NORM: "output_norm.weight",
             L.OUTPUT: "output.weight"}
    per_layer = {L.ATTN_NORM: "attn_norm", L.WQ: "attn_q", L.WK: "attn_k", L.WV: "attn_v", L.WO: "attn_output",
                 L.FFN_NORM: "ffn_norm", L.W_GATE: "ffn_gate", L.W_UP: "ffn_up", L.W_DOWN: "ffn_down"}
    return model[slot] if slot in model else f"blk.{layer}.{per_layer[slot]}.weight"


def write_gguf(path, cfg, slots, **kw):
    """A Llama GGUF file holding the bytes of `slots` (as tiny_weights returns
    them); keyword arguments go to gguf_writer.llama_builder."""
    from rdlquant import gguf_writer
    by_name = {gguf_name(s, l): a for s, l, a in slots}
    b = gguf_writer.llama_builder(cfg, lambda name: by_name[name], **kw)
    b.write(path)
    return b
