"""Seeded tiny Llama-style models for the decoder tests (CPU oracle and GPU)."""
import numpy as np

from rdlquant import synth


def tiny_config(**kw):
    from rdlquant.llama import LlamaConfig
    base = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=320,
                max_seq=64, norm_eps=1e-5, rope_theta=10000.0, kv_f16=False, max_batch=16)
    base.update(kw)
    return LlamaConfig(**base)


def tiny_weights(cfg, seed=1234):
    """(gpu_slots, oracle_weights): the same seeded bytes for both sides."""
    from rdlquant import llama as L
    from oracle import oracle as orc
    rng = np.random.default_rng(seed)
    q, kv = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    slots, ref = [], {}
    s = seed

    def q4(n, k):
        nonlocal s
        s += 1
        return synth.q4_0_weights(n, k, s)

    def norm():
        return (1.0 + 0.1 * rng.standard_normal(cfg.dim)).astype(np.float32)

    emb = q4(cfg.vocab, cfg.dim)
    slots.append((L.TOKEN_EMBEDDING, 0, emb))
    ref["emb_f32"] = orc.to_f32("q4_0", emb, cfg.vocab * cfg.dim).reshape(cfg.vocab, cfg.dim)
    for layer in range(cfg.n_layers):
        for slot, name, arr in ((L.ATTN_NORM, "attn_norm", norm()), (L.WQ, "wq", q4(q, cfg.dim)),
                                (L.WK, "wk", q4(kv, cfg.dim)), (L.WV, "wv", q4(kv, cfg.dim)),
                                (L.WO, "wo", q4(cfg.dim, q)), (L.FFN_NORM, "ffn_norm", norm()),
                                (L.W_GATE, "w_gate", q4(cfg.ffn_dim, cfg.dim)),
                                (L.W_UP, "w_up", q4(cfg.ffn_dim, cfg.dim)),
                                (L.W_DOWN, "w_down", q4(cfg.dim, cfg.ffn_dim))):
            slots.append((slot, layer, arr))
            ref[(name, layer)] = arr
    s += 1
    out = synth.weights(cfg.output_dtype, cfg.vocab, cfg.dim, s)
    fin = norm()
    slots += [(L.FINAL_NORM, 0, fin), (L.OUTPUT, 0, out)]
    ref["final_norm"], ref["output"] = fin, out
    ref["output_kind"] = {2: "q4", 3: "q4_1", 8: "q8", 12: "q4k", 14: "q6k"}[cfg.output_dtype]
    return slots, ref


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
