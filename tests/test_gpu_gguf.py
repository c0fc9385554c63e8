"""GGUF loading on the GPU: tensor bytes from the file mapping into HBM
(rdl_gguf_upload_tensor) and the decoder built from a file
(rdl_llama_load_gguf), checked bit-exact against the set_weight path with the
same bytes and, for one model, against the CPU oracle's decode."""
import dataclasses

import numpy as np
import pytest

from llama_fixtures import gguf_name, tiny_config, tiny_weights, write_gguf
from parity import assert_close

pytestmark = pytest.mark.gpu


def from_slots(cfg, slots):
    from rdlquant.llama import LlamaModel
    m = LlamaModel(cfg)
    for slot, layer, arr in slots:
        m.set_weight(slot, layer, arr)
    return m


def run(m, prompt, n_gen):
    m.reset()
    logits = m.forward_with_cache(prompt)
    m.reset()
    toks = m.generate_greedy(prompt, n_gen)
    return logits, toks


@pytest.mark.parametrize("sizes", [[18 * 5], [4 * 1000, 2 * 7, 3], [(96 << 20) + 18 * 3]])
def test_upload_tensor_bytes(rq, gpu, tmp_path, sizes):
    """Raw bytes into device memory, one tensor per size (the last spans
    several 32 MiB staging chunks)."""
    import torch

    from rdlquant import gguf, gguf_writer as W
    rng = np.random.default_rng(len(sizes))
    blobs = []
    b = W.GgufBuilder().add_string("general.architecture", "llama")
    for i, n in enumerate(sizes):
        # a type whose block size divides n: Q4_0 (18 B), F16 (2 B) or F32 (4 B)
        t = W.GGML_Q4_0 if n % 18 == 0 else W.GGML_F32 if n % 4 == 0 else W.GGML_F16
        bs, bb = W.GGML_BLOCK[t]
        n = n - n % bb
        blob = rng.integers(0, 256, n, dtype=np.uint8)
        blobs.append(blob)
        b.add_tensor_data(f"t{i}", [n // bb * bs], t, blob)
    p = tmp_path / "t.gguf"
    b.write(p)
    f = gguf.GGUFFile.parse_header(p)
    for i, blob in enumerate(blobs):
        dst = torch.full((blob.size + 64,), 0xAB, dtype=torch.uint8, device=gpu)
        f.upload_tensor(f"t{i}", dst.data_ptr(), dst.numel())
        got = dst.cpu().numpy()
        assert np.array_equal(got[:blob.size], blob), f"t{i}"
        assert (got[blob.size:] == 0xAB).all()
    with pytest.raises(rq.ShapeMismatch):
        dst = torch.empty(blobs[0].size - 1, dtype=torch.uint8, device=gpu)
        f.upload_tensor("t0", dst.data_ptr(), dst.numel())


@pytest.mark.parametrize("kv_f16", [False, True])
def test_model_from_gguf_matches_set_weight(rq, gpu, tmp_path, kv_f16):
    from rdlquant.llama import LlamaModel
    cfg = tiny_config(kv_f16=kv_f16)
    slots, _ = tiny_weights(cfg, seed=77)
    p = tmp_path / "tiny.gguf"
    write_gguf(p, cfg, slots)
    m = LlamaModel.from_gguf(str(p), max_batch=cfg.max_batch, kv_f16=kv_f16)
    # the file holds eps as f32
    assert m.config == dataclasses.replace(cfg, norm_eps=float(np.float32(cfg.norm_eps)))
    prompt = [5, 17, 300, 2, 99, 1, 42]
    got = run(m, prompt, 12)
    want = run(from_slots(cfg, slots), prompt, 12)
    assert np.array_equal(got[0], want[0])
    assert np.array_equal(got[1], want[1])


def test_model_from_gguf_matches_oracle(rq, gpu, tmp_path):
    from oracle.llama_ref import LlamaRef
    from rdlquant.llama import LlamaModel
    cfg = tiny_config()
    slots, ref_w = tiny_weights(cfg, seed=78)
    p = tmp_path / "tiny.gguf"
    write_gguf(p, cfg, slots)
    m = LlamaModel.from_gguf(str(p), max_batch=cfg.max_batch, kv_f16=False)
    prompt = [3, 9, 27, 81, 243]
    got = m.forward_with_cache(prompt)
    want = LlamaRef(cfg, ref_w).forward_with_cache(prompt)
    assert_close(got, want)


def test_file_order_extras_and_f16_norms(rq, gpu, tmp_path):
    """Tensors in reverse order, an unmapped extra tensor, a duplicate name
    (the later one wins, as the reference's HashMap insert), F16 norm weights."""
    from rdlquant import gguf_writer as W
    from rdlquant.llama import LlamaModel
    cfg = tiny_config()
    slots, _ = tiny_weights(cfg, seed=79)
    # norms exactly representable in f16, so F32 and F16 files hold the same values
    slots = [(s, l, np.float16(a).astype(np.float32) if a.dtype == np.float32 else a) for s, l, a in slots]
    by_name = {gguf_name(s, l): a for s, l, a in slots}
    shapes = W.llama_tensor_shapes(cfg)
    b = W.llama_builder(cfg, lambda n: by_name[n], skip=set(shapes))
    b.add_tensor_data("rope_freqs.weight", [cfg.head_dim // 2], W.GGML_F32,
                      np.ones(cfg.head_dim // 2, np.float32))
    decoy = np.zeros_like(by_name["blk.1.attn_v.weight"])
    b.add_tensor_data("blk.1.attn_v.weight", shapes["blk.1.attn_v.weight"][0], W.GGML_Q4_0, decoy)
    for name in reversed(list(shapes)):
        dims, t = shapes[name]
        data = by_name[name]
        if t == W.GGML_F32:
            t, data = W.GGML_F16, data.astype(np.float16)
        b.add_tensor_data(name, dims, t, data)
    p = tmp_path / "mixed.gguf"
    b.write(p)
    m = LlamaModel.from_gguf(str(p), max_batch=cfg.max_batch, kv_f16=False)
    prompt = [11, 12, 13]
    got, want = run(m, prompt, 6), run(from_slots(cfg, slots), prompt, 6)
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])


def test_max_seq_from_file_and_override(rq, gpu, tmp_path):
    from rdlquant.llama import LlamaModel
    cfg = tiny_config()
    slots, _ = tiny_weights(cfg, seed=80)
    p = tmp_path / "tiny.gguf"
    write_gguf(p, cfg, slots, context_length=48)
    assert LlamaModel.from_gguf(str(p)).config.max_seq == 48
    m = LlamaModel.from_gguf(str(p), max_seq=20, max_batch=4)
    assert (m.config.max_seq, m.config.max_batch) == (20, 4)
    with pytest.raises(rq.InvalidData):
        m.generate_greedy(list(range(18)), 5)


def test_7b_layer_shapes_staged_in_chunks(rq, gpu, tmp_path):
    """One layer at the 7B shapes: the [gate; up] interleave of 33 MB per
    matrix crosses the 32 MiB staging chunk (strided copy in several chunks)."""
    from rdlquant import synth
    from rdlquant.llama import LlamaConfig, LlamaModel
    import rdlquant.llama as L
    cfg = LlamaConfig(dim=4096, n_layers=1, n_heads=32, n_kv_heads=8, head_dim=128, ffn_dim=14336, vocab=32000,
                      max_seq=64, kv_f16=True, max_batch=16)
    q, kv = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
    seeds = iter(range(0x5EED0200, 0x5EED0300))
    w = lambda n, k: synth.q4_0_weights(n, k, next(seeds))  # noqa: E731
    rng = np.random.default_rng(5)
    norm = lambda: (1 + 0.1 * rng.standard_normal(cfg.dim)).astype(np.float32)  # noqa: E731
    slots = [(L.TOKEN_EMBEDDING, 0, w(cfg.vocab, cfg.dim)), (L.ATTN_NORM, 0, norm()), (L.WQ, 0, w(q, cfg.dim)),
             (L.WK, 0, w(kv, cfg.dim)), (L.WV, 0, w(kv, cfg.dim)), (L.WO, 0, w(cfg.dim, q)),
             (L.FFN_NORM, 0, norm()), (L.W_GATE, 0, w(cfg.ffn_dim, cfg.dim)),
             (L.W_UP, 0, w(cfg.ffn_dim, cfg.dim)), (L.W_DOWN, 0, w(cfg.dim, cfg.ffn_dim)),
             (L.FINAL_NORM, 0, norm()), (L.OUTPUT, 0, w(cfg.vocab, cfg.dim))]
    p = tmp_path / "layer7b.gguf"
    write_gguf(p, cfg, slots)
    m = LlamaModel.from_gguf(str(p), max_batch=cfg.max_batch)
    prompt = [1, 2, 3, 4, 5, 6, 7, 8, 9]
    got = run(m, prompt, 8)
    m.close()
    want = run(from_slots(cfg, slots), prompt, 8)
    assert np.array_equal(got[0], want[0])
    assert np.array_equal(got[1], want[1])


def test_q6_k_output_from_gguf(rq, gpu, tmp_path):
    """A file with a Q6_K output.weight (as llama.cpp writes Q4_0 models)."""
    from rdlquant.llama import LlamaModel
    cfg = tiny_config(output_dtype=14)
    slots, _ = tiny_weights(cfg, seed=81)
    p = tmp_path / "q6k_out.gguf"
    write_gguf(p, cfg, slots)
    m = LlamaModel.from_gguf(str(p), max_batch=cfg.max_batch, kv_f16=False)
    assert m.config.output_dtype == 14
    prompt = [4, 40, 44, 144]
    got, want = run(m, prompt, 7), run(from_slots(cfg, slots), prompt, 7)
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])


def test_mixed_type_file(rq, gpu, tmp_path):
    """A file mixing GGUF types per tensor (as llama.cpp's Q4_K_M files do)."""
    from llama_fixtures import gguf_types
    from rdlquant.llama import LlamaModel
    from test_gpu_llama import mixed_types
    cfg = tiny_config(n_layers=3, output_dtype=8)
    types = mixed_types()
    slots, _ = tiny_weights(cfg, seed=82, types=types)
    p = tmp_path / "mixed.gguf"
    write_gguf(p, cfg, slots, types=gguf_types(types))
    m = LlamaModel.from_gguf(str(p), max_batch=cfg.max_batch, kv_f16=False)
    ref = LlamaModel(cfg, types=types)
    for slot, layer, arr in slots:
        ref.set_weight(slot, layer, arr)
    prompt = [7, 77, 177, 277, 17]
    got, want = run(m, prompt, 7), run(ref, prompt, 7)
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
