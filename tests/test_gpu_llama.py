"""GPU decoder (include/rdl_llama.h) against the CPU restatement of the
rustml decode path (oracle/llama_ref.py) on seeded tiny models, plus
properties of the full BASELINE config-5 model (7B shape, synthetic weights)."""
import numpy as np
import pytest

from oracle.llama_ref import LlamaRef, argmax
from parity import ATOL, RTOL, assert_close

from llama_fixtures import tiny_config, tiny_weights

pytestmark = pytest.mark.gpu


def build(cfg, seed=1234, centered=False):
    from rdlquant.llama import LlamaModel
    slots, ref_w = tiny_weights(cfg, seed, centered=centered)
    m = LlamaModel(cfg)
    for slot, layer, arr in slots:
        m.set_weight(slot, layer, arr)
    # an f16 cache: the oracle stores K / V rounded to f16 the same way
    return m, LlamaRef(cfg, ref_w, kv_f16=bool(cfg.kv_f16))


# Bound between an f16 KV cache and the reference's f32 KVCache
# (kv_cache.rs:23-114): rounding K and V to f16 (11 significant bits) moved
# the logits of the config-5 geometry tests by 1.8e-4 to 2.6e-4 of the
# largest one on MI355X; the bound is 2e-3.  This is the parity gap of the
# default decoder (kv_f16 = 1) to the reference; the f16 tests also compare,
# at the f32 bar, against the oracle that stores K / V rounded alike.
F16_CACHE_BOUND = 2e-3


def assert_within_f16_cache_bound(got, want32):
    err = np.abs(np.asarray(got, np.float64) - want32).max()
    bound = F16_CACHE_BOUND * np.abs(want32).max()
    print(f"  f16 cache vs f32 reference: max err {err:.3g} = {err / np.abs(want32).max():.2e} of the largest logit")
    assert err <= bound, (err, bound)


def assert_greedy_chain(gen, ref, logits, bar=None):
    """gen: the GPU's greedy tokens; ref: the oracle at the same position;
    logits: the oracle's logits that pick gen[0].  Each token is the oracle's
    argmax, except at a step where the oracle's two best logits are within
    twice the parity bar of each other (an order the bar cannot fix): there
    the GPU's token must be one of those, and the chains may part after it.
    bar: a bound relative to the largest logit in place of the parity bar."""
    for i, t in enumerate(np.asarray(gen).tolist()):
        want = argmax(logits)
        if t != want:
            gap = float(logits[want]) - float(logits[t])
            tol = (ATOL + RTOL * abs(float(logits[want]))) if bar is None else bar * float(np.abs(logits).max())
            assert gap <= 2 * tol, (i, t, want, gap)
            print(f"  greedy step {i}: near-tie {t} vs {want} (gap {gap:.3g}); chains part here")
            return
        if i + 1 < len(gen):
            logits = ref.forward_with_cache([t])


def test_rope_tables_match_oracle(rq, gpu):
    from oracle import oracle as orc
    cfg = tiny_config()
    m, _ = build(cfg)
    c, s = m.rope_tables()
    oc, os_ = orc.rope_tables(cfg.head_dim, cfg.max_seq, cfg.rope_theta)
    assert np.array_equal(c, oc) and np.array_equal(s, os_)


def test_prefill_and_decode_logits(rq, gpu):
    cfg = tiny_config()
    m, ref = build(cfg)
    prompt = [3, 141, 59, 26, 53, 58, 97, 93, 23]  # 9 rows: the GEMM path
    assert_close(m.forward_with_cache(prompt), ref.forward_with_cache(prompt))
    tok = 11
    for _ in range(6):  # one-row steps: the fused GEMV path
        got = m.decode_step(tok)
        want = ref.forward_with_cache([tok])
        assert_close(got, want)
        tok = argmax(want)
    assert m.position == ref.pos == len(prompt) + 6


def test_generate_greedy_matches_eager_steps(rq, gpu):
    cfg = tiny_config()
    m, _ = build(cfg)
    prompt = [7, 8, 9, 10, 200]
    gen = m.generate_greedy(prompt, 12)  # prefill + 11 graph replays
    m.reset()
    logits = m.forward_with_cache(prompt)
    eager = []
    for _ in range(12):
        t = int(np.argmax(logits))  # numpy argmax: first maximum, as sampling::argmax
        eager.append(t)
        logits = m.decode_step(t)
    assert gen.tolist() == eager
    # a second call replays the captured graph again from a fresh cache
    m.reset()
    assert m.generate_greedy(prompt, 12).tolist() == eager


@pytest.mark.parametrize("kw", [dict(dim=256, n_heads=2, n_kv_heads=1, head_dim=64),
                                dict(dim=128, n_heads=4, n_kv_heads=2, head_dim=64)])
def test_decode_with_head_width_unlike_dim(rq, gpu, kw):
    """n_heads * head_dim != dim: the o projection (fused into the decode
    launch) maps the attention outputs back to dim; logits against the
    oracle after prefill and fused decode steps."""
    cfg = tiny_config(**kw)
    m, ref = build(cfg, seed=77)
    prompt = [4, 9, 16, 25, 36, 49]
    assert_close(m.forward_with_cache(prompt), ref.forward_with_cache(prompt))
    tok = 3
    for _ in range(4):
        got = m.decode_step(tok)
        want = ref.forward_with_cache([tok])
        assert_close(got, want)
        tok = argmax(want)


def test_greedy_sampling_ties_pick_the_first_maximum(rq, gpu):
    """Output rows repeat with period 37, so each maximum logit is shared by
    8-9 token ids in different workgroups of the lm_head launch: the decode
    graph's sampling (per-workgroup argmax partials) picks the first, as
    numpy's argmax over the eager logits does (sampling.rs:8-18)."""
    from rdlquant.llama import LlamaModel, OUTPUT
    cfg = tiny_config()
    slots, _ = tiny_weights(cfg, 4321)
    m = LlamaModel(cfg)
    for slot, layer, arr in slots:
        if slot == OUTPUT:
            arr = arr.reshape(cfg.vocab, -1)[np.arange(cfg.vocab) % 37].copy()
        m.set_weight(slot, layer, arr)
    prompt = [5, 6, 7]
    gen = m.generate_greedy(prompt, 10)
    m.reset()
    logits = m.forward_with_cache(prompt)
    eager = []
    for _ in range(10):
        t = int(np.argmax(logits))
        assert np.count_nonzero(logits == logits[t]) > 1  # a real tie
        eager.append(t)
        logits = m.decode_step(t)
    assert gen.tolist() == eager


def test_generate_greedy_matches_oracle_tokens(rq, gpu):
    cfg = tiny_config()
    m, ref = build(cfg, seed=99)
    prompt = [1, 2, 3, 4, 5, 6]
    gen = m.generate_greedy(prompt, 8)
    want, logits = [], ref.forward_with_cache(prompt)
    for _ in range(8):
        t = argmax(logits)
        want.append(t)
        logits = ref.forward_with_cache([t])
    assert gen.tolist() == want


def test_f16_kv_cache(rq, gpu):
    # the f16 cache rounds K and V to 11 significant bits; against the oracle
    # that stores them rounded the same way the logits meet the f32 tolerance
    cfg = tiny_config(kv_f16=True)
    m, ref = build(cfg)
    prompt = list(range(20, 31))
    assert_close(m.forward_with_cache(prompt), ref.forward_with_cache(prompt))
    for t in (5, 6, 7):
        assert_close(m.decode_step(t), ref.forward_with_cache([t]))


def test_chunked_prefill_matches_single_pass(rq, gpu):
    cfg = tiny_config(max_batch=16)
    m, ref = build(cfg)
    prompt = list(np.random.default_rng(5).integers(0, cfg.vocab, 40))  # 3 chunks of <= 16
    gen = m.generate_greedy(prompt, 3)
    want, logits = [], ref.forward_with_cache(prompt)
    for _ in range(3):
        want.append(argmax(logits))
        logits = ref.forward_with_cache([want[-1]])
    assert gen.tolist() == want


def test_errors(rq, gpu):
    cfg = tiny_config(max_seq=16)
    m, _ = build(cfg)
    with pytest.raises(rq.InvalidData):
        m.forward_with_cache([cfg.vocab])  # out of the embedding
    with pytest.raises(rq.ShapeMismatch):
        m.forward_with_cache([1] * (cfg.max_batch + 1))
    m.forward_with_cache([1] * 10)
    with pytest.raises(rq.InvalidData):
        m.forward_with_cache([1] * 7)  # 10 + 7 > max_seq
    assert m.position == 10


def test_config5_shape_synthetic_weights(rq, gpu):
    # 32 layers, 4096 hidden, 32/8 heads x 128, SwiGLU 14336,
    # vocab 32000, f16 KV up to 2048; seeded synthetic Q4_0 weights
    from rdlquant.llama import LlamaConfig, LlamaModel
    cfg = LlamaConfig()
    m = LlamaModel(cfg)
    m.init_random(0x5EED0005)
    prompt = np.random.default_rng(0x5EED0005).integers(0, cfg.vocab, 128)
    a = m.generate_greedy(prompt, 6)
    assert a.min() >= 0 and a.max() < cfg.vocab
    assert m.position == 128 + 5
    m.reset()
    b = m.generate_greedy(prompt, 6)
    assert a.tolist() == b.tolist()  # deterministic
    # This seeded model is almost blind to its input: its Q4_0 codes are
    # uniform in 0..15, so every weight carries a mean of -d/2 and the
    # residual stream is dominated by that common mode (the logits move by
    # about 2e-5 of 8 from one step to the next).  Logits here therefore
    # check determinism and that the 7B launch shapes agree with each other;
    # oracle parity of this attention geometry is
    # test_config5_attention_path_f16_cache's.
    # (1) Decode steps against a prefill of the same sequence (GEMM and
    # prompt-chunk attention): the paths round differently (GEMV against GEMM
    # sums, K / V from either rounded to f16).
    m.reset()
    seq = list(prompt) + a[:-1].tolist()
    m.forward_with_cache(prompt)
    dec = [m.decode_step(t) for t in a[:-1].tolist()]
    m.reset()
    m.forward_with_cache(seq[:cfg.max_batch])
    pre = m.forward_with_cache(seq[cfg.max_batch:])
    assert np.all(np.isfinite(pre)) and np.all(np.isfinite(dec[-1]))
    scale = np.abs(pre).max()
    err = np.abs(dec[-1].astype(np.float64) - pre).max()
    print(f"  7B decode vs prefill logits: max err {err:.3g} of max |logit| {scale:.3g}")
    assert err <= 1e-3 * scale, (err, scale)
    # (2) The fused decode launch (q/k/v + attention + o at 4 query heads per
    # KV head, head dim 128, f16 cache) against the three separate launches,
    # bit for bit, at every step.
    c0 = m.path_counts()
    m.reset()
    m.set_fused_attention(False)
    m.forward_with_cache(prompt)
    dec3 = [m.decode_step(t) for t in a[:-1].tolist()]
    m.set_fused_attention(True)
    assert m.path_counts()["fused_decode"] == c0["fused_decode"]
    for i, (f, u) in enumerate(zip(dec, dec3)):
        assert np.array_equal(f.view(np.uint32), u.view(np.uint32)), f"step {i}"
    # (3) Each layer's down projection leading the next layer's fused launch
    # (level 2; one workgroup a CU, the 256 down workgroups fill the device):
    # the same logits, bit for bit.
    m.reset()
    m.set_fused_attention(2)
    m.forward_with_cache(prompt)
    dec2 = [m.decode_step(t) for t in a[:-1].tolist()]
    m.set_fused_attention(1)
    assert m.path_counts()["fused_down"] - c0["fused_down"] == len(dec2) * (cfg.n_layers - 1)
    for i, (f, u) in enumerate(zip(dec, dec2)):
        assert np.array_equal(f.view(np.uint32), u.view(np.uint32)), f"step {i} (level 2)"


@pytest.mark.parametrize("kw", [
    dict(kv_f16=False),                                  # grouped kernel, f32 cache, 2 heads per KV head
    dict(kv_f16=True),                                   # grouped kernel, f16 cache
    dict(kv_f16=False, dim=384, n_heads=6, n_kv_heads=2),  # 3 heads per KV head: per-head kernel
    # head dim 128: f16 rows take the coalesced 16-lane layout (transposed
    # score sums), f32 rows the per-key layout
    dict(kv_f16=True, dim=256, n_heads=2, n_kv_heads=1, head_dim=128),
    dict(kv_f16=False, dim=256, n_heads=2, n_kv_heads=1, head_dim=128),
])
def test_long_context_spans(rq, gpu, kw):
    # more than 512 cached keys: several attention workgroups per row, whose
    # softmax partials the last one to finish combines
    cfg = tiny_config(max_seq=1100, max_batch=128, **kw)
    m, ref = build(cfg, seed=7)
    prompt = np.random.default_rng(11).integers(0, cfg.vocab, 700)
    for c0 in range(0, 700, 128):  # prefill chunks of up to 128 rows (the GEMM path)
        got = m.forward_with_cache(prompt[c0:c0 + 128])
        want = ref.forward_with_cache(prompt[c0:c0 + 128])
    # f16 caches: the oracle rounds K / V alike, so both meet the f32 bar
    assert_close(got, want)
    tok = argmax(want)
    for _ in range(3):  # one-row steps at 700 .. 702 cached keys
        got, want = m.decode_step(tok), ref.forward_with_cache([tok])
        assert_close(got, want)
        tok = argmax(want)
    # graph-replayed greedy steps cross no span boundary differently from eager ones
    gen = m.generate_greedy([tok], 4)
    # f16 caches too: equal tokens unless the oracle's best two are within the bar
    assert_greedy_chain(gen, ref, ref.forward_with_cache([tok]))


@pytest.mark.parametrize("kw,chunks", [
    (dict(kv_f16=False), [8]),                                     # one group of 8 rows, one page
    (dict(kv_f16=True), [9, 70]),                                  # a ragged group; rows crossing a page
    (dict(kv_f16=False, dim=256, n_heads=2, n_kv_heads=1, head_dim=128), [77, 3, 40]),  # 3 rows: per-row kernel
    (dict(kv_f16=True, dim=256, n_heads=2, n_kv_heads=1, head_dim=128), [128, 128]),
    (dict(kv_f16=False, dim=256, n_heads=1, n_kv_heads=1, head_dim=256), [33, 31]),   # head dim 256
    (dict(kv_f16=False, dim=384, n_heads=6, n_kv_heads=2), [128] * 5),  # 32+ rows past 512 keys
    (dict(kv_f16=True), [128] * 4 + [16, 40]),   # 16 rows past 512 keys: per-row kernel; 40 rows: 10 pages
    (dict(kv_f16=True, dim=256, n_heads=1, n_kv_heads=1, head_dim=256), [40, 33]),  # f16, head dim 256
])
def test_prefill_attention_chunks(rq, gpu, kw, chunks):
    """Prompt chunks of 32 rows or more (on the matrix cores with an f16
    cache), and of 8 rows or more whose rows see at most 8 cache pages, take
    the kernels that walk a row group's pages; the rest take the per-row
    kernel.  Every chunk's logits against the oracle."""
    cfg = tiny_config(max_seq=700, max_batch=128, **kw)
    print(f"case prefill chunks {kw} {chunks}", flush=True)
    m, _ = build(cfg, seed=5)
    # the oracle stores K / V rounded to f16 as the f16 cache does, so both
    # cache types meet the f32 tolerance
    ref = LlamaRef(cfg, tiny_weights(cfg, 5)[1], kv_f16=kw["kv_f16"])
    prompt = np.random.default_rng(3).integers(0, cfg.vocab, sum(chunks))
    c0 = 0
    for n in chunks:
        got = m.forward_with_cache(prompt[c0:c0 + n])
        want = ref.forward_with_cache(prompt[c0:c0 + n])
        c0 += n
        assert_close(got, want)
    assert m.position == ref.pos == c0


@pytest.mark.parametrize("out_dtype", [14, 8, 12])
def test_output_matrix_types(rq, gpu, out_dtype):
    """An output matrix in Q6_K / Q8_0 / Q4_K (llama.cpp files keep lm_head in
    Q6_K): prefill, fused decode steps and greedy generation against the
    oracle's forward (the reference dequantizes K-quants at load and runs the
    F32 Linear)."""
    cfg = tiny_config(output_dtype=out_dtype)
    m, ref = build(cfg, seed=4321)
    prompt = [9, 8, 7, 6, 5, 4, 3, 2, 1]
    assert_close(m.forward_with_cache(prompt), ref.forward_with_cache(prompt))
    tok = 12
    for _ in range(4):
        got = m.decode_step(tok)
        want = ref.forward_with_cache([tok])
        assert_close(got, want)
        tok = argmax(want)
    m.reset()
    toks = m.generate_greedy(prompt, 6)
    m.reset()
    eager = [argmax(m.forward_with_cache(prompt))]
    for _ in range(5):
        eager.append(argmax(m.forward_with_cache([eager[-1]])))
    assert list(toks) == eager
    with pytest.raises(rq.DeviceError):
        m.init_random(1)


def mixed_types():
    """Layer 0 all Q4_0 (fused launches); layer 1 as llama.cpp's Q4_K_M mixes
    (q, k Q4_K, v Q6_K: split q/k/v; gate Q4_K, up Q6_K: split gate/up; o
    Q8_0; down Q6_K); layer 2 non-Q4_0 but combined (q/k/v Q8_0, gate/up
    Q4_1, down Q4_K); a Q6_K embedding table and a Q8_0 output matrix."""
    import rdlquant.llama as L
    t = {(L.TOKEN_EMBEDDING, 0): 14, (L.OUTPUT, 0): 8}
    t.update({(L.WQ, 1): 12, (L.WK, 1): 12, (L.WV, 1): 14, (L.WO, 1): 8, (L.W_GATE, 1): 12, (L.W_UP, 1): 14,
              (L.W_DOWN, 1): 14})
    t.update({(L.WQ, 2): 8, (L.WK, 2): 8, (L.WV, 2): 8, (L.W_GATE, 2): 3, (L.W_UP, 2): 3, (L.W_DOWN, 2): 12})
    return t


def build_typed(cfg, types, seed):
    from rdlquant.llama import LlamaModel
    slots, ref_w = tiny_weights(cfg, seed, types=types)
    m = LlamaModel(cfg, types=types)
    for slot, layer, arr in slots:
        m.set_weight(slot, layer, arr)
    return m, LlamaRef(cfg, ref_w, kv_f16=bool(cfg.kv_f16)), slots


@pytest.mark.parametrize("kv_f16", [False, True])
def test_mixed_type_layers(rq, gpu, kv_f16):
    """Fused and per-type layers in one model: prefill (the GEMM and the
    records paths), decode steps and greedy generation against the oracle."""
    cfg = tiny_config(n_layers=3, kv_f16=kv_f16, output_dtype=8)
    m, ref, _ = build_typed(cfg, mixed_types(), 99)
    prompt = [3, 141, 59, 26, 53, 58, 97, 93, 23]
    if kv_f16:  # f16 cache: the oracle rounds K / V alike
        assert_close(m.forward_with_cache(prompt), ref.forward_with_cache(prompt))
        return
    assert_close(m.forward_with_cache(prompt), ref.forward_with_cache(prompt))
    tok = 11
    for _ in range(4):
        got = m.decode_step(tok)
        want = ref.forward_with_cache([tok])
        assert_close(got, want)
        tok = argmax(want)
    m.reset()
    toks = m.generate_greedy(prompt, 6)
    m.reset()
    eager = [argmax(m.forward_with_cache(prompt))]
    for _ in range(5):
        eager.append(argmax(m.forward_with_cache([eager[-1]])))
    assert list(toks) == eager


def test_mixed_type_prompt_chunk_on_the_gemms(rq, gpu):
    """The mixed-type model above with a 40-row prompt chunk: layer 0's Q4_0
    GEMMs, layer 1's [Wq; Wk] (Q4_K), Q6_K v, Q8_0 o and split gate (Q4_K) /
    up (Q6_K) / down (Q6_K) on the tile GEMM, layer 2's Q8_0 q/k/v with the
    RMSNorm in its x prep, Q4_1 gate/up with the SwiGLU folded into the Q4_K
    down's x prep; then decode steps and greedy generation, against the
    oracle."""
    cfg = tiny_config(n_layers=3, output_dtype=8, max_batch=40, max_seq=64)
    m, ref, _ = build_typed(cfg, mixed_types(), 101)
    prompt = [int(v) for v in np.random.default_rng(41).integers(0, cfg.vocab, size=40)]
    check_typed_model(m, ref, prompt, 17, steps=2)


def check_typed_model(m, ref, prompt, tok, steps=4):
    """Prefill (rows four at a time through the fused GEMVs), decode steps and
    greedy generation against the oracle's forward."""
    assert_close(m.forward_with_cache(prompt), ref.forward_with_cache(prompt))
    for _ in range(steps):
        got = m.decode_step(tok)
        want = ref.forward_with_cache([tok])
        assert_close(got, want)
        tok = argmax(want)
    m.reset()
    toks = m.generate_greedy(prompt, 5)
    m.reset()
    eager = [argmax(m.forward_with_cache(prompt))]
    for _ in range(4):
        eager.append(argmax(m.forward_with_cache([eager[-1]])))
    assert list(toks) == eager


def q4_k_m_mix():
    import rdlquant.llama as L
    t = {(L.TOKEN_EMBEDDING, 0): 12, (L.OUTPUT, 0): 14}
    for layer in range(2):
        for slot in (L.WQ, L.WK, L.WV, L.WO, L.W_GATE, L.W_UP, L.W_DOWN):
            t[(slot, layer)] = 12
    t[(L.WV, 0)] = t[(L.W_DOWN, 0)] = 14
    return t


def test_q4_k_m_layers(rq, gpu):
    """llama.cpp's Q4_K_M mix: layer 0 with Q6_K attn_v / ffn_down (split q/k/v,
    RMSNorm in each part's GEMV; gate/up combined Q4_K with the SwiGLU in the
    GEMV; residual adds in the o / down GEMVs), layer 1 all Q4_K (one q/k/v
    launch), Q4_K embedding, Q6_K output matrix (final norm in its GEMV)."""
    cfg = tiny_config(output_dtype=14)
    m, ref, _ = build_typed(cfg, q4_k_m_mix(), 2024)
    check_typed_model(m, ref, [5, 17, 33, 2, 250, 7, 91, 64, 8, 1], 31)


@pytest.mark.parametrize("kv_f16", [False, True])
def test_q4_k_m_prompt_chunks_on_the_gemm(rq, gpu, kv_f16):
    """The Q4_K_M mix above with a 56-row prompt chunk: its Q4_K
    matrices take the tile GEMM (layer 1: one q/k/v GEMM with the RMSNorm in
    its x prep and RoPE after it, o and down adding into the residual rows,
    gate/up with the SwiGLU folded into down's x prep; layer 0: the q and k
    parts and gate/up on the GEMM beside Q6_K v and down on the GEMVs), then
    decode steps and greedy generation, against the oracle."""
    cfg = tiny_config(output_dtype=14, kv_f16=kv_f16, max_batch=56, max_seq=96)
    m, ref, _ = build_typed(cfg, q4_k_m_mix(), 2025 + kv_f16)
    prompt = [int(v) for v in np.random.default_rng(56).integers(0, cfg.vocab, size=56)]
    check_typed_model(m, ref, prompt, 31, steps=2)


def test_q6_k_prompt_chunk_on_the_gemm(rq, gpu):
    """Every layer matrix Q6_K with a 40-row prompt chunk: one q/k/v GEMM with
    the RMSNorm in its x prep, gate/up with the SwiGLU folded into down's x
    prep, residual adds in the o / down stores; then decode steps on the Q6_K
    GEMVs, against the oracle."""
    import rdlquant.llama as L
    t = {(slot, layer): 14 for layer in range(2)
         for slot in (L.WQ, L.WK, L.WV, L.WO, L.W_GATE, L.W_UP, L.W_DOWN)}
    t[(L.OUTPUT, 0)] = 8
    cfg = tiny_config(output_dtype=8, max_batch=40, max_seq=64)
    m, ref, _ = build_typed(cfg, t, 78)
    prompt = [int(v) for v in np.random.default_rng(40).integers(0, cfg.vocab, size=40)]
    check_typed_model(m, ref, prompt, 12, steps=2)


def test_wide_q4_k_prompt_on_the_gemm(rq, gpu):
    """A 24-row prompt chunk over dim 4352 / ffn 4608 Q4_K layers: the tile
    GEMM at 17 super-blocks a row (chunks not dividing them)."""
    import rdlquant.llama as L
    t = {(slot, 0): 12 for slot in (L.WQ, L.WK, L.WV, L.WO, L.W_GATE, L.W_UP, L.W_DOWN)}
    t[(L.OUTPUT, 0)] = 12
    cfg = tiny_config(dim=4352, n_layers=1, n_heads=34, n_kv_heads=2, head_dim=128, ffn_dim=4608, vocab=256,
                      max_seq=32, max_batch=24, output_dtype=12)
    m, ref, _ = build_typed(cfg, t, 4353)
    prompt = [int(v) for v in np.random.default_rng(24).integers(0, cfg.vocab, size=24)]
    check_typed_model(m, ref, prompt, 7, steps=1)


def test_q6_k_combined_layers(rq, gpu):
    """Every layer matrix Q6_K: one q/k/v launch with the RMSNorm prologue,
    gate/up rows combined with the SwiGLU epilogue, residual epilogues, all in
    the Q6_K kernel; a Q8_0 output matrix behind a separate norm."""
    import rdlquant.llama as L
    t = {(L.OUTPUT, 0): 8}
    for layer in range(2):
        for slot in (L.WQ, L.WK, L.WV, L.WO, L.W_GATE, L.W_UP, L.W_DOWN):
            t[(slot, layer)] = 14
    cfg = tiny_config(output_dtype=8)
    m, ref, _ = build_typed(cfg, t, 77)
    check_typed_model(m, ref, [9, 3, 100, 200, 300, 44], 12)


@pytest.mark.parametrize("qtype", [12, 14])
def test_k_quant_rope_epilogue_f16_cache(rq, gpu, qtype):
    """Combined Q4_K / Q6_K q/k/v with the RoPE epilogue writing an f16 cache:
    prefill (rows four at a time, positions 0..8) and decode steps against
    the oracle with K / V stored rounded to f16, at the f32 tolerance."""
    import rdlquant.llama as L
    t = {(slot, layer): qtype for layer in range(2)
         for slot in (L.WQ, L.WK, L.WV, L.WO, L.W_GATE, L.W_UP, L.W_DOWN)}
    cfg = tiny_config(kv_f16=True)
    m, ref, _ = build_typed(cfg, t, 515 + qtype)
    got, want = m.forward_with_cache([7, 70, 170, 2, 9, 31, 44, 5, 300]), ref.forward_with_cache(
        [7, 70, 170, 2, 9, 31, 44, 5, 300])
    assert_close(got, want)
    tok = argmax(want)
    for _ in range(3):
        got, want = m.decode_step(tok), ref.forward_with_cache([tok])
        assert_close(got, want)
        tok = argmax(want)


def test_wide_k_quant_layers(rq, gpu):
    """Rows longer than 4096 (dim 4352, ffn 4608): the split-K Q4_K kernel with
    the RMSNorm prologue and the SwiGLU / residual epilogues (layer 0), the
    Q6_K kernel split over four waves (layer 1)."""
    import rdlquant.llama as L
    t = {(L.TOKEN_EMBEDDING, 0): 12, (L.OUTPUT, 0): 12}
    for slot in (L.WQ, L.WK, L.WV, L.WO, L.W_GATE, L.W_UP, L.W_DOWN):
        t[(slot, 0)] = 12
        t[(slot, 1)] = 14
    cfg = tiny_config(dim=4352, n_heads=34, n_kv_heads=2, head_dim=128, ffn_dim=4608, vocab=256, max_seq=32,
                      output_dtype=12)
    m, ref, _ = build_typed(cfg, t, 4352)
    check_typed_model(m, ref, [1, 2, 3, 4, 5, 6], 7, steps=2)


def test_typed_create_rejects(rq, gpu):
    import rdlquant.llama as L
    from rdlquant.llama import LlamaModel
    cfg = tiny_config(ffn_dim=288)
    with pytest.raises(rq.DeviceError) as e:  # K-quant down over ffn 288
        LlamaModel(cfg, types={(L.W_DOWN, 0): 12})
    assert "256" in str(e.value)
    with pytest.raises(rq.DeviceError):
        LlamaModel(tiny_config(), types={(L.WQ, 1): 13})  # Q5_K is not resident
    m = LlamaModel(tiny_config(), types={(L.WO, 0): 8})
    with pytest.raises(rq.DeviceError):
        m.init_random(1)


def config5_attention_config(**kw):
    """BASELINE config 5's attention geometry (hidden 4096, 32 query heads over
    8 KV heads of dim 128, f16 cache) on two layers with a narrow FFN and
    vocabulary, so that the oracle runs in seconds.  Its tests use centered
    Q4_0 codes, which keep the logits sensitive to the attention (a dropped
    current key moves most of them past the parity bar; with BASELINE's codes
    it moves none: test_oracle_llama.py)."""
    base = dict(dim=4096, n_layers=2, n_heads=32, n_kv_heads=8, head_dim=128, ffn_dim=512, vocab=320,
                max_seq=1024, max_batch=128, kv_f16=True)
    base.update(kw)
    return tiny_config(**base)


def test_config5_attention_path_f16_cache(rq, gpu):
    """Config 5's own attention path against the oracle: 128-row prompt chunks
    on the matrix-core prompt attention (prefill_attention_mfma_kernel<128>)
    and one-row steps on the fused q/k/v + attention + o launch
    (qkv_attention_kernel<_Float16, 128>), at 4 query heads per KV head, over
    128-131 cached keys (one span) and 644-647 (two spans and their combine),
    then graph-replayed greedy steps.  Logits within 1e-3 rel + 1e-4 abs of
    LlamaRef(kv_f16=True) and within the f16-cache bound of the reference's
    f32 cache (LlamaRef(kv_f16=False)); greedy tokens equal to the oracle's
    (repeat_kv, ops.rs:955-995; attention.rs:401-446)."""
    cfg = config5_attention_config()
    print("case config-5 attention path, f16 cache, 32/8 x 128, dim 4096", flush=True)
    m, ref = build(cfg, seed=505, centered=True)
    ref32 = LlamaRef(cfg, ref.w, kv_f16=False)
    prompt = np.random.default_rng(5005).integers(0, cfg.vocab, 640)

    def step(tokens):
        got = m.forward_with_cache(tokens)
        want, want32 = ref.forward_with_cache(tokens), ref32.forward_with_cache(tokens)
        assert_close(got, want)
        assert_within_f16_cache_bound(got, want32)
        return want

    c0 = m.path_counts()
    want = step(prompt[:128])
    c1 = m.path_counts()
    assert c1["prefill_mfma"] - c0["prefill_mfma"] == cfg.n_layers
    tok = argmax(want)
    for _ in range(4):  # 128 .. 131 cached keys: one span
        want = step([tok])
        tok = argmax(want)
    c2 = m.path_counts()
    assert c2["fused_decode"] - c1["fused_decode"] == 4 * cfg.n_layers
    assert c2["attention"] == c1["attention"]  # no unfused decode attention
    feed = prompt[128:640]
    for i in range(0, feed.size, 128):  # more prompt after the decode steps: 132 .. 643
        want = step(feed[i:i + 128])
    tok = argmax(want)
    for _ in range(4):  # 644 .. 647 cached keys: two spans
        want = step([tok])
        tok = argmax(want)
    c3 = m.path_counts()
    assert c3["fused_decode"] - c2["fused_decode"] == 4 * cfg.n_layers
    assert c3["prefill_mfma"] - c2["prefill_mfma"] == 4 * cfg.n_layers
    assert c3["attention"] == c0["attention"] and c3["prefill_rows"] == c0["prefill_rows"]
    gen = m.generate_greedy([tok], 6)  # prefill of one row, then 5 graph replays of the fused step
    assert m.position == ref.pos + 6
    assert_greedy_chain(gen, ref, ref.forward_with_cache([tok]))


def test_config5_f16_kernels_against_f32_reference(rq, gpu):
    """Every f16-cache attention kernel at config 5's grouping against the
    reference's f32 KVCache, within the f16-cache bound, and against the
    oracle that rounds K / V alike at the f32 bar: a 128-row chunk (matrix
    cores), a 16-row chunk over 3 pages (a wave a row, LDS-staged pages), a
    3-row chunk (the per-row span kernel) and fused one-row steps."""
    cfg = config5_attention_config(max_seq=256)
    print("case config-5 f16 kernels vs f32 cache", flush=True)
    m, ref = build(cfg, seed=606, centered=True)
    ref32 = LlamaRef(cfg, ref.w, kv_f16=False)
    prompt = np.random.default_rng(6006).integers(0, cfg.vocab, 147)
    c0 = m.path_counts()
    c_prev, want = c0, None
    for rows, kernel in ((128, "prefill_mfma"), (16, "prefill_rows"), (3, "attention")):
        toks = prompt[ref.pos:ref.pos + rows]
        got = m.forward_with_cache(toks)
        want, want32 = ref.forward_with_cache(toks), ref32.forward_with_cache(toks)
        assert_close(got, want)
        assert_within_f16_cache_bound(got, want32)
        c = m.path_counts()
        assert c[kernel] - c_prev[kernel] == cfg.n_layers, (kernel, c)
        c_prev = c
    tok = argmax(want)
    for _ in range(3):
        got = m.decode_step(tok)
        want, want32 = ref.forward_with_cache([tok]), ref32.forward_with_cache([tok])
        assert_close(got, want)
        assert_within_f16_cache_bound(got, want32)
        tok = argmax(want)
    assert m.path_counts()["fused_decode"] - c_prev["fused_decode"] == 3 * cfg.n_layers


@pytest.mark.parametrize("kv_f16,hd", [(True, 128), (True, 64), (False, 64)])
def test_fused_decode_two_rows_a_wave(rq, gpu, kv_f16, hd):
    """Hidden sizes past 4096 (4352: 136 blocks a row) give the fused q/k/v +
    attention launch two rows a wave and four block columns a lane
    (qkv_attention_kernel<KV, HD, 2, 4>): bit-equal to the q/k/v launch
    followed by the attention and o launches, and within the bar of the
    oracle (f16 caches: K / V rounded alike), at 64+ cached keys.  Also with
    the first layer's down projection leading the second layer's launch
    (level 2): 272 down workgroups ahead of 384 q/k/v workgroups that poll
    its output (with head_dim 64 and an f16 cache two workgroups share a CU,
    so the pollers start while the down workgroups still run)."""
    nh = 4096 // hd
    cfg = tiny_config(dim=4352, n_layers=2, n_heads=nh, n_kv_heads=nh // 4, head_dim=hd, ffn_dim=512,
                      vocab=320, max_seq=128, max_batch=64, kv_f16=kv_f16)
    print(f"case fused decode R=2 kv_f16={kv_f16} hd={hd}", flush=True)
    a, ref = build(cfg, seed=4352, centered=True)
    b, _ = build(cfg, seed=4352, centered=True)
    c, _ = build(cfg, seed=4352, centered=True)
    b.set_fused_attention(False)
    c.set_fused_attention(2)
    prompt = np.random.default_rng(4353).integers(0, cfg.vocab, 64)
    la, lb, lc = a.forward_with_cache(prompt), b.forward_with_cache(prompt), c.forward_with_cache(prompt)
    want = ref.forward_with_cache(prompt)
    assert_close(la, want)
    assert np.array_equal(la, lb) and np.array_equal(la, lc)
    c0, d0 = a.path_counts(), c.path_counts()
    tok = argmax(want)
    for _ in range(4):
        la, lb, lc = a.decode_step(tok), b.decode_step(tok), c.decode_step(tok)
        want = ref.forward_with_cache([tok])
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
        assert np.array_equal(la.view(np.uint32), lc.view(np.uint32))
        assert_close(la, want)
        tok = argmax(want)
    assert a.path_counts()["fused_decode"] - c0["fused_decode"] == 4 * cfg.n_layers
    assert c.path_counts()["fused_down"] - d0["fused_down"] == 4 * (cfg.n_layers - 1)
    assert b.path_counts()["fused_decode"] == 0
    ga = a.generate_greedy([tok], 5).tolist()
    assert ga == b.generate_greedy([tok], 5).tolist() == c.generate_greedy([tok], 5).tolist()


def test_config5_head_grouping_against_oracle(rq, gpu):
    """BASELINE config 5's attention grouping (32 query heads over 8 KV heads
    of dim 128, hidden 4096) on a 2-layer model with an f32 cache: prefill
    and decode logits within the bar of LlamaRef, greedy tokens equal."""
    cfg = tiny_config(dim=4096, n_layers=2, n_heads=32, n_kv_heads=8, head_dim=128, ffn_dim=512,
                      vocab=320, max_seq=64, kv_f16=False)
    print("case config-5 grouping 32/8 x 128, 2 layers", flush=True)
    m, ref = build(cfg, seed=505)
    prompt = [3, 141, 59, 26, 53, 58, 97, 93, 23]
    assert_close(m.forward_with_cache(prompt), ref.forward_with_cache(prompt))
    tok = 17
    for _ in range(4):
        got = m.decode_step(tok)
        want = ref.forward_with_cache([tok])
        assert_close(got, want)
        tok = argmax(want)
    m.reset()
    gen = m.generate_greedy(prompt, 5)
    ref2 = LlamaRef(cfg, ref.w, kv_f16=bool(cfg.kv_f16))
    want_toks, logits = [], ref2.forward_with_cache(prompt)
    for _ in range(5):
        want_toks.append(argmax(logits))
        logits = ref2.forward_with_cache([want_toks[-1]])
    assert gen.tolist() == want_toks


@pytest.mark.parametrize("kv_f16", [False, True])
def test_long_context_four_spans(rq, gpu, kv_f16):
    """1,900-1,906 cached keys at head dim 128: four 512-key attention
    workgroups per row whose partials the last one to finish combines."""
    cfg = tiny_config(dim=256, n_heads=2, n_kv_heads=1, head_dim=128, max_seq=2048, max_batch=128,
                      kv_f16=kv_f16)
    print(f"case four spans kv_f16={kv_f16}", flush=True)
    m, ref = build(cfg, seed=19)
    prompt = np.random.default_rng(23).integers(0, cfg.vocab, 1900)
    for c0 in range(0, 1900, 128):
        got = m.forward_with_cache(prompt[c0:c0 + 128])
        want = ref.forward_with_cache(prompt[c0:c0 + 128])

    # f16 caches: the oracle rounds K / V alike, so both meet the f32 bar
    assert_close(got, want)
    tok = argmax(want)
    for _ in range(3):
        got, want = m.decode_step(tok), ref.forward_with_cache([tok])
        assert_close(got, want)
        tok = argmax(want)
    gen = m.generate_greedy([tok], 3)
    assert_greedy_chain(gen, ref, ref.forward_with_cache([tok]))
    assert m.position == 1900 + 3 + 3


@pytest.mark.parametrize("kv_f16", [False, True])
def test_paged_cache_shuffled_pages(rq, gpu, kv_f16):
    """The KV cache through a shuffled page table (physical page order
    reversed and interleaved): 1,900+ cached keys cross 30 page boundaries and
    four attention spans; prefill, eager decode steps and graph-replayed
    greedy steps against the oracle, whose cache is contiguous."""
    cfg = tiny_config(dim=256, n_heads=2, n_kv_heads=1, head_dim=128, max_seq=2048, max_batch=128,
                      kv_f16=kv_f16)
    print(f"case paged cache kv_f16={kv_f16}", flush=True)
    m, ref = build(cfg, seed=29)
    ps, n_pages = m.kv_pages()
    assert ps == 64 and n_pages == 32
    table = np.random.default_rng(31).permutation(n_pages).astype(np.int32)
    m.set_kv_page_table(table)
    prompt = np.random.default_rng(37).integers(0, cfg.vocab, 1900)
    for c0 in range(0, 1900, 128):
        got = m.forward_with_cache(prompt[c0:c0 + 128])
        want = ref.forward_with_cache(prompt[c0:c0 + 128])

    # f16 caches: the oracle rounds K / V alike, so both meet the f32 bar
    assert_close(got, want)
    tok = argmax(want)
    for _ in range(2):
        got, want = m.decode_step(tok), ref.forward_with_cache([tok])
        assert_close(got, want)
        tok = argmax(want)
    gen = m.generate_greedy([tok], 3)
    assert_greedy_chain(gen, ref, ref.forward_with_cache([tok]))


def test_paged_cache_same_tokens_under_any_table(rq, gpu):
    # the page table changes where rows live, not what attention computes:
    # greedy tokens over 300 positions (5 pages) agree bit for bit
    cfg = tiny_config(max_seq=320, max_batch=64)
    m, _ = build(cfg, seed=41)
    prompt = list(np.random.default_rng(43).integers(0, cfg.vocab, 100))
    base = m.generate_greedy(prompt, 200)
    _, n_pages = m.kv_pages()
    for seed in (1, 2):
        m.reset()
        m.set_kv_page_table(np.random.default_rng(seed).permutation(n_pages))
        assert m.generate_greedy(prompt, 200).tolist() == base.tolist()


def test_paged_cache_table_errors(rq, gpu):
    cfg = tiny_config(max_seq=200)
    m, _ = build(cfg)
    _, n_pages = m.kv_pages()
    assert n_pages == 4  # ceil(200 / 64)
    with pytest.raises(rq.ShapeMismatch):
        m.set_kv_page_table([0, 1, 2])
    with pytest.raises(rq.InvalidData):
        m.set_kv_page_table([0, 1, 1, 3])  # not a permutation
    with pytest.raises(rq.InvalidData):
        m.set_kv_page_table([0, 1, 2, 4])  # out of range
    m.forward_with_cache([1, 2, 3])
    with pytest.raises(rq.InvalidData):
        m.set_kv_page_table([3, 2, 1, 0])  # cache not empty
    m.reset()
    m.set_kv_page_table([3, 2, 1, 0])


@pytest.mark.parametrize("kw,n_prompt", [
    (dict(kv_f16=False), 40),                                               # f32 cache, head dim 64
    (dict(kv_f16=True), 40),                                                # f16 cache, head dim 64
    (dict(kv_f16=True, dim=256, n_heads=2, n_kv_heads=1, head_dim=128), 40),  # f16, head dim 128
    (dict(kv_f16=True, dim=256, n_heads=2, n_kv_heads=1, head_dim=128, max_seq=1100, max_batch=128), 1000),
    (dict(kv_f16=False, dim=512, n_heads=8, n_kv_heads=2, head_dim=64, max_seq=700, max_batch=128), 600),
    (dict(kv_f16=True, dim=256, n_heads=2, n_kv_heads=1, head_dim=64), 40),   # o input 128 < dim 256
    (dict(kv_f16=False, dim=128, n_heads=4, n_kv_heads=2, head_dim=64), 40),  # o input 256 > dim 128
])
def test_fused_attention_equals_two_launches(rq, gpu, kw, n_prompt):
    """Decode steps with the attention fused into the q/k/v launch, with and
    without the previous layer's down projection leading that launch, give
    the same logits, bit for bit, as the q/k/v launch followed by the
    attention launch (eager steps and graph-replayed greedy steps; one to two
    spans of 512 keys)."""
    cfg = tiny_config(**kw)
    print(f"case fused attention {kw} prompt {n_prompt}", flush=True)
    a, _ = build(cfg, seed=61)
    b, _ = build(cfg, seed=61)
    c, _ = build(cfg, seed=61)
    b.set_fused_attention(False)
    c.set_fused_attention(2)
    prompt = np.random.default_rng(67).integers(0, cfg.vocab, n_prompt)
    for c0 in range(0, n_prompt, cfg.max_batch):
        la = a.forward_with_cache(prompt[c0:c0 + cfg.max_batch])
        lb = b.forward_with_cache(prompt[c0:c0 + cfg.max_batch])
        lc = c.forward_with_cache(prompt[c0:c0 + cfg.max_batch])
    assert np.array_equal(la, lb) and np.array_equal(la, lc)
    tok = int(np.argmax(la))
    p0 = c.path_counts()
    for _ in range(5):
        la, lb, lc = a.decode_step(tok), b.decode_step(tok), c.decode_step(tok)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
        assert np.array_equal(la.view(np.uint32), lc.view(np.uint32))
        tok = int(np.argmax(la))
    p1 = c.path_counts()
    assert p1["fused_down"] - p0["fused_down"] == 5 * (cfg.n_layers - 1)
    assert a.path_counts()["fused_down"] == 0
    ga = a.generate_greedy([tok], 6).tolist()
    assert ga == b.generate_greedy([tok], 6).tolist() == c.generate_greedy([tok], 6).tolist()


NATIVE_KIND = {"q4": "q4_native", "q4_1": "q4_1_native"}
LAYER_MATS = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")


def native_ref(cfg, w, layers, kv_f16):
    """LlamaRef with Linear::use_native_q4 on the given layers: their Q4_0 /
    Q4_1 matrices take matmul_f32_q4_native / _q4_1_native (linear.rs:128-150)."""
    w = dict(w)
    kinds = dict(w.get("kinds", {}))
    for layer in layers:
        for name in LAYER_MATS:
            k = kinds.get((name, layer), "q4")
            if k in NATIVE_KIND:
                kinds[(name, layer)] = NATIVE_KIND[k]
    w["kinds"] = kinds
    return LlamaRef(cfg, w, kv_f16=kv_f16)


# Q8_0 activation quantization (quantize.rs:326-394) is discontinuous: each
# block's scale amax / 127 is rounded to f16 and each code to the nearest
# integer, so where an input sits within float noise (about 1e-7 of its size)
# of such a rounding tie, two correct implementations whose float sums differ
# in the last bit take neighbouring scales or codes, and the layers after
# carry the step on.  On MI355X such a tie moved the logits of one case in
# several dozen by up to 3.1e-3 of the largest one.  Each case below starts
# from an empty cache, so a tie touches that case only: every case holds the
# parity bar but at most one in six, which must stay within NATIVE_TIE_BOUND
# (a mistake in the native algorithm -- float activations, an unrounded
# scale, a dropped block -- misses the bar in every case).
NATIVE_TIE_BOUND = 1e-2


def native_cases(m, cfg, w, layers, kv_f16, prompt, extra):
    """(name, GPU logits, oracle logits) of independent cases, each from an
    empty cache: the prefill of prompt + extra[:j] (native GEMM rows), then
    one decode step of extra[j] (the native GEMV)."""
    for j, tok in enumerate(extra):
        seq = list(prompt) + list(extra[:j])
        m.reset()
        ref = native_ref(cfg, w, layers, kv_f16)
        yield f"prefill of {len(seq)}", m.forward_with_cache(seq), ref.forward_with_cache(seq)
        yield f"decode at {len(seq)}", m.decode_step(tok), ref.forward_with_cache([tok])


def within_bar(got, want):
    return bool(np.all(np.abs(got - want) <= ATOL + RTOL * np.abs(want)))


def assert_native_cases(cases):
    ties, n = [], 0
    for name, got, want in cases:
        n += 1
        if within_bar(got, want):
            continue
        worst = float(np.abs(got - want).max() / np.abs(want).max())
        assert worst <= NATIVE_TIE_BOUND, (name, worst)
        ties.append((name, worst))
    print(f"  {n - len(ties)}/{n} cases within the bar; Q8_0 ties: {ties}")
    assert len(ties) <= n // 6, ties


@pytest.mark.parametrize("kv_f16,layer", [(False, -1), (True, -1), (False, 1)])
def test_native_q4_layers_against_oracle(rq, gpu, kv_f16, layer):
    """TransformerBlock::set_native_q4_matmul (transformer_block.rs:248-255) on
    every layer (as gemma3_gguf.rs:126-128) or on one: prompt rows through the
    native GEMM (int8 matrix cores on the Q8_0 codes), decode steps through
    the native GEMV, against the oracle whose layers use
    matmul_f32_q4_native; most float-mode logits sit outside the bar from
    them (the activation quantization shows)."""
    cfg = tiny_config(kv_f16=kv_f16)
    print(f"case native q4 layers kv_f16={kv_f16} layer={layer}", flush=True)
    m, ref_float = build(cfg, seed=808, centered=True)
    layers = range(cfg.n_layers) if layer < 0 else [layer]
    m.set_native_q4_matmul(True, layer)
    prompt = [3, 141, 59, 26, 53, 58, 97, 93, 23]
    extra = [73, 289, 289, 271, 227, 164]
    # the float path's logits sit outside the bar for most entries
    got = m.forward_with_cache(prompt)
    f = ref_float.forward_with_cache(prompt)
    assert np.count_nonzero(np.abs(got - f) > ATOL + RTOL * np.abs(f)) > f.size // 2
    c0 = m.path_counts()
    assert_native_cases(native_cases(m, cfg, ref_float.w, layers, kv_f16, prompt, extra))
    # native layers leave the fused decode launch; the others keep it
    fused_layers = 0 if layer < 0 else cfg.n_layers - 1
    assert m.path_counts()["fused_decode"] - c0["fused_decode"] == len(extra) * fused_layers
    m.reset()
    ref = native_ref(cfg, ref_float.w, layers, kv_f16)
    want = ref.forward_with_cache(prompt)
    gen = m.generate_greedy(prompt, 5)
    assert_greedy_chain(gen, ref, want, bar=NATIVE_TIE_BOUND)


def test_native_q4_1_layer(rq, gpu):
    """A Q4_1 layer (the Linear dispatch's Q4_1 branch, linear.rs:137-153)
    with native Q4 on: matmul_f32_q4_1_native through the decoder."""
    import rdlquant.llama as L
    t = {(s, 1): 3 for s in (L.WQ, L.WK, L.WV, L.WO, L.W_GATE, L.W_UP, L.W_DOWN)}
    cfg = tiny_config()
    m, ref_float, _ = build_typed(cfg, t, 909)
    m.set_native_q4_matmul(True)
    assert_native_cases(native_cases(m, cfg, ref_float.w, range(cfg.n_layers), False,
                                     [5, 17, 33, 2, 250, 7, 91, 64, 8, 1], [31, 4, 200, 77]))


def test_native_q4_switch_errors(rq, gpu):
    m, _ = build(tiny_config())
    with pytest.raises(rq.InvalidData):
        m.set_native_q4_matmul(True, 2)  # 2 layers
    m.set_native_q4_matmul(False, 1)
