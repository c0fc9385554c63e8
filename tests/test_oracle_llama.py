"""Pins of the decoder oracle (CPU): RoPE tables and RMSNorm against closed
forms, argmax against the reference's tie and NaN rules, and the cached
decode against a full causal pass of the same oracle."""
import numpy as np
import pytest

from oracle import oracle as orc
from oracle.llama_ref import LlamaRef, argmax

from llama_fixtures import tiny_config, tiny_weights


def test_rope_tables_closed_form():
    c, s = orc.rope_tables(128, 64, 10000.0)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)  # pos 0: angle 0
    i = np.arange(64, dtype=np.float64)
    freq = 1.0 / 10000.0 ** (2.0 * i / 128.0)
    ang = np.arange(64, dtype=np.float64)[:, None] * freq[None]
    # f32 angle rounding: |angle| < 64 -> error below 64 * 2^-24 in the argument
    assert np.max(np.abs(c - np.cos(ang))) < 1e-5
    assert np.max(np.abs(s - np.sin(ang))) < 1e-5
    assert np.allclose(c ** 2 + s ** 2, 1.0, atol=1e-6)


@pytest.mark.parametrize("dim", [4096, 24, 40, 7, 256])
def test_rms_norm_row_closed_form(dim):
    rng = np.random.default_rng(dim)
    x = rng.standard_normal((3, dim)).astype(np.float32) * 3
    g = rng.standard_normal(dim).astype(np.float32)
    got = orc.rms_norm(x, g, 1e-5)
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd ** 2).mean(axis=1, keepdims=True) + 1e-5) * g
    assert np.allclose(got, want, rtol=2e-6, atol=1e-6)


def test_rms_norm_planted_eps_is_visible():
    # a dropped eps must fail this pin: near-zero rows make it dominant
    x = np.full((1, 64), 1e-4, np.float32)
    g = np.ones(64, np.float32)
    got = orc.rms_norm(x, g, 1e-5)
    assert abs(got[0, 0] - 1e-4 / np.sqrt(1e-8 + 1e-5)) < 1e-6
    assert abs(got[0, 0] - 1.0) > 0.5


def test_argmax_rules():
    assert argmax([1.0, 3.0, 3.0, 2.0]) == 1           # first maximum wins
    assert argmax([np.nan, 2.0, np.nan, 5.0]) == 3     # NaN never wins
    assert argmax([np.nan, np.nan]) == 0               # all NaN -> 0
    assert argmax([-np.inf, -np.inf]) == 0
    r = np.random.default_rng(0).standard_normal(1000).astype(np.float32)
    assert argmax(r) == int(np.argmax(r))


def test_cached_decode_matches_full_causal_pass():
    # token-by-token decode through the cache == the last row of one causal pass
    cfg = tiny_config(n_layers=1)
    _, ref_w = tiny_weights(cfg, seed=77)
    toks = [5, 17, 250, 3, 99, 42, 7]
    a = LlamaRef(cfg, ref_w)
    for t in toks:
        step = a.forward_with_cache([t])
    b = LlamaRef(cfg, ref_w)
    full = b.forward_with_cache(toks)
    assert np.allclose(step, full, rtol=1e-4, atol=1e-5)
    # and the cache positions advanced alike
    assert a.pos == b.pos == len(toks)


def test_f16_cache_rows_are_the_nearest_halves():
    # kv_f16: every stored K / V value is an f16 value, the nearest one to the
    # f32 row (within half an f16 spacing), and the rounding reaches the logits
    cfg = tiny_config(n_layers=1)
    _, ref_w = tiny_weights(cfg, seed=78)
    toks = [9, 200, 31, 4]
    a = LlamaRef(cfg, ref_w)
    b = LlamaRef(cfg, ref_w, kv_f16=True)
    la, lb = a.forward_with_cache(toks), b.forward_with_cache(toks)
    for kv in (0, 1):
        v32 = a.kv[0][kv][:, :len(toks)]
        v16 = b.kv[0][kv][:, :len(toks)]
        assert np.array_equal(v16.astype(np.float16).astype(np.float32), v16)
        half = np.spacing(np.abs(v32).astype(np.float16)).astype(np.float32) / 2
        assert np.all(np.abs(v16 - v32) <= half)
        assert not np.array_equal(v16, v32)
    assert not np.array_equal(la, lb)
    assert np.allclose(la, lb, rtol=1e-2, atol=1e-2 * np.abs(la).max())


# ---- closed-form pins of the pieces LlamaRef composes ---------------------------------------
from oracle import llama_ref as LR  # noqa: E402


@pytest.mark.parametrize("hd,pos", [(8, 3), (128, 37), (64, 0)])
def test_rope_unit_vectors_rotate_half_split_pairs(hd, pos):
    # rope.rs:189-190: element i pairs with i + D/2 (not 2i / 2i+1), and the
    # pair rotates by pos * theta^(-2i/D)
    cos, sin = orc.rope_tables(hd, pos + 1, 10000.0)
    half = hd // 2
    ang = pos * (1.0 / 10000.0 ** (2.0 * np.arange(half) / hd))
    for i in range(half):
        e = np.zeros((1, 1, hd), np.float32)
        e[0, 0, i] = 1.0
        out = LR.rope_apply(e, cos, sin, pos)[0, 0].astype(np.float64)
        want = np.zeros(hd)
        want[i], want[i + half] = np.cos(ang[i]), np.sin(ang[i])
        assert np.max(np.abs(out - want)) < 2e-5, i
        e[0, 0, i], e[0, 0, i + half] = 0.0, 1.0
        out = LR.rope_apply(e, cos, sin, pos)[0, 0].astype(np.float64)
        want[i], want[i + half] = -np.sin(ang[i]), np.cos(ang[i])
        assert np.max(np.abs(out - want)) < 2e-5, i


def test_rope_rows_follow_start_position():
    # a row at offset j of a chunk starting at `start` rotates as position start + j
    cos, sin = orc.rope_tables(16, 12, 10000.0)
    x = np.random.default_rng(3).standard_normal((2, 4, 16)).astype(np.float32)
    chunk = LR.rope_apply(x, cos, sin, 5)
    for j in range(4):
        assert np.array_equal(chunk[:, j:j + 1], LR.rope_apply(x[:, j:j + 1], cos, sin, 5 + j))


def test_attention_one_cached_key_returns_its_value_row():
    # softmax over one key is exactly 1, whatever q: the context is V's row
    rng = np.random.default_rng(8)
    q = rng.standard_normal((3, 1, 32)).astype(np.float32) * 50
    kc = rng.standard_normal((3, 1, 32)).astype(np.float32)
    vc = rng.standard_normal((3, 1, 32)).astype(np.float32)
    ctx = LR.attention(q, kc, vc, 0)
    assert np.array_equal(ctx[:, 0], vc[:, 0])


def test_attention_gqa_head_map():
    # 8 query heads over 2 KV heads: head h reads KV head h // 4
    # (repeat_kv repeats each KV head n_rep times in a row, ops.rs:981-987,
    # attention.rs:406-409); equal scores (q = 0) over 4 keys and a constant
    # V per KV head make each head's context exactly that constant
    nh, nkv, t, hd = 8, 2, 4, 16
    q = np.zeros((nh, 1, hd), np.float32)
    kc = np.random.default_rng(1).standard_normal((nkv, t, hd)).astype(np.float32)
    vc = np.stack([np.full((t, hd), 10.0 * (g + 1), np.float32) for g in range(nkv)])
    ctx = LR.attention(q, kc, vc, t - 1)
    for h in range(nh):
        assert np.all(ctx[h, 0] == 10.0 * (h // 4 + 1)), h
    # a modulo map (h % n_kv) would give head 1 the second KV head
    assert ctx[1, 0, 0] != 10.0 * (1 % nkv + 1)


def test_attention_two_key_softmax_and_scale():
    # scores q.k / sqrt(D) (attention.rs:414-415), softmax (ops.rs:582-628):
    # with q.k1 - q.k2 = 3 and D = 4 the weights are 1 / (1 + e^-1.5) and the rest
    hd = 4
    q = np.array([[[1.0, 0, 0, 0]]], np.float32)
    kc = np.array([[[2.0, 0, 0, 0], [-1.0, 0, 0, 0]]], np.float32)
    vc = np.array([[[1.0, 0, 0, 0], [0, 1.0, 0, 0]]], np.float32)
    ctx = LR.attention(q, kc, vc, 1)[0, 0].astype(np.float64)
    w1 = 1.0 / (1.0 + np.exp(-3.0 / np.sqrt(hd)))
    assert abs(ctx[0] - w1) < 1e-6 and abs(ctx[1] - (1 - w1)) < 1e-6
    assert ctx[2] == 0 and ctx[3] == 0
    # unscaled scores would weight the first key 1 / (1 + e^-3)
    assert abs(ctx[0] - 1.0 / (1.0 + np.exp(-3.0))) > 0.1


def test_attention_causal_rows():
    # a prefill chunk of 2 rows at positions 0, 1: row 0 sees key 0 only
    # (Tensor::causal_mask keeps j <= i + offset, ops.rs:905-916)
    rng = np.random.default_rng(4)
    q = rng.standard_normal((1, 2, 8)).astype(np.float32)
    kc = rng.standard_normal((1, 2, 8)).astype(np.float32)
    vc = rng.standard_normal((1, 2, 8)).astype(np.float32)
    ctx = LR.attention(q, kc, vc, 0)
    assert np.array_equal(ctx[0, 0], vc[0, 0])
    assert not np.allclose(ctx[0, 1], vc[0, 0])


def test_swiglu_is_silu_of_gate_times_up():
    # feed_forward.rs:146-148: silu(gate) * up, silu(g) = g / (1 + e^-g)
    g = np.array([1.0, -2.0, 0.5, 3.0], np.float32)
    u = np.array([3.0, 0.25, -1.0, 2.0], np.float32)
    got = LR.swiglu(g, u).astype(np.float64)
    gd, ud = g.astype(np.float64), u.astype(np.float64)
    want = gd / (1.0 + np.exp(-gd)) * ud
    assert np.allclose(got, want, rtol=1e-6, atol=0)
    swapped = ud / (1.0 + np.exp(-ud)) * gd
    assert not np.allclose(got, swapped, rtol=1e-2)


def test_forward_uses_the_pinned_pieces(monkeypatch):
    # the decode oracle composes exactly the functions pinned above
    calls = {"rope": 0, "att": 0, "swiglu": 0}

    def wrap(name, f):
        def g(*a, **k):
            calls[name] += 1
            return f(*a, **k)
        return g

    monkeypatch.setattr(LR, "rope_apply", wrap("rope", LR.rope_apply))
    monkeypatch.setattr(LR, "attention", wrap("att", LR.attention))
    monkeypatch.setattr(LR, "swiglu", wrap("swiglu", LR.swiglu))
    cfg = tiny_config(n_layers=2)
    _, ref_w = tiny_weights(cfg, seed=5)
    LlamaRef(cfg, ref_w).forward_with_cache([1, 2, 3])
    assert calls == {"rope": 4, "att": 2, "swiglu": 2}


def test_config5_geometry_logits_see_attention_mistakes(monkeypatch):
    """The GPU test of config 5's attention path (test_gpu_llama.py,
    test_config5_attention_path_f16_cache) compares logits of a 2-layer model
    at hidden 4096, 32 query heads over 8 KV heads of dim 128.  That
    comparison can only catch an attention mistake if the model's logits
    move by more than the parity bar when the attention is wrong: here the
    oracle's own attention is replaced by plausible mistakes (the h % n_kv
    head map instead of h // 4, no 1/sqrt(D) scale, the current key left out)
    and each must move the logits of a 128-row prompt and of a decode step at
    128 cached keys well outside 1e-3 rel + 1e-4 abs.  The model has the
    GPU test's centered Q4_0 codes; with BASELINE's codes (uniform in 0..15,
    a common mode of -d/2 a weight) the dropped key moves no logit past the
    bar, which is why the GPU test does not use them."""
    import oracle.llama_ref as lr

    cfg = tiny_config(dim=4096, n_layers=2, n_heads=32, n_kv_heads=8, head_dim=128, ffn_dim=512, vocab=320,
                      max_seq=256, max_batch=128, kv_f16=True)
    _, w = tiny_weights(cfg, 505, centered=True)
    prompt = np.random.default_rng(5005).integers(0, cfg.vocab, 128)
    good = LlamaRef(cfg, w, kv_f16=True)
    want = [good.forward_with_cache(prompt)]
    want.append(good.forward_with_cache([argmax(want[0])]))
    right = lr.attention

    def head_mod(q, kc, vc, start):  # query head h reads KV head h % n_kv
        nh, nkv = q.shape[0], kc.shape[0]
        perm = np.array([h % nkv for h in range(nh)]) * (nh // nkv) + np.array([h // nkv for h in range(nh)])
        return right(q[np.argsort(perm)], kc, vc, start)[perm]

    def unscaled(q, kc, vc, start):
        return right(q * np.float32(np.sqrt(q.shape[-1])), kc, vc, start)

    def no_current_key(q, kc, vc, start):
        if q.shape[1] != 1:
            return right(q, kc, vc, start)
        return right(q, kc[:, :-1], vc[:, :-1], start - 1)

    for name, fn in (("h % n_kv", head_mod), ("unscaled", unscaled), ("current key dropped", no_current_key)):
        monkeypatch.setattr(lr, "attention", fn)
        bad = LlamaRef(cfg, w, kv_f16=True)
        got = [bad.forward_with_cache(prompt)]
        got.append(bad.forward_with_cache([argmax(want[0])]))
        monkeypatch.setattr(lr, "attention", right)
        for step, (g, t) in enumerate(zip(got, want)):
            tol = 1e-4 + 1e-3 * np.abs(t)
            if name == "current key dropped" and step == 0:
                continue  # a prompt row always sees its own key in this planted form
            assert np.count_nonzero(np.abs(g - t) > tol) > t.size // 2, (name, step)
