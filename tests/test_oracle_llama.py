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
