"""Pins the oracle's quantize_row_q8_0 (rustml/quant/main/src/core/quantize.rs:164-193)
by closed-form properties and special cases, independent of its own code path:
numpy's float16 for the scale, exact f64 rounding for the codes."""
import numpy as np
import pytest


def ref_codes(x, rt):
    """round-half-away(x * (1/rt)) clamped to [-128, 127] with the f32 product."""
    inv = np.float32(0.0) if rt == 0 else np.float32(1.0) / np.float32(rt)
    prod = (x.astype(np.float32) * inv).astype(np.float64)
    r = np.sign(prod) * np.floor(np.abs(prod) + 0.5)
    r = np.where(np.isnan(r), 0, r)
    return np.clip(r, -128, 127).astype(np.int8)


def check_block(x, out, sc):
    amax = np.float32(0.0)
    for v in x:  # f32::max fold from 0.0 (NaN ignored)
        a = np.float32(abs(v))
        if not np.isnan(a):
            amax = max(amax, a)
    scale = np.float32(0.0) if amax == 0 else np.float32(amax) / np.float32(127.0)
    h = np.array([scale], dtype=np.float32).astype(np.float16)
    rt = h.astype(np.float32)[0]
    assert int(out[0]) | (int(out[1]) << 8) == int(h.view(np.uint16)[0])
    assert np.float32(sc).view(np.uint32) == rt.view(np.uint32)
    got = out[2:34].view(np.int8)
    assert np.array_equal(got, ref_codes(x, rt))


def test_random_rows(orc):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(4096) * np.float32(10.0) ** rng.integers(-6, 3, 4096)).astype(np.float32)
    out, sc = orc.quantize_row_q8_0(x)
    for b in range(128):
        check_block(x[b * 32:(b + 1) * 32], out[b * 34:(b + 1) * 34], sc[b])


def test_special_blocks(orc):
    blocks = [
        np.zeros(32, np.float32),                                     # amax = 0 -> scale 0, codes 0
        np.linspace(-1, 1, 32, dtype=np.float32),                     # +-amax -> +-127
        (np.arange(32, dtype=np.float32) - 15.5) * np.float32(127 / 16.5),  # ties around .5
        np.full(32, 1e-9, np.float32),                                # f16-subnormal scale
        np.full(32, 1e-12, np.float32),                               # scale rounds to 0 in f16
        np.array([np.nan] + [0.5] * 31, np.float32),                  # NaN ignored by amax, code 0
        np.array([np.inf] + [0.5] * 31, np.float32),                  # inf scale -> inv 0 -> codes 0
        np.array([1e9] + [1.0] * 31, np.float32),                     # scale overflows f16
    ]
    x = np.concatenate(blocks)
    out, sc = orc.quantize_row_q8_0(x)
    for b, blk in enumerate(blocks):
        check_block(blk, out[b * 34:(b + 1) * 34], sc[b])
    # closed forms
    assert np.all(out[2:34] == 0) and sc[0] == 0
    codes = out[34 + 2:34 + 34].view(np.int8)
    assert codes[0] == -127 and codes[-1] == 127
    assert np.all(out[5 * 34 + 2] == 0)


def test_dequant_error_bound(orc):
    # |q*rt - x| <= rt/2 (up to one f32 rounding) whenever rt is a normal f16
    rng = np.random.default_rng(12)
    x = rng.standard_normal(32 * 256).astype(np.float32)
    out, sc = orc.quantize_row_q8_0(x)
    q = out.reshape(-1, 34)[:, 2:].view(np.int8).astype(np.float64)
    err = np.abs(q * sc[:, None].astype(np.float64) - x.reshape(-1, 32))
    assert np.all(err <= sc[:, None] * 0.5 * (1 + 2 ** -10) + 1e-12)
    assert np.all(np.abs(q).max(axis=1) >= 126)
