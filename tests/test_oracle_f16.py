"""Pins the oracle's binary16 conversions (half 2.7.1 f16::from_f32 / to_f32,
used at rustml/quant/main/src/core/quantize.rs:178-179 and parser.rs:506-508)
against numpy's independent float16 implementation."""
import numpy as np


def test_f16_to_f32_all_patterns(orc):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_rne_matches_numpy(orc):
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000).astype(np.float32),
        # exact ties between adjacent f16 values (normal and subnormal range)
        (np.arange(1, 2000, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -24),
        (np.float32(1.0) + (np.arange(0, 1024, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10)),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, np.inf, -np.inf,
                  2.0 ** -25, 2.0 ** -24, 2.0 ** -25 * 1.0000001, 6.1e-5, 5.96e-8], dtype=np.float32),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(float(vals[i]), hex(got[i]), hex(want[i])) for i in bad[:5]]


def test_f32_to_f16_nan_is_quiet_nan(orc):
    h = orc.f32_to_f16(float("nan"))
    assert (h & 0x7C00) == 0x7C00 and (h & 0x3FF) != 0
