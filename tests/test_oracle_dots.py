"""Pins the oracle's block dots (rustml/quant/main/src/core/simd.rs).

Known answers come from the reference's own tests
(rustml/experimentation/llmforge/tests/simd_test.rs, same kernel semantics) and
simd.rs:629-695; the float dots are bounded by an f64 brute force over the
GGUF-order dequantization."""
import numpy as np
import pytest


def test_q4q8_known_answer_minus_246(orc):
    # simd_test.rs:161-182
    packed = np.full(16, 0x88, dtype=np.uint8)
    packed[0] = 0x53
    packed[1] = 0xF0
    q8 = np.zeros(32, dtype=np.int8)
    q8[0], q8[1], q8[16], q8[17] = 10, 20, 5, -3
    assert orc.dot_q4q8_block(packed, q8) == -246


def test_q4q8_max_values_28448(orc):
    # simd_test.rs:215-224: 32 * 7 * 127
    assert orc.dot_q4q8_block(np.full(16, 0xFF, np.uint8), np.full(32, 127, np.int8)) == 28448


def test_q4q8_all_zero_q8(orc):
    # simd_test.rs:206-213
    assert orc.dot_q4q8_block(np.zeros(16, np.uint8), np.zeros(32, np.int8)) == 0


def test_q4q8_dispatch_vector(orc):
    # simd_test.rs:184-204 inputs; the integer value by brute force
    packed = np.array([(i * 7 + 3) & 0xFF for i in range(16)], dtype=np.uint8)
    q8 = np.fmod(np.arange(32) * 13 - 50, 128).astype(np.int8)  # Rust % truncates
    lo = (packed & 0xF).astype(np.int64) - 8
    hi = (packed >> 4).astype(np.int64) - 8
    want = int((lo * q8[:16]).sum() + (hi * q8[16:]).sum())
    assert orc.dot_q4q8_block(packed, q8) == want


def test_q4q8_brute_force_random(orc):
    rng = np.random.default_rng(1)
    for _ in range(500):
        packed = rng.integers(0, 256, 16, dtype=np.uint8)
        q8 = rng.integers(-128, 128, 32, dtype=np.int16).astype(np.int8)
        w = np.concatenate([(packed & 0xF), (packed >> 4)]).astype(np.int64) - 8
        assert orc.dot_q4q8_block(packed, q8) == int((w * q8).sum())


def test_q4_1_q8_simd_rs_vector(orc):
    # simd.rs:665-680 inputs; (unsigned dot, q8 sum) by brute force
    packed = np.array([(((j + 1) << 4) & 0xFF) | j for j in range(16)], dtype=np.uint8)  # u8 shl wraps
    q8 = np.arange(32, dtype=np.int64) - 16
    nib = np.concatenate([packed & 0xF, packed >> 4]).astype(np.int64)
    assert orc.dot_q4_1_q8_block(packed, q8.astype(np.int8)) == (int((nib * q8).sum()), int(q8.sum()))


def test_float_dots_lane_restatement_equals_avx2_bits(orc):
    # The lane-by-lane restatement of the AVX2 tree and the intrinsic version
    # must give identical bits (no contraction on either side).
    rng = np.random.default_rng(2)
    for _ in range(300):
        x = rng.standard_normal(32).astype(np.float32)
        q = rng.integers(-128, 128, 32, dtype=np.int16).astype(np.int8)
        p = rng.integers(0, 256, 16, dtype=np.uint8)
        s = np.float32(abs(rng.standard_normal()))
        a = np.float32(orc.dot_q8_block(x, q, s)); b = np.float32(orc.dot_q8_block(x, q, s, "_lanes"))
        assert a.view(np.uint32) == b.view(np.uint32)
        a = np.float32(orc.dot_q4_block(x, p, s)); b = np.float32(orc.dot_q4_block(x, p, s, "_lanes"))
        assert a.view(np.uint32) == b.view(np.uint32)


def test_float_dots_vs_f64(orc):
    rng = np.random.default_rng(3)
    for _ in range(300):
        x = rng.standard_normal(32).astype(np.float32)
        q = rng.integers(-128, 128, 32, dtype=np.int16).astype(np.int8)
        p = rng.integers(0, 256, 16, dtype=np.uint8)
        s = np.float32(abs(rng.standard_normal()) * 0.01)
        want8 = float((x.astype(np.float64) * q).sum()) * float(s)
        w4 = np.concatenate([(p & 0xF), (p >> 4)]).astype(np.float64) - 8
        want4 = float((x.astype(np.float64) * w4).sum()) * float(s)
        bound8 = 32 * 2.0 ** -23 * float((np.abs(x) * np.abs(q)).sum()) * float(s) + 1e-30
        bound4 = 32 * 2.0 ** -23 * float((np.abs(x) * np.abs(w4)).sum()) * float(s) + 1e-30
        assert abs(orc.dot_q8_block(x, q, s) - want8) <= bound8
        assert abs(orc.dot_q4_block(x, p, s) - want4) <= bound4
        assert abs(orc.dot_q4_block(x, p, s, "_scalar") - want4) <= bound4


@pytest.mark.parametrize("variant", ["", "_scalar"])
def test_simd_rs_scalar_vs_dispatch_tolerance(orc, variant):
    # simd.rs:633-663 inputs: scalar and dispatched agree to 1e-3
    x = np.arange(32, dtype=np.float32) * np.float32(0.1)
    q = (np.arange(32) - 16).astype(np.int8)
    assert abs(orc.dot_q8_block(x, q, 0.5, variant) - orc.dot_q8_block(x, q, 0.5, "_scalar")) < 1e-3
    packed = np.array([((((j + 1) % 8) + 8) << 4) | ((j % 8) + 8) for j in range(16)], dtype=np.uint8)
    assert abs(orc.dot_q4_block(x, packed, 0.5, variant) - orc.dot_q4_block(x, packed, 0.5, "_scalar")) < 1e-3


def test_zero_scale_gives_zero(orc):
    # simd_test.rs:141-157
    assert orc.dot_q8_block(np.ones(32, np.float32), np.full(32, 100, np.int8), 0.0) == 0.0
    assert orc.dot_q4_block(np.ones(32, np.float32), np.full(16, 0xFF, np.uint8), 0.0) == 0.0
