"""Pins the oracle's matmuls and dequantizers (rustml/quant/main/src/core/quantize.rs,
rustml/core/main/src/core/tensor/tensor.rs:535-639, rustml/gguf/main/src/core/parser.rs:510-593)."""
import numpy as np
import pytest

from rdlquant import synth


def f64_gemm(x, wdeq, m, k, n):
    return x.reshape(m, k).astype(np.float64) @ wdeq.reshape(n, k).astype(np.float64).T


def test_to_f32_q4_0_gguf_order(orc):
    # tensor.rs:553-563: byte j -> element j (lo) and j+16 (hi), value d*(q-8)
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.array([1.0], np.float16).view(np.uint8)  # d = 1
    blk[2:] = np.array([(((j + 1) & 15) << 4) | j for j in range(16)], np.uint8)
    out = orc.to_f32("q4_0", blk, 32)
    want = np.array([j - 8 for j in range(16)] + [((j + 1) & 15) - 8 for j in range(16)], np.float32)
    assert np.array_equal(out, want)


def test_to_f32_q8_0_and_q4_1(orc):
    rng = np.random.default_rng(5)
    w8 = synth.q8_0_weights(3, 64, 1)
    out = orc.to_f32("q8_0", w8, 3 * 64).reshape(-1, 32)
    b = w8.reshape(-1, 34)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)
    assert np.array_equal(out, d * b[:, 2:].view(np.int8).astype(np.float32))
    w41 = synth.q4_1_weights(2, 64, 2)
    out = orc.to_f32("q4_1", w41, 128).reshape(-1, 32)
    b = w41.reshape(-1, 20)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)
    mv = b[:, 2:4].copy().view(np.float16).astype(np.float32)
    nib = np.concatenate([b[:, 4:] & 0xF, b[:, 4:] >> 4], axis=1).astype(np.float32)
    assert np.array_equal(out, d * nib + mv)


@pytest.mark.parametrize("kind,gen,deq", [
    ("q8", synth.q8_0_weights, "q8_0"),
    ("q4", synth.q4_0_weights, "q4_0"),
    ("q4_1", synth.q4_1_weights, "q4_1"),
])
def test_float_matmul_vs_f64(orc, kind, gen, deq):
    m, k, n = 3, 512, 40
    x = synth.activations(m, k, 3)
    w = gen(n, k, 4)
    y = orc.matmul(kind, x, w, m, k, n, threads=2).reshape(m, n)
    wd = orc.to_f32(deq, w, n * k)
    want = f64_gemm(x, wd, m, k, n)
    bound = 2.0 ** -20 * (np.abs(x.reshape(m, k)) @ np.abs(wd.reshape(n, k)).T) + 1e-12
    assert np.all(np.abs(y - want) <= bound)


def test_native_vs_float_agreement(orc):
    # llmforge simd_test.rs:245-276 style: native and float paths agree within 2%
    x = ((np.arange(128, dtype=np.float32) - 64) * np.float32(0.02)).reshape(1, 128)
    w = synth.q4_0_weights(4, 128, 9)
    a = orc.matmul("q4", x, w, 1, 128, 4)
    b = orc.matmul("q4_native", x, w, 1, 128, 4)
    assert np.all(np.abs(a - b) <= 0.02 * np.abs(a) + 1e-3)


def test_native_equals_partials_composition(orc):
    # y = sum_b (float(int_dot_b) * sx_b) * sw_b in block order (quantize.rs:383-384)
    m, k, n = 2, 256, 5
    x = synth.activations(m, k, 21)
    w = synth.q4_0_weights(n, k, 22)
    part = orc.block_dots(x, w, m, k, n)
    y = orc.matmul("q4_native", x, w, m, k, n).reshape(m, n)
    wb = w.reshape(n, k // 32, 18)
    ws = wb[:, :, 0:2].copy().view(np.float16).astype(np.float32)[..., 0]
    for r in range(m):
        _, sx = orc.quantize_row_q8_0(x[r])
        for c in range(n):
            acc = np.float32(0)
            for b in range(k // 32):
                acc = np.float32(acc + np.float32(np.float32(np.float32(part[r, c, b]) * sx[b]) * ws[c, b]))
            assert acc == y[r, c]
    # and the partials are the integer dots against the Q8_0 codes
    q8, _ = orc.quantize_row_q8_0(x[0])
    codes = q8.reshape(-1, 34)[:, 2:].view(np.int8).astype(np.int64)
    nib = np.concatenate([wb[..., 2:] & 0xF, wb[..., 2:] >> 4], axis=2).astype(np.int64) - 8
    assert np.array_equal(part[0], (nib * codes[None]).sum(axis=2))


def _q8_values(orc, row):
    """quantize_row_q8_0's codes times their f16-rounded block scales, in f64
    (the activation the native paths dot against; pinned by the closed forms
    of tests/test_oracle_quant.py)."""
    codes, sx = orc.quantize_row_q8_0(row)
    q = codes.reshape(-1, 34)[:, 2:].view(np.int8).astype(np.float64)
    return (q * sx.astype(np.float64)[:, None]).reshape(-1)


@pytest.mark.parametrize("shape", [(3, 512, 24), (1, 4096, 8)])
def test_q4_1_native_vs_f64(orc, shape):
    """matmul_f32_q4_1_native (quantize.rs:501-572) is the product of the
    Q8_0-quantized activation with the Q4_1 weights: y = sum_b sum_j
    (sx_b q8_j) (d_b nib_j + m_b).  The exact value comes from two
    independently pinned pieces, the Q8_0 codes / scales and to_f32's Q4_1
    values; the oracle's f32 result (per block sx (d isum + m qsum), then a
    sequential sum) must sit within a few f32 roundings of it.  A dropped or
    sign-flipped m term, a float (unquantized) x or the Q4_0 offset of 8
    each break the bound."""
    m, k, n = shape
    x = synth.activations(m, k, 51)
    w = synth.q4_1_weights(n, k, 52)
    y = orc.matmul("q4_1_native", x, w, m, k, n).reshape(m, n)
    wd = orc.to_f32("q4_1", w, n * k).reshape(n, k).astype(np.float64)
    b = w.reshape(n, k // 32, 20)
    d = b[..., 0:2].copy().view(np.float16).astype(np.float64)
    mv = b[..., 2:4].copy().view(np.float16).astype(np.float64)
    nib = np.concatenate([b[..., 4:] & 0xF, b[..., 4:] >> 4], axis=2).astype(np.float64)
    mag = (np.abs(d * nib) + np.abs(mv)).reshape(n, k)  # size of each weight's two terms
    for r in range(m):
        xq = _q8_values(orc, x[r])
        want = wd @ xq
        bound = 2.0 ** -18 * (mag @ np.abs(xq)) + 1e-12
        err = np.abs(y[r].astype(np.float64) - want)
        assert np.all(err <= bound), float((err / bound).max())
        # the mistakes a restatement could make fail the same bound
        planted = {"m dropped": (wd - mv[..., 0].repeat(32, axis=1)) @ xq,
                   "m negated": (wd - 2 * mv[..., 0].repeat(32, axis=1)) @ xq,
                   "x unquantized": wd @ x[r].astype(np.float64),
                   "q4_0 offset": (wd - 8 * d[..., 0].repeat(32, axis=1)) @ xq}
        for name, v in planted.items():
            assert np.count_nonzero(np.abs(v - want) > bound) >= n // 2, name


def test_q4k_exact_small_integers(orc):
    # d, dmin powers of two, small integer q/sc/mn: every product is exact, so
    # the dequantization has a closed form to compare bit for bit.
    rng = np.random.default_rng(8)
    n, k = 2, 512
    ns = k // 256
    q = rng.integers(0, 16, size=(n, ns, 4, 2, 32), dtype=np.uint8)
    sc = rng.integers(0, 64, size=(n, ns, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, size=(n, ns, 8), dtype=np.uint8)
    blob = np.zeros((n, ns, 144), np.uint8)
    blob[..., 0:2] = np.array([0.25], np.float16).view(np.uint8)
    blob[..., 2:4] = np.array([0.5], np.float16).view(np.uint8)
    blob[..., 4:16] = synth.pack_q4k_scales(sc, mn)
    blob[..., 16:] = (q[..., 0, :] | (q[..., 1, :] << 4)).reshape(n, ns, 128)
    out = orc.to_f32("q4k", blob.reshape(-1), n * k).reshape(n, ns, 4, 2, 32)
    # sub-block j = 2*chunk + (0 lo | 1 hi)
    scj = sc.reshape(n, ns, 4, 2, 1).astype(np.float32)
    mnj = mn.reshape(n, ns, 4, 2, 1).astype(np.float32)
    want = 0.25 * scj * q.astype(np.float32) - 0.5 * mnj
    assert np.array_equal(out, want.astype(np.float32))


def test_q4k_scale_pack_roundtrip():
    # synth.pack_q4k_scales must invert parser.rs:562-569 exactly
    rng = np.random.default_rng(9)
    sc = rng.integers(0, 64, size=(100, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, size=(100, 8), dtype=np.uint8)
    s = synth.pack_q4k_scales(sc, mn).astype(np.int64)
    usc = np.concatenate([s[:, 0:4] & 63, ((s[:, 0:4] >> 6) & 3) | ((s[:, 8:12] & 0xF) << 2)], axis=1)
    umn = np.concatenate([s[:, 4:8] & 63, ((s[:, 4:8] >> 6) & 3) | ((s[:, 8:12] >> 4) << 2)], axis=1)
    assert np.array_equal(usc, sc) and np.array_equal(umn, mn)


def test_q4k_matmul_vs_f64(orc):
    m, k, n = 2, 1024, 24
    x = synth.activations(m, k, 31)
    w = synth.q4_k_weights(n, k, 32)
    y = orc.matmul("q4k", x, w, m, k, n, threads=2).reshape(m, n)
    wd = orc.to_f32("q4k", w, n * k)
    want = f64_gemm(x, wd, m, k, n)
    bound = 2.0 ** -13 * (np.abs(x.reshape(m, k)) @ np.abs(wd.reshape(n, k)).T) + 1e-9
    assert np.all(np.abs(y - want) <= bound)


def test_q6k_known_block(orc):
    """A block worked by hand from parser.rs:525-541: ql bytes 0x21 (low nibble
    1, high 2), qh bytes 0xE4 (bit pairs 0, 1, 2, 3 for t = 0..3), scales
    1..16, d = 0.5.  Element 128h + 32t + l has code (1 or 2) + 16t and scale
    index 8h + 2t + l // 16."""
    blk = np.zeros(210, np.uint8)
    blk[0:128] = 0x21
    blk[128:192] = 0xE4
    blk[192:208] = np.arange(1, 17, dtype=np.int8).view(np.uint8)
    blk[208:210] = np.array([0.5], np.float16).view(np.uint8)
    out = orc.to_f32("q6k", blk, 256)
    want = np.empty(256, np.float32)
    for h in range(2):
        for t in range(4):
            code = (1 if t < 2 else 2) + 16 * t
            for l in range(32):
                want[128 * h + 32 * t + l] = 0.5 * (8 * h + 2 * t + l // 16 + 1) * (code - 32)
    assert np.array_equal(out, want)


def test_q6k_pack_roundtrip_and_signed_scales(orc):
    """synth.pack_q6_k inverts the unpack: every code, negative scales, and
    (d * scale) * (code - 32) exact in f32."""
    rng = np.random.default_rng(10)
    n, k = 3, 768
    ns = k // 256
    codes = rng.integers(0, 64, size=(n, ns, 256), dtype=np.uint8)
    codes[0, 0] = np.arange(256) % 64  # every code in every position class
    scales = rng.integers(-128, 128, size=(n, ns, 16), dtype=np.int16).astype(np.int8)
    d = synth.f16_bits(np.abs(rng.normal(0, 0.01, size=(n, ns))))
    blob = synth.pack_q6_k(codes, scales, d)
    out = orc.to_f32("q6k", blob.reshape(-1), n * k).reshape(n, ns, 256)
    df = d.view(np.float16).astype(np.float32)[..., None]
    sc = np.repeat(scales.astype(np.float32), 16, axis=-1)  # element e -> scale e // 16
    want = (df * sc) * (codes.astype(np.float32) - 32)
    assert np.array_equal(out, want.astype(np.float32))


def test_q6k_matmul_vs_f64(orc):
    m, k, n = 2, 1024, 24
    x = synth.activations(m, k, 33)
    w = synth.q6_k_weights(n, k, 34)
    y = orc.matmul("q6k", x, w, m, k, n, threads=2).reshape(m, n)
    wd = orc.to_f32("q6k", w, n * k)
    want = f64_gemm(x, wd, m, k, n)
    bound = 2.0 ** -13 * (np.abs(x.reshape(m, k)) @ np.abs(wd.reshape(n, k)).T) + 1e-9
    assert np.all(np.abs(y - want) <= bound)


@pytest.mark.parametrize("kind", ["q8", "q4", "q4_native", "q4_1", "q4_1_native"])
def test_block_alignment_error(orc, kind):
    with pytest.raises(orc.OracleError) as e:
        orc.matmul(kind, np.zeros(33, np.float32), np.zeros(100, np.uint8), 1, 33, 1)
    assert e.value.code == 3


def test_short_weight_is_shape_mismatch(orc):
    with pytest.raises(orc.OracleError) as e:
        orc.matmul("q4", np.zeros(64, np.float32), np.zeros(35, np.uint8), 1, 64, 1)
    assert e.value.code == 2


def test_cols_split_equals_row_split(orc):
    m, k, n = 1, 1024, 33
    x = synth.activations(m, k, 41)
    w = synth.q4_0_weights(n, k, 42)
    assert np.array_equal(orc.matmul("q4", x, w, m, k, n, 1), orc.matmul("q4_cols", x, w, m, k, n, 4))
