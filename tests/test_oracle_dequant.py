"""Pins the oracle's load-time dequantizers (rustml/gguf/main/src/core/parser.rs:
371-776) with packers written in the encoding direction: each test draws codes,
scales and minimums, lays them into GGUF blocks by the format's description,
and requires the oracle to give back d * scale * code (- min) exactly -- a
transposed index, a wrong shift or a dropped term on either side breaks the
round trip.  Q3_K's scale packing also gets a block worked by hand."""
import numpy as np
import pytest

from rdlquant import synth


def f16(v):
    return np.asarray(v, np.float32).astype(np.float16)


def f16_bytes(v):
    return f16(v).view(np.uint8).reshape(np.shape(v) + (2,))


def f32_of(v):
    return f16(v).astype(np.float32)


def rng(seed):
    return np.random.default_rng(seed)


NB = 5  # blocks per case


def test_q5_0_roundtrip(orc):
    r = rng(1)
    q = r.integers(0, 32, size=(NB, 32))
    d = np.abs(r.normal(0, 0.05, NB))
    blk = np.zeros((NB, 22), np.uint8)
    blk[:, 0:2] = f16_bytes(d)
    qh = np.zeros(NB, np.uint64)
    for j in range(32):
        qh |= ((q[:, j] >> 4).astype(np.uint64) & 1) << np.uint64(j)
    blk[:, 2:6] = qh.astype("<u4").view(np.uint8).reshape(NB, 4)
    blk[:, 6:22] = (q[:, :16] & 0xF) | ((q[:, 16:] & 0xF) << 4)
    want = f32_of(d)[:, None] * (q.astype(np.float32) - 16.0)
    assert np.array_equal(orc.to_f32("q5_0", blk.reshape(-1), NB * 32).reshape(NB, 32), want)


def test_q5_1_and_q4_1_roundtrip(orc):
    r = rng(2)
    q = r.integers(0, 32, size=(NB, 32))
    d, m = np.abs(r.normal(0, 0.05, NB)), r.normal(0, 0.1, NB)
    blk = np.zeros((NB, 24), np.uint8)
    blk[:, 0:2], blk[:, 2:4] = f16_bytes(d), f16_bytes(m)
    qh = np.zeros(NB, np.uint64)
    for j in range(32):
        qh |= ((q[:, j] >> 4).astype(np.uint64) & 1) << np.uint64(j)
    blk[:, 4:8] = qh.astype("<u4").view(np.uint8).reshape(NB, 4)
    blk[:, 8:24] = (q[:, :16] & 0xF) | ((q[:, 16:] & 0xF) << 4)
    want = (f32_of(d)[:, None] * q.astype(np.float32)).astype(np.float32) + f32_of(m)[:, None]
    assert np.array_equal(orc.to_f32("q5_1", blk.reshape(-1), NB * 32).reshape(NB, 32), want)
    # the 4-bit legacy form: the same with nibbles only
    q4 = q & 0xF
    b4 = np.zeros((NB, 20), np.uint8)
    b4[:, 0:2], b4[:, 2:4] = f16_bytes(d), f16_bytes(m)
    b4[:, 4:20] = q4[:, :16] | (q4[:, 16:] << 4)
    want4 = (f32_of(d)[:, None] * q4.astype(np.float32)).astype(np.float32) + f32_of(m)[:, None]
    assert np.array_equal(orc.to_f32("q4_1_legacy", b4.reshape(-1), NB * 32).reshape(NB, 32), want4)
    assert np.array_equal(orc.to_f32("q4_1", b4.reshape(-1), NB * 32).reshape(NB, 32), want4)


def test_q8_1_and_q8_k_roundtrip(orc):
    r = rng(3)
    q = r.integers(-128, 128, size=(NB, 32)).astype(np.int8)
    d = r.normal(0, 0.01, NB).astype(np.float32)
    blk = np.zeros((NB, 40), np.uint8)
    blk[:, 0:4] = d.view(np.uint8).reshape(NB, 4)
    blk[:, 4:8] = r.integers(0, 256, size=(NB, 4))  # the sum field: not read
    blk[:, 8:40] = q.view(np.uint8)
    want = d[:, None] * q.astype(np.float32)
    assert np.array_equal(orc.to_f32("q8_1", blk.reshape(-1), NB * 32).reshape(NB, 32), want)
    qk = r.integers(-128, 128, size=(2, 256)).astype(np.int8)
    dk = r.normal(0, 0.01, 2).astype(np.float32)
    bk = np.zeros((2, 292), np.uint8)
    bk[:, 0:4] = dk.view(np.uint8).reshape(2, 4)
    bk[:, 4:260] = qk.view(np.uint8)
    bk[:, 260:] = r.integers(0, 256, size=(2, 32))  # bsums: not read
    assert np.array_equal(orc.to_f32("q8k", bk.reshape(-1), 512).reshape(2, 256), dk[:, None] * qk.astype(np.float32))


def test_q5_k_roundtrip(orc):
    r = rng(4)
    n = 3
    q = r.integers(0, 32, size=(n, 256))
    sc, mn = r.integers(0, 64, size=(n, 8)), r.integers(0, 64, size=(n, 8))
    d, dmin = np.abs(r.normal(0, 0.01, n)), np.abs(r.normal(0, 0.01, n))
    blk = np.zeros((n, 176), np.uint8)
    blk[:, 0:2], blk[:, 2:4] = f16_bytes(d), f16_bytes(dmin)
    blk[:, 4:16] = synth.pack_q4k_scales(sc.astype(np.uint8), mn.astype(np.uint8))
    qh = np.zeros((n, 32), np.uint8)
    qs = np.zeros((n, 128), np.uint8)
    for c in range(4):  # element 64c + l: low nibble of qs[32c + l], bit 2c of qh[l]; +32: high nibble, bit 2c+1
        lo, hi = q[:, 64 * c:64 * c + 32], q[:, 64 * c + 32:64 * c + 64]
        qs[:, 32 * c:32 * c + 32] = (lo & 0xF) | ((hi & 0xF) << 4)
        qh |= (((lo >> 4) & 1) << (2 * c)).astype(np.uint8) | (((hi >> 4) & 1) << (2 * c + 1)).astype(np.uint8)
    blk[:, 16:48], blk[:, 48:176] = qh, qs
    sub = np.repeat(np.arange(8), 32)  # sub-block of each element
    d1 = (f32_of(d)[:, None] * sc[:, sub].astype(np.float32)).astype(np.float32)
    m1 = (f32_of(dmin)[:, None] * mn[:, sub].astype(np.float32)).astype(np.float32)
    want = (d1 * q.astype(np.float32)).astype(np.float32) - m1
    assert np.array_equal(orc.to_f32("q5k", blk.reshape(-1), n * 256).reshape(n, 256), want)


def _k_order():
    """(element -> scale index, byte of qs / hmask, shift step j) of the Q2_K /
    Q3_K element order: halves of 128, four 2-bit steps, 16 + 16 elements."""
    scale, qbyte, step = np.zeros(256, int), np.zeros(256, int), np.zeros(256, int)
    e = 0
    for h in range(2):
        for j in range(4):
            for part in range(2):
                for l in range(16):
                    scale[e] = 8 * h + 2 * j + part
                    qbyte[e] = 32 * h + 16 * part + l  # qs byte; the hmask byte is qbyte - 32h
                    step[e] = j  # 2-bit field 2j of the qs byte; hmask bit 4h + j
                    e += 1
    return scale, qbyte, step


def test_q2_k_roundtrip(orc):
    r = rng(5)
    n = 3
    q = r.integers(0, 4, size=(n, 256))
    sc, mn = r.integers(0, 16, size=(n, 16)), r.integers(0, 16, size=(n, 16))
    d, dmin = np.abs(r.normal(0, 0.01, n)), np.abs(r.normal(0, 0.01, n))
    scale, qbyte, step = _k_order()
    blk = np.zeros((n, 84), np.uint8)
    blk[:, 0:16] = sc | (mn << 4)
    qs = np.zeros((n, 64), np.int64)
    for e in range(256):
        qs[:, qbyte[e]] |= q[:, e] << (2 * step[e])
    blk[:, 16:80] = qs
    blk[:, 80:82], blk[:, 82:84] = f16_bytes(d), f16_bytes(dmin)
    dl = (f32_of(d)[:, None] * sc[:, scale].astype(np.float32)).astype(np.float32)
    ml = (f32_of(dmin)[:, None] * mn[:, scale].astype(np.float32)).astype(np.float32)
    want = (dl * q.astype(np.float32)).astype(np.float32) - ml
    assert np.array_equal(orc.to_f32("q2k", blk.reshape(-1), n * 256).reshape(n, 256), want)


def pack_q3k_scales(s):
    """Sixteen 6-bit scales -> 12 bytes: low nibbles of scales 0..7 in the low
    nibbles of bytes 0..7, of scales 8..15 in their high nibbles; the high bit
    pair of scale i at bits 2 (i // 4) of byte 8 + i % 4."""
    s = np.asarray(s, np.int64)
    out = np.zeros(s.shape[:-1] + (12,), np.int64)
    out[..., 0:8] = (s[..., 0:8] & 0xF) | ((s[..., 8:16] & 0xF) << 4)
    for i in range(16):
        out[..., 8 + i % 4] |= (s[..., i] >> 4) << (2 * (i // 4))
    return out.astype(np.uint8)


def test_q3_k_roundtrip(orc):
    r = rng(6)
    n = 3
    v = r.integers(-4, 4, size=(n, 256))  # the value q2 - 4 * (hmask bit clear)
    s = r.integers(0, 64, size=(n, 16))
    d = np.abs(r.normal(0, 0.01, n))
    scale, qbyte, step = _k_order()
    hbit = (v >= 0).astype(np.int64)  # set: no -4
    q2 = v + 4 * (1 - hbit)
    blk = np.zeros((n, 110), np.uint8)
    hm = np.zeros((n, 32), np.int64)
    qs = np.zeros((n, 64), np.int64)
    for e in range(256):
        h = qbyte[e] // 32
        qs[:, qbyte[e]] |= q2[:, e] << (2 * step[e])
        hm[:, qbyte[e] - 32 * h] |= hbit[:, e] << (4 * h + step[e])
    blk[:, 0:32], blk[:, 32:96] = hm, qs
    blk[:, 96:108] = pack_q3k_scales(s)
    blk[:, 108:110] = f16_bytes(d)
    dl = (f32_of(d)[:, None] * (s[:, scale].astype(np.float32) - 32.0)).astype(np.float32)
    want = dl * v.astype(np.float32)
    assert np.array_equal(orc.to_f32("q3k", blk.reshape(-1), n * 256).reshape(n, 256), want)


def test_q3_k_scales_by_hand(orc):
    """Scales 0..15 stored as 2i + 17 (so each has both nibble and high bits),
    every code 0 with its hmask bit set (value 0 - 0 = 0) except one element
    per scale group given code 1: the output is d * (scale - 32) there.
    Bytes worked by hand: scale i low nibble (2i + 17) & 15, high pair
    (2i + 17) >> 4."""
    s = np.array([2 * i + 17 for i in range(16)])
    sb = np.zeros(12, np.uint8)
    for i in range(8):
        sb[i] = ((s[i] & 15) | ((s[i + 8] & 15) << 4))
    for i in range(16):
        sb[8 + i % 4] |= (s[i] >> 4) << (2 * (i // 4))
    assert np.array_equal(sb, pack_q3k_scales(s))
    blk = np.zeros(110, np.uint8)
    blk[0:32] = 0xFF  # every hmask bit set: no -4 anywhere
    # element 0 of each 16-group: group g = 2 (4h + j) + part -> qs byte 32h + 16 part, shift 2j
    for h in range(2):
        for j in range(4):
            for part in range(2):
                blk[32 + 32 * h + 16 * part] |= 1 << (2 * j)
    blk[96:108] = sb
    blk[108:110] = f16_bytes([0.5])[0]
    out = orc.to_f32("q3k", blk, 256).reshape(16, 16)
    assert np.array_equal(out[:, 0], 0.5 * (s - 32).astype(np.float32))
    assert not out[:, 1:].any()


def test_partial_block_counts_leave_zeros(orc):
    """n_elements not a multiple of the block: whole blocks only, zeros after
    (the reference's n_elements / block_size blocks into a zeroed Vec)."""
    w = synth.q6_k_weights(1, 512, 9)
    out = orc.to_f32("q2k", np.resize(w, 2 * 84), 300)
    assert out.shape == (300,) and not out[256:].any()
