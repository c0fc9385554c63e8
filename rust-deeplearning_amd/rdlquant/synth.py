"""Seeded synthetic inputs in GGUF block layout for the BASELINE.json configs.

Blocks are generated directly as packed bytes (BASELINE specifies packed GGUF
bytes, not a quantizer run).  Element order inside a Q4_0 / Q4_1 block is the
GGUF one the reference kernels use: byte j holds element j in its low nibble
and element j+16 in its high nibble (rustml/quant/main/src/core/simd.rs:21-31,
rustml/core/main/src/core/tensor/tensor.rs:553-563).  Q4_K scale/min bytes are
packed as the exact inverse of the reference unpack
(rustml/gguf/main/src/core/parser.rs:562-569).
"""
from __future__ import annotations

import numpy as np

SEED_BASE = 0x5EED0000


def _rng(seed):
    return np.random.default_rng(seed)


def f16_bits(values) -> np.ndarray:
    """IEEE binary16 bit patterns (round to nearest even) of f32 values."""
    return np.asarray(values, dtype=np.float32).astype(np.float16).view(np.uint16)


def activations(m, k, seed):
    """x ~ N(0, 1), f32 [m, k]."""
    return _rng(seed).standard_normal((m, k), dtype=np.float32)


def pack_q4_nibbles(q: np.ndarray) -> np.ndarray:
    """q uint8 [..., 32] in 0..15 -> 16 bytes per block (lo = q[j], hi = q[j+16])."""
    q = q.astype(np.uint8)
    return (q[..., :16] | (q[..., 16:] << 4)).astype(np.uint8)


def q8_0_weights(n, k, seed, d_sigma=0.02):
    """Config 1: q ~ U{-127..127}, d = f16(|N(0, d_sigma)| / 127); [n, k/32] blocks of 34 B."""
    r = _rng(seed)
    nb = k // 32
    q = r.integers(-127, 128, size=(n, nb, 32), dtype=np.int16).astype(np.int8)
    d = f16_bits(np.abs(r.normal(0.0, d_sigma, size=(n, nb))) / 127.0)
    out = np.empty((n, nb, 34), dtype=np.uint8)
    out[..., 0:2] = d[..., None].view(np.uint8).reshape(n, nb, 2)
    out[..., 2:] = q.view(np.uint8)
    return out.reshape(-1)


def q4_0_weights(n, k, seed, d_sigma=0.02):
    """Config 2: q ~ U{0..15}, d = f16(|N(0, d_sigma)| / 8); [n, k/32] blocks of 18 B."""
    r = _rng(seed)
    nb = k // 32
    q = r.integers(0, 16, size=(n, nb, 32), dtype=np.uint8)
    d = f16_bits(np.abs(r.normal(0.0, d_sigma, size=(n, nb))) / 8.0)
    out = np.empty((n, nb, 18), dtype=np.uint8)
    out[..., 0:2] = d[..., None].view(np.uint8).reshape(n, nb, 2)
    out[..., 2:] = pack_q4_nibbles(q)
    return out.reshape(-1)


def q4_1_weights(n, k, seed, d_sigma=0.02, m_sigma=0.01):
    """Q4_1 (not a BASELINE config): q ~ U{0..15}, d = f16(|N(0,d_sigma)|/16), m = f16(N(0,m_sigma))."""
    r = _rng(seed)
    nb = k // 32
    q = r.integers(0, 16, size=(n, nb, 32), dtype=np.uint8)
    d = f16_bits(np.abs(r.normal(0.0, d_sigma, size=(n, nb))) / 16.0)
    mn = f16_bits(r.normal(0.0, m_sigma, size=(n, nb)))
    out = np.empty((n, nb, 20), dtype=np.uint8)
    out[..., 0:2] = d[..., None].view(np.uint8).reshape(n, nb, 2)
    out[..., 2:4] = mn[..., None].view(np.uint8).reshape(n, nb, 2)
    out[..., 4:] = pack_q4_nibbles(q)
    return out.reshape(-1)


def pack_q4k_scales(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Inverse of parser.rs:562-569: sc, mn uint8 [..., 8] in 0..63 -> 12 bytes."""
    sc = sc.astype(np.uint8)
    mn = mn.astype(np.uint8)
    s = np.empty(sc.shape[:-1] + (12,), dtype=np.uint8)
    s[..., 0:4] = sc[..., 0:4] | ((sc[..., 4:8] & 3) << 6)
    s[..., 4:8] = mn[..., 0:4] | ((mn[..., 4:8] & 3) << 6)
    s[..., 8:12] = ((sc[..., 4:8] >> 2) & 0xF) | (((mn[..., 4:8] >> 2) & 0xF) << 4)
    return s


def q4_k_weights(n, k, seed, d_sigma=0.01):
    """Config 3: q ~ U{0..15}, sc, mn ~ U{0..63}, d, dmin = f16(|N(0, d_sigma)|); 144 B super-blocks."""
    r = _rng(seed)
    ns = k // 256
    q = r.integers(0, 16, size=(n, ns, 4, 2, 32), dtype=np.uint8)  # [chunk][lo/hi][32]
    sc = r.integers(0, 64, size=(n, ns, 8), dtype=np.uint8)
    mn = r.integers(0, 64, size=(n, ns, 8), dtype=np.uint8)
    d = f16_bits(np.abs(r.normal(0.0, d_sigma, size=(n, ns))))
    dmin = f16_bits(np.abs(r.normal(0.0, d_sigma, size=(n, ns))))
    out = np.empty((n, ns, 144), dtype=np.uint8)
    out[..., 0:2] = d[..., None].view(np.uint8).reshape(n, ns, 2)
    out[..., 2:4] = dmin[..., None].view(np.uint8).reshape(n, ns, 2)
    out[..., 4:16] = pack_q4k_scales(sc, mn)
    qs = q[..., 0, :] | (q[..., 1, :] << 4)  # [n, ns, 4, 32]
    out[..., 16:] = qs.reshape(n, ns, 128)
    return out.reshape(-1)


def pack_q6_k(codes, scales, d_bits) -> np.ndarray:
    """Q6_K super-blocks from codes [..., 256] in 0..63 (value = code - 32),
    int8 scales [..., 16] and f16 bit patterns d [...]: the inverse of the
    unpack in dequantize_q6k (rustml/gguf/main/src/core/parser.rs:510-547).
    Element 128*h + 32*t + l: low nibble in ql[64*h + 32*(t&1) + l] (low
    half for t < 2, high half for t >= 2), high bit pair at bits 2t, 2t+1 of
    qh[32*h + l]."""
    c = np.asarray(codes, dtype=np.uint8)
    lead = c.shape[:-1]
    c = c.reshape(lead + (2, 4, 32))  # [half][t][l]
    lo = c & 0x0F
    ql = np.empty(lead + (2, 2, 32), dtype=np.uint8)  # [half][t & 1][l]
    ql[..., 0, :] = lo[..., 0, :] | (lo[..., 2, :] << 4)
    ql[..., 1, :] = lo[..., 1, :] | (lo[..., 3, :] << 4)
    hb = (c >> 4) & 3
    qh = hb[..., 0, :] | (hb[..., 1, :] << 2) | (hb[..., 2, :] << 4) | (hb[..., 3, :] << 6)  # [half][l]
    out = np.empty(lead + (210,), dtype=np.uint8)
    out[..., 0:128] = ql.reshape(lead + (128,))
    out[..., 128:192] = qh.reshape(lead + (64,))
    out[..., 192:208] = np.asarray(scales, dtype=np.int8).view(np.uint8)
    out[..., 208:210] = np.asarray(d_bits, dtype=np.uint16)[..., None].view(np.uint8).reshape(lead + (2,))
    return out


def q6_k_weights(n, k, seed, d_sigma=0.002):
    """Q6_K: codes ~ U{0..63}, scales ~ U{-128..127}, d = f16(|N(0, d_sigma)|); 210 B super-blocks."""
    r = _rng(seed)
    ns = k // 256
    codes = r.integers(0, 64, size=(n, ns, 256), dtype=np.uint8)
    scales = r.integers(-128, 128, size=(n, ns, 16), dtype=np.int16).astype(np.int8)
    d = f16_bits(np.abs(r.normal(0.0, d_sigma, size=(n, ns))))
    return pack_q6_k(codes, scales, d).reshape(-1)


def weights(dtype, n, k, seed):
    """Weights of GGML type id `dtype` (2 = Q4_0, 3 = Q4_1, 8 = Q8_0, 12 = Q4_K, 14 = Q6_K)."""
    return {2: q4_0_weights, 3: q4_1_weights, 8: q8_0_weights, 12: q4_k_weights,
            14: q6_k_weights}[dtype](n, k, seed)
