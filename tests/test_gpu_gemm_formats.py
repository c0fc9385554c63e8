"""GPU parity of the prompt GEMM (matrix cores) for the weight formats other
than Q4_0: products of KQ_GEMM_MIN_M (16) or more rows of the reference's
Q4_K and Q6_K Linears (dequantize_q4k / dequantize_q6k at load,
rustml/gguf/main/src/core/parser.rs:510-593, then the F32 matmul), of
matmul_f32_q8 (quantize.rs:201-260) and of matmul_f32_q4_1 (float mode,
quantize.rs:429-495), through the C ABI, against the CPU restatement and the
exact (f64) value of the reference computation."""
import numpy as np
import pytest

from parity import assert_close, check_parity, exact_f64, exact_f64_cond
from rdlquant import synth

pytestmark = pytest.mark.gpu

THREADS = 16


def product(rq, kind):
    return {"q4k": rq.matmul_f32_q4_k, "q6k": rq.matmul_f32_q6_k, "q8": rq.matmul_f32_q8,
            "q4_1": rq.matmul_f32_q4_1}[kind]


def weights(kind, n, k, seed):
    return {"q4k": synth.q4_k_weights, "q6k": synth.q6_k_weights, "q8": synth.q8_0_weights,
            "q4_1": synth.q4_1_weights}[kind](n, k, seed)


ALL = ["q4k", "q6k", "q8", "q4_1"]


# Bar: check_parity with each output's condition (Q6_K's synthetic rows of
# 4096 give outputs near 100 that cancel to 0.03 in places, where the
# reference's own f32 path misses the exact value by more than 1e-4).
def run(rq, orc, m, n, k, seed, rows=None, x=None, w=None, kind="q4k"):
    x = synth.activations(m, k, seed) if x is None else x
    w = weights(kind, n, k, seed + 1) if w is None else w
    got = product(rq, kind)(x, w, m, k, n).reshape(m, n)
    if rows is not None:
        x, got, m = x.reshape(-1, k)[rows], got[rows], len(rows)
    want = orc.matmul(kind, x, w, m, k, n, threads=THREADS)
    exact, cond = exact_f64_cond(orc, kind, x, w, m, k, n)
    check_parity(got.reshape(-1), want, exact, cond=cond)


# Tile shapes by row count (the LDS GEMM's choice).  Q4_K: 16 rows (16 x 16
# tiles, 32-block chunks), 17-47 (16 x 32), 48-127 with the 32 x 64 tiles of
# 4 or 8 waves, 128 (64 x 64 when 32-row tiles overflow a round, 128 x 64
# when they fill the CUs), 256 and 1024 (128 x 128).  Q6_K: 16 x 16 (16-block
# chunks), 16 x 32, then 32 x 64 tiles below a round of 64 x 64 ones.  Q8_0
# and Q4_1 take Q4_K's shapes (Q8_0 16 x 16 tiles with 16-block chunks).
@pytest.mark.parametrize("kind", ALL)
@pytest.mark.parametrize("m,n,k", [(16, 4096, 4096), (16, 64, 256), (24, 300, 1024), (47, 1000, 2048),
                                   (64, 4096, 4096), (64, 12288, 512), (128, 4096, 4096), (128, 12288, 1024),
                                   (128, 22016, 512), (256, 4096, 1024), (1024, 512, 768)])
def test_kquant_gemm_tile_shapes(rq, orc, gpu, m, n, k, kind):
    run(rq, orc, m, n, k, 0x5EED4000 + m + n, kind=kind)


# ragged: partial tiles in both dimensions, one output column, super-block
# counts not dividing the chunk, the longest row the x prep holds (16384).
# Q6_K's 210-byte super-blocks start on a dword or 2 bytes past one; odd
# super-block counts a row (768, 1280, 2304) alternate the rows' alignment,
# and (16, 1, 256) / (19, 37, 768) end the matrix with a super-block on a
# dword (its d read from 2 bytes before its dword).
@pytest.mark.parametrize("kind", ALL)
@pytest.mark.parametrize("m,n,k", [(16, 1, 256), (19, 37, 768), (70, 130, 1280), (130, 257, 2304),
                                   (300, 100, 256), (33, 40, 16384), (1030, 33, 512), (48, 3, 768)])
def test_kquant_gemm_ragged(rq, orc, gpu, m, n, k, kind):
    run(rq, orc, m, n, k, 61 + m + n + k, kind=kind)


# Q8_0 / Q4_1 rows of any whole number of 32-element blocks: odd block counts
# (Q8_0's 34-byte blocks then alternate between starting on a dword and 2
# bytes past one, across rows too; (16, 1, 32), (17, 5, 96) and (48, 3, 160)
# end the matrix with a block on a dword, its last dword read 2 bytes early)
@pytest.mark.parametrize("kind", ["q8", "q4_1"])
@pytest.mark.parametrize("m,n,k", [(16, 1, 32), (17, 5, 96), (48, 3, 160), (20, 33, 1056), (130, 77, 4128),
                                   (64, 301, 416), (300, 64, 14336)])
def test_q8_q4_1_gemm_block_counts(rq, orc, gpu, m, n, k, kind):
    run(rq, orc, m, n, k, 91 + m + n + k, kind=kind)


@pytest.mark.parametrize("kind", ALL)
def test_kquant_gemm_large_rows_sampled(rq, orc, gpu, kind):
    # 2048 rows: each output row depends only on its x row, so 40 spread rows
    # pin all tiles
    rows = np.unique(np.linspace(0, 2047, 40).astype(int))
    run(rq, orc, 2048, 4096, 1024, 0x5EED4800, rows=rows, kind=kind)


@pytest.mark.parametrize("kind", ALL)
def test_kquant_longer_rows_take_the_records_path(rq, orc, gpu, kind):
    # k = 16640 > 16384: the x prep cannot hold the row; the records GEMV runs
    run(rq, orc, 20, 30, 16640, 0x5EED4900, kind=kind)


@pytest.mark.parametrize("kind", ALL)
def test_kquant_gemm_matches_gemv_rows(rq, gpu, kind):
    # the same rows through the GEMV (4 rows) and the GEMM (16 rows) agree
    # within the bar: the two paths split and sum differently
    m, n, k = 16, 512, 2048
    x = synth.activations(m, k, 8080)
    w = weights(kind, n, k, 8081)
    f = product(rq, kind)
    g = f(x, w, m, k, n).reshape(m, n)
    v = np.concatenate([f(x[4 * r:4 * r + 4], w, 4, k, n).reshape(4, n) for r in range(m // 4)])
    assert_close(g, v, rtol=2e-3, atol=2e-4)


def test_q4k_gemm_extreme_scales(rq, orc, gpu):
    # super-block scales across the f16 range (d, dmin from 2^-14 to 2^10),
    # 6-bit sub-block scales and mins at 0 and 63, and x rows from 1e-6 to 1e4.
    # Such rows cancel: outputs reach 1 / 400000 of sum |w x|, where no f32
    # evaluation (the reference's included) meets a bar relative to the value.
    # Bar: |got - exact| <= 1e-6 sum |w x| on every output (a wrong scale, min
    # or sub-block moves an output by O(sum |w x|)), and the value bar where
    # |exact| >= 1e-2 sum |w x|.
    m, n, k = 32, 64, 1024
    r = np.random.default_rng(99)
    w = synth.q4_k_weights(n, k, 98).reshape(n, k // 256, 144).copy()
    d = synth.f16_bits(2.0 ** r.integers(-14, 11, size=(n, k // 256)))
    dmin = synth.f16_bits(2.0 ** r.integers(-14, 11, size=(n, k // 256)))
    w[..., 0:2] = d[..., None].view(np.uint8).reshape(n, k // 256, 2)
    w[..., 2:4] = dmin[..., None].view(np.uint8).reshape(n, k // 256, 2)
    w[0, :, 4:16] = 0xFF  # every 6-bit scale and min 63
    w[1, :, 4:16] = 0x00  # every scale and min 0: the row is zero
    w = w.reshape(-1)
    x = synth.activations(m, k, 97) * (10.0 ** r.uniform(-6, 4, size=(m, 1))).astype(np.float32)
    got = rq.matmul_f32_q4_k(x, w, m, k, n).reshape(m, n).astype(np.float64)
    wd = np.abs(orc.to_f32("q4k", w, n * k).reshape(n, k).astype(np.float64))
    cond = np.abs(x.astype(np.float64)) @ wd.T
    exact = exact_f64(orc, "q4k", x, w, m, k, n).reshape(m, n)
    want = orc.matmul("q4k", x, w, m, k, n, threads=THREADS).reshape(m, n).astype(np.float64)
    assert np.all(np.abs(got - exact) <= 1e-6 * cond)
    assert np.all(np.abs(got - want) <= 1e-6 * cond)
    assert np.all(got[:, 1] == 0.0)  # weight row 1: every scale and min 0
    well = np.abs(exact) >= 1e-2 * cond
    assert well.sum() > m * n // 2
    assert_close(got[well], exact[well])


def test_q6k_gemm_extreme_scales(rq, orc, gpu):
    # super-block d across the f16 range (2^-14 .. 2^10), sub-block scales at
    # -128 and 127 (weight row 0) and 0 (row 1: a zero column), x rows from
    # 1e-6 to 1e4; bars as for Q4_K above
    m, n, k = 32, 64, 1024
    r = np.random.default_rng(199)
    ns = k // 256
    codes = r.integers(0, 64, size=(n, ns, 256), dtype=np.uint8)
    scales = r.integers(-128, 128, size=(n, ns, 16), dtype=np.int16).astype(np.int8)
    scales[0] = np.where(np.arange(16) % 2 == 0, -128, 127).astype(np.int8)
    scales[1] = 0
    d = synth.f16_bits(2.0 ** r.integers(-14, 11, size=(n, ns)))
    w = synth.pack_q6_k(codes, scales, d).reshape(-1)
    x = synth.activations(m, k, 197) * (10.0 ** r.uniform(-6, 4, size=(m, 1))).astype(np.float32)
    got = rq.matmul_f32_q6_k(x, w, m, k, n).reshape(m, n).astype(np.float64)
    wd = np.abs(orc.to_f32("q6k", w, n * k).reshape(n, k).astype(np.float64))
    cond = np.abs(x.astype(np.float64)) @ wd.T
    exact = exact_f64(orc, "q6k", x, w, m, k, n).reshape(m, n)
    want = orc.matmul("q6k", x, w, m, k, n, threads=THREADS).reshape(m, n).astype(np.float64)
    assert np.all(np.abs(got - exact) <= 1e-6 * cond)
    assert np.all(np.abs(got - want) <= 1e-6 * cond)
    assert np.all(got[:, 1] == 0.0)
    well = np.abs(exact) >= 1e-2 * cond
    assert well.sum() > m * n // 2
    assert_close(got[well], exact[well])


@pytest.mark.parametrize("kind", ALL)
def test_kquant_gemm_nan_row_stays_in_its_row(rq, gpu, kind):
    m, n, k = 20, 48, 512
    x = synth.activations(m, k, 5)
    x[3, 100] = np.nan
    w = weights(kind, n, k, 6)
    y = product(rq, kind)(x, w, m, k, n).reshape(m, n)
    assert np.isnan(y[3]).all()
    assert np.isfinite(np.delete(y, 3, axis=0)).all()
