"""GPU parity of the Q4_K prompt GEMM (matrix cores): products of
KQ_GEMM_MIN_M (16) or more rows of the reference's Q4_K Linear
(dequantize_q4k at load, rustml/gguf/main/src/core/parser.rs:549-593, then
the F32 matmul) through the C ABI, against the CPU restatement and the exact
(f64) value of the reference computation."""
import numpy as np
import pytest

from parity import assert_close, check_parity, exact_f64
from rdlquant import synth

pytestmark = pytest.mark.gpu

THREADS = 16


def run(rq, orc, m, n, k, seed, rows=None, x=None, w=None):
    x = synth.activations(m, k, seed) if x is None else x
    w = synth.q4_k_weights(n, k, seed + 1) if w is None else w
    got = rq.matmul_f32_q4_k(x, w, m, k, n).reshape(m, n)
    if rows is not None:
        x, got, m = x.reshape(-1, k)[rows], got[rows], len(rows)
    want = orc.matmul("q4k", x, w, m, k, n, threads=THREADS)
    check_parity(got.reshape(-1), want, exact_f64(orc, "q4k", x, w, m, k, n))


# Tile shapes by row count (the LDS GEMM's choice): 16 rows (16 x 16 tiles,
# 32-block chunks), 17-47 (16 x 32), 48-127 with the 32 x 64 tiles of 4 or 8
# waves, 128 (64 x 64 when 32-row tiles overflow a round, 128 x 64 when they
# fill the CUs), 256 and 1024 (128 x 128).
@pytest.mark.parametrize("m,n,k", [(16, 4096, 4096), (16, 64, 256), (24, 300, 1024), (47, 1000, 2048),
                                   (64, 4096, 4096), (64, 12288, 512), (128, 4096, 4096), (128, 12288, 1024),
                                   (128, 22016, 512), (256, 4096, 1024), (1024, 512, 768)])
def test_q4k_gemm_tile_shapes(rq, orc, gpu, m, n, k):
    run(rq, orc, m, n, k, 0x5EED4000 + m + n)


# ragged: partial tiles in both dimensions, one output column, super-block
# counts not dividing the chunk, the longest row the x prep holds (16384)
@pytest.mark.parametrize("m,n,k", [(16, 1, 256), (19, 37, 768), (70, 130, 1280), (130, 257, 2304),
                                   (300, 100, 256), (33, 40, 16384), (1030, 33, 512)])
def test_q4k_gemm_ragged(rq, orc, gpu, m, n, k):
    run(rq, orc, m, n, k, 61 + m + n + k)


def test_q4k_gemm_large_rows_sampled(rq, orc, gpu):
    # 2048 rows (128 x 128 tiles, 8 x 16 = 128 tiles a column of x tiles):
    # each output row depends only on its x row, so 40 spread rows pin all tiles
    rows = np.unique(np.linspace(0, 2047, 40).astype(int))
    run(rq, orc, 2048, 4096, 1024, 0x5EED4800, rows=rows)


def test_q4k_longer_rows_take_the_records_path(rq, orc, gpu):
    # k = 16640 > 16384: the x prep cannot hold the row; the records GEMV runs
    run(rq, orc, 20, 30, 16640, 0x5EED4900)


def test_q4k_gemm_matches_gemv_rows(rq, gpu):
    # the same rows through the GEMV (4 rows) and the GEMM (16 rows) agree
    # within the bar: the two paths split and sum differently
    m, n, k = 16, 512, 2048
    x = synth.activations(m, k, 8080)
    w = synth.q4_k_weights(n, k, 8081)
    g = rq.matmul_f32_q4_k(x, w, m, k, n).reshape(m, n)
    v = np.concatenate([rq.matmul_f32_q4_k(x[4 * r:4 * r + 4], w, 4, k, n).reshape(4, n)
                        for r in range(m // 4)])
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


def test_q4k_gemm_nan_row_stays_in_its_row(rq, gpu):
    m, n, k = 20, 48, 512
    x = synth.activations(m, k, 5)
    x[3, 100] = np.nan
    w = synth.q4_k_weights(n, k, 6)
    y = rq.matmul_f32_q4_k(x, w, m, k, n).reshape(m, n)
    assert np.isnan(y[3]).all()
    assert np.isfinite(np.delete(y, 3, axis=0)).all()
