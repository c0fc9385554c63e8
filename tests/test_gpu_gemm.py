"""GPU parity of the Q4_0 prefill GEMM (matrix cores): the many-row case of
matmul_f32_q4 (quantize.rs:265-320) through the C ABI, against the CPU
restatement and the exact (f64) value of the reference computation."""
import numpy as np
import pytest

from parity import assert_close, check_parity, exact_f64
from rdlquant import synth

pytestmark = pytest.mark.gpu

THREADS = 16


def run(rq, orc, m, n, k, seed, rows=None):
    x = synth.activations(m, k, seed)
    w = synth.q4_0_weights(n, k, seed + 1)
    got = rq.matmul_f32_q4(x, w, m, k, n).reshape(m, n)
    if rows is not None:
        x, got, m = x[rows], got[rows], len(rows)
    want = orc.matmul("q4", x, w, m, k, n, threads=THREADS)
    check_parity(got.reshape(-1), want, exact_f64(orc, "q4", x, w, m, k, n))


# W 4096x4096 Q4_0, M in {16, 64, 512, 2048}
@pytest.mark.parametrize("m", [16, 64, 512])
def test_config4_prefill(rq, orc, gpu, m):
    run(rq, orc, m, 4096, 4096, 0x5EED0004 + m)


def test_prefill_chunk_of_a_tall_matrix(rq, orc, gpu):
    # 128 rows against 16512 weight rows: the 128 x 64 tiles fill the CUs
    # (the prefill chunk's gate/up shape, narrower K)
    run(rq, orc, 128, 16512, 256, 0x5EED0128)


@pytest.mark.parametrize("n,k", [(4096, 4096), (6144, 1024), (200, 2080), (24640, 256)])
def test_prefill_chunk_tile_shapes(rq, orc, gpu, n, k):
    # 128 rows: 8-wave 32 x 64 tiles (one round), 64 x 64 tiles (32-row
    # tiles overflow a round), a matrix too small for either, and 128 x 128
    # tiles (the gate/up shape)
    run(rq, orc, 128, n, k, 0x5EED0200 + n)


def test_config4_prefill_2048_sampled_rows(rq, orc, gpu):
    # each output row depends only on its x row: check 48 spread rows, all tiles
    rows = np.unique(np.linspace(0, 2047, 48).astype(int))
    run(rq, orc, 2048, 4096, 4096, 0x5EED0804, rows=rows)


# ragged: partial tiles in both dimensions, odd block counts (block windows
# straddling the matrix end), chunk counts not dividing the blocks
@pytest.mark.parametrize("m,n,k", [(5, 1, 32), (5, 17, 96), (17, 100, 4128), (33, 130, 1056),
                                   (100, 64, 2080), (300, 257, 544), (1030, 33, 160)])
def test_gemm_ragged(rq, orc, gpu, m, n, k):
    run(rq, orc, m, n, k, 31 + m + n + k)


def test_gemm_matches_gemv_rows(rq, gpu):
    # the same rows through the one-row GEMV and the GEMM agree within the bar
    m, n, k = 24, 320, 2048
    x = synth.activations(m, k, 41)
    w = synth.q4_0_weights(n, k, 42)
    gemm = rq.matmul_f32_q4(x, w, m, k, n).reshape(m, n)
    for r in (0, 7, 23):
        gemv = rq.matmul_f32_q4(x[r:r + 1], w, 1, k, n)
        assert_close(gemm[r], gemv, rtol=2e-3, atol=2e-4)


def test_large_scales_stay_within_the_bar(rq, orc, gpu):
    # |d| = 20000: (q - 8) * d would overflow f16; the GEMM keeps (q - 8) in
    # its operands and applies d in f32 after each block's MFMA
    m, n, k = 8, 40, 256
    w = synth.q4_0_weights(n, k, 51)
    blocks = w.reshape(n, -1, 18)
    blocks[3, 2, 0:2] = np.frombuffer(np.float16(20000.0).tobytes(), np.uint8)
    x = synth.activations(m, k, 52)
    check_parity(rq.matmul_f32_q4(x, w, m, k, n), orc.matmul("q4", x, w, m, k, n),
                 exact_f64(orc, "q4", x, w, m, k, n))


def test_wide_dynamic_range_rows(rq, orc, gpu):
    # rows scaled by 2^-40 .. 2^+40: the per-row power-of-two scaling keeps each
    # row's relative accuracy
    m, n, k = 12, 48, 512
    x = synth.activations(m, k, 61)
    x *= (2.0 ** np.linspace(-40, 40, m)).astype(np.float32)[:, None]
    w = synth.q4_0_weights(n, k, 62)
    got = rq.matmul_f32_q4(x, w, m, k, n).reshape(m, n)
    exact = exact_f64(orc, "q4", x, w, m, k, n).reshape(m, n)
    for r in range(m):
        scale = np.abs(exact[r]).max()
        assert_close(got[r] / scale, exact[r] / scale)


def test_nan_row_stays_in_its_row(rq, gpu):
    m, n, k = 20, 64, 256
    x = synth.activations(m, k, 71)
    w = synth.q4_0_weights(n, k, 72)
    x[6, 100] = np.nan
    y = rq.matmul_f32_q4(x, w, m, k, n).reshape(m, n)
    assert np.all(np.isnan(y[6]))
    assert np.all(np.isfinite(np.delete(y, 6, axis=0)))


# small M (m <= 64): the x-tile kernel that splits x per block itself
@pytest.mark.parametrize("m,n,k", [(5, 16, 256), (15, 33, 1024), (16, 4096, 4096), (17, 48, 4128),
                                   (31, 7, 96), (32, 256, 4096), (48, 100, 2080), (63, 130, 1056),
                                   (64, 4096, 4096), (20, 16400, 256)])
def test_small_m_shapes(rq, orc, gpu, m, n, k):
    # 16400 rows: two row tiles a workgroup with a ragged last tile
    run(rq, orc, m, n, k, 7 + m + n + k)


@pytest.mark.parametrize("m", [16, 24])
def test_small_m_block_extremes(rq, orc, gpu, m):
    # per-block scaling: all-zero, subnormal, huge and mixed-magnitude blocks
    # each keep the bar; an infinite element makes its row non-finite only
    # (m = 16 and m = 24: the two K-split kernels for small m)
    n, k = 80, 1024
    x = synth.activations(m, k, 91)
    w = synth.q4_0_weights(n, k, 92)
    x[1, 0:32] = 0.0                                   # a zero block
    x[2, 64:96] = np.float32(3e-41)                    # subnormal block
    x[3, 128:160] *= np.float32(1e30)                  # huge block
    x[4, :] *= (2.0 ** np.repeat(np.linspace(-60, 60, k // 32), 32)).astype(np.float32)  # blocks 2^-60 .. 2^60
    x[5, :] = 0.0                                      # a zero row
    check_parity(rq.matmul_f32_q4(x, w, m, k, n), orc.matmul("q4", x, w, m, k, n),
                 exact_f64(orc, "q4", x, w, m, k, n))
    x[6, 200] = np.inf
    y = rq.matmul_f32_q4(x, w, m, k, n).reshape(m, n)
    assert not np.any(np.isfinite(y[6]))
    assert np.all(np.isfinite(np.delete(y, 6, axis=0)))


# ---- native mode (matmul_f32_q4_native) on the int8 matrix cores ---------------------
def _native_exact(orc, x, w, m, k, n):
    part = orc.block_dots(x, w, m, k, n).astype(np.float64)
    sw = w.reshape(n, k // 32, 18)[:, :, 0:2].copy().view(np.float16).astype(np.float64)[..., 0]
    sx = np.stack([orc.quantize_row_q8_0(x[r])[1] for r in range(m)]).astype(np.float64)
    return (part.reshape(m, n, k // 32) * sx[:, None, :] * sw[None]).sum(axis=2).reshape(-1)


@pytest.mark.parametrize("m,n", [(512, 256), (2048, 64)])
def test_native_gemm_block_dots_bit_exact(rq, orc, gpu, m, n):
    """The int8 MFMA stage of the native GEMM (rows > 4) gives the exact int32
    block dots of simd::dot_q4q8_block (simd.rs:562-581) for every (row,
    column, block) at config-4 row counts."""
    k = 4096
    print(f"case native partials m={m} n={n}", flush=True)
    x = synth.activations(m, k, 0x5EED0904 + m)
    w = synth.q4_0_weights(n, k, 0x5EED0905)
    assert np.array_equal(rq.q4_0_q8_0_block_dots(x, w, m, k, n), orc.block_dots(x, w, m, k, n))


@pytest.mark.parametrize("m,n,k", [(5, 1, 32), (6, 17, 96), (17, 100, 4128), (33, 130, 1056),
                                   (100, 64, 2080), (300, 257, 544), (1030, 33, 160)])
def test_native_gemm_ragged(rq, orc, gpu, m, n, k):
    x = synth.activations(m, k, 91 + m + n + k)
    w = synth.q4_0_weights(n, k, 92 + m + n + k)
    assert np.array_equal(rq.q4_0_q8_0_block_dots(x, w, m, k, n), orc.block_dots(x, w, m, k, n))
    check_parity(rq.matmul_f32_q4_native(x, w, m, k, n), orc.matmul("q4_native", x, w, m, k, n, THREADS),
                 _native_exact(orc, x, w, m, k, n))


def test_native_gemm_nan_and_zero_rows(rq, orc, gpu):
    # quantize_row_q8_0 maps NaN to code 0 and a zero block to scale 0
    # (quantize.rs:176-187): such rows stay finite, as in the reference
    m, n, k = 9, 40, 256
    x = synth.activations(m, k, 93)
    x[2, 5] = np.nan
    x[4] = 0.0
    w = synth.q4_0_weights(n, k, 94)
    got = rq.matmul_f32_q4_native(x, w, m, k, n)
    want = orc.matmul("q4_native", x, w, m, k, n)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert_close(np.nan_to_num(got), np.nan_to_num(want))
