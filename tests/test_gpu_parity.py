"""GPU parity: librdlquant (HIP, gfx950) against the CPU restatement.

Bars: integer work bit-exact (Q8_0 activation bytes,
int32 block dots); f32 outputs within 1e-3 relative + 1e-4 absolute of the
reference CPU path on identical seeded inputs."""
import numpy as np
import pytest

from rdlquant import synth

pytestmark = pytest.mark.gpu

from parity import ATOL, RTOL, assert_close, check_parity, exact_f64  # noqa: E402,F401


# ---- quantize_row_q8_0: byte-exact --------------------------------------------------
def test_quantize_row_q8_0_bit_exact(rq, orc, gpu):
    rng = np.random.default_rng(100)
    x = (rng.standard_normal(32 * 1024) * np.float32(10.0) ** rng.integers(-8, 4, 32 * 1024)).astype(np.float32)
    specials = np.concatenate([
        np.zeros(32, np.float32), np.full(32, 1e-9, np.float32), np.full(32, 1e-12, np.float32),
        np.array([np.nan] + [0.5] * 31, np.float32), np.array([np.inf] + [0.5] * 31, np.float32),
        np.array([-np.inf] + [-0.25] * 31, np.float32), np.full(32, np.nan, np.float32),
        np.array([1e9] + [1.0] * 31, np.float32),
        (np.arange(32, dtype=np.float32) - 15.5) * np.float32(127 / 16.5),
    ])
    x = np.concatenate([x, specials])
    out, sc = rq.quantize_row_q8_0(x)
    want_out, want_sc = orc.quantize_row_q8_0(x)
    assert np.array_equal(out, want_out)
    assert np.array_equal(sc.view(np.uint32), want_sc.view(np.uint32))


# ---- float-mode GEMV at the BASELINE shapes ---------------------------------------------
@pytest.mark.parametrize("name,dtype,n,k,kind,seed", [
    ("config1_q8_0", 8, 4096, 4096, "q8", 0x5EED0001),
    ("config2_q4_0", 2, 11008, 4096, "q4", 0x5EED0002),
    ("config3_q4_k_up", 12, 14336, 4096, "q4k", 0x5EED0003),
    ("config3_q4_k_down", 12, 4096, 14336, "q4k", 0x5EED0013),
    ("q4_0_down_14336", 2, 4096, 14336, "q4", 0x5EED0023),
    ("q4_1_small", 3, 1000, 2048, "q4_1", 0x5EED0033),
])
def test_gemv_float_baseline_shapes(rq, orc, gpu, name, dtype, n, k, kind, seed):
    print(f"case {name}: n={n} k={k}", flush=True)
    x = synth.activations(1, k, seed + 100)
    w = synth.weights(dtype, n, k, seed)
    fn = {"q8": rq.matmul_f32_q8, "q4": rq.matmul_f32_q4, "q4k": rq.matmul_f32_q4_k,
          "q4_1": rq.matmul_f32_q4_1}[kind]
    y = fn(x, w, 1, k, n)
    want = orc.matmul(kind, x, w, 1, k, n, threads=8)
    check_parity(y, want, exact_f64(orc, kind, x, w, 1, k, n))


# (1, 6000, 256) and (2, 14336, 512) take the fused kernel's 2- and 4-row-per-wave
# reductions on a 256-CU device (the baseline shapes take 1 and 3).  K > 8192
# splits K over 4 waves: an odd block count (8224), ragged rows, the largest K.
@pytest.mark.parametrize("m,n,k", [(1, 1, 32), (1, 3, 64), (2, 17, 96), (3, 65, 4096 + 32),
                                   (1, 129, 2048), (4, 7, 8192), (5, 300, 320),
                                   (1, 6000, 256), (2, 14336, 512),
                                   (3, 37, 8224), (1, 1000, 12288), (2, 21, 16384)])
@pytest.mark.parametrize("dtype,kind", [(2, "q4"), (8, "q8"), (3, "q4_1")])
def test_gemv_float_ragged(rq, orc, gpu, m, n, k, dtype, kind):
    x = synth.activations(m, k, 7 + n)
    w = synth.weights(dtype, n, k, 11 + k)
    fn = {"q8": rq.matmul_f32_q8, "q4": rq.matmul_f32_q4, "q4_1": rq.matmul_f32_q4_1}[kind]
    check_parity(fn(x, w, m, k, n), orc.matmul(kind, x, w, m, k, n), exact_f64(orc, kind, x, w, m, k, n))


# K <= 4096 on a 256-CU device spreads the rows over 512 workgroups of 8
# waves: (1, 6000, 2048) takes 2 rows a wave, (1, 10000, 1024) and
# (2, 9000, 4096) 3, (1, 17000, 512) 5, (2, 22016, 1024) 6, (1, 26000, 256) 7,
# (1, 28673, 512) 8 and (1, 40000, 256) 8 with more workgroups than one round.
# K > 4096 splits K over 2 (K <= 8192) or 4 waves of a workgroup: ragged row
# counts, a last slice shorter than the others (K = 4352, 8448, 16128) and
# the largest K.
@pytest.mark.parametrize("m,n,k", [(1, 1, 256), (2, 5, 512), (1, 33, 1280), (3, 8, 14336),
                                   (1, 10000, 1024), (2, 9000, 4096), (1, 6000, 2048),
                                   (1, 17000, 512), (2, 22016, 1024), (1, 26000, 256), (1, 28673, 512),
                                   (1, 40000, 256),
                                   (1, 37, 4352), (2, 100, 8192), (1, 77, 8448), (4, 50, 16128),
                                   (1, 130, 16384), (1, 4096, 14336)])
def test_gemv_q4k_ragged(rq, orc, gpu, m, n, k):
    x = synth.activations(m, k, 3 + n)
    w = synth.q4_k_weights(n, k, 5 + k)
    check_parity(rq.matmul_f32_q4_k(x, w, m, k, n), orc.matmul("q4k", x, w, m, k, n),
                 exact_f64(orc, "q4k", x, w, m, k, n))


# Q6_K (dequantize_q6k + F32 Linear in the reference): K split over 1 (K <= 2048),
# 2, 4 or 8 waves of 64 columns; odd super-block counts (K = 768, 1280, 4352,
# 8448) put every other row on a 2-byte boundary; ragged last slices; the
# lm_head shape; 5-15 rows take the records kernel (16 or more the tile GEMM,
# tests/test_gpu_gemm_formats.py).
@pytest.mark.parametrize("m,n,k", [(1, 1, 256), (2, 5, 768), (1, 33, 1280), (3, 8, 14336),
                                   (1, 1000, 2048), (4, 300, 4096), (1, 32000, 4096), (1, 37, 4352),
                                   (2, 100, 8192), (1, 77, 8448), (1, 130, 16384), (5, 40, 4096),
                                   (9, 70, 768), (6, 3, 16640)])
def test_gemv_q6k_ragged(rq, orc, gpu, m, n, k):
    x = synth.activations(m, k, 13 + n)
    w = synth.q6_k_weights(n, k, 17 + k)
    check_parity(rq.matmul_f32_q6_k(x, w, m, k, n), orc.matmul("q6k", x, w, m, k, n, threads=8),
                 exact_f64(orc, "q6k", x, w, m, k, n))


# ---- native mode: int32 partials bit-exact, outputs within tolerance --------------------
def test_native_block_dots_bit_exact(rq, orc, gpu):
    m, n, k = 2, 64, 512
    x = synth.activations(m, k, 201)
    w = synth.q4_0_weights(n, k, 202)
    assert np.array_equal(rq.q4_0_q8_0_block_dots(x, w, m, k, n), orc.block_dots(x, w, m, k, n))


def test_native_block_dots_config2(rq, orc, gpu):
    n, k = 11008, 4096
    x = synth.activations(1, k, 0x5EED0102)
    w = synth.q4_0_weights(n, k, 0x5EED0002)
    assert np.array_equal(rq.q4_0_q8_0_block_dots(x, w, 1, k, n), orc.block_dots(x, w, 1, k, n))


@pytest.mark.parametrize("m,n,k", [(1, 11008, 4096), (1, 4096, 14336), (3, 33, 96), (1, 1, 32), (2, 45, 8224)])
def test_native_gemv(rq, orc, gpu, m, n, k):
    x = synth.activations(m, k, 300 + n)
    w = synth.q4_0_weights(n, k, 301 + k)
    # exact value of the native computation: sum_b int_dot * sx_b * sw_b in f64
    part = orc.block_dots(x, w, m, k, n).astype(np.float64)
    sw = w.reshape(n, k // 32, 18)[:, :, 0:2].copy().view(np.float16).astype(np.float64)[..., 0]
    sx = np.stack([orc.quantize_row_q8_0(x[r])[1] for r in range(m)]).astype(np.float64)
    exact = (part * sx[:, None, :] * sw[None]).sum(axis=2).reshape(-1)
    check_parity(rq.matmul_f32_q4_native(x, w, m, k, n), orc.matmul("q4_native", x, w, m, k, n, 8), exact)


def test_native_q4_1(rq, orc, gpu):
    m, n, k = 2, 257, 1024
    x = synth.activations(m, k, 401)
    w = synth.q4_1_weights(n, k, 402)
    assert_close(rq.matmul_f32_q4_1_native(x, w, m, k, n), orc.matmul("q4_1_native", x, w, m, k, n))


# ---- edge cases -----------------------------------------------------------------------
def test_k_zero_gives_zeros(rq, gpu):
    y = rq.matmul_f32_q4(np.zeros(0, np.float32), np.zeros(0, np.uint8), 2, 0, 5)
    assert np.array_equal(y, np.zeros(10, np.float32))


def test_zero_scales_and_zero_input(rq, orc, gpu):
    n, k = 9, 128
    w = synth.q4_0_weights(n, k, 5)
    w.reshape(n, -1, 18)[:, :, 0:2] = 0  # all scales 0
    x = synth.activations(1, k, 6)
    assert np.array_equal(rq.matmul_f32_q4(x, w, 1, k, n), np.zeros(n, np.float32))
    w2 = synth.q4_0_weights(n, k, 7)
    assert np.array_equal(rq.matmul_f32_q4(np.zeros(k, np.float32), w2, 1, k, n), np.zeros(n, np.float32))


def test_f16_subnormal_weight_scales(rq, orc, gpu):
    # config-1 style scales: many below the f16 normal minimum; they must not flush
    n, k = 64, 1024
    w = synth.q8_0_weights(n, k, 9, d_sigma=0.0005)
    d = w.reshape(n, -1, 34)[:, :, 0:2].copy().view(np.uint16)
    assert np.mean((d & 0x7C00) == 0) > 0.5
    x = synth.activations(1, k, 10)
    # a flushed subnormal scale would zero whole blocks: far outside this bar
    check_parity(rq.matmul_f32_q8(x, w, 1, k, n), orc.matmul("q8", x, w, 1, k, n),
                 exact_f64(orc, "q8", x, w, 1, k, n), atol=1e-6)


def test_nan_activation_poisons_outputs(rq, gpu):
    n, k = 4, 64
    w = synth.q4_0_weights(n, k, 12)
    x = synth.activations(1, k, 13)
    x[0, 40] = np.nan
    assert np.all(np.isnan(rq.matmul_f32_q4(x, w, 1, k, n)))


# ---- native mode at prefill row counts (config-4 weight, 4096 x 4096) -----------------
def _native_exact(orc, x, w, m, k, n):
    """f64 value of matmul_f32_q4_native (quantize.rs:326-394): the exact int32
    block dots times the f16-rounded activation scale and the weight scale."""
    part = orc.block_dots(x, w, m, k, n).astype(np.float64)
    sw = w.reshape(n, k // 32, 18)[:, :, 0:2].copy().view(np.float16).astype(np.float64)[..., 0]
    sx = np.stack([orc.quantize_row_q8_0(x[r])[1] for r in range(m)]).astype(np.float64)
    return (part.reshape(m, n, k // 32) * sx[:, None, :] * sw[None]).sum(axis=2).reshape(-1), part


@pytest.mark.parametrize("m", [5, 16, 64, 512])
def test_native_q4_0_prefill_rows_config4(rq, orc, gpu, m):
    n = k = 4096
    print(f"case native q4_0 m={m} n={n} k={k}", flush=True)
    x = synth.activations(m, k, 0x5EED0104 + m)
    w = synth.q4_0_weights(n, k, 0x5EED0004)
    if m <= 16:
        exact, part = _native_exact(orc, x, w, m, k, n)
        # the integer stage, bit for bit (simd.rs:562-581)
        assert np.array_equal(rq.q4_0_q8_0_block_dots(x, w, m, k, n).astype(np.float64), part)
        check_parity(rq.matmul_f32_q4_native(x, w, m, k, n), orc.matmul("q4_native", x, w, m, k, n, 8), exact)
    else:
        want = orc.matmul("q4_native", x, w, m, k, n, 8)
        assert_close(rq.matmul_f32_q4_native(x, w, m, k, n), want)


@pytest.mark.parametrize("m", [5, 16, 64, 512])
def test_native_q4_1_prefill_rows_config4(rq, orc, gpu, m):
    n = k = 4096
    print(f"case native q4_1 m={m} n={n} k={k}", flush=True)
    x = synth.activations(m, k, 0x5EED0204 + m)
    w = synth.q4_1_weights(n, k, 0x5EED0014)
    assert_close(rq.matmul_f32_q4_1_native(x, w, m, k, n), orc.matmul("q4_1_native", x, w, m, k, n, 8))
