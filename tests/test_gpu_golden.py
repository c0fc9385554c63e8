"""The HIP path, through the C ABI, against the committed golden fixtures
(tests/golden/*.npz): float outputs within 1e-3 rel + 1e-4 abs, int32 block
partials, Q8_0 activation bytes and dequantized rows bit-exact."""
import os

import numpy as np
import pytest

from parity import assert_close

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name))


@pytest.mark.parametrize("name,fn,native_fn", [
    ("q8_0", "matmul_f32_q8", None),
    ("q4_0", "matmul_f32_q4", "matmul_f32_q4_native"),
    ("q4_1", "matmul_f32_q4_1", "matmul_f32_q4_1_native"),
    ("q4_k", "matmul_f32_q4_k", None),
    ("q6_k", "matmul_f32_q6_k", None),
])
def test_linear_fixture(rq, gpu, name, fn, native_fn):
    d = load(f"linear_{name}.npz")
    m, k, n = (int(v) for v in d["shape"])
    assert_close(getattr(rq, fn)(d["x"], d["w"], m, k, n).reshape(m, n), d["y_float"])
    if native_fn:
        assert_close(getattr(rq, native_fn)(d["x"], d["w"], m, k, n).reshape(m, n), d["y_native"])


@pytest.mark.parametrize("fixture", ["linear_q4_0.npz", "block_dots_q4_0_64x512.npz"])
def test_block_dots_fixture(rq, gpu, fixture):
    d = load(fixture)
    m, n, nb = d["partials"].shape
    got = rq.q4_0_q8_0_block_dots(d["x"], d["w"], m, nb * 32, n)
    assert np.array_equal(got, d["partials"])


def test_quantize_row_fixture(rq, gpu):
    d = load("quantize_row_q8_0.npz")
    q, s = rq.quantize_row_q8_0(d["x"])
    assert np.array_equal(q, d["q"])
    assert np.array_equal(s, d["scales"])


@pytest.mark.parametrize("name,dtype", [("q8_0", 8), ("q4_0", 2), ("q4_1", 3), ("q4_k", 12), ("q6_k", 14)])
def test_dequantized_rows_fixture(rq, gpu, name, dtype):
    import torch
    d = load(f"linear_{name}.npz")
    m, k, n = (int(v) for v in d["shape"])
    w = rq.Weight.upload(d["w"], dtype, n, k)
    rows = torch.arange(n, dtype=torch.int32, device=gpu)
    out = torch.empty(n, k, dtype=torch.float32, device=gpu)
    w.dequantize_rows_dev(rows.data_ptr(), n, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), d["w_f32"])
