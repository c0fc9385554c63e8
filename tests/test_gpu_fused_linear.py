"""rdl_linear_fused_dev: the Q4_0 Linear with an RMSNorm / SwiGLU prologue and
a residual epilogue (one launch), against the same operations done apart on
the CPU restatement."""
import numpy as np
import pytest

from oracle import oracle as orc
from parity import check_parity, exact_f64
from rdlquant import synth

pytestmark = pytest.mark.gpu

# (2, 20000, 2048), (1, 33001, 4096): taller than one round of workgroups at
# 4 rows a wave, so the store epilogue takes 8 rows a wave (ragged last group)
SHAPES = [(1, 320, 256), (3, 1000, 4096), (1, 4096, 14336), (4, 64, 512), (2, 20000, 2048), (1, 33001, 4096)]


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def run(rq, torch, w, x, xs, m, n, prologue, g=None, eps=0.0, y0=None):
    W = rq.Weight.upload(w, rq.DTYPE_Q4_0, n, x.shape[1] if prologue != rq.PROLOGUE_SWIGLU else x.shape[1] // 2)
    xd = dev(torch, x)
    yd = dev(torch, y0) if y0 is not None else torch.empty(m * n, dtype=torch.float32, device="cuda:0")
    gd = dev(torch, g) if g is not None else None
    W.forward_fused_dev(xd.data_ptr(), xs, m, yd.data_ptr(), prologue, gd.data_ptr() if gd is not None else 0,
                        eps, rq.EPILOGUE_RESIDUAL if y0 is not None else rq.EPILOGUE_STORE)
    torch.cuda.synchronize()
    return yd.cpu().numpy().reshape(-1)


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_plain_equals_linear_forward(rq, gpu, m, n, k):
    import torch
    w = synth.q4_0_weights(n, k, 3)
    x = synth.activations(m, k, 4)
    got = run(rq, torch, w, x, k, m, n, rq.PROLOGUE_NONE)
    W = rq.Weight.upload(w, rq.DTYPE_Q4_0, n, k)
    xd, yd = dev(torch, x), torch.empty(m * n, dtype=torch.float32, device="cuda:0")
    W.forward_dev(xd.data_ptr(), m, yd.data_ptr())
    torch.cuda.synchronize()
    assert np.array_equal(got, yd.cpu().numpy())


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_rmsnorm_prologue(rq, orc, gpu, m, n, k):
    import torch
    w = synth.q4_0_weights(n, k, 5)
    x = synth.activations(m, k, 6) * np.float32(3.0)
    g = (1.0 + 0.2 * np.random.default_rng(7).standard_normal(k)).astype(np.float32)
    got = run(rq, torch, w, x, k, m, n, rq.PROLOGUE_RMSNORM, g, 1e-5)
    xn = orc.rms_norm(x, g, 1e-5)
    check_parity(got, orc.matmul("q4", xn, w, m, k, n, threads=8), exact_f64(orc, "q4", xn, w, m, k, n))


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_swiglu_prologue_with_residual(rq, orc, gpu, m, n, k):
    import torch
    w = synth.q4_0_weights(n, k, 8)
    gu = synth.activations(m, 2 * k, 9) * np.float32(2.0)
    y0 = synth.activations(m, n, 10).reshape(-1)
    got = run(rq, torch, w, gu, 2 * k, m, n, rq.PROLOGUE_SWIGLU, y0=y0)
    gate, up = gu[:, :k], gu[:, k:]
    h = ((gate * (np.float32(1.0) / (np.float32(1.0) + np.exp(-gate)))) * up).astype(np.float32)
    want = orc.matmul("q4", h, w, m, k, n, threads=8) + y0
    exact = exact_f64(orc, "q4", h, w, m, k, n) + y0.astype(np.float64)
    check_parity(got, want, exact)


def test_residual_epilogue(rq, orc, gpu):
    import torch
    m, n, k = 2, 700, 1024
    w = synth.q4_0_weights(n, k, 11)
    x = synth.activations(m, k, 12)
    y0 = synth.activations(m, n, 13).reshape(-1)
    got = run(rq, torch, w, x, k, m, n, rq.PROLOGUE_NONE, y0=y0)
    check_parity(got, orc.matmul("q4", x, w, m, k, n) + y0,
                 exact_f64(orc, "q4", x, w, m, k, n) + y0.astype(np.float64))


def test_rejects_unsupported_shapes(rq, gpu):
    import torch
    w = synth.q4_0_weights(8, 96, 1)  # 3 blocks per row: odd
    W = rq.Weight.upload(w, rq.DTYPE_Q4_0, 8, 96)
    x = torch.zeros(96, device="cuda:0")
    y = torch.zeros(8, device="cuda:0")
    with pytest.raises(rq.QuantError):
        W.forward_fused_dev(x.data_ptr(), 96, 1, y.data_ptr())


@pytest.mark.parametrize("m,ffn,k", [(1, 160, 256), (3, 1000, 4096), (4, 14336, 4096), (1, 32, 8192)])
def test_swiglu_pair_epilogue(rq, orc, gpu, m, ffn, k):
    import torch
    gate = synth.q4_0_weights(ffn, k, 21).reshape(ffn, -1)
    up = synth.q4_0_weights(ffn, k, 22).reshape(ffn, -1)
    inter = np.empty((2 * ffn, gate.shape[1]), np.uint8)
    inter[0::2], inter[1::2] = gate, up  # rows 2j, 2j+1 = gate_j, up_j
    x = synth.activations(m, k, 23)
    g = (1.0 + 0.1 * np.random.default_rng(24).standard_normal(k)).astype(np.float32)
    W = rq.Weight.upload(inter.reshape(-1), rq.DTYPE_Q4_0, 2 * ffn, k)
    xd, gd = dev(torch, x), dev(torch, g)
    yd = torch.empty(m * ffn, dtype=torch.float32, device="cuda:0")
    W.forward_fused_dev(xd.data_ptr(), k, m, yd.data_ptr(), rq.PROLOGUE_RMSNORM, gd.data_ptr(), 1e-5,
                        rq.EPILOGUE_SWIGLU)
    torch.cuda.synchronize()
    got = yd.cpu().numpy().reshape(m, ffn)
    xn = orc.rms_norm(x, g, 1e-5)
    a = orc.matmul("q4", xn, gate.reshape(-1), m, k, ffn, threads=8).reshape(m, ffn)
    b = orc.matmul("q4", xn, up.reshape(-1), m, k, ffn, threads=8).reshape(m, ffn)
    want = (a * (np.float32(1.0) / (np.float32(1.0) + np.exp(-a)))) * b
    # the product of two in-tolerance factors: bar on each scaled by the other
    assert np.all(np.abs(got - want) <= 2e-3 * np.abs(want) + 2e-4 * (np.abs(b) + np.abs(a) + 1.0))
