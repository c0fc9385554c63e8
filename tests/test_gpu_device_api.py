"""GPU tests of the device-resident entry points (weights in HBM, torch streams)."""
import numpy as np
import pytest

from rdlquant import synth

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-4
KIND = {2: "q4", 3: "q4_1", 8: "q8", 12: "q4k", 14: "q6k"}
DEQ = {2: "q4_0", 3: "q4_1", 8: "q8_0", 12: "q4k", 14: "q6k"}


def close(got, want, exact):
    got, want = np.asarray(got, np.float64).ravel(), np.asarray(want, np.float64).ravel()
    assert np.all(np.abs(got - exact) <= ATOL + RTOL * np.abs(exact))
    assert np.all(np.abs(got - want) <= ATOL + RTOL * np.abs(want) + np.abs(want - exact))


def dev_weight(rq, torch, w, dtype, n, k):
    t = torch.from_numpy(w).cuda()
    return t, rq.Weight.wrap_device(t.data_ptr(), t.numel(), dtype, n, k, keepalive=t)


@pytest.mark.parametrize("dtype,n,k", [(2, 11008, 4096), (8, 4096, 4096), (12, 4096, 14336),
                                       (2, 4096, 14336), (3, 100, 512), (2, 7, 20480),
                                       (14, 32000, 4096), (14, 4096, 14336), (14, 9, 1280)])
@pytest.mark.parametrize("m", [1, 2])
def test_prepared_records_path(rq, orc, gpu, dtype, n, k, m):
    import torch

    x = synth.activations(m, k, 50 + n)
    w = synth.weights(dtype, n, k, 51 + k)
    _, h = dev_weight(rq, torch, w, dtype, n, k)
    xt = torch.from_numpy(x.reshape(-1)).cuda()
    rec = torch.empty(rq.activation_record_bytes(m, k, rq.MODE_FLOAT), dtype=torch.uint8, device="cuda")
    yt = torch.empty(m * n, dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    rq.prepare_activations_dev(xt.data_ptr(), m, k, rq.MODE_FLOAT, rec.data_ptr(), s)
    h.forward_prepared_dev(rec.data_ptr(), m, yt.data_ptr(), rq.MODE_FLOAT, s)
    torch.cuda.synchronize()
    want = orc.matmul(KIND[dtype], x, w, m, k, n, threads=8)
    wd = orc.to_f32(DEQ[dtype], w, n * k).reshape(n, k).astype(np.float64)
    close(yt.cpu().numpy(), want, (x.astype(np.float64) @ wd.T).ravel())
    # the fused single-launch path on the same data
    yf = torch.empty_like(yt)
    h.forward_dev(xt.data_ptr(), m, yf.data_ptr(), rq.MODE_FLOAT, s)
    torch.cuda.synchronize()
    close(yf.cpu().numpy(), want, (x.astype(np.float64) @ wd.T).ravel())


def test_prepared_native_bit_equal_to_fused(rq, gpu):
    import torch

    n, k = 3000, 4096
    x = synth.activations(1, k, 61)
    w = synth.q4_0_weights(n, k, 62)
    _, h = dev_weight(rq, torch, w, 2, n, k)
    xt = torch.from_numpy(x.reshape(-1)).cuda()
    s = torch.cuda.current_stream().cuda_stream
    rec = torch.empty(rq.activation_record_bytes(1, k, rq.MODE_NATIVE), dtype=torch.uint8, device="cuda")
    y1 = torch.empty(n, dtype=torch.float32, device="cuda")
    y2 = torch.empty(n, dtype=torch.float32, device="cuda")
    rq.prepare_activations_dev(xt.data_ptr(), 1, k, rq.MODE_NATIVE, rec.data_ptr(), s)
    h.forward_prepared_dev(rec.data_ptr(), 1, y1.data_ptr(), rq.MODE_NATIVE, s)
    h.forward_dev(xt.data_ptr(), 1, y2.data_ptr(), rq.MODE_NATIVE, s)
    torch.cuda.synchronize()
    # both reduce exact int32 block dots; only the f32 summation order may differ
    a, b = y1.cpu().numpy().astype(np.float64), y2.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(a - b) <= 1e-5 + 1e-5 * np.abs(a))


@pytest.mark.parametrize("dtype,kind", [(2, "q4_0"), (8, "q8_0"), (3, "q4_1"), (12, "q4k"), (14, "q6k")])
def test_dequantize_rows_exact(rq, orc, gpu, dtype, kind):
    import torch

    n, k = 300, 4096
    w = synth.weights(dtype, n, k, 70 + dtype)
    _, h = dev_weight(rq, torch, w, dtype, n, k)
    rows = np.array([0, 299, 17, 17, 150], dtype=np.int32)
    rt = torch.from_numpy(rows).cuda()
    out = torch.empty(len(rows) * k, dtype=torch.float32, device="cuda")
    h.dequantize_rows_dev(rt.data_ptr(), len(rows), out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    full = orc.to_f32(kind, w, n * k).reshape(n, k)
    assert np.array_equal(out.cpu().numpy().reshape(len(rows), k), full[rows])


def test_block_dots_dev_exact(rq, orc, gpu):
    import torch

    n, k = 1000, 4096
    x = synth.activations(1, k, 81)
    w = synth.q4_0_weights(n, k, 82)
    _, h = dev_weight(rq, torch, w, 2, n, k)
    xt = torch.from_numpy(x.reshape(-1)).cuda()
    part = torch.empty(n * (k // 32), dtype=torch.int32, device="cuda")
    h.block_dots_dev(xt.data_ptr(), part.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(part.cpu().numpy().reshape(1, n, k // 32), orc.block_dots(x, w, 1, k, n))


def test_graph_replays_match_eager(rq, gpu):
    """Captured launches replayed several times, with eager work in between,
    reproduce the eager result bit for bit (the kernels are deterministic)."""
    import torch

    n, k = 4096, 4096
    hs = []
    for i in range(3):
        hs.append(dev_weight(rq, torch, synth.q4_0_weights(n, k, 90 + i), 2, n, k))
    xt = torch.from_numpy(synth.activations(1, k, 93).reshape(-1)).cuda()
    ys = [torch.empty(n, dtype=torch.float32, device="cuda") for _ in range(3)]
    s = torch.cuda.current_stream().cuda_stream
    for (_, h), y in zip(hs, ys):
        h.forward_dev(xt.data_ptr(), 1, y.data_ptr(), rq.MODE_FLOAT, s)
    torch.cuda.synchronize()
    eager = [y.cpu().numpy().copy() for y in ys]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        cs = torch.cuda.current_stream().cuda_stream
        for (_, h), y in zip(hs, ys):
            h.forward_dev(xt.data_ptr(), 1, y.data_ptr(), rq.MODE_FLOAT, cs)
    for rep in range(4):
        for y in ys:
            y.fill_(-1.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for y, e in zip(ys, eager):
            assert np.array_equal(y.cpu().numpy(), e), f"replay {rep}"
        _ = (xt * 2).sum().item()  # unrelated eager work between replays


def test_skinny_gemm_calls_on_one_handle(rq, gpu):
    """Prefill products of 5 .. 64 rows through one device handle: its
    stream's work memory grows with the largest call, the split GEMM's
    counters return to zero after every launch, and each result equals the
    synchronous entry point's (same kernels, same split) bit for bit."""
    import torch

    n, k = 4096, 4096
    w = synth.q4_0_weights(n, k, 140)
    _, h = dev_weight(rq, torch, w, 2, n, k)
    s = torch.cuda.current_stream().cuda_stream
    for m in (16, 64, 16, 5, 40, 64):
        x = synth.activations(m, k, 141 + m)
        xt = torch.from_numpy(x.reshape(-1)).cuda()
        yt = torch.empty(m * n, dtype=torch.float32, device="cuda")
        h.forward_dev(xt.data_ptr(), m, yt.data_ptr(), rq.MODE_FLOAT, s)
        torch.cuda.synchronize()
        want = rq.matmul_f32_q4(x, w, m, k, n)
        assert np.array_equal(yt.cpu().numpy(), want.reshape(-1)), f"m={m}"


def test_sliced_gemm_shapes_share_the_stream_work_memory(rq, gpu):
    """Products of at most 16 rows (128-row strips, K-slices joined through
    partials and a counter per strip in the stream's work memory): three
    weights of different layouts alternate on one stream, and every result
    equals the synchronous entry point's (fresh work memory) bit for bit --
    each launch leaves the shared counters at zero for the next, whatever its
    shape."""
    import torch

    shapes = [(4096, 4096, 160), (1000, 2048, 161), (6144, 4096, 162)]
    hs = []
    for n, k, seed in shapes:
        w = synth.q4_0_weights(n, k, seed)
        _, h = dev_weight(rq, torch, w, 2, n, k)
        hs.append((n, k, w, h))
    s = torch.cuda.current_stream().cuda_stream
    for rep, (i, m) in enumerate([(0, 16), (1, 9), (2, 16), (0, 3 + 2), (1, 16), (2, 11), (0, 16)]):
        n, k, w, h = hs[i]
        x = synth.activations(m, k, 170 + rep)
        xt = torch.from_numpy(x.reshape(-1)).cuda()
        yt = torch.empty(m * n, dtype=torch.float32, device="cuda")
        h.forward_dev(xt.data_ptr(), m, yt.data_ptr(), rq.MODE_FLOAT, s)
        torch.cuda.synchronize()
        want = rq.matmul_f32_q4(x, w, m, k, n)
        assert np.array_equal(yt.cpu().numpy(), want.reshape(-1)), f"call {rep}: n={n} k={k} m={m}"


@pytest.mark.parametrize("dtype,n,k,m,mode", [(2, 4096, 4096, 1, 0), (2, 4096, 4096, 16, 0), (2, 300, 1024, 70, 0),
                                            (2, 4096, 4096, 3, 1), (8, 1000, 2048, 2, 0), (12, 2048, 4096, 5, 0),
                                            (3, 257, 1024, 2, 1)])
def test_linear_bias(rq, orc, gpu, dtype, n, k, m, mode):
    """Linear::forward's optional bias (linear.rs:172-176: output.add(bias)):
    the product plus bias[j] in f32, equal bit for bit to the unbiased
    device product plus the bias on the host, and within the bar of the
    oracle's product plus the bias; a NULL bias is the plain product."""
    import torch

    x = synth.activations(m, k, 190 + n + m)
    w = synth.weights(dtype, n, k, 191 + k)
    _, h = dev_weight(rq, torch, w, dtype, n, k)
    bias = np.random.default_rng(192 + n).standard_normal(n).astype(np.float32)
    xt = torch.from_numpy(x.reshape(-1)).cuda()
    bt = torch.from_numpy(bias).cuda()
    y0 = torch.empty(m * n, dtype=torch.float32, device="cuda")
    y1 = torch.empty(m * n, dtype=torch.float32, device="cuda")
    y2 = torch.empty(m * n, dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    md = rq.MODE_NATIVE if mode else rq.MODE_FLOAT
    h.forward_dev(xt.data_ptr(), m, y0.data_ptr(), md, s)
    h.forward_bias_dev(xt.data_ptr(), m, bt.data_ptr(), y1.data_ptr(), md, s)
    h.forward_bias_dev(xt.data_ptr(), m, 0, y2.data_ptr(), md, s)
    torch.cuda.synchronize()
    plain = y0.cpu().numpy().reshape(m, n)
    got = y1.cpu().numpy().reshape(m, n)
    assert np.array_equal(got, (plain + bias[None, :]).astype(np.float32))
    assert np.array_equal(y2.cpu().numpy().reshape(m, n), plain)
    kind = KIND[dtype] + ("_native" if mode else "")
    want = orc.matmul(kind, x, w, m, k, n, threads=8).reshape(m, n) + bias[None, :]
    if mode:  # the native products: exact int32 block dots, as the oracle's
        assert np.all(np.abs(got - want) <= ATOL + RTOL * np.abs(want))
    else:  # float: the exact (f64) value, and the oracle within its own rounding
        wd = orc.to_f32(DEQ[dtype], w, n * k).reshape(n, k).astype(np.float64)
        close(got, want, (x.astype(np.float64).reshape(m, k) @ wd.T + bias[None, :]).ravel())


def test_release_stream_work(rq, gpu):
    """rdl_release_stream_work frees a stream's work memory: products on a
    stream of their own before and after the release (which allocates again)
    equal the synchronous entry point's bit for bit; releasing a stream with
    no work memory, or twice, is a no-op."""
    import torch

    n, k = 4096, 4096
    w = synth.q4_0_weights(n, k, 180)
    _, h = dev_weight(rq, torch, w, 2, n, k)
    st = torch.cuda.Stream()
    rq.release_stream_work(st.cuda_stream)  # nothing kept yet
    for rep, m in enumerate((16, 7, 1, 40)):
        x = synth.activations(m, k, 181 + rep)
        xt = torch.from_numpy(x.reshape(-1)).cuda()
        yt = torch.empty(m * n, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        h.forward_dev(xt.data_ptr(), m, yt.data_ptr(), rq.MODE_FLOAT, st.cuda_stream)
        rq.release_stream_work(st.cuda_stream)  # waits for the stream, then frees
        want = rq.matmul_f32_q4(x, w, m, k, n)
        assert np.array_equal(yt.cpu().numpy(), want.reshape(-1)), f"m={m}"
    rq.release_stream_work(st.cuda_stream)


def test_skinny_gemm_graph_replays_match_eager(rq, gpu):
    """A 16-row prefill product captured in a graph (graph-owned scratch and
    counters, zeroed by a kernel on every replay) reproduces the eager result
    bit for bit on every replay."""
    import torch

    n, k, m = 4096, 4096, 16
    _, h = dev_weight(rq, torch, synth.q4_0_weights(n, k, 150), 2, n, k)
    xt = torch.from_numpy(synth.activations(m, k, 151).reshape(-1)).cuda()
    y = torch.empty(m * n, dtype=torch.float32, device="cuda")
    h.forward_dev(xt.data_ptr(), m, y.data_ptr(), rq.MODE_FLOAT, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    eager = y.cpu().numpy().copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        h.forward_dev(xt.data_ptr(), m, y.data_ptr(), rq.MODE_FLOAT, torch.cuda.current_stream().cuda_stream)
    for rep in range(4):
        y.fill_(-1.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), eager), f"replay {rep}"
        _ = (xt * 2).sum().item()  # unrelated eager work between replays


def test_stream_read_folds_every_word(rq, gpu):
    """The plain-read measurement kernel reads every 16-byte unit once: the
    XOR of its per-workgroup words is the XOR of all 32-bit words."""
    import torch

    nbytes = 3 * 2**20 + 48
    data = np.random.default_rng(5).integers(0, 2**32, nbytes // 4, dtype=np.uint32)
    buf = torch.from_numpy(data.view(np.int32)).cuda()
    out = torch.zeros(2048, dtype=torch.int32, device="cuda")
    rq.stream_read_dev(buf.data_ptr(), nbytes, out.data_ptr(), out.numel(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32)) == np.bitwise_xor.reduce(data)


def test_time_next_launch(rq, gpu):
    import torch

    n, k = 11008, 4096
    _, h = dev_weight(rq, torch, synth.q4_0_weights(n, k, 95), 2, n, k)
    xt = torch.from_numpy(synth.activations(1, k, 96).reshape(-1)).cuda()
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(); b.record()
    torch.cuda.synchronize()
    rq.time_next_launch(a.cuda_event, b.cuda_event)
    h.forward_dev(xt.data_ptr(), 1, y.data_ptr(), rq.MODE_FLOAT, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b)
    assert 0.0005 < ms < 5.0, ms


@pytest.mark.parametrize("m", [16, 32, 48, 64])
def test_gemm_combine_paths_bit_equal(rq, gpu, m):
    """The K-slice combine of the 5-64-row GEMMs both ways: XCD-local (each
    strip's slices on one XCD, partials through its L2; the default where the
    placement probe passes) and agent-coherent (rdl_set_gemm_combine
    (RDL_COMBINE_COHERENT): write-through partials, device-scope counter).
    Eager calls and graph replays, equal bit for bit to each other and to the
    synchronous entry point."""
    import torch

    n, k = 4096, 4096
    w = synth.q4_0_weights(n, k, 180 + m)
    x = synth.activations(m, k, 190 + m)
    _, h = dev_weight(rq, torch, w, 2, n, k)
    xt = torch.from_numpy(x.reshape(-1)).cuda()
    y = torch.empty(m * n, dtype=torch.float32, device="cuda")
    print(f"case combine paths m={m}", flush=True)
    got = {}
    try:
        for mode in (rq.COMBINE_AUTO, rq.COMBINE_COHERENT):
            rq.set_gemm_combine(mode)
            y.fill_(-1.0)
            h.forward_dev(xt.data_ptr(), m, y.data_ptr(), rq.MODE_FLOAT, torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            eager = y.cpu().numpy().copy()
            assert rq.gemm_combine() == (mode, mode == rq.COMBINE_AUTO)  # the local path did run by default
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                h.forward_dev(xt.data_ptr(), m, y.data_ptr(), rq.MODE_FLOAT, torch.cuda.current_stream().cuda_stream)
            for rep in range(3):
                y.fill_(-1.0)
                torch.cuda.synchronize()
                g.replay()
                torch.cuda.synchronize()
                assert np.array_equal(y.cpu().numpy(), eager), f"mode {mode} replay {rep}"
                _ = (xt * 2).sum().item()  # unrelated eager work between replays
            got[mode] = eager
    finally:
        rq.set_gemm_combine(rq.COMBINE_AUTO)
    assert np.array_equal(got[rq.COMBINE_AUTO].view(np.uint32), got[rq.COMBINE_COHERENT].view(np.uint32))
    assert np.array_equal(got[rq.COMBINE_AUTO], rq.matmul_f32_q4(x, w, m, k, n))

