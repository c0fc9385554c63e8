"""rdl_linear_forward_dev_noalloc (static per-GPU scratch, no device
allocation) against rdl_linear_forward_dev on the same inputs: two calls in
a row, the second with fewer rows, for each path that uses scratch memory
(the prefill GEMMs' activation split, native-mode and Q8_0 activation
records).  Both entry points run the same kernels, so the outputs must be
bit-identical."""
import numpy as np
import pytest

from rdlquant import synth

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,mode,n,k,rows", [
    (2, 0, 4096, 4096, (96, 40)),    # Q4_0 float: matrix-core GEMM, x split in scratch
    (2, 0, 4096, 4096, (16, 5)),     # Q4_0 float, one x tile: K-slice partials in scratch
    (2, 0, 4096, 4096, (64, 33)),    # Q4_0 float, four then three x tiles
    (2, 1, 4096, 4096, (24, 6)),     # Q4_0 native: Q8_0 records in scratch
    (3, 1, 1000, 2048, (9, 5)),      # Q4_1 native records
    (8, 0, 512, 1024, (33, 7)),      # Q8_0 float: tile GEMM (33 rows), then records (7 rows)
    (12, 0, 1024, 4096, (40, 16)),   # Q4_K float: tile GEMM, x split and x' block sums in scratch
    (14, 0, 1000, 2048, (20, 17)),   # Q6_K float: tile GEMM, x split in scratch
])
def test_noalloc_matches_allocating_entry_point(rq, gpu, dtype, mode, n, k, rows):
    import torch
    print(f"case noalloc dtype={dtype} mode={mode} n={n} k={k} rows={rows}", flush=True)
    w = rq.Weight.upload(synth.weights(dtype, n, k, 31 + dtype), dtype, n, k)
    stream = torch.cuda.current_stream().cuda_stream
    for i, m in enumerate(rows):
        x = torch.from_numpy(synth.activations(m, k, 70 + i)).to(gpu)
        want = torch.full((m, n), np.nan, dtype=torch.float32, device=gpu)
        got = torch.full((m, n), np.nan, dtype=torch.float32, device=gpu)
        w.forward_dev(x.data_ptr(), m, want.data_ptr(), mode, stream)
        w.forward_dev_noalloc(x.data_ptr(), m, got.data_ptr(), mode, stream)
        torch.cuda.synchronize()
        g, r = got.cpu().numpy(), want.cpu().numpy()
        assert np.all(np.isfinite(r))
        assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), f"call {i}, m={m}"
    w.free()


def test_noalloc_rejects_products_beyond_its_scratch(rq, gpu):
    import torch
    n, k, m = 256, 4096, 2048  # the GEMM's activation split needs 32 MiB > 16 MiB
    w = rq.Weight.upload(synth.weights(2, n, k, 5), 2, n, k)
    x = torch.zeros((m, k), dtype=torch.float32, device=gpu)
    y = torch.zeros((m, n), dtype=torch.float32, device=gpu)
    with pytest.raises(rq.QuantError) as e:
        w.forward_dev_noalloc(x.data_ptr(), m, y.data_ptr(), rq.MODE_FLOAT, torch.cuda.current_stream().cuda_stream)
    assert e.value.status == rq.ERR_UNSUPPORTED
    w.free()
