"""Device expansion of every GGML type to f32 (rdl_dequantize_gguf_dev,
rdl_gguf_upload_tensor_f32) against the oracle's restatement of the
reference's load-time dequantizers (rustml/gguf/main/src/core/parser.rs:
371-776) and Tensor::to_f32 (tensor.rs:535-639): bit-exact, including the
zero tail past the last whole block."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# GGML type id -> (block elements, block bytes, oracle kind, f16 fields, f32 fields)
TYPES = {
    2: (32, 18, "q4_0", [0], []),
    3: (32, 20, "q4_1_legacy", [0, 2], []),
    6: (32, 22, "q5_0", [0], []),
    7: (32, 24, "q5_1", [0, 2], []),
    8: (32, 34, "q8_0", [0], []),
    9: (32, 40, "q8_1", [], [0]),
    10: (256, 84, "q2k", [80, 82], []),
    11: (256, 110, "q3k", [108], []),
    12: (256, 144, "q4k", [0, 2], []),
    13: (256, 176, "q5k", [0, 2], []),
    14: (256, 210, "q6k", [208], []),
    15: (256, 292, "q8k", [], [0]),
}


def random_blocks(t, nblocks, seed):
    """Random bytes with finite scale fields (so no NaN payload rules enter)."""
    bs, bb, _, f16s, f32s = TYPES[t]
    r = np.random.default_rng(seed)
    blk = r.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)
    for off in f16s:
        blk[:, off:off + 2] = r.normal(0, 0.05, nblocks).astype(np.float16).view(np.uint8).reshape(nblocks, 2)
    for off in f32s:
        blk[:, off:off + 4] = r.normal(0, 0.05, nblocks).astype(np.float32).view(np.uint8).reshape(nblocks, 4)
    return blk.reshape(-1)


def oracle_f32(orc, t, raw, n_elements):
    bs = TYPES[t][0]
    full = n_elements // bs * bs
    out = np.zeros(n_elements, np.float32)
    if full:
        out[:full] = orc.to_f32(TYPES[t][2], raw, full)
    return out


@pytest.mark.parametrize("t", sorted(TYPES))
@pytest.mark.parametrize("extra", [0, 7])
def test_dequantize_every_type(rq, orc, gpu, t, extra):
    import torch

    from rdlquant import gguf
    bs = TYPES[t][0]
    nblocks = 37
    raw = random_blocks(t, nblocks, 100 + t)
    n = nblocks * bs + extra
    src = torch.from_numpy(raw).to(gpu)
    dst = torch.full((n + 8,), 7.0, dtype=torch.float32, device=gpu)
    gguf.dequantize_gguf_dev(t, src.data_ptr(), src.numel(), n, dst.data_ptr())
    torch.cuda.synchronize()
    got = dst.cpu().numpy()
    assert np.array_equal(got[:n], oracle_f32(orc, t, raw, n))
    assert (got[n:] == 7.0).all()


def test_f16_and_f32(rq, gpu):
    import torch

    from rdlquant import gguf
    r = np.random.default_rng(5)
    h = r.normal(0, 3, 1000).astype(np.float16)
    h[:4] = [0.0, -0.0, 6.1e-5, -2.0 ** -24]  # zeros, a normal at the bottom, the smallest subnormal
    src = torch.from_numpy(h.view(np.uint8).copy()).to(gpu)
    dst = torch.empty(1000, dtype=torch.float32, device=gpu)
    gguf.dequantize_gguf_dev(1, src.data_ptr(), src.numel(), 1000, dst.data_ptr())
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy().view(np.uint32), h.astype(np.float32).view(np.uint32))
    f = r.normal(0, 1, 100).astype(np.float32)
    src = torch.from_numpy(f.view(np.uint8).copy()).to(gpu)
    dst = torch.empty(100, dtype=torch.float32, device=gpu)
    gguf.dequantize_gguf_dev(0, src.data_ptr(), src.numel(), 100, dst.data_ptr())
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy(), f)


def test_upload_tensor_f32_every_type(rq, orc, gpu, tmp_path):
    """A file holding one tensor of every type: load_tensors' F32 view of each."""
    import torch

    from rdlquant import gguf, gguf_writer as W
    b = W.GgufBuilder().add_string("general.architecture", "llama")
    want = {}
    for t in sorted(TYPES):
        bs = TYPES[t][0]
        raw = random_blocks(t, 6, 200 + t)
        n = 6 * bs
        b.add_tensor_data(f"t{t}", [bs, 6], t, raw)
        want[f"t{t}"] = oracle_f32(orc, t, raw, n)
    h = np.random.default_rng(3).normal(0, 1, 96).astype(np.float16)
    b.add_tensor_data("f16", [96], W.GGML_F16, h)
    want["f16"] = h.astype(np.float32)
    p = tmp_path / "types.gguf"
    b.write(p)
    f = gguf.GGUFFile.parse_header(p)
    for name, w in want.items():
        dst = torch.empty(w.size, dtype=torch.float32, device=gpu)
        f.upload_tensor_f32(name, dst.data_ptr(), dst.numel())
        assert np.array_equal(dst.cpu().numpy(), w), name
    with pytest.raises(rq.ShapeMismatch):
        dst = torch.empty(10, dtype=torch.float32, device=gpu)
        f.upload_tensor_f32("t14", dst.data_ptr(), dst.numel())
