"""GGUF reader (include/rdl_gguf.h) on the CPU: no device is touched.

Pins, in order:
  * the reference's own tests: parser.rs:768-794 (bad magic, minimal v3 file)
    and the values rustml/gguf/tests/cli.rs asserts for its builder fixture
    (cli.rs:107-130 file, :112-143 info, :164-260 meta, :262-300 tensors),
    run against both the native reader and the oracle (oracle/gguf_ref.py);
  * the native reader against the oracle on seeded random files holding every
    value type, nested arrays, non-ASCII strings, repeated keys and every GGML
    type; on every prefix of a file (all must fail with the reference's
    end-of-file error); and on single-field corruptions;
  * the writer (rdlquant.gguf_writer) byte-for-byte against the layout the
    cli.rs builder writes;
  * the Llama loader's checks that run before any allocation (missing weight,
    wrong type, wrong dims, unsupported architecture, config validation).
"""
import os
import struct

import numpy as np
import pytest

from oracle import gguf_ref as ref


@pytest.fixture(scope="module")
def G(rq):
    from rdlquant import gguf

    return gguf


@pytest.fixture(scope="module")
def W():
    from rdlquant import gguf_writer

    return gguf_writer


def cli_llama_gguf(W):
    """cli.rs:107-130, build_llama_gguf."""
    b = W.GgufBuilder()
    (b.add_string("general.architecture", "llama")
      .add_u32("llama.embedding_length", 4096)
      .add_u32("llama.feed_forward_length", 11008)
      .add_u32("llama.block_count", 32)
      .add_u32("llama.attention.head_count", 32)
      .add_u32("llama.attention.head_count_kv", 8)
      .add_u32("llama.context_length", 2048)
      .add_f32("llama.attention.layer_norm_rms_epsilon", 1e-5)
      .add_f32("llama.rope.freq_base", 10000.0)
      .add_u32("tokenizer.ggml.bos_token_id", 1)
      .add_u32("tokenizer.ggml.eos_token_id", 2)
      .add_string("general.name", "LLaMA-7B")
      .add_bool("general.quantized", True)
      .add_tensor("token_embd.weight", [4096, 32000], 0, 0)
      .add_tensor("blk.0.attn_q.weight", [4096, 4096], 2, 524288000)
      .add_tensor("blk.0.attn_k.weight", [1024, 4096], 2, 524296192)
      .add_tensor("output.weight", [4096, 32000], 0, 999999999))
    return b.build()


# ---- the reference's unit tests (parser.rs:768-794) --------------------------
def test_magic_check(G):
    bad = bytes(20)
    with pytest.raises(G.InvalidFormat) as e:
        G.GGUFFile.parse_bytes(bad)
    assert "Invalid GGUF magic" in str(e.value)
    with pytest.raises(ref.OracleError) as o:
        ref.parse_bytes(bad)
    assert o.value.kind == "InvalidFormat"


def test_valid_minimal(G):
    data = b"GGUF" + struct.pack("<IQQ", 3, 0, 0)
    f = G.GGUFFile.parse_bytes(data)
    assert f.version == 3 and f.metadata == {} and f.tensor_infos == []
    o = ref.parse_bytes(data)
    assert o.version == 3 and o.metadata == {} and o.tensor_infos == []
    assert f.data_offset == o.data_offset == 32


# ---- the cli.rs fixture and the values its tests assert ---------------------
def test_cli_fixture_info(G, W):
    data = cli_llama_gguf(W)
    for f in (G.GGUFFile.parse_bytes(data), ref.parse_bytes(data)):
        assert f.version == 3
        assert len(f.tensor_infos) == 4
    c = G.GGUFFile.parse_bytes(data).to_model_config()
    assert (c.architecture, c.dim, c.hidden_dim, c.n_layers, c.n_heads, c.n_kv_heads, c.vocab_size,
            c.max_seq_len) == ("llama", 4096, 11008, 32, 32, 8, 32000, 2048)
    o = ref.to_model_config(ref.parse_bytes(data))
    assert (o["architecture"], o["dim"], o["hidden_dim"], o["n_layers"], o["n_heads"], o["n_kv_heads"],
            o["vocab_size"], o["max_seq_len"]) == ("llama", 4096, 11008, 32, 32, 8, 32000, 2048)
    assert (c.bos_token_id, c.eos_token_id) == (1, 2)


def test_cli_fixture_meta(G, W):
    f = G.GGUFFile.parse_bytes(cli_llama_gguf(W))
    md = f.metadata
    assert md["general.architecture"].value == "llama"
    assert md["general.name"].value == "LLaMA-7B"
    assert md["general.quantized"].value is True
    assert md["llama.embedding_length"].value == 4096
    assert md["llama.feed_forward_length"].value == 11008
    assert md["llama.block_count"].value == 32
    assert md["llama.rope.freq_base"].value == 10000.0
    assert abs(md["llama.attention.layer_norm_rms_epsilon"].value - 0.00001) < 1e-12
    assert f.get_u32("llama.block_count") == 32
    assert f.metadata_find("general.name").value == "LLaMA-7B"
    with pytest.raises(G.NotFound) as e:
        f.metadata_find("nonexistent.key")
    assert "Key not found: nonexistent.key" in str(e.value)


def test_cli_fixture_tensors(G, W):
    f = G.GGUFFile.parse_bytes(cli_llama_gguf(W))
    names = [t.name for t in f.tensor_infos]
    assert names == ["token_embd.weight", "blk.0.attn_q.weight", "blk.0.attn_k.weight", "output.weight"]
    q = f.tensor_infos[1]
    assert q.dimensions == [4096, 4096] and q.ggml_type == 2 and q.offset == 524288000
    assert q.n_bytes == 4096 * 4096 // 32 * 18
    # the header alone: load_tensors' bound check fails for every tensor
    with pytest.raises(G.GgufIoError) as e:
        f.tensor_data("output.weight")
    assert "Tensor 'output.weight' data exceeds file bounds" in str(e.value)


def test_minimal_has_no_model_config(G, W):
    """cli.rs:146-160: a file without metadata gives no config (MissingMetadata)."""
    f = G.GGUFFile.parse_bytes(W.GgufBuilder().build())
    assert len(f.tensor_infos) == 0
    with pytest.raises(G.MissingMetadata) as e:
        f.to_model_config()
    assert "llama.embedding_length" in str(e.value)
    with pytest.raises(ref.OracleError) as o:
        ref.to_model_config(ref.parse_bytes(W.GgufBuilder().build()))
    assert o.value.kind == "MissingMetadata" and o.value.message == "llama.embedding_length"


def test_long_string_and_u32_array(G, W):
    """cli.rs:262-289: a 300-byte string and a u32 array of length 5."""
    b = W.GgufBuilder().add_string("long.key", "x" * 300).add_u32_array("test.array", [1, 2, 3, 4, 5])
    md = G.GGUFFile.parse_bytes(b.build()).metadata
    assert md["long.key"].value == "x" * 300
    assert [e.value for e in md["test.array"].value] == [1, 2, 3, 4, 5]
    assert all(e.type == W.U32 for e in md["test.array"].value)


# ---- writer layout ---------------------------------------------------------
def test_writer_matches_cli_builder_layout(W):
    """The bytes cli.rs:72-103 writes for one string, one u32 and one tensor info."""
    b = W.GgufBuilder().add_string("a", "bc").add_u32("n", 7).add_tensor("t", [32, 2], 2, 64)
    want = (b"GGUF" + struct.pack("<IQQ", 3, 1, 2)
            + struct.pack("<Q", 1) + b"a" + struct.pack("<I", 8) + struct.pack("<Q", 2) + b"bc"
            + struct.pack("<Q", 1) + b"n" + struct.pack("<II", 4, 7)
            + struct.pack("<Q", 1) + b"t" + struct.pack("<I", 2) + struct.pack("<QQ", 32, 2)
            + struct.pack("<IQ", 2, 64))
    assert b.build() == want


def test_writer_data_alignment_and_views(G, W, tmp_path):
    rng = np.random.default_rng(7)
    blobs = {"a": rng.integers(0, 256, 18 * 3, dtype=np.uint8), "b": rng.integers(0, 256, 4 * 5, dtype=np.uint8),
             "c": rng.integers(0, 256, 2 * 7, dtype=np.uint8)}
    b = W.GgufBuilder().add_string("k", "v")
    b.add_tensor_data("a", [96], W.GGML_Q4_0, blobs["a"])
    b.add_tensor_data("b", [5], W.GGML_F32, blobs["b"])
    b.add_tensor_data("c", [7], W.GGML_F16, lambda: blobs["c"].tobytes())
    path = tmp_path / "t.gguf"
    size = b.write(path)
    assert size == os.path.getsize(path)
    data = path.read_bytes()
    f = G.GGUFFile.parse_header(path)
    assert f.data_offset % 32 == 0 and all(t.offset % 32 == 0 for t in f.tensor_infos)
    o = ref.parse_bytes(data)
    for i, name in enumerate("abc"):
        got = f.tensor_data(name)
        assert np.array_equal(got, blobs[name])
        assert ref.tensor_bytes(o, data, i) == blobs[name].tobytes()
        assert not got.flags.writeable
    assert f.file_size == len(data)


# ---- native vs oracle on random files ---------------------------------------
_INT_RANGE = {0: (0, 1 << 8), 1: (-(1 << 7), 1 << 7), 2: (0, 1 << 16), 3: (-(1 << 15), 1 << 15),
              4: (0, 1 << 32), 5: (-(1 << 31), 1 << 31), 10: (0, 1 << 64), 11: (-(1 << 63), 1 << 63)}
_ALPHABET = ["a", "Z", "\u00e9", "\u00df", "\u6f22", "\u5b57", "\U0001f642", " ", ".", "\u0000"]


def _rand_of(rng, t, depth):
    """A random value of GGUF type t (arrays: (elem_type, elements))."""
    if t in _INT_RANGE:
        lo, hi = _INT_RANGE[t]
        return lo + int.from_bytes(rng.bytes(8), "little") % (hi - lo)
    if t == 6:
        return float(np.float32(rng.standard_normal() * 10.0 ** int(rng.integers(-5, 5))))
    if t == 12:
        return float(rng.standard_normal() * 10.0 ** int(rng.integers(-50, 50)))
    if t == 7:
        return bool(rng.integers(0, 2))
    if t == 8:
        return "".join(str(rng.choice(_ALPHABET)) for _ in range(int(rng.integers(0, 12))))
    et = _rand_type(rng, depth + 1)
    return (et, [_rand_of(rng, et, depth + 1) for _ in range(int(rng.integers(0, 6)))])


def _rand_type(rng, depth):
    return int(rng.integers(0, 13)) if depth < 3 else int(rng.choice([0, 4, 6, 8, 12]))


def _rand_value(rng, W, depth=0):
    t = _rand_type(rng, depth)
    return t, _rand_of(rng, t, depth)


def _rand_file(rng, W):
    b = W.GgufBuilder(version=int(rng.choice([2, 3])))
    keys = [f"k{i}.{'é' if i % 3 == 0 else 'x'}" for i in range(int(rng.integers(0, 12)))]
    if keys and rng.integers(0, 2):
        keys.append(keys[0])  # a repeated key: the later value wins
    for k in keys:
        t, v = _rand_value(rng, W)
        b.add_value(k, t, v)
    for i in range(int(rng.integers(0, 6))):
        t = int(rng.choice(list(W.GGML_BLOCK)))
        bs, _ = W.GGML_BLOCK[t]
        dims = [int(bs * rng.integers(1, 4))] + [int(rng.integers(1, 4)) for _ in range(int(rng.integers(0, 3)))]
        b.add_tensor(f"blk.{i}.w" if i != 2 else "blk.0.w", dims, t, int(rng.integers(0, 1 << 20)))
    return b.build()


def _plain(v):
    """GGUFValue -> the oracle's (type, value) form."""
    if v.type == 9:
        return (9, [_plain(e) for e in v.value])
    return (v.type, v.value)


def _same_value(a, b):
    if a[0] != b[0]:
        return False
    if a[0] == 9:
        return len(a[1]) == len(b[1]) and all(_same_value(x, y) for x, y in zip(a[1], b[1]))
    if isinstance(a[1], float) and np.isnan(a[1]):
        return np.isnan(b[1])
    return a[1] == b[1]


def _compare(G, data):
    try:
        o = ref.parse_bytes(data)
        oerr = None
    except ref.OracleError as e:
        o, oerr = None, e
    try:
        f = G.GGUFFile.parse_bytes(data)
        ferr = None
    except G.GgufError as e:
        f, ferr = None, e
    if oerr is not None:
        assert ferr is not None, f"oracle raised {oerr}, native parsed"
        kinds = {"Io": G.GgufIoError, "InvalidFormat": G.InvalidFormat, "UnsupportedType": G.UnsupportedType}
        assert isinstance(ferr, kinds[oerr.kind]), (oerr, ferr)
        assert oerr.message in str(ferr), (oerr.message, str(ferr))
        return None
    assert ferr is None, f"native raised {ferr}, oracle parsed"
    assert f.version == o.version and f.data_offset == o.data_offset
    md = f.metadata
    assert list(md) == list(o.metadata)
    for k in md:
        assert _same_value(_plain(md[k]), o.metadata[k]), k
    assert [(t.name, t.dimensions, t.ggml_type, t.offset) for t in f.tensor_infos] == \
        [(n, d, t, off) for n, d, t, off in o.tensor_infos]
    # sizes beyond 64 bits saturate (the reference's usize product would wrap)
    assert [t.n_bytes for t in f.tensor_infos] == \
        [min(ref.tensor_nbytes(d, t), 2**64 - 1) for _, d, t, _ in o.tensor_infos]
    return f, o


def test_random_files_match_oracle(G, W):
    rng = np.random.default_rng(0x5EED0100)
    for _ in range(150):
        _compare(G, _rand_file(rng, W))


def test_every_prefix_is_unexpected_eof(G, W):
    rng = np.random.default_rng(0x5EED0101)
    data = _rand_file(rng, W)
    while len(data) < 200:
        data = _rand_file(rng, W)
    full = _compare(G, data)
    assert full is not None
    for n in range(len(data)):
        _compare(G, data[:n])


def test_corruptions_match_oracle(G, W):
    """Single-byte and single-field corruptions of a valid file."""
    rng = np.random.default_rng(0x5EED0102)
    data = bytearray(_rand_file(rng, W))
    while len(data) < 120:
        data = bytearray(_rand_file(rng, W))
    for pos in range(len(data)):
        for val in (0x00, 0xFF, 0x0D, 0x80):
            d = bytearray(data)
            d[pos] = val
            _compare(G, bytes(d))


@pytest.mark.parametrize("version", [0, 1, 4, 0xFFFFFFFF])
def test_unsupported_versions(G, version):
    data = b"GGUF" + struct.pack("<IQQ", version, 0, 0)
    with pytest.raises(G.InvalidFormat) as e:
        G.GGUFFile.parse_bytes(data)
    assert f"Unsupported GGUF version: {version}" in str(e.value)


def test_unknown_value_and_ggml_types(G, W):
    b = W.GgufBuilder().add_raw("k", 13, b"")
    with pytest.raises(G.UnsupportedType) as e:
        G.GGUFFile.parse_bytes(b.build())
    assert "Unknown GGUF value type: 13" in str(e.value)
    # an empty array of an unknown element type reads nothing (read_value is never called)
    f = G.GGUFFile.parse_bytes(W.GgufBuilder().add_raw("e", 9, struct.pack("<IQ", 99, 0)).build())
    assert f.metadata["e"].value == []
    with pytest.raises(G.UnsupportedType):
        G.GGUFFile.parse_bytes(W.GgufBuilder().add_raw("e", 9, struct.pack("<IQ", 99, 1)).build())
    for t in (4, 5, 16, 30):
        with pytest.raises(G.UnsupportedType) as e:
            G.GGUFFile.parse_bytes(W.GgufBuilder().add_tensor("x", [32], t, 0).build())
        assert f"GGML type: {t}" in str(e.value)


@pytest.mark.parametrize("raw", [b"\xff", b"\xc0\xaf", b"\xed\xa0\x80", b"\xf4\x90\x80\x80", b"a\xe2\x82"])
def test_invalid_utf8(G, W, raw):
    data = W.GgufBuilder().add_raw("k", 8, struct.pack("<Q", len(raw)) + raw).build()
    with pytest.raises(G.GgufIoError) as e:
        G.GGUFFile.parse_bytes(data)
    with pytest.raises(ref.OracleError) as o:
        ref.parse_bytes(data)
    assert o.value.kind == "Io" and o.value.message in str(e.value)


def test_typed_getters_follow_ggufvalue_conversions(G, W):
    b = (W.GgufBuilder().add_i32("neg", -5).add_u64("big", (7 << 32) + 9).add_f64("d", 0.1)
         .add_value("u16", W.U16, 5).add_string("s", "hé"))
    f = G.GGUFFile.parse_bytes(b.build())
    assert f.get_u32("neg") == (-5) & 0xFFFFFFFF
    assert f.get_u32("big") == 9
    assert f.get_f32("d") == float(np.float32(0.1))
    assert f.get_string("s") == "hé"
    with pytest.raises(G.MissingMetadata):
        f.get_u32("u16")  # as_u32 takes only U32, I32, U64
    with pytest.raises(G.MissingMetadata):
        f.get_f32("neg")
    with pytest.raises(G.MissingMetadata):
        f.get_u32("absent")


def _cfg_file(W, **md):
    b = W.GgufBuilder()
    for k, (t, v) in md.items():
        b.add_value(k.replace("__", "."), t, v)
    return b.build()


@pytest.mark.parametrize("case", ["vocab_key", "tokens_count", "tokens_array", "default", "other_arch",
                                  "arch_not_string", "optional", "f64_eps"])
def test_model_config_rules(G, W, case):
    base = {"general__architecture": (W.STRING, "llama"), "llama__embedding_length": (W.U32, 64),
            "llama__attention__head_count": (W.U32, 4), "llama__block_count": (W.I32, 2)}
    if case == "vocab_key":
        base.update(llama__vocab_size=(W.U32, 77), tokenizer__ggml__tokens_count=(W.U32, 5))
    elif case == "tokens_count":
        base.update(tokenizer__ggml__tokens_count=(W.U64, 66), tokenizer__ggml__tokens=(W.ARRAY, (W.STRING, ["a"])))
    elif case == "tokens_array":
        base.update(tokenizer__ggml__tokens=(W.ARRAY, (W.STRING, ["a", "b", "c"])))
    elif case == "other_arch":
        base = {"general__architecture": (W.STRING, "mistral"), "mistral__embedding_length": (W.U32, 32),
                "mistral__attention__head_count": (W.U32, 2), "mistral__block_count": (W.U32, 1),
                "mistral__feed_forward_length": (W.U32, 96), "mistral__attention__sliding_window": (W.U32, 16)}
    elif case == "arch_not_string":
        base["general__architecture"] = (W.U32, 3)
    elif case == "optional":
        base.update(llama__attention__head_count_kv=(W.U32, 2), llama__context_length=(W.U32, 4096),
                    llama__rope__freq_base=(W.F32, 500000.0), llama__attention__key_length=(W.U32, 16),
                    tokenizer__chat_template=(W.STRING, "{{x}}"), tokenizer__ggml__bos_token_id=(W.I32, 0))
    elif case == "f64_eps":
        base.update(llama__attention__layer_norm_rms_epsilon=(W.F64, 1e-6))
    data = _cfg_file(W, **base)
    c = G.GGUFFile.parse_bytes(data).to_model_config()
    o = ref.to_model_config(ref.parse_bytes(data))
    got = {k: getattr(c, k) for k in o}
    for k in ("norm_eps", "rope_theta"):
        assert got[k] == pytest.approx(o[k], rel=0, abs=0), k
    assert got == o


# ---- loader checks that run before allocation (no device needed) ------------
def _small_cfg(**kw):
    from rdlquant.llama import LlamaConfig

    c = dict(dim=64, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=16, ffn_dim=96, vocab=40, max_seq=32,
             max_batch=8)
    c.update(kw)
    return LlamaConfig(**c)


def _zeros_for(W, cfg, types=None):
    shapes = W.llama_tensor_shapes(cfg)

    def data(name):
        dims, t = shapes[name]
        t = (types or {}).get(name, t)
        return np.zeros(W.tensor_nbytes(dims, t), np.uint8)
    return data


def _load_error(G, W, tmp_path, builder):
    from rdlquant.llama import LlamaModel

    p = tmp_path / "m.gguf"
    builder.write(p)
    with pytest.raises(Exception) as e:
        LlamaModel.from_gguf(str(p))
    return e.value


def test_loader_missing_weight(G, W, tmp_path):
    cfg = _small_cfg()
    e = _load_error(G, W, tmp_path, W.llama_builder(cfg, _zeros_for(W, cfg), skip={"blk.1.attn_k.weight"}))
    assert isinstance(e, G.NotFound)
    assert "Missing weight: layers.1.attention.k_proj.weight" in str(e)
    e = _load_error(G, W, tmp_path, W.llama_builder(cfg, _zeros_for(W, cfg), skip={"output.weight"}))
    assert "Missing weight: output.weight" in str(e)
    e = _load_error(G, W, tmp_path, W.llama_builder(cfg, _zeros_for(W, cfg), skip={"token_embd.weight"}))
    assert "Missing weight: token_embedding.weight" in str(e)


def test_loader_rejects_types_shapes_arch(G, W, tmp_path, rq):
    cfg = _small_cfg()
    shapes = W.llama_tensor_shapes(cfg)

    def with_type(name, t):
        b = W.GgufBuilder()
        full = W.llama_builder(cfg, _zeros_for(W, cfg))
        b.metadata = full.metadata
        for n, (dims, tt) in shapes.items():
            tt = t if n == name else tt
            b.add_tensor_data(n, dims, tt, np.zeros(W.tensor_nbytes(dims, tt), np.uint8))
        return b

    # matrices may be Q4_0, Q8_0, Q4_1, Q4_K or Q6_K; Q5_K is not resident
    e = _load_error(G, W, tmp_path, with_type("blk.0.ffn_down.weight", W.GGML_Q5_K))
    assert isinstance(e, rq.DeviceError) and "blk.0.ffn_down.weight" in str(e) and "Q5K" in str(e)
    e = _load_error(G, W, tmp_path, with_type("output_norm.weight", W.GGML_Q4_0))
    assert "output_norm.weight" in str(e)
    # dims that disagree with the config
    b = W.GgufBuilder()
    b.metadata = W.llama_builder(cfg, _zeros_for(W, cfg)).metadata
    for n, (dims, t) in shapes.items():
        if n == "blk.1.attn_output.weight":
            dims = [dims[0], dims[1] + 32]
        b.add_tensor_data(n, dims, t, np.zeros(W.tensor_nbytes(dims, t), np.uint8))
    e = _load_error(G, W, tmp_path, b)
    assert isinstance(e, rq.ShapeMismatch) and "blk.1.attn_output.weight" in str(e)
    e = _load_error(G, W, tmp_path, W.llama_builder(cfg, _zeros_for(W, cfg), arch="gemma3"))
    assert "gemma3" in str(e)
    e = _load_error(G, W, tmp_path, W.llama_builder(cfg, _zeros_for(W, cfg), skip={"blk.0.ffn_gate.weight"}))
    assert "SwiGLU" in str(e)


def test_loader_config_validation(G, W, tmp_path, rq):
    cfg = _small_cfg()
    b = W.llama_builder(cfg, _zeros_for(W, cfg), extra_metadata={"llama.attention.head_count_kv": (W.U32, 3)})
    e = _load_error(G, W, tmp_path, b)
    assert isinstance(e, rq.InvalidData) and "n_heads (4) must be divisible by n_kv_heads (3)" in str(e)
    b = W.llama_builder(cfg, _zeros_for(W, cfg), extra_metadata={"llama.attention.head_count": (W.U32, 5)})
    e = _load_error(G, W, tmp_path, b)
    assert "dim (64) must be divisible by n_heads (5)" in str(e)


def test_loader_truncated_file(G, W, tmp_path):
    cfg = _small_cfg()
    p = tmp_path / "m.gguf"
    W.llama_builder(cfg, _zeros_for(W, cfg)).write(p)
    data = p.read_bytes()
    p.write_bytes(data[:-10])
    from rdlquant.llama import LlamaModel

    with pytest.raises(G.GgufIoError) as e:
        LlamaModel.from_gguf(str(p))
    assert "output.weight" in str(e.value) and "exceeds file bounds" in str(e.value)


def test_open_missing_file(G, tmp_path):
    with pytest.raises(G.GgufIoError) as e:
        G.GGUFFile.parse_header(tmp_path / "absent.gguf")
    assert "os error 2" in str(e.value)


def test_dequantize_rejects_unknown_types_and_short_sources(G):
    with pytest.raises(G.UnsupportedType) as e:
        G.dequantize_gguf_dev(4, 0, 0, 32, 0)
    assert "GGML type: 4" in str(e.value)
    with pytest.raises(G.UnsupportedType):
        G.dequantize_gguf_dev(16, 0, 0, 32, 0)
    import rdlquant as rq
    with pytest.raises(rq.ShapeMismatch):
        G.dequantize_gguf_dev(14, 0, 209, 256, 0)  # one Q6_K block is 210 bytes
