"""The committed golden fixtures (tests/golden/*.npz) against the oracle, and
the fixtures themselves against what the mathematics fixes: f64 brute force
over the dequantized weights, exact integer block dots, and the closed-form
cases of quantize_row_q8_0 (quantize.rs:164-193).  CPU only."""
import os

import numpy as np
import pytest

from parity import ATOL, RTOL

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
LINEAR = {"q8_0": ("q8", None), "q4_0": ("q4", "q4_native"), "q4_1": ("q4_1", "q4_1_native"),
          "q4_k": ("q4k", None), "q6_k": ("q6k", None)}


def load(name):
    return np.load(os.path.join(GOLDEN, name))  # allow_pickle defaults to False


@pytest.mark.parametrize("name", sorted(LINEAR))
def test_oracle_reproduces_linear_fixture(orc, name):
    d = load(f"linear_{name}.npz")
    m, k, n = (int(v) for v in d["shape"])
    fk, nk = LINEAR[name]
    assert np.array_equal(orc.matmul(fk, d["x"], d["w"], m, k, n).reshape(m, n), d["y_float"])
    if nk:
        assert np.array_equal(orc.matmul(nk, d["x"], d["w"], m, k, n).reshape(m, n), d["y_native"])
    kind = {"q4_k": "q4k", "q6_k": "q6k"}.get(name, name)
    assert np.array_equal(orc.to_f32(kind, d["w"], n * k).reshape(n, k), d["w_f32"])


@pytest.mark.parametrize("name", sorted(LINEAR))
def test_linear_fixture_against_f64_brute_force(name):
    d = load(f"linear_{name}.npz")
    exact = d["x"].astype(np.float64) @ d["w_f32"].astype(np.float64).T
    y = d["y_float"].astype(np.float64)
    assert np.all(np.abs(y - exact) <= 1e-6 + 1e-5 * np.abs(exact)), np.max(np.abs(y - exact))


def _q4_0_fields(w, n, k):
    blk = w.reshape(n, k // 32, 18)
    d = blk[..., :2].copy().view(np.float16)[..., 0].astype(np.float64)
    nib = blk[..., 2:]
    # GGUF order: byte j holds element j (low nibble) and j + 16 (high nibble)
    q = np.concatenate([nib & 15, nib >> 4], axis=-1).astype(np.int64) - 8
    return d, q


def test_q4_0_dequant_fixture_is_the_gguf_formula():
    d = load("linear_q4_0.npz")
    m, k, n = (int(v) for v in d["shape"])
    scale, q = _q4_0_fields(d["w"], n, k)
    assert np.array_equal(d["w_f32"], (q * scale[..., None]).reshape(n, k).astype(np.float32))


def _q8_codes(qbytes, nb):
    blk = qbytes.reshape(nb, 34)
    return blk[:, 2:].view(np.int8).astype(np.int64), blk[:, :2].copy().view(np.float16)[:, 0]


@pytest.mark.parametrize("fixture", ["linear_q4_0.npz", "block_dots_q4_0_64x512.npz"])
def test_block_dots_fixture_is_the_integer_dot(orc, fixture):
    d = load(fixture)
    x, w, part = d["x"], d["w"], d["partials"]
    m, n, nb = part.shape
    k = nb * 32
    assert np.array_equal(orc.block_dots(x, w, m, k, n), part)
    _, q = _q4_0_fields(w, n, k)
    for r in range(m):
        qb, _ = orc.quantize_row_q8_0(x[r])
        q8, _ = _q8_codes(qb, nb)
        assert np.array_equal(np.einsum("nbj,bj->nb", q, q8), part[r])


def test_native_fixture_is_scaled_partials():
    # matmul_f32_q4_native (quantize.rs:367-379): y = sum_b (p_b * sx_b) * d_b, in order
    d = load("linear_q4_0.npz")
    m, k, n = (int(v) for v in d["shape"])
    from oracle import oracle as orc
    scale = d["w"].reshape(n, k // 32, 18)[..., :2].copy().view(np.float16)[..., 0].astype(np.float32)
    for r in range(m):
        _, sx = orc.quantize_row_q8_0(d["x"][r])
        for c in range(n):
            acc = np.float32(0)
            for b in range(k // 32):
                acc = np.float32(acc + np.float32(np.float32(d["partials"][r, c, b]) * sx[b]) * scale[c, b])
            assert acc == d["y_native"][r, c]


def test_quantize_row_fixture_closed_forms(orc):
    d = load("quantize_row_q8_0.npz")
    x, qb, sc = d["x"], d["q"], d["scales"]
    q, s16 = _q8_codes(qb, x.size // 32)
    out_q, out_s = orc.quantize_row_q8_0(x)
    assert np.array_equal(out_q, qb) and np.array_equal(out_s, sc)
    xb = x.reshape(-1, 32)
    # f16(amax / 127) with round-to-nearest-even, and the f32 value handed back
    amax = np.abs(xb).max(axis=1)
    assert np.array_equal(s16, (amax / np.float32(127)).astype(np.float16))
    assert np.array_equal(sc, s16.astype(np.float32))
    assert not q[0].any() and sc[0] == 0  # all-zero block
    assert list(q[2]) == [127] + [((-1) ** j) * (j + 1) for j in range(31)]  # halves away from zero
    assert q[3][0] == -127 and q[3][-1] == 127
    assert 0 < sc[4] < 2.0 ** -14  # subnormal scale
    assert sc[8] == 0 and not q[8].any()  # scale rounds to zero: codes 0
    assert q[9][np.argmax(np.abs(xb[9]))] == -127
    nz = np.flatnonzero(xb[6])
    assert list(nz) == [17] and q[6][17] == -127 and np.count_nonzero(q[6]) == 1
    # every code is within half a step of x / scale (the scale being nonzero)
    for b in range(xb.shape[0]):
        if sc[b] > 0:
            assert np.all(np.abs(xb[b].astype(np.float64) / sc[b] - q[b]) <= 0.5 + 1e-4)


def test_fixture_files_hold_no_pickles():
    for f in os.listdir(GOLDEN):
        if f.endswith(".npz"):
            with np.load(os.path.join(GOLDEN, f)) as z:
                for key in z.files:
                    assert z[key].dtype != object
