"""Writes the golden fixtures of this directory from the C oracle (oracle/).

Each fixture is a small .npz of plain arrays (no pickles): seeded inputs in
GGUF block layout and the oracle's outputs for them.  The reference (Rust)
cannot be built or run here, so the expected outputs come from the oracle,
which tests/test_golden.py pins independently (f64 brute force over the
dequantized weights, exact integer dots, closed forms of quantize_row_q8_0).

Run from the repository root:  python tests/golden/make_golden.py [linear case ...]
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.join(ROOT, "rust-deeplearning_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

from oracle import oracle as orc  # noqa: E402
from rdlquant import synth  # noqa: E402

SEED = 0x601D0000

# name -> (GGML type id, n, k, m, oracle float kind, oracle native kind or None)
LINEAR_CASES = {
    "q8_0": (8, 4, 256, 2, "q8", None),
    "q4_0": (2, 4, 256, 2, "q4", "q4_native"),
    "q4_1": (3, 4, 256, 2, "q4_1", "q4_1_native"),
    "q4_k": (12, 2, 512, 2, "q4k", None),
    "q6_k": (14, 3, 768, 2, "q6k", None),
}


def linear_fixture(name):
    dtype, n, k, m, fk, nk = LINEAR_CASES[name]
    seed = SEED + dtype
    x = synth.activations(m, k, seed + 100)
    w = synth.weights(dtype, n, k, seed)
    out = {"x": x, "w": w, "shape": np.array([m, k, n], np.int64),
           "y_float": orc.matmul(fk, x, w, m, k, n).reshape(m, n)}
    if nk is not None:
        out["y_native"] = orc.matmul(nk, x, w, m, k, n).reshape(m, n)
    if dtype == 2:
        out["partials"] = orc.block_dots(x, w, m, k, n)
    kind = {8: "q8_0", 2: "q4_0", 3: "q4_1", 12: "q4k", 14: "q6k"}[dtype]
    out["w_f32"] = orc.to_f32(kind, w, n * k).reshape(n, k)
    return out


def quantize_row_input():
    """Ten 32-element blocks covering the cases quantize_row_q8_0 distinguishes."""
    r = np.random.default_rng(SEED + 7)
    b = np.zeros((10, 32), np.float32)
    # 0: all zeros (amax = 0 -> scale 0, codes 0)
    b[1] = r.standard_normal(32)
    # 2: amax 127 -> scale exactly 1: halves round away from zero
    b[2] = np.array([127.0] + [((-1) ** j) * (j + 0.5) for j in range(31)], np.float32)
    b[3] = np.linspace(-3.0, 3.0, 32)  # +-amax -> +-127
    b[4] = r.standard_normal(32) * 1e-4  # scale is an f16 subnormal
    b[5] = r.standard_normal(32) * 1e4
    b[6, 17] = -0.25  # one nonzero element
    b[7] = np.round(r.standard_normal(32) * 40) / 2  # many exact .5 products
    b[8] = r.standard_normal(32) * 1e-6  # amax / 127 rounds to an f16 zero: codes 0
    b[9] = -np.abs(r.standard_normal(32))  # the block maximum is negative -> -127
    return b.reshape(-1)


def main(names=None):
    for name in names or LINEAR_CASES:
        np.savez_compressed(os.path.join(HERE, f"linear_{name}.npz"), **linear_fixture(name))
    if names:
        return
    x = quantize_row_input()
    q, s = orc.quantize_row_q8_0(x)
    np.savez_compressed(os.path.join(HERE, "quantize_row_q8_0.npz"), x=x, q=q, scales=s)
    # config-2 element order at a shape the int32 partials stay small for
    xb = synth.activations(1, 512, SEED + 200)
    wb = synth.q4_0_weights(64, 512, SEED + 201)
    np.savez_compressed(os.path.join(HERE, "block_dots_q4_0_64x512.npz"), x=xb, w=wb,
                        partials=orc.block_dots(xb, wb, 1, 512, 64))
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main(sys.argv[1:] or None)
