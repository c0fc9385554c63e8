"""Shared parity checks for the GPU tests.

Bars: integer work bit-exact (Q8_0 activation bytes,
int32 block dots); f32 outputs within 1e-3 relative + 1e-4 absolute of the
reference CPU path on identical seeded inputs."""
import numpy as np

RTOL, ATOL = 1e-3, 1e-4


def assert_close(got, want, rtol=RTOL, atol=ATOL, slack=0.0):
    got = np.asarray(got, np.float64).reshape(-1)
    want = np.asarray(want, np.float64).reshape(-1)
    err = np.abs(got - want)
    tol = atol + rtol * np.abs(want) + slack
    bad = np.nonzero(~(err <= tol))[0]
    assert bad.size == 0, (
        f"{bad.size}/{want.size} outside tol; worst idx {bad[np.argmax(err[bad])]} "
        f"got {got[bad[0]]} want {want[bad[0]]}")


DEQ = {"q8": "q8_0", "q4": "q4_0", "q4_1": "q4_1", "q4k": "q4k", "q6k": "q6k"}


def exact_f64(orc, kind, x, w, m, k, n):
    """The reference's float-path product evaluated exactly (f64) over its own
    f32 dequantized weights (Tensor::to_f32 / dequantize_q4k / dequantize_q6k)."""
    wd = orc.to_f32(DEQ[kind], w, n * k).reshape(n, k).astype(np.float64)
    return (np.asarray(x, np.float64).reshape(m, k) @ wd.T).reshape(-1)


def exact_f64_cond(orc, kind, x, w, m, k, n):
    """exact_f64 and each output's condition sum_k |x_ik| |w_jk| (f64)."""
    wd = orc.to_f32(DEQ[kind], w, n * k).reshape(n, k).astype(np.float64)
    xd = np.asarray(x, np.float64).reshape(m, k)
    return (xd @ wd.T).reshape(-1), (np.abs(xd) @ np.abs(wd).T).reshape(-1)


def check_parity(got, want, exact, rtol=RTOL, atol=ATOL, cond=None):
    """got: GPU; want: the reference CPU path (oracle, f32); exact: f64 value of
    the same computation.  (1) the GPU result is within the bar of the exact
    value; (2) it agrees with the CPU path within the bar plus the CPU path's
    own f32 rounding error |want - exact| (the reference's summation order --
    faer for Q4_K -- is not pinned, so only that much of its noise is defined).
    cond (sum |x| |w| of each output): outputs that cancel to far below their
    terms are beyond any f32 evaluation's bar, the reference's included; (1)
    then also allows rho cond, rho = the CPU path's own largest |want - exact|
    / cond over the case: the GPU may miss the exact value by as much,
    relative to an output's terms, as the reference path does somewhere."""
    want = np.asarray(want, np.float64).reshape(-1)
    exact = np.asarray(exact, np.float64).reshape(-1)
    slack = 0.0
    if cond is not None:
        cond = np.asarray(cond, np.float64).reshape(-1)
        pos = cond > 0
        rho = float((np.abs(want - exact)[pos] / cond[pos]).max()) if pos.any() else 0.0
        slack = rho * cond
    assert_close(got, exact, rtol, atol, slack=slack)
    assert_close(got, want, rtol, atol, slack=np.abs(want - exact))
