"""The build check of the fused GEMV kernels' hand-counted load wait
(rust-deeplearning_amd/check_vmcnt.py): it passes on the compiled kernels and
fails on planted mistakes in small assembly fragments."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "rust-deeplearning_amd")
sys.path.insert(0, PKG)

import check_vmcnt as cv  # noqa: E402

XLOAD = ";;#ASMSTART\nglobal_load_dwordx4 v[4:7], v[2:3], off\n;;#ASMEND"


def wait(n):
    return f";;#ASMSTART\ns_waitcnt vmcnt({n})\n;;#ASMEND"


def fn(*body, name="_Z1kv"):
    return "\n".join([f"{name}:"] + list(body) + [".Lfunc_end0:"])


LOADS3 = ["buffer_load_dwordx4 v[8:11], v1, s[0:3], 0 offen"] * 3


def run(text):
    return cv.check(text)


def test_compiled_kernels_hold():
    path = os.path.join(PKG, "build", "gemv_fused.s")
    if not os.path.exists(path):
        pytest.skip("build/gemv_fused.s is written by the library build (make -C rust-deeplearning_amd)")
    problems, checked = cv.check(open(path).read())
    assert checked > 0 and not problems, problems[:5]


def test_enough_loads_pass():
    problems, checked = run(fn(XLOAD, *LOADS3, wait(3)))
    assert checked == 1 and not problems


def test_too_few_loads_fail():
    problems, checked = run(fn(XLOAD, *LOADS3, wait(4)))
    assert checked == 1 and problems and "after only 3 loads" in problems[0]


def test_loads_before_the_x_loads_do_not_count():
    problems, _ = run(fn(*LOADS3, XLOAD, LOADS3[0], wait(2)))
    assert problems


def test_loads_in_a_skippable_block_do_not_count():
    body = [XLOAD, LOADS3[0], "s_cbranch_execz .LBB0_2", LOADS3[0], LOADS3[0], ".LBB0_2:", LOADS3[0]]
    assert not run(fn(*body, wait(2)))[0]
    assert run(fn(*body, wait(3)))[0]


def test_backward_branch_fails():
    body = [XLOAD, ".LBB0_1:", LOADS3[0], "s_cbranch_scc1 .LBB0_1", LOADS3[0], wait(1)]
    problems, _ = run(fn(*body))
    assert problems and "control flow" in problems[0]


def test_branch_out_of_the_range_fails():
    body = [XLOAD, LOADS3[0], "s_cbranch_execz .LBB0_9", LOADS3[0], wait(1), ".LBB0_9:", "s_endpgm"]
    problems, _ = run(fn(*body))
    assert problems


def test_jump_into_the_range_fails():
    body = ["s_cbranch_execz .LBB0_3", XLOAD, LOADS3[0], LOADS3[0], ".LBB0_3:", LOADS3[0], wait(1)]
    problems, _ = run(fn(*body))
    assert problems and "control flow" in problems[0]


def test_a_wait_without_x_loads_is_not_checked():
    problems, checked = run(fn(*LOADS3, wait(9)))
    assert checked == 0 and not problems
