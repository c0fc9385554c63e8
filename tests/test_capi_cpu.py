"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and rejects bad shapes with the reference's error kinds
before touching a device (rustml/quant/main/src/core/quantize.rs:208-213,
272-277, 333-338 -> QuantError::BlockAlignment)."""
import ctypes as C

import numpy as np
import pytest


def test_exports_every_declared_symbol(rq):
    names = rq.declared_symbols()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(rq.lib, n)]
    assert not missing, missing


def test_integration_names_every_declared_symbol(rq):
    """The integration guide's entry point index covers every function
    the headers declare (a new entry point needs its row there)."""
    import os
    doc = open(os.path.join(os.path.dirname(__file__), "..", "INTEGRATION.md")).read()
    unnamed = [n for n in rq.declared_symbols() if n not in doc]
    assert not unnamed, unnamed


def test_status_strings(rq):
    for code in range(14):
        assert rq.lib.rdl_status_string(code)
    assert rq.version().startswith("rdlquant")


@pytest.mark.parametrize("fn", ["matmul_f32_q8", "matmul_f32_q4", "matmul_f32_q4_native",
                                "matmul_f32_q4_1", "matmul_f32_q4_1_native"])
def test_block_alignment(rq, fn):
    with pytest.raises(rq.BlockAlignment) as e:
        getattr(rq, fn)(np.zeros(33, np.float32), np.zeros(64, np.uint8), 1, 33, 1)
    assert "33" in str(e.value)


def test_q4k_block_alignment(rq):
    with pytest.raises(rq.BlockAlignment):
        rq.matmul_f32_q4_k(np.zeros(288, np.float32), np.zeros(200, np.uint8), 1, 288, 1)


def test_short_weight_is_shape_mismatch(rq):
    # QuantError::ShapeMismatch { expected, actual } (error.rs:9-10): both
    # extents cross the ABI (rdl_last_shape_mismatch), not only the text
    with pytest.raises(rq.ShapeMismatch) as e:
        rq.matmul_f32_q4(np.zeros(64, np.float32), np.zeros(35, np.uint8), 1, 64, 1)
    assert (e.value.expected, e.value.actual) == ([36], [35])
    assert "expected [36], got [35]" in str(e.value)


def test_short_input_is_shape_mismatch(rq):
    with pytest.raises(rq.ShapeMismatch) as e:
        rq.matmul_f32_q8(np.zeros(63, np.float32), np.zeros(68, np.uint8), 1, 64, 1)
    assert (e.value.expected, e.value.actual) == ([64], [63])


def test_shape_detail_only_for_shape_mismatch(rq):
    # another status leaves no extents behind, and the query does not reset the status
    with pytest.raises(rq.ShapeMismatch):
        rq.matmul_f32_q4(np.zeros(64, np.float32), np.zeros(35, np.uint8), 1, 64, 1)
    assert rq.last_shape_mismatch() == ([36], [35])
    assert rq.last_shape_mismatch() == ([36], [35])
    with pytest.raises(rq.BlockAlignment):
        rq.matmul_f32_q4(np.zeros(33, np.float32), np.zeros(35, np.uint8), 1, 33, 1)
    assert rq.last_shape_mismatch() is None
    h = C.c_size_t()
    assert rq.lib.rdl_last_shape_mismatch(None, C.byref(h), None, C.byref(h)) == rq.ERR_NULL_POINTER


def test_quantize_row_alignment(rq):
    with pytest.raises(rq.BlockAlignment):
        rq.quantize_row_q8_0(np.zeros(40, np.float32))


def test_empty_shapes_are_ok_without_device(rq):
    # m = 0 or n = 0: nothing to compute, no device needed (an empty Vec in the reference)
    assert rq.matmul_f32_q4(np.zeros(0, np.float32), np.zeros(0, np.uint8), 0, 64, 4).size == 0
    assert rq.matmul_f32_q4(np.zeros(64, np.float32), np.zeros(0, np.uint8), 1, 64, 0).size == 0


def test_weight_upload_rejects_bad_dtype(rq):
    h = C.c_void_p()
    assert rq.lib.rdl_weight_upload(None, 0, 5, 1, 32, C.byref(h)) == rq.ERR_DTYPE_MISMATCH
    assert not h.value


def test_no_device_is_reported(rq):
    if rq.device_count() > 0:
        pytest.skip("a gfx950 device is visible; covered by the gpu tests")
    with pytest.raises(rq.DeviceError) as e:
        rq.matmul_f32_q4(np.zeros(64, np.float32), np.zeros(72, np.uint8), 1, 64, 2)
    assert e.value.status == rq.ERR_NO_DEVICE


def test_record_bytes(rq):
    assert rq.activation_record_bytes(1, 4096, rq.MODE_FLOAT) == 128 * 128
    assert rq.activation_record_bytes(2, 4096, rq.MODE_NATIVE) == 2 * 128 * 48


def test_gemm_combine_switch(rq):
    # the testing switch of the split GEMMs' combine: modes 0 / 1 only, no device needed
    with pytest.raises(rq.InvalidData):
        rq.set_gemm_combine(2)
    rq.set_gemm_combine(rq.COMBINE_COHERENT)
    assert rq.gemm_combine() == (rq.COMBINE_COHERENT, False)
    rq.set_gemm_combine(rq.COMBINE_AUTO)
    assert rq.gemm_combine()[0] == rq.COMBINE_AUTO
