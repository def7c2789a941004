"""CPU-side checks of the C ABI: the library loads, exports every function
include/aq.h declares, and fails with status codes (never a crash) where the
reference's QMatMul would return an error.  No kernel is launched here."""
import ctypes
import os
import re

import numpy as np
import pytest

import arm_ai_amd as A
from arm_ai_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    src = open(os.path.join(ROOT, "include", "aq.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(aq_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    L = _lib.load()
    names = _declared_functions()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # the ctypes table mirrors the header one-to-one
    assert sorted(_lib.SIGNATURES) == names


def test_abi_version_and_error_string():
    L = _lib.load()
    assert L.aq_abi_version() == 1
    assert isinstance(L.aq_last_error(), bytes)


def test_null_arguments_are_errors_not_crashes():
    L = _lib.load()
    assert L.aq_ctx_create(0, None) == _lib.AQ_ERR_INVALID_ARG
    assert L.aq_ctx_synchronize(None) == _lib.AQ_ERR_INVALID_ARG
    assert L.aq_qmatmul_f32(None, None, None, 1, 256, None) == _lib.AQ_ERR_INVALID_ARG
    assert L.aq_qweight_info(None, None, None, None, None) == _lib.AQ_ERR_INVALID_ARG
    assert L.aq_ctx_destroy(None) == _lib.AQ_OK
    assert L.aq_qweight_free(None) == _lib.AQ_OK
    assert L.aq_device_count(None) == _lib.AQ_ERR_INVALID_ARG


@pytest.mark.skipif(A.device_count() > 0, reason="checks the no-device path")
def test_no_device_is_reported():
    with pytest.raises(A.AqError) as e:
        A.Context(0)
    assert e.value.code == _lib.AQ_ERR_NO_DEVICE
    assert b"no HIP device" in _lib.load().aq_last_error()


def test_qtensor_shape_checks_mirror_candle():
    with pytest.raises(A.QMatMulError):
        A.QTensor(A.GgmlDType.Q4K, (4, 300), np.zeros(4 * 144, np.uint8))  # k not a multiple of 256
    with pytest.raises(A.QMatMulError):
        A.QTensor(A.GgmlDType.Q4K, (4, 256), np.zeros(3 * 144, np.uint8))  # wrong byte count
    qt = A.QTensor(A.GgmlDType.Q6K, (2, 512), np.zeros(2 * 2 * 210, np.uint8))
    assert qt.storage_size_in_bytes() == 840


def test_qmatmul_input_checks_mirror_candle():
    mm = A.QMatMul(None, ctypes.c_void_p(1), A.GgmlDType.Q4K, (8, 256))
    mm._h = None  # never touches the library
    with pytest.raises(A.QMatMulError, match="only one dimension"):
        mm._check_input(np.zeros(256, np.float32))
    with pytest.raises(A.QMatMulError, match="incompatible"):
        mm._check_input(np.zeros((1, 512), np.float32))
    with pytest.raises(A.QMatMulError, match="not contiguous"):
        mm._check_input(np.zeros((512, 2), np.float32).T[:, :256].copy(order="F"))
    with pytest.raises(A.QMatMulError):
        mm._check_input(np.zeros((1, 256), np.float64))


def test_header_types_match_gguf_ids():
    src = open(os.path.join(ROOT, "include", "aq.h")).read()
    for name, val in (("Q8_0", 8), ("Q4_K", 12), ("Q6_K", 14), ("Q8_K", 15)):
        assert re.search(rf"AQ_TYPE_{name}\s*=\s*{val}\b", src)
        assert int(getattr(A.GgmlDType, name.replace("_K", "K") if name != "Q8_0" else name)) == val


def test_swiglu_fused_query():
    """aq_swiglu_fused: which paired gate|up weights get silu(g) * u inside the
    matvec launch (the row-per-lane forms with the fused norm, whole 8-row
    blocks); a pure host query."""
    L = _lib.load()
    Q4K, Q6K, Q8_0, Q5_0 = 12, 14, 8, 6
    assert L.aq_swiglu_fused(Q4K, 11264, 2048) == 1   # TinyLlama w1|w3
    assert L.aq_swiglu_fused(Q4K, 28672, 4096) == 1   # Llama-3-8B w1|w3
    assert L.aq_swiglu_fused(Q6K, 1024, 4096) == 1
    assert L.aq_swiglu_fused(Q8_0, 2048, 2048) == 1
    assert L.aq_swiglu_fused(Q5_0, 3072, 576) == 0    # SmolLM-135M: rows of 576
    assert L.aq_swiglu_fused(Q4K, 200, 1024) == 0     # below 256 rows
    assert L.aq_swiglu_fused(Q4K, 11260, 2048) == 0   # not whole 8-row blocks
    assert L.aq_swiglu_fused(Q4K, 11264, 16384) == 0  # too long a row for the fused norm
    assert L.aq_swiglu_fused(Q4K, 0, 2048) == 0 and L.aq_swiglu_fused(99, 11264, 2048) == 0
