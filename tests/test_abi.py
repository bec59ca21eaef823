"""CPU-side checks of the C ABI: the library loads, exports every declared
symbol, and rejects bad arguments on the host before touching a GPU."""
import ctypes

import numpy as np
import pytest

from unillm_amd import _capi


@pytest.fixture(scope="module")
def lib():
    return _capi.lib()


def test_every_header_symbol_is_exported(lib):
    declared = _capi.header_symbols()
    assert len(declared) >= 16
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/unillm_hip.h but not exported"
    assert sorted(_capi.SIGNATURES) == declared


def test_header_constants_match_binding():
    text = open(_capi.HEADER).read()
    for macro, value in [("UNILLM_QTYPE_Q4_0", _capi.Q4_0), ("UNILLM_QTYPE_Q8_0", _capi.Q8_0),
                         ("UNILLM_PATH_GEMV", _capi.PATH_GEMV),
                         ("UNILLM_PATH_DECODE_MFMA", _capi.PATH_DECODE_MFMA),
                         ("UNILLM_PATH_PREFILL_MFMA", _capi.PATH_PREFILL_MFMA),
                         ("UNILLM_QTYPE_F32", _capi.F32), ("UNILLM_QTYPE_F16", _capi.F16),
                         ("UNILLM_QTYPE_BF16", _capi.BF16), ("UNILLM_PATH_DENSE", _capi.PATH_DENSE),
                         ("UNILLM_ERR_INVALID_ARG", _capi.ERR_INVALID_ARG),
                         ("UNILLM_ERR_UNSUPPORTED", _capi.ERR_UNSUPPORTED)]:
        assert f"#define {macro} {value}" in text or f"#define {macro} ({value})" in text, macro


def _create(lib, qtype, n, k, nbytes, flags=0, data=True):
    h = ctypes.c_void_p()
    buf = np.zeros(max(nbytes, 1), np.uint8)
    ptr = buf.ctypes.data if data else None
    rc = lib.unillm_hip_qweight_create(qtype, n, k, ptr, nbytes, flags, ctypes.byref(h))
    return rc, h


def test_create_rejects_bad_qtype(lib):
    rc, h = _create(lib, 3, 4, 64, 4 * 2 * 18)
    assert rc == _capi.ERR_UNSUPPORTED and h.value is None
    assert "unsupported qtype 3" in _capi.last_error()


@pytest.mark.parametrize("n,k", [(0, 64), (4, 48), (4, 0), (-1, 64)])
def test_create_rejects_bad_shape(lib, n, k):
    rc, _ = _create(lib, _capi.Q4_0, n, k, 18)
    assert rc == _capi.ERR_INVALID_ARG
    assert "multiple of 32" in _capi.last_error()


@pytest.mark.parametrize("qtype,esize", [(_capi.F32, 4), (_capi.F16, 2), (_capi.BF16, 2)])
def test_dense_create_checks_shape_and_bytes_on_the_host(lib, qtype, esize):
    # dense weights take any k >= 1 (candle's dequantized QMatMul has no block size),
    # and n * k elements of their GGUF type; both are checked before any device work
    rc, _ = _create(lib, qtype, 0, 7, esize)
    assert rc == _capi.ERR_INVALID_ARG and "need n, k >= 1" in _capi.last_error()
    rc, _ = _create(lib, qtype, 3, 7, 3 * 7 * esize + 1)
    assert rc == _capi.ERR_INVALID_ARG and "nbytes" in _capi.last_error()


def test_dense_types_have_one_element_blocks():
    for q, esize in ((_capi.F32, 4), (_capi.F16, 2), (_capi.BF16, 2)):
        assert _capi.BLOCK_ELEMS[q] == 1 and _capi.BLOCK_BYTES[q] == esize
        assert q in _capi.DENSE


def test_create_rejects_wrong_byte_count(lib):
    rc, _ = _create(lib, _capi.Q8_0, 4, 64, 4 * 2 * 18)
    assert rc == _capi.ERR_INVALID_ARG and "nbytes" in _capi.last_error()


def test_create_rejects_null_and_flags(lib):
    rc, _ = _create(lib, _capi.Q4_0, 4, 64, 4 * 2 * 18, data=False)
    assert rc == _capi.ERR_INVALID_ARG and "NULL" in _capi.last_error()
    rc, _ = _create(lib, _capi.Q4_0, 4, 64, 4 * 2 * 18, flags=1)
    assert rc == _capi.ERR_INVALID_ARG and "layout_flags" in _capi.last_error()
    assert lib.unillm_hip_qweight_create(2, 4, 64, None, 0, 0, None) == _capi.ERR_INVALID_ARG


def test_qmatmul_rejects_null_weight(lib):
    rc = lib.unillm_hip_qmatmul(None, None, 1, None, None)
    assert rc == _capi.ERR_INVALID_ARG
    assert _capi.last_error().startswith("QMatMul forward failed")


def test_select_path_rejects_null(lib):
    assert lib.unillm_hip_select_path(None, 1) == _capi.ERR_INVALID_ARG


def test_quantize_rejects_bad_shape(lib):
    assert lib.unillm_hip_quantize(2, None, 4, 33, None, None) == _capi.ERR_INVALID_ARG


def test_destroy_null_is_noop(lib):
    assert lib.unillm_hip_qweight_destroy(None) == _capi.OK


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_capi, "_lib", None)
    monkeypatch.setattr(_capi, "LIB_PATH", str(tmp_path / "nope.so"))
    with pytest.raises(ImportError, match="no CPU fallback"):
        _capi.lib()


def test_graph_and_stream_entry_points_reject_null_on_the_host(lib):
    # no GPU needed: every check below fails before the library touches a device
    assert lib.unillm_hip_graph_begin(None) == _capi.ERR_INVALID_ARG
    assert "null stream" in _capi.last_error()
    out = ctypes.c_void_p(1)
    assert lib.unillm_hip_graph_end(None, ctypes.byref(out)) == _capi.ERR_INVALID_ARG
    assert lib.unillm_hip_graph_launch(None, None) == _capi.ERR_INVALID_ARG
    assert lib.unillm_hip_graph_destroy(None) == _capi.OK
    assert lib.unillm_hip_stream_destroy(None) == _capi.OK
    assert lib.unillm_hip_stream_create(None) == _capi.ERR_INVALID_ARG
