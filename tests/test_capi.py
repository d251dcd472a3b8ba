"""CPU tests of the C-ABI library: it loads, exports every symbol its header
declares, and rejects bad arguments before touching a device, with the status
codes the Java adapter maps back to the reference's exceptions."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from gollek_amd import _native
from gollek_amd import tensor_ops as ops

HEADER = Path(__file__).resolve().parents[1] / "include" / "gollek_hip.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(gollek_hip_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    names = declared_functions()
    assert len(names) >= 12
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_library_resolves_all_of_its_own_symbols():
    # Loading binds lazily here, so an unresolved kernel launch stub (which
    # hipcc can leave behind for a kernel template) would only fail on first
    # use; dlopen with RTLD_NOW resolves every symbol up front.
    lib_path = _native.load()._name
    ctypes.CDLL(lib_path, mode=ctypes.RTLD_GLOBAL | 0x2)  # RTLD_NOW


def test_python_signatures_cover_header():
    assert set(declared_functions()) <= set(_native.SIGNATURES)


def test_version():
    assert _native.load().gollek_hip_version() >= 10000


def _err():
    return _native.ErrBuf()


def test_upload_rejects_unsupported_type():
    lib = _native.load()
    e = _err()
    buf = np.zeros(64, np.uint8)
    h = lib.gollek_hip_weight_upload(1, buf.ctypes.data, 1, 32, 64, e.buf, e.size)  # F16
    assert not h
    assert lib.gollek_hip_last_status() == _native.ERR_UNSUPPORTED
    assert "Unsupported" in e.text


def test_upload_rejects_non_block_multiple():
    lib = _native.load()
    e = _err()
    buf = np.zeros(1024, np.uint8)
    h = lib.gollek_hip_weight_upload(_native.Q4_K, buf.ctypes.data, 1, 300, 144, e.buf, e.size)
    assert not h
    assert lib.gollek_hip_last_status() == _native.ERR_ARG
    assert "not a multiple of block size 256" in e.text


def test_upload_rejects_wrong_row_bytes_and_null():
    lib = _native.load()
    e = _err()
    buf = np.zeros(1024, np.uint8)
    assert not lib.gollek_hip_weight_upload(_native.Q8_0, buf.ctypes.data, 2, 64, 70, e.buf, e.size)
    assert lib.gollek_hip_last_status() == _native.ERR_ARG
    assert not lib.gollek_hip_weight_upload(_native.Q8_0, None, 2, 64, 68, e.buf, e.size)
    assert lib.gollek_hip_last_status() == _native.ERR_NULL


def test_null_handle_calls_fail_with_null_status():
    lib = _native.load()
    e = _err()
    x = np.zeros(32, np.float32)
    y = np.zeros(4, np.float32)
    assert lib.gollek_hip_matvec_rows(None, x.ctypes.data, 32, y.ctypes.data, 4, 1, e.buf,
                                      e.size) == _native.ERR_NULL
    assert lib.gollek_hip_dot_row(None, 0, x.ctypes.data, 32, y.ctypes.data, e.buf,
                                  e.size) == _native.ERR_NULL
    assert lib.gollek_hip_dequantize_rows(None, 0, 1, y.ctypes.data, 4, e.buf,
                                          e.size) == _native.ERR_NULL
    assert lib.gollek_hip_matvec_device(None, None, None, 0, None, e.buf, e.size) == _native.ERR_NULL
    assert lib.gollek_hip_weight_info(None, None, None, None, None) == _native.ERR_NULL
    lib.gollek_hip_weight_free(None)  # ignored


def test_error_buffer_truncates():
    lib = _native.load()
    small = ctypes.create_string_buffer(8)
    buf = np.zeros(64, np.uint8)
    assert not lib.gollek_hip_weight_upload(99, buf.ctypes.data, 1, 32, 34, small, 8)
    assert len(small.value) == 7


def test_testing_option_is_outside_the_public_abi():
    # The kernel-family switch the parity tests use is exported by a
    # test-only header, not by include/gollek_hip.h.
    assert "gollek_hip_testing_set_option" not in declared_functions()
    assert "gollek_hip_set_option" not in declared_functions()
    ops.set_option("gemv_variant", 0)
    with pytest.raises(ops.IllegalArgumentError):
        ops.set_option("no_such_option", 1)
    with pytest.raises(ops.IllegalArgumentError):
        ops.set_option("gemv_variant", 2)


def test_tensor_shape_rules():
    t = ops.GgufTensor("blk.0.ffn_up.weight", (4096, 11008), 2, np.zeros(1, np.uint8))
    assert (t.columns, t.rows, t.row_bytes) == (4096, 11008, 2304)
    t = ops.GgufTensor("ffn_gate_exps", (2048, 768, 128), 12, np.zeros(1, np.uint8))
    assert (t.columns, t.rows, t.row_bytes) == (2048, 768 * 128, 1152)


def test_python_mirror_null_checks():
    with pytest.raises(ops.NullPointerError):
        ops.mat_vec_rows(None, np.zeros(4, np.float32), np.zeros(4, np.float32), 1)
    with pytest.raises(ops.NullPointerError):
        ops.dot_row(None, 0, np.zeros(4, np.float32))
