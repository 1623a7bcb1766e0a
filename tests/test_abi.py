"""CPU-side checks of the C ABI (no GPU needed, no compute calls).

* the built libgemma4_qmm.so loads and exports every function include/gemma4_qmm.h declares;
* argument validation follows the reference conventions: status codes and a
  thread-local last-error message (native/gemma4_mlx/src/runtime.cc:116-133,
  crates/gemma4d-ffi/src/lib.rs:1589-1594 for the null-pointer tests it mirrors),
  and a NULL free is a no-op;
* the ctypes structures match the header's layout (the reference pins its ABI
  structs the same way, crates/gemma4d-ffi/src/lib.rs:1470-1508).
"""

import ctypes
import os
import re
import threading

import pytest

from helios_amd import build as hbuild
from helios_amd import qmm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gemma4_qmm.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"Gemma4Status\s+(\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(hbuild.LIB_PATH):
        hbuild.build()
    return qmm.load_library()


def test_library_exports_every_declared_symbol(lib):
    names = header_functions()
    assert len(names) >= 8
    for name in names:
        assert hasattr(lib, name), name


def test_runtime_version(lib):
    v = qmm.runtime_version()
    assert v["abi_version"] == 2 and v["backend_name"] == "gemma4_qmm"
    assert qmm.last_error() == ""


def test_null_and_invalid_arguments_set_last_error(lib):
    out = ctypes.c_void_p()
    assert lib.gemma4_qlinear_create(None, None, None, None, ctypes.byref(out)) == qmm.Status.INVALID_ARGUMENT
    assert "non-null desc" in qmm.last_error()
    assert lib.gemma4_qlinear_create(None, None, None, None, None) == qmm.Status.INVALID_ARGUMENT
    assert "out pointer" in qmm.last_error()
    desc = qmm._Desc(16, 64, 2, 64)
    assert lib.gemma4_qlinear_create(ctypes.byref(desc), None, None, None, ctypes.byref(out)) == \
        qmm.Status.UNSUPPORTED_CONFIG
    assert "bits=2" in qmm.last_error()
    desc = qmm._Desc(16, 64, 8, 32)
    assert lib.gemma4_qlinear_create(ctypes.byref(desc), None, None, None, ctypes.byref(out)) == \
        qmm.Status.UNSUPPORTED_CONFIG
    desc = qmm._Desc(16, 64, 8, 64)  # 8-bit is accepted: the next check is the pointers
    assert lib.gemma4_qlinear_create(ctypes.byref(desc), None, None, None, ctypes.byref(out)) == \
        qmm.Status.INVALID_ARGUMENT
    desc = qmm._Desc(16, 100, 4, 64)
    assert lib.gemma4_qlinear_create(ctypes.byref(desc), None, None, None, ctypes.byref(out)) == \
        qmm.Status.INVALID_ARGUMENT
    assert "multiple of 64" in qmm.last_error()
    desc = qmm._Desc(16, 64, 4, 64)
    assert lib.gemma4_qlinear_create(ctypes.byref(desc), None, None, None, ctypes.byref(out)) == \
        qmm.Status.INVALID_ARGUMENT
    assert "non-null weight" in qmm.last_error()
    assert out.value is None
    # handles are magic-checked: a bogus pointer is rejected, NULL free is a no-op
    bogus = ctypes.create_string_buffer(64)
    assert lib.gemma4_qlinear_forward(ctypes.cast(bogus, ctypes.c_void_p), None, None, 1, None, 0) == \
        qmm.Status.INVALID_ARGUMENT
    assert "invalid handle" in qmm.last_error()
    assert lib.gemma4_qlinear_free(None) == qmm.Status.OK
    assert qmm.last_error() == ""
    assert lib.gemma4_qlinear_free(ctypes.cast(bogus, ctypes.c_void_p)) == qmm.Status.INVALID_ARGUMENT
    info = qmm._Info()
    assert lib.gemma4_qlinear_info(None, ctypes.byref(info)) == qmm.Status.INVALID_ARGUMENT
    assert lib.gemma4_qlinear_dequantize(None, None, None) == qmm.Status.INVALID_ARGUMENT
    assert lib.gemma4_qmm_get_last_error(None, 0) == qmm.Status.INVALID_ARGUMENT


def test_geglu_pair_argument_checks(lib):
    out = ctypes.c_void_p()
    assert lib.gemma4_qgeglu_create(None, None, None, None, None, None, None, ctypes.byref(out)) == \
        qmm.Status.INVALID_ARGUMENT
    assert "non-null desc" in qmm.last_error()
    desc = qmm._Desc(15360, 3840, 4, 64)
    assert lib.gemma4_qgeglu_create(ctypes.byref(desc), None, None, None, None, None, None, None) == \
        qmm.Status.INVALID_ARGUMENT
    assert "out pointer" in qmm.last_error()
    assert lib.gemma4_qgeglu_create(ctypes.byref(desc), None, None, None, None, None, None, ctypes.byref(out)) == \
        qmm.Status.INVALID_ARGUMENT
    assert "gate and up" in qmm.last_error()
    desc = qmm._Desc(64, 64, 3, 64)
    assert lib.gemma4_qgeglu_create_device(ctypes.byref(desc), None, None, None, None, None, None, None,
                                           ctypes.byref(out)) == qmm.Status.UNSUPPORTED_CONFIG
    assert out.value is None
    bogus = ctypes.create_string_buffer(64)
    assert lib.gemma4_qgeglu_forward(ctypes.cast(bogus, ctypes.c_void_p), None, None, 1, None, 0) == \
        qmm.Status.INVALID_ARGUMENT
    assert "invalid handle" in qmm.last_error()


def test_process_wide_settings(lib):
    """gemma4_qmm_set_decode_kernel, _set_gemm_form and _set_gemm_min_rows return the
    previous setting; a value out of range selects the default (0) and a row count past
    INT_MAX is clamped to it; the Python mirror rejects out-of-range values instead."""
    for setter, top in ((lib.gemma4_qmm_set_decode_kernel, 2), (lib.gemma4_qmm_set_gemm_form, 1)):
        prev = setter(top)
        try:
            assert setter(top + 5) == top   # out of range: stored as the default
            assert setter(1) == 0
            assert setter(0) == 1
        finally:
            setter(prev)
    prev = lib.gemma4_qmm_set_gemm_min_rows(2 ** 32 - 1)
    try:
        assert lib.gemma4_qmm_set_gemm_min_rows(64) == 2 ** 31 - 1
        assert lib.gemma4_qmm_set_gemm_min_rows(0) == 64
    finally:
        lib.gemma4_qmm_set_gemm_min_rows(prev)
    for fn, bad in ((qmm.set_decode_kernel, 3), (qmm.set_gemm_form, 2), (qmm.set_gemm_min_rows, -1)):
        with pytest.raises(ValueError):
            fn(bad)
    with qmm.decode_kernel(2), qmm.gemm_form(1), qmm.gemm_min_rows(32):
        assert lib.gemma4_qmm_set_decode_kernel(2) == 2 and lib.gemma4_qmm_set_gemm_form(1) == 1
        assert lib.gemma4_qmm_set_gemm_min_rows(32) == 32
    assert lib.gemma4_qmm_set_decode_kernel(0) == 0 and lib.gemma4_qmm_set_gemm_form(0) == 0
    assert lib.gemma4_qmm_set_gemm_min_rows(0) == 0


def test_last_error_is_thread_local(lib):
    out = ctypes.c_void_p()
    assert lib.gemma4_qlinear_create(None, None, None, None, ctypes.byref(out)) != 0
    seen = {}

    def other():
        seen["msg"] = qmm.last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == ""
    assert qmm.last_error() != ""


def test_struct_layouts_match_header():
    assert ctypes.sizeof(qmm._Desc) == 16
    assert ctypes.sizeof(qmm._Info) == 32
    assert qmm._Info.device_bytes.offset == 16 and qmm._Info.device.offset == 24
    assert qmm._Info.flags.offset == 28
    assert ctypes.sizeof(qmm._Version) == 24


def test_python_mirror_rejects_unsupported_specs():
    with pytest.raises(qmm.Gemma4Error) as e:
        qmm.quantized_matmul(None, None, None, None, bits=3)
    assert e.value.status == qmm.Status.UNSUPPORTED_CONFIG
    with pytest.raises(qmm.Gemma4Error):
        qmm.quantized_matmul(None, None, None, None, transpose=False)
    with pytest.raises(qmm.Gemma4Error):
        qmm.dequantize(None, None, None, mode="mxfp4")
