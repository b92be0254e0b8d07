"""CPU checks of the C-ABI library: it loads, exports every symbol that
include/cvs_hip.h declares, and fails cleanly (no crash, clear message) when
no GPU is present.  No compute is launched here."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cvs_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cvs_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree(cvs):
    assert set(declared_symbols()) == set(cvs.exported_symbols())


def test_library_exports_every_declared_symbol(cvs):
    lib = ctypes.CDLL(cvs.library_path())
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_library_is_built_for_gfx950(cvs):
    blob = open(cvs.library_path(), "rb").read()
    assert b"gfx950" in blob


def test_dispatch_counter_resets(cvs):
    cvs.reset_dispatch_count()
    assert cvs.dispatch_count() == 0


def test_null_arguments_are_rejected(cvs):
    lib = cvs.load()
    assert lib.cvs_device_count(None) == cvs.CVS_ERR_INVALID_ARGUMENT
    assert "null" in lib.cvs_last_error().decode()
    assert lib.cvs_context_create(0, None) == cvs.CVS_ERR_INVALID_ARGUMENT
    assert lib.cvs_context_synchronize(None) == cvs.CVS_ERR_INVALID_ARGUMENT
    assert lib.cvs_dataset_shape(None, None, None) == cvs.CVS_ERR_INVALID_ARGUMENT
    assert lib.cvs_context_destroy(None) == cvs.CVS_OK
    assert lib.cvs_dataset_destroy(None) == cvs.CVS_OK
    out = ctypes.c_double(0)
    assert lib.cvs_calibrate_mfma(None, None, 0, 1, 2, 0, 1, ctypes.byref(out)) == cvs.CVS_ERR_INVALID_ARGUMENT
    assert lib.cvs_calibrate_stream_read(None, 1 << 20, 1, 1, ctypes.byref(out)) == cvs.CVS_ERR_INVALID_ARGUMENT


def test_no_device_is_an_error_not_a_fallback(cvs):
    if cvs.device_count() > 0:
        pytest.skip("a GPU is visible")
    with pytest.raises(RuntimeError, match="no HIP device"):
        cvs.Context(0)
