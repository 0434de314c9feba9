"""C-ABI checks that need no GPU: the library loads, and it exports exactly the
entry points include/cormorant_amd.h declares (no compute calls here)."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

from cormorant_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cormorant_amd.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cm_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert header_functions() == sorted(_native.EXPORTS)


def test_library_loads_and_exports_every_symbol():
    lib = _native.load()
    for name in header_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _native.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (cm_[a-z0-9_]+)\b", out))
    assert set(header_functions()) <= exported
    assert lib.cm_version().decode().startswith("cormorant_amd")


def test_invalid_arguments_are_rejected_before_any_launch():
    """Null pointers return CM_ERR_INVALID without touching the GPU."""
    lib = _native.load()
    assert lib.cm_vectorop(None, None, None, 8, 0, 1, 0, 0, None) == _native.CM_ERR_INVALID
    assert "null" in _native.last_error()
    assert lib.cm_matmul(None, None, None, 2, 2, 2, 1, 0, 0, 0, None) == _native.CM_ERR_INVALID
    assert lib.cm_conv(None, None, None, None, *([1] * 17), None) == _native.CM_ERR_INVALID
    assert lib.cm_pool(None, None, *([1] * 17), None) == _native.CM_ERR_INVALID
    # zero-sized work is a no-op success
    assert lib.cm_vectorop(None, None, None, 0, 0, 1, 0, 0, None) == _native.CM_OK
    assert lib.cm_run_op(None, None, None, 8, 0, 1, 0, 0) == _native.CM_ERR_INVALID


def test_bad_epilogues_are_rejected_before_any_launch():
    """cm_matmul_ex / cm_conv_ex validate the epilogue before launching (the
    pointers below are never dereferenced: every call returns CM_ERR_INVALID)."""
    lib = _native.load()
    fake = 4096

    def epi(add, mode, act):
        e = _native.CmEpilogue()
        e.add, e.add_mode, e.act = add, mode, act
        return ctypes.byref(e)

    def mm(e):
        return lib.cm_matmul_ex(fake, fake, fake, 2, 2, 2, 1, 0, 0, 0, e, None)

    def conv(e):
        return lib.cm_conv_ex(fake, fake, None, fake, *([1] * 15), 0, 0, e, None)

    assert mm(epi(fake, 3, 0)) == _native.CM_ERR_INVALID
    assert mm(epi(fake, _native.CM_EPI_ADD_SAME, 3)) == _native.CM_ERR_INVALID
    assert mm(epi(None, _native.CM_EPI_ADD_COLUMN, 0)) == _native.CM_ERR_INVALID
    assert "null add" in _native.last_error()
    assert conv(epi(fake, _native.CM_EPI_ADD_COLUMN, 0)) == _native.CM_ERR_INVALID
    assert "add_mode" in _native.last_error()
    assert conv(epi(None, _native.CM_EPI_ADD_SAME, 0)) == _native.CM_ERR_INVALID


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(_native.NativeLibraryError):
        saved = _native._lib
        _native._lib = None
        try:
            _native.load(str(tmp_path / "nope.so"))
        finally:
            _native._lib = saved
