"""ctypes binding of libcormorant_amd.so (the gfx950 kernel library).

The library is built in-tree by ``python -m cormorant_amd.build``.  There is no
fallback: if the shared object is missing or fails to load, every entry point
raises ``NativeLibraryError``.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcormorant_amd.so")

# Every symbol the C header declares (include/cormorant_amd.h).
EXPORTS = (
    "cm_vectorop", "cm_matmul", "cm_matmul_at", "cm_conv", "cm_pool",
    "cm_buf_pool_init", "cm_buf_pool_deinit", "cm_buf_alloc", "cm_buf_free", "cm_buf_ptr",
    "cm_buf_dev", "cm_buf_count", "cm_buf_init_view", "cm_buf_sync_to_device",
    "cm_buf_sync_from_device", "cm_run_op", "cm_run_matmul", "cm_run_matmul_at", "cm_run_conv",
    "cm_run_pool", "cm_set_stream", "cm_get_stream", "cm_sync", "cm_last_error", "cm_version",
    "cm_selftest_div", "cm_selftest_finalize", "cm_matmul_ex", "cm_conv_ex",
    "cm_matmul_workspace_size", "cm_conv_workspace_size", "cm_set_workspace",
    "cm_matmul_noalloc", "cm_conv_packed_size", "cm_conv_pack", "cm_conv_packed_ex",
    "cm_conv_pair_packed_size", "cm_conv_pair_pack", "cm_conv_pair_packed_ex",
    "cm_conv_gap_supported", "cm_conv_gap",
)

CM_OK = 0
CM_ERR_INVALID = -1
CM_ERR_HIP = -2
CM_ERR_RANGE = -3
CM_ERR_NOMEM = -4

# cm_epilogue_t add_mode / act
CM_EPI_ADD_NONE, CM_EPI_ADD_SAME, CM_EPI_ADD_COLUMN = 0, 1, 2
CM_EPI_ACT_NONE, CM_EPI_ACT_RELU, CM_EPI_ACT_RELU6 = 0, 1, 2


class NativeLibraryError(RuntimeError):
    pass


class CmError(RuntimeError):
    """A C-ABI call returned a negative status."""

    def __init__(self, func: str, code: int, msg: str):
        super().__init__(f"{func} failed with {code}: {msg}")
        self.func = func
        self.code = code


class CmBuf(ctypes.Structure):
    """Mirror of cm_buf_t (include/cormorant_amd.h)."""
    _fields_ = [
        ("host", ctypes.c_void_p),
        ("dev", ctypes.c_void_p),
        ("count", ctypes.c_uint32),
        ("is_owner", ctypes.c_uint8),
    ]


class CmEpilogue(ctypes.Structure):
    """Mirror of cm_epilogue_t (include/cormorant_amd.h)."""
    _fields_ = [
        ("add", ctypes.c_void_p),
        ("add_mode", ctypes.c_uint32),
        ("act", ctypes.c_uint32),
    ]


_u32 = ctypes.c_uint32
_vp = ctypes.c_void_p
_i = ctypes.c_int
_BUFP = ctypes.POINTER(CmBuf)

_SIGS = {
    "cm_vectorop": (_i, [_vp, _vp, _vp] + [_u32] * 5 + [_vp]),
    "cm_matmul": (_i, [_vp, _vp, _vp] + [_u32] * 7 + [_vp]),
    "cm_matmul_at": (_i, [_vp, _u32, _vp, _u32, _vp, _u32] + [_u32] * 7 + [_vp]),
    "cm_conv": (_i, [_vp, _vp, _vp, _vp] + [_u32] * 17 + [_vp]),
    "cm_pool": (_i, [_vp, _vp] + [_u32] * 17 + [_vp]),
    "cm_buf_pool_init": (_i, []),
    "cm_buf_pool_deinit": (None, []),
    "cm_buf_alloc": (_BUFP, [_u32]),
    "cm_buf_free": (None, [_BUFP]),
    "cm_buf_ptr": (_vp, [_BUFP]),
    "cm_buf_dev": (_vp, [_BUFP]),
    "cm_buf_count": (_u32, [_BUFP]),
    "cm_buf_init_view": (None, [_BUFP, _BUFP, _u32, _u32]),
    "cm_buf_sync_to_device": (_i, [_BUFP]),
    "cm_buf_sync_from_device": (_i, [_BUFP]),
    "cm_run_op": (_i, [_BUFP, _BUFP, _BUFP] + [_u32] * 5),
    "cm_run_matmul": (_i, [_BUFP, _BUFP, _BUFP] + [_u32] * 7),
    "cm_run_matmul_at": (_i, [_BUFP, _u32, _BUFP, _u32, _BUFP, _u32] + [_u32] * 7),
    "cm_run_conv": (_i, [_BUFP, _BUFP, _BUFP, _BUFP] + [_u32] * 17),
    "cm_run_pool": (_i, [_BUFP, _BUFP] + [_u32] * 17),
    "cm_set_stream": (_i, [_vp]),
    "cm_get_stream": (_vp, []),
    "cm_sync": (_i, [_vp]),
    "cm_last_error": (ctypes.c_char_p, []),
    "cm_version": (ctypes.c_char_p, []),
    "cm_selftest_div": (_i, [_u32, _u32, ctypes.POINTER(ctypes.c_uint64),
                                ctypes.POINTER(ctypes.c_uint64), _vp]),
    "cm_selftest_finalize": (_i, [_u32, _u32, _u32, _u32, ctypes.POINTER(ctypes.c_uint64), _vp]),
    "cm_matmul_ex": (_i, [_vp, _vp, _vp] + [_u32] * 7 +
                     [ctypes.POINTER(CmEpilogue), _vp, ctypes.c_size_t, _vp]),
    "cm_conv_ex": (_i, [_vp, _vp, _vp, _vp] + [_u32] * 17 +
                   [ctypes.POINTER(CmEpilogue), _vp, ctypes.c_size_t, _vp]),
    "cm_matmul_workspace_size": (ctypes.c_size_t, [_u32] * 7),
    "cm_conv_workspace_size": (ctypes.c_size_t, [_u32] * 17),
    "cm_set_workspace": (_i, [_vp, ctypes.c_size_t]),
    "cm_matmul_noalloc": (_i, [_vp, _vp, _vp] + [_u32] * 7 + [ctypes.POINTER(CmEpilogue), _vp]),
    "cm_conv_packed_size": (ctypes.c_size_t, [_u32] * 17),
    "cm_conv_pack": (_i, [_vp] + [_u32] * 17 + [_vp, ctypes.c_size_t, _vp]),
    "cm_conv_packed_ex": (_i, [_vp, _vp, _vp, _vp] + [_u32] * 17 + [ctypes.POINTER(CmEpilogue), _vp]),
    "cm_conv_pair_packed_size": (ctypes.c_size_t, [_u32] * 14),
    "cm_conv_pair_pack": (_i, [_vp, _vp] + [_u32] * 14 + [_vp, ctypes.c_size_t, _vp]),
    "cm_conv_pair_packed_ex": (_i, [_vp, _vp, _vp, _vp, _vp] + [_u32] * 15 +
                               [ctypes.POINTER(CmEpilogue), _vp]),
    "cm_conv_gap_supported": (_i, [_u32] * 4),
    "cm_conv_gap": (_i, [_vp, _vp, _vp, _vp] + [_u32] * 5 + [_vp]),
}

_lib = None


def load(path: str | None = None):
    """Load (once) and return the configured ctypes library."""
    global _lib
    if _lib is not None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise NativeLibraryError(
            f"{p} is missing: build it with `python -m cormorant_amd.build` (no CPU fallback exists)")
    try:
        L = ctypes.CDLL(p)
    except OSError as e:
        raise NativeLibraryError(f"cannot load {p}: {e}") from e
    for name, (res, args) in _SIGS.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def last_error() -> str:
    return load().cm_last_error().decode(errors="replace")


def check(func: str, rc: int) -> int:
    if rc != CM_OK:
        raise CmError(func, rc, last_error())
    return rc


def call(func: str, *args) -> int:
    """Call an int-returning entry point and raise CmError on failure."""
    return check(func, getattr(load(), func)(*args))
