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
        return lib.cm_matmul_ex(fake, fake, fake, 2, 2, 2, 1, 0, 0, 0, e, None, 0, None)

    def conv(e):
        return lib.cm_conv_ex(fake, fake, None, fake, *([1] * 15), 0, 0, e, None, 0, None)

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


def test_workspace_size_queries():
    """cm_*_workspace_size: a dry run of the launch decision (no GPU work).  Large
    MatMuls (>= 256 output tiles of 128 x 128) pack B into limb fragments: 2 KB per
    16 columns and 64 k, plus uint32 column sums per k chunk of the pack grid
    (about 1024 blocks); other shapes whose tiles fill the GPU never split; few
    tiles over a long k range split into at most 16 parts of uint32 partials,
    rows x cols rounded up to 8 columns."""
    lib = _native.load()
    # 4096^3: 64 k steps x 256 column tiles x 2 KB; 32 column groups -> 32 k chunks of 2 steps
    assert lib.cm_matmul_workspace_size(4096, 4096, 4096, 1, 0, 0, 0) == \
        64 * 256 * 2048 + 32 * 256 * 16 * 4
    # batch 32 of 1024^3: 32 x (16 x 64 x 2 KB) and 8 groups x 32 batches -> 4 k chunks
    assert lib.cm_matmul_workspace_size(1024, 1024, 1024, 32, 1 << 20, 1 << 20, 1 << 20) == \
        32 * (16 * 64 * 2048 + 4 * 64 * 16 * 4)
    # a broadcast B is packed once: 8 groups -> 16 k chunks of one step
    assert lib.cm_matmul_workspace_size(1024, 1024, 1024, 32, 1 << 20, 0, 1 << 20) == \
        16 * 64 * 2048 + 16 * 64 * 16 * 4
    # m not a multiple of 8: the general path, no split
    assert lib.cm_matmul_workspace_size(4096, 4096, 4092, 1, 0, 0, 0) == 0
    # one tile, 79 k steps: 16 splits of 100 x 64 (60 rounded up) words
    assert lib.cm_matmul_workspace_size(100, 5000, 60, 1, 0, 0, 0) == 16 * 100 * 64 * 4
    # 16 x 1280 x 1000 (16,000 outputs, 20 k steps) takes the register-only kernel: none
    assert lib.cm_matmul_workspace_size(16, 1280, 1000, 1, 0, 0, 0) == 0
    # 16 x 1280 x 20000: 157 tiles, 20 k steps -> 2 splits of 16 x 20000 words
    assert lib.cm_matmul_workspace_size(16, 1280, 20000, 1, 0, 0, 0) == 2 * 16 * 20000 * 4
    # batched without overlap: one launch over every batch, no split
    assert lib.cm_matmul_workspace_size(100, 5000, 60, 4, 500000, 300000, 6000) == 0
    # batches whose outputs overlap run one launch each, each of which may split
    assert lib.cm_matmul_workspace_size(100, 5000, 60, 3, 500000, 300000, 10) == 16 * 100 * 64 * 4
    assert lib.cm_matmul_workspace_size(0, 5000, 60, 1, 0, 0, 0) == 0
    # convolution: a 7x7 3x3 layer 256 -> 160 at batch 16 with column stride 2 (K =
    # 2304 is past the register-only kernel: the gather path over 16 * 7 * 4 = 448
    # columns, split over k)
    conv = lib.cm_conv_workspace_size(16, 256, 7, 7, 160, 7, 4, 3, 3, 1, 2, 1, 1, 1, 1, 1, 0)
    assert conv > 0 and conv % (160 * 448 * 4) == 0
    # the same layer with stride 1 takes the patch-GEMM path: two row tiles of 128
    # channels, 36 k steps (four chunks of 64 channels x 9 taps), 3 planes of
    # 128 x 64 bytes per tile and step
    assert lib.cm_conv_workspace_size(16, 256, 7, 7, 160, 7, 7, 3, 3, 1, 1, 1, 1, 1, 1, 1, 0) == \
        2 * 36 * 3 * 128 * 64 + 8 * 256
    # a small strided layer (16 x 160 x 14 x 14 -> 7 x 7, K = 1440) on the
    # register-only kernel: none
    assert lib.cm_conv_workspace_size(16, 160, 14, 14, 160, 7, 7, 3, 3, 2, 2, 1, 1, 1, 1, 1, 0) == 0
    # conv A of the benchmark block: the patch-GEMM path, whose workspace holds the
    # weights as two int8 limb planes and one int8 plane (9 k steps x 128 rows x 64 k
    # x 3), 128 row sums and 128 int8 flags; depthwise never uses a workspace
    assert lib.cm_conv_workspace_size(32, 64, 56, 56, 128, 56, 56, 3, 3, 1, 1, 1, 1, 1, 1, 1, 0) == \
        9 * 128 * 64 * 3 + 128 * 8
    assert lib.cm_conv_workspace_size(1, 64, 56, 56, 64, 56, 56, 3, 3, 1, 1, 1, 1, 1, 1, 0, 1) == 0
