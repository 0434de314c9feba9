"""CPU oracle for the Cormorant Q8.8 kernels -- TEST INFRASTRUCTURE ONLY.

Two independent restatements of the reference arithmetic live here:

* ``libcm_oracle.so`` (built from ``cm_oracle.c`` by ``oracle/Makefile``): the
  C-simulation semantics of VectorOPKernel / MatmulKernel / ConvKernel /
  PoolingKernel (kernels/*/kernel/*.cpp), in the reference loop order, with an
  OpenMP variant of each for the multi-thread CPU baseline.
* ``numpy_sim``: the scheduler's float64 numpy simulation
  (inference-scheduler/src/codegen/_simulate.py:49-383).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
may import this package, and only to check results.  The product package
``cormorant_amd`` never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libcm_oracle.so")
_lib = None

_u32 = ctypes.c_uint32
_p16 = ctypes.c_void_p


def build(force: bool = False) -> str:
    """Compile libcm_oracle.so with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        for name in ("ora_vectorop", "ora_vectorop_omp"):
            f = getattr(L, name)
            f.argtypes = [_p16, _p16, _p16] + [_u32] * 5
            f.restype = None
        for name in ("ora_matmul", "ora_matmul_omp"):
            f = getattr(L, name)
            f.argtypes = [_p16, _p16, _p16] + [_u32] * 7
            f.restype = None
        L.ora_matmul_row.argtypes = [_p16, _p16, _p16, _u32, _u32]
        L.ora_matmul_row.restype = None
        for name in ("ora_conv", "ora_conv_omp"):
            f = getattr(L, name)
            f.argtypes = [_p16, _p16, _p16, _p16] + [_u32] * 17
            f.restype = None
        for name in ("ora_pool", "ora_pool_omp"):
            f = getattr(L, name)
            f.argtypes = [_p16, _p16] + [_u32] * 17
            f.restype = None
        L.ora_q88_mul.argtypes = [ctypes.c_int16, ctypes.c_int16]
        L.ora_q88_mul.restype = ctypes.c_int16
        L.ora_q88_div.argtypes = [ctypes.c_int16, ctypes.c_int16]
        L.ora_q88_div.restype = ctypes.c_int16
        L.ora_avg_finalize.argtypes = [_u32, _u32]
        L.ora_avg_finalize.restype = ctypes.c_int16
        L.ora_lp2_finalize.argtypes = [_u32]
        L.ora_lp2_finalize.restype = ctypes.c_int16
        L.ora_lp2_checksum.argtypes = [_u32, _u32]
        L.ora_lp2_checksum.restype = ctypes.c_uint64
        L.ora_avg_checksum.argtypes = [_u32, _u32, _u32]
        L.ora_avg_checksum.restype = ctypes.c_uint64
        L.ora_set_threads.argtypes = [ctypes.c_int]
        L.ora_set_threads.restype = None
        L.ora_get_threads.argtypes = []
        L.ora_get_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _ptr(a):
    if a is None:
        return None
    assert a.dtype == np.int16 and a.flags["C_CONTIGUOUS"], "oracle takes contiguous int16"
    return a.ctypes.data


def set_threads(n: int) -> None:
    lib().ora_set_threads(int(n))


def get_threads() -> int:
    return int(lib().ora_get_threads())


def vectorop(a, b, c, size, op, outer=1, a_inc=0, b_inc=0, threads: bool = False):
    """VectorOPKernel(a, b, c, size, op, outer, a_inc, b_inc) on the CPU (in place on c)."""
    f = lib().ora_vectorop_omp if threads else lib().ora_vectorop
    f(_ptr(a), _ptr(b), _ptr(c), size, op, outer, a_inc, b_inc)
    return c


def matmul(a, b, c, n, k, m, batch=1, a_bs=0, b_bs=0, c_bs=0, threads: bool = False):
    """MatmulKernel(a, b, c, n, k, m, batch, strides) on the CPU (in place on c)."""
    f = lib().ora_matmul_omp if threads else lib().ora_matmul
    f(_ptr(a), _ptr(b), _ptr(c), n, k, m, batch, a_bs, b_bs, c_bs)
    return c


def matmul_row(a_row, b, k, m):
    out = np.zeros(m, dtype=np.int16)
    lib().ora_matmul_row(_ptr(np.ascontiguousarray(a_row)), _ptr(b), _ptr(out), k, m)
    return out


def conv(x, w, bias, y, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw,
         sh, sw, dh, dw, pad_top, pad_left, has_bias, is_dw, threads: bool = False):
    """ConvKernel(...) on the CPU (in place on y)."""
    f = lib().ora_conv_omp if threads else lib().ora_conv
    f(_ptr(x), _ptr(w), _ptr(bias) if has_bias else None, _ptr(y), batch, in_ch, in_h, in_w,
      out_ch, out_h, out_w, kh, kw, sh, sw, dh, dw, pad_top, pad_left, has_bias, is_dw)
    return y


def pool(x, y, batch, ch, in_h, in_w, out_h, out_w, ph, pw, sh, sw, pad_top, pad_left,
         dh, dw, pool_type, lp_order, cip, threads: bool = False):
    """PoolingKernel(...) on the CPU (in place on y)."""
    f = lib().ora_pool_omp if threads else lib().ora_pool
    f(_ptr(x), _ptr(y), batch, ch, in_h, in_w, out_h, out_w, ph, pw, sh, sw, pad_top,
      pad_left, dh, dw, pool_type, lp_order, cip)
    return y


def q88_mul(a: int, b: int) -> int:
    return int(lib().ora_q88_mul(a, b))


def q88_div(a: int, b: int) -> int:
    return int(lib().ora_q88_div(a, b))


def avg_finalize(acc: int, denom: int) -> int:
    return int(lib().ora_avg_finalize(acc & 0xFFFFFFFF, denom))


def lp2_finalize(acc: int) -> int:
    return int(lib().ora_lp2_finalize(acc & 0xFFFFFFFF))


def lp2_checksum(lo: int, hi: int) -> int:
    """Sum over a in [lo, hi) of (uint16)lp2_finalize(a) * (a | 1) mod 2^64."""
    return int(lib().ora_lp2_checksum(lo, hi))


def avg_checksum(lo: int, count: int, d: int) -> int:
    """Sum over v in [lo, lo+count) of (uint16)avg_finalize(v << 8, d) * (v | 1) mod 2^64."""
    return int(lib().ora_avg_checksum(lo, count, d))


def checksum_of(values, keys) -> int:
    """The same checksum for arrays computed elsewhere (numpy closed forms)."""
    import numpy as _np
    v = _np.asarray(values).astype(_np.int16).view(_np.uint16).astype(_np.uint64)
    k = _np.asarray(keys).astype(_np.uint64) | _np.uint64(1)
    with _np.errstate(over="ignore"):
        return int((v * k).sum(dtype=_np.uint64))
