"""cm_matmul_noalloc (split-K partials in the library's static device array)
against cm_matmul_ex with a caller workspace and against the CPU oracle, bit for
bit, through the C ABI: two calls in a row, the second with a smaller input
(full-range operands whose sums wrap), then a shape whose partials exceed the
array (rejected, nothing launched)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from cormorant_amd import _native
from cormorant_amd import kernels as K
from cormorant_amd import workloads as wl
import oracle
from tests.gpu_util import dev, empty_dev, host, oracle_threads, say

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20


def _noalloc(a, b, c, n, k, m, batch=1, a_bs=0, b_bs=0, c_bs=0, epi=None):
    import torch
    lib = _native.load()
    return lib.cm_matmul_noalloc(a.data_ptr(), b.data_ptr(), c.data_ptr(), n, k, m, batch, a_bs,
                                 b_bs, c_bs, ctypes.byref(epi) if epi is not None else None,
                                 torch.cuda.current_stream().cuda_stream)


def test_noalloc_matches_workspace_entry_point():
    import torch
    g = wl.rng(990)
    # first call: 16 x 1280 x 20000 with a fused column Add and Relu6 (splits 2 ways);
    # second, smaller: 64 x 4160 x 96 full-range operands whose sums wrap (16 splits)
    cases = [(16, 1280, 20000, 1.0, True), (64, 4160, 96, None, False)]
    for n, k, m, r, fused in cases:
        need = K.matmul_workspace_size(n, k, m)
        assert 0 < need <= SCRATCH_BYTES, need
        say(f"matmul_noalloc {n}x{k}x{m}, partials {need} bytes")
        if r is None:
            a = g.integers(-32768, 32768, n * k, dtype=np.int16)
            b = g.integers(-32768, 32768, k * m, dtype=np.int16)
        else:
            a = wl.uniform_q88(g, n * k, -r, r)
            b = wl.uniform_q88(g, k * m, -r, r)
        da, db = dev(a), dev(b)
        add = dev(g.integers(-32768, 32768, m, dtype=np.int16)) if fused else None
        ws = torch.empty(need // 4, dtype=torch.int32, device="cuda")
        want = empty_dev(n * m)
        K.MatmulKernel(da, db, want, n, k, m, add=add, add_column=fused,
                       act=K.ACT_RELU6 if fused else K.ACT_NONE, workspace=ws)
        got = empty_dev(n * m)
        epi = None
        if fused:
            epi = _native.CmEpilogue()
            epi.add, epi.add_mode, epi.act = add.data_ptr(), _native.CM_EPI_ADD_COLUMN, _native.CM_EPI_ACT_RELU6
        rc = _noalloc(da, db, got, n, k, m, epi=epi)
        assert rc == 0, _native.last_error()
        np.testing.assert_array_equal(host(got), host(want))
        # and against the oracle directly: MatMul, then the Add of the column
        # vector per row and Clip(0,6) as the separate VectorOP calls compute them
        ref = np.zeros(n * m, np.int16)
        oracle.set_threads(oracle_threads())
        oracle.matmul(a, b, ref, n, k, m, threads=True)
        if fused:
            tmp = ref.copy()
            oracle.vectorop(tmp, host(add), ref, m, 0, n, m, 0)
            oracle.vectorop(ref.copy(), ref.copy(), ref, n * m, 5)
        np.testing.assert_array_equal(host(got), ref)


def test_noalloc_rejects_partials_beyond_the_array():
    n, k, m = 1280, 2048, 1536
    need = K.matmul_workspace_size(n, k, m)
    assert need > SCRATCH_BYTES, need
    say(f"matmul_noalloc rejection {n}x{k}x{m}, partials {need} bytes")
    a, b = empty_dev(n * k, 0), empty_dev(k * m, 0)
    c = empty_dev(n * m)
    rc = _noalloc(a, b, c, n, k, m)
    assert rc == _native.CM_ERR_RANGE
    assert "static scratch" in _native.last_error()
    assert np.all(host(c) == np.int16(0x5A5A))   # nothing was launched
