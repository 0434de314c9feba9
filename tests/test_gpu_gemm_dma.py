"""GPU parity of the large-MatMul path that streams operands into LDS with
direct-to-LDS loads (csrc/gemm_dma.hip): B packed once per call into MFMA-ready
limb fragments in the caller's workspace, A raw in LDS and split per fragment.
Every case runs MatmulKernel with the workspace that cm_matmul_workspace_size
reports and compares the whole output with the CPU oracle bit for bit: full-range
operands whose sums wrap, ragged n / m / k (m and k multiples of 8), a broadcast
B, batch outputs with gaps, the fused Add (same-shaped and per column) with each
activation, and the benchmark's two configurations at full size."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from cormorant_amd import kernels as K
from cormorant_amd import workloads as wl
from tests.gpu_util import dev, empty_dev, host, oracle_threads, say
from tests.test_gpu_epilogue import apply_epilogue, full_range

pytestmark = pytest.mark.gpu


def workspace(nbytes: int):
    import torch
    t = torch.empty(max(nbytes, 4) // 4 + 1, dtype=torch.int32, device="cuda")
    t.fill_(0x3C5A7E11)   # the path must not depend on the workspace's old contents
    return t


def run_both(a, b, n, k, m, batch=1, a_bs=0, b_bs=0, c_bs=None, add=None, column=False,
             act=K.ACT_NONE):
    c_bs = n * m if c_bs is None else c_bs
    c_len = (batch - 1) * c_bs + n * m
    need = K.matmul_workspace_size(n, k, m, batch, a_bs, b_bs, c_bs)
    c = empty_dev(c_len)
    K.MatmulKernel(dev(a), dev(b), c, n, k, m, batch, a_bs, b_bs, c_bs,
                   add=None if add is None else dev(add), add_column=column, act=act,
                   workspace=workspace(need))
    want = np.full(c_len, 0x5A5A, np.int16)
    oracle.set_threads(oracle_threads())
    oracle.matmul(np.ascontiguousarray(a.reshape(-1)), np.ascontiguousarray(b.reshape(-1)), want,
                  n, k, m, batch, a_bs, b_bs, c_bs, threads=True)
    if add is not None or act != K.ACT_NONE:
        assert batch == 1 or column is False
        want = apply_epilogue(want, add, column, act, n * batch if c_bs == n * m else n, m)
    return host(c), want, need


SHAPES = [
    # name, batch, n, k, m, b broadcast, c gap  (the path takes >= 256 output tiles of 128 x 128)
    ("square", 1, 2048, 512, 2048, False, 0),
    ("ragged_n", 1, 2000, 264, 2048, False, 0),       # n past a tile, k not a multiple of 64
    ("ragged_m", 1, 2304, 512, 1832, False, 0),       # m a multiple of 8, not of 128
    ("batched", 8, 512, 1024, 1024, False, 0),
    ("broadcast_b", 6, 1024, 320, 768, True, 0),
    ("gapped_c", 4, 1024, 256, 1024, False, 8),       # batch outputs with 8-element gaps
    ("long_k", 1, 2048, 8192, 2048, False, 0),
    # the kernel is persistent (one block per CU walking its tiles, the next tile's
    # first steps loaded during the current one's last): several tiles per block,
    # shares of unequal length, odd step counts, ragged edges on every side
    ("many_tiles_ragged", 1, 3000, 264, 2600, False, 0),   # 24 x 21 = 504 tiles, 5 steps
    ("batched_odd_steps", 5, 1000, 320, 1000, False, 0),   # 320 tiles, 5 steps
    ("broadcast_many", 9, 640, 256, 904, True, 16),        # 9 x 5 x 8 = 360 tiles, 4 steps, gaps
]


@pytest.mark.parametrize("case", SHAPES, ids=[s[0] for s in SHAPES])
def test_full_range_shapes(case):
    name, batch, n, k, m, bcast, gap = case
    say(f"gemm_dma {name}: batch {batch} {n}x{k}x{m}")
    g = wl.rng(930, batch, n, k, m)
    a = full_range(g, batch * n * k)
    b = full_range(g, (1 if bcast else batch) * k * m)
    got, want, need = run_both(a, b, n, k, m, batch, n * k, 0 if bcast else k * m, n * m + gap)
    assert need > 0
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("column", [False, True])
@pytest.mark.parametrize("act", [K.ACT_NONE, K.ACT_RELU, K.ACT_RELU6])
def test_fused_epilogue(column, act):
    n, k, m = 2048, 512, 2048
    say(f"gemm_dma epilogue column={column} act={act}")
    g = wl.rng(931, int(column), act)
    a = wl.uniform_q88(g, n * k, -2.0, 2.0)
    b = wl.uniform_q88(g, k * m, -2.0, 2.0)
    add = full_range(g, m if column else n * m)
    got, want, _ = run_both(a, b, n, k, m, add=add, column=column, act=act)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("cid", [0, 1], ids=[c.name for c in wl.GEMM_CASES])
def test_benchmark_configurations(cid):
    case = wl.GEMM_CASES[cid]
    say(f"gemm_dma {case.name}")
    a, b = wl.gemm_operands(case, cid)
    n, k, m, bt = case.n, case.k, case.m, case.batch
    got, want, _ = run_both(a, b, n, k, m, bt, n * k, k * m, n * m)
    np.testing.assert_array_equal(got, want)
