"""GPU parity of the conv + pool block at full size: conv A (3x3 s1 p1) and
conv B (3x3 s2 d2 p2), N=32, 64 -> 128 channels on 56x56 with bias, each
followed by MaxPool 3x3/s2, AveragePool 3x3/s2 pad 1 count_include_pad,
LpPool p=2 2x2/s2 and GlobalAveragePool.  The pools read the convolution's
device output (nothing goes back through the host between the kernels); the
oracle runs the same chain on the CPU and every tensor is compared bit for bit."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from cormorant_amd import kernels as K
from cormorant_amd import workloads as wl
from tests.gpu_util import dev, empty_dev, host, oracle_threads, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", wl.CONV_CASES, ids=[c.name for c in wl.CONV_CASES])
def test_conv_then_pools_chained(case):
    import torch
    say(f"block: {case.name} then the four pools")
    x, w, b = wl.conv_operands(case)
    o = case.out_hw
    args = (case.batch, case.in_ch, case.hw, case.hw, case.out_ch, o, o, case.k, case.k,
            case.stride, case.stride, case.dil, case.dil, case.pad, case.pad, 1, 0)
    y = empty_dev(case.batch * case.out_ch * o * o)
    need = K.conv_workspace_size(*args)
    ws = torch.empty(max(need, 4) // 4, dtype=torch.int32, device="cuda")
    K.ConvKernel(dev(x), dev(w), dev(b), y, *args, workspace=ws)
    oracle.set_threads(oracle_threads())
    y_ref = np.zeros(y.numel(), np.int16)
    oracle.conv(x.reshape(-1), w.reshape(-1), b, y_ref, *args, threads=True)
    np.testing.assert_array_equal(host(y), y_ref, err_msg=case.name)
    for pc in wl.POOL_CASES:
        say(f"block: {pc.name} on {case.name} ({o}x{o})")
        a = wl.pool_args(pc, case.batch, case.out_ch, o)
        ny = case.batch * case.out_ch * a["out_h"] * a["out_w"]
        z = empty_dev(ny)
        K.PoolingKernel(y, z, **a)
        want = np.zeros(ny, np.int16)
        oracle.pool(y_ref, want, *a.values(), threads=True)
        np.testing.assert_array_equal(host(z), want, err_msg=f"{pc.name} on {case.name}")
