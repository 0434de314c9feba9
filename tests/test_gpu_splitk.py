"""GPU parity of split-K launches: MatMul / Conv calls whose output tiles
cannot fill the GPU are computed as k-split partial sums plus a reduction pass
(the partials of every k range obey the same limb identity, and the uint32
sum of the partials is the wrapping accumulator).  The partials live in a
workspace the caller passes; compared bit for bit with the oracle, including
full-range operands whose sums wrap, with the full workspace, a smaller one
(fewer splits) and none (no split)."""
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
    """A device workspace pre-filled with garbage (partials must not depend on it)."""
    import torch
    t = torch.empty(max(nbytes, 4) // 4, dtype=torch.int32, device="cuda")
    t.fill_(0x3C5A7E11)
    return t

MM = [
    # name, n, k, m, operand range (None = full int16 range)
    ("one_tile_k5000", 100, 5000, 60, 2.0),
    ("fc_16x1280x20000", 16, 1280, 20000, 1.0),   # 16 x 1280 x 1000 takes the register-only kernel
    ("odd_steps_k449", 130, 449, 2100, 4.0),
    ("wrap_full_range", 64, 4160, 96, None),
    ("k256_two_tiles", 200, 256, 1400, 8.0),
    ("tiles64_k640", 1024, 640, 1024, 1.0),    # 64 tiles: split with two k steps per split
]


@pytest.mark.parametrize("case", MM, ids=[c[0] for c in MM])
def test_matmul_split(case):
    name, n, k, m, rng_ = case
    say(f"split-K matmul {name}")
    g = wl.rng(910, n, k, m)
    if rng_ is None:
        a, b = full_range(g, n * k), full_range(g, k * m)
    else:
        a = wl.uniform_q88(g, n * k, -rng_, rng_)
        b = wl.uniform_q88(g, k * m, -rng_, rng_)
    want = np.zeros(n * m, np.int16)
    oracle.set_threads(oracle_threads())
    oracle.matmul(a, b, want, n, k, m, threads=True)
    need = K.matmul_workspace_size(n, k, m)
    assert need > 0, "the case is meant to split"
    # the full workspace, one for two splits only, one too small to split, none
    for ws_bytes in (need, 2 * n * ((m + 7) // 8 * 8) * 4, 4 * n, None):
        c = empty_dev(n * m)
        K.MatmulKernel(dev(a), dev(b), c, n, k, m,
                       workspace=None if ws_bytes is None else workspace(ws_bytes))
        np.testing.assert_array_equal(host(c), want, err_msg=f"workspace {ws_bytes}")


@pytest.mark.parametrize("extra", [16, 0])
def test_matmul_split_unaligned_workspace(extra):
    """A workspace that starts 2 bytes past a 16-byte boundary (an int16 view at an
    odd element offset): the partials (16-byte vector stores) go to its first aligned
    byte on, with fewer splits when the rest is too small; the result is the oracle's."""
    import torch
    n, k, m = 64, 4160, 96
    say(f"split-K matmul, workspace at +2 bytes, {extra} spare bytes")
    g = wl.rng(914, extra)
    a, b = full_range(g, n * k), full_range(g, k * m)
    want = np.zeros(n * m, np.int16)
    oracle.set_threads(oracle_threads())
    oracle.matmul(a, b, want, n, k, m, threads=True)
    need = K.matmul_workspace_size(n, k, m)
    base = workspace(need + extra + 16).view(torch.int16)
    ws = base[1: 1 + (need + extra) // 2]
    assert ws.data_ptr() % 16 == 2
    c = empty_dev(n * m)
    K.MatmulKernel(dev(a), dev(b), c, n, k, m, workspace=ws)
    np.testing.assert_array_equal(host(c), want)


@pytest.mark.parametrize("act", [K.ACT_NONE, K.ACT_RELU6])
def test_matmul_split_column_add(act):
    say(f"split-K matmul column add act {act}")
    n, k, m = 16, 1280, 1000
    g = wl.rng(911, act)
    a = wl.uniform_q88(g, n * k, -1.0, 1.0)
    b = wl.uniform_q88(g, k * m, -0.5, 0.5)
    bias = full_range(g, m)
    c = empty_dev(n * m)
    K.MatmulKernel(dev(a), dev(b), c, n, k, m, add=dev(bias), add_column=True, act=act,
                   workspace=workspace(K.matmul_workspace_size(n, k, m)))
    y = np.zeros(n * m, np.int16)
    oracle.matmul(a, b, y, n, k, m)
    np.testing.assert_array_equal(host(c), apply_epilogue(y, bias, True, act, n, m))


CONV = [
    # name, N, C, H, W, M, k, s, p
    ("7x7x160", 16, 160, 7, 7, 160, 3, 1, 1),
    ("14x14x256_s2", 16, 256, 14, 14, 96, 3, 2, 1),   # K = 2304: past the register-only kernel
    ("14x14x64", 16, 64, 14, 14, 64, 3, 1, 1),
    ("5x5_kernel_c40", 2, 40, 9, 9, 50, 5, 1, 2),
]


@pytest.mark.parametrize("case", CONV, ids=[c[0] for c in CONV])
def test_conv_split(case):
    name, N, C, H, W, M, k, s, p = case
    say(f"split-K conv {name}")
    g = wl.rng(912, N, C, M)
    OH = (H + 2 * p - k) // s + 1
    x = wl.uniform_q88(g, N * C * H * W, -4.0, 4.0)
    w = full_range(g, M * C * k * k)
    bias = full_range(g, M)
    res = full_range(g, N * M * OH * OH)
    args = (N, C, H, W, M, OH, OH, k, k, s, s, 1, 1, p, p, 1, 0)
    y = np.zeros(N * M * OH * OH, np.int16)
    oracle.set_threads(oracle_threads())
    oracle.conv(x, w, bias, y, *args, threads=True)
    need = K.conv_workspace_size(*args)
    assert need > 0, "the case is meant to split"
    ws = workspace(need)
    for w_ in (ws, None):
        out = empty_dev(y.size)
        K.ConvKernel(dev(x), dev(w), dev(bias), out, *args, workspace=w_)
        np.testing.assert_array_equal(host(out), y)
    out2 = empty_dev(y.size)
    K.ConvKernel(dev(x), dev(w), dev(bias), out2, *args, add=dev(res), act=K.ACT_RELU, workspace=ws)
    np.testing.assert_array_equal(host(out2), apply_epilogue(y, res, False, K.ACT_RELU, 0, 0))
