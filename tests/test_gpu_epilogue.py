"""GPU parity of the fused MatMul / Conv epilogues (cm_matmul_ex / cm_conv_ex).

Expected values come from the unfused sequence on the oracle: the C-simulation
MatMul / Conv, then VectorOP Add (flat, or broadcast per column) and then
VectorOP Relu / Relu6 -- exactly the calls the epilogue replaces."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from cormorant_amd import kernels as K
from cormorant_amd import workloads as wl
from tests.gpu_util import dev, empty_dev, host, oracle_threads, say

pytestmark = pytest.mark.gpu

ACT_OPS = {K.ACT_NONE: None, K.ACT_RELU: 4, K.ACT_RELU6: 5}


def full_range(g, n):
    return g.integers(-32768, 32768, n, dtype=np.int64).astype(np.int16)


def apply_epilogue(y, add, column, act, rows, m, row_stride=None):
    """Unfused VectorOP calls on the oracle, in place on y."""
    if add is not None:
        out = np.empty_like(y)
        if column:
            stride = m if row_stride is None else row_stride
            out[:] = y
            oracle.vectorop(y, add, out, m, 0, rows, stride, 0)
        else:
            oracle.vectorop(y, add, out, y.size, 0)
        y = out
    if ACT_OPS[act] is not None:
        out = np.empty_like(y)
        oracle.vectorop(y, None, out, y.size, ACT_OPS[act])
        y = out
    return y


MM_CASES = [
    # name, n, k, m, batch, add mode ("same" / "column" / None), act
    ("same_relu6_b3", 37, 100, 45, 3, "same", K.ACT_RELU6),
    ("same_none", 130, 64, 129, 1, "same", K.ACT_NONE),
    ("column_relu", 64, 784, 256, 1, "column", K.ACT_RELU),
    ("column_none_k1280", 16, 1280, 1000, 1, "column", K.ACT_NONE),
    ("act_only_relu", 200, 72, 33, 2, None, K.ACT_RELU),
    ("act_only_relu6", 8, 5000, 8, 1, None, K.ACT_RELU6),
]


@pytest.mark.parametrize("case", MM_CASES, ids=[c[0] for c in MM_CASES])
def test_matmul_epilogue(case):
    name, n, k, m, batch, mode, act = case
    say(f"matmul epilogue {name}")
    g = wl.rng(901, n, k, m)
    a = wl.uniform_q88(g, batch * n * k, -2.0, 2.0)
    b = wl.uniform_q88(g, batch * k * m, -2.0, 2.0)
    add = None if mode is None else full_range(g, m if mode == "column" else batch * n * m)
    c = empty_dev(batch * n * m)
    K.MatmulKernel(dev(a), dev(b), c, n, k, m, batch, n * k, k * m, n * m,
                   add=None if add is None else dev(add), add_column=mode == "column", act=act)
    y = np.zeros(batch * n * m, np.int16)
    oracle.set_threads(oracle_threads())
    oracle.matmul(a, b, y, n, k, m, batch, n * k, k * m, n * m, threads=True)
    want = apply_epilogue(y, add, mode == "column", act, batch * n, m)
    np.testing.assert_array_equal(host(c), want)


def test_matmul_column_add_strided_rows():
    """Batched single-row MatMul with padded output rows (the scheduler's
    row-strided form) + bias: only the data columns of each row change."""
    say("matmul epilogue strided rows")
    n, k, m, batch, c_bs = 1, 256, 10, 64, 16
    g = wl.rng(902)
    a = wl.uniform_q88(g, (batch - 1) * 256 + n * k, -1.0, 1.0)
    b = wl.uniform_q88(g, k * m, -1.0, 1.0)
    add = full_range(g, m)
    c = empty_dev(batch * c_bs)
    K.MatmulKernel(dev(a), dev(b), c, n, k, m, batch, 256, 0, c_bs, add=dev(add), add_column=True)
    y = np.full(batch * c_bs, 0x5A5A, np.int16)
    oracle.matmul(a, b, y, n, k, m, batch, 256, 0, c_bs)
    want = y.copy()
    oracle.vectorop(y, add, want, m, 0, batch, c_bs, 0)
    np.testing.assert_array_equal(host(c), want)


CONV_CASES = [
    # name, N, C, H, W, M, k, s, d, p, depthwise
    ("3x3_s1_patch", 16, 16, 20, 20, 24, 3, 1, 1, 1, 0),
    ("3x3_s2_patch", 64, 8, 17, 15, 40, 3, 2, 1, 1, 0),
    ("3x3_s2_small", 3, 8, 17, 15, 40, 3, 2, 1, 1, 0),
    ("3x3_s1_tab", 2, 20, 20, 20, 24, 3, 1, 1, 1, 0),
    ("1x1_pointwise", 2, 24, 14, 14, 32, 1, 1, 1, 0, 0),
    ("3x3_inc_k2304", 1, 256, 9, 9, 20, 3, 1, 1, 1, 0),
    ("depthwise_3x3", 2, 12, 11, 13, 12, 3, 1, 1, 1, 1),
    ("direct_1x1", 2, 24, 130, 130, 24, 1, 1, 1, 0, 0),
]


def conv_case(case, seed):
    name, N, C, H, W, M, k, s, d, p, dwise = case
    g = wl.rng(903, seed)
    OH = (H + 2 * p - d * (k - 1) - 1) // s + 1
    OW = (W + 2 * p - d * (k - 1) - 1) // s + 1
    x = wl.uniform_q88(g, N * C * H * W, -2.0, 2.0)
    w = wl.uniform_q88(g, M * (1 if dwise else C) * k * k, -0.5, 0.5)
    bias = wl.uniform_q88(g, M, -1.0, 1.0)
    args = (N, C, H, W, M, OH, OW, k, k, s, s, d, d, p, p, 1, dwise)
    y = np.zeros(N * M * OH * OW, np.int16)
    oracle.set_threads(oracle_threads())
    oracle.conv(x, w, bias, y, *args, threads=True)
    return g, x, w, bias, args, y


@pytest.mark.parametrize("act", [K.ACT_NONE, K.ACT_RELU, K.ACT_RELU6])
@pytest.mark.parametrize("case", CONV_CASES, ids=[c[0] for c in CONV_CASES])
def test_conv_epilogue(case, act):
    say(f"conv epilogue {case[0]} act {act}")
    g, x, w, bias, args, y = conv_case(case, act)
    add = full_range(g, y.size)
    out = empty_dev(y.size)
    K.ConvKernel(dev(x), dev(w), dev(bias), out, *args, add=dev(add), act=act)
    np.testing.assert_array_equal(host(out), apply_epilogue(y, add, False, act, 0, 0))
    out2 = empty_dev(y.size)
    K.ConvKernel(dev(x), dev(w), dev(bias), out2, *args, act=act)
    if act != K.ACT_NONE:
        np.testing.assert_array_equal(host(out2), apply_epilogue(y, None, False, act, 0, 0))


def test_conv_epilogue_in_place_add():
    """add == output buffer (a residual Add writing over its operand)."""
    say("conv epilogue in place")
    g, x, w, bias, args, y = conv_case(CONV_CASES[0], 7)
    res = full_range(g, y.size)
    buf = dev(res)
    K.ConvKernel(dev(x), dev(w), dev(bias), buf, *args, add=buf, act=K.ACT_RELU6)
    np.testing.assert_array_equal(host(buf), apply_epilogue(y, res, False, K.ACT_RELU6, 0, 0))


ROWS_CASES = [
    # batch, k, m, a_bs, c_bs, add mode, act: single-row products sharing B (one
    # product on the register-only kernel, A rows a_bs apart, C rows c_bs apart)
    (64, 256, 10, 256, 16, "column", K.ACT_NONE),
    (100, 784, 33, 792, 40, "same", K.ACT_RELU),
    (7, 72, 1, 72, 3, None, K.ACT_RELU6),
    (300, 128, 64, 136, 64, "column", K.ACT_RELU6),
    (33, 20, 17, 24, 17, "same", K.ACT_NONE),
    (5, 1000, 200, 1000, 256, None, K.ACT_NONE),
]


@pytest.mark.parametrize("case", ROWS_CASES, ids=[str(c[:5]) for c in ROWS_CASES])
def test_matmul_single_row_batches(case):
    """Batches of single-row products with a shared B and padded output rows, with
    and without the fused Add / activation, full-range operands (sums wrap):
    each written row equals the oracle's MatMul followed by the unfused VectorOP
    calls, and the padding between rows keeps its contents."""
    batch, k, m, a_bs, c_bs, mode, act = case
    say(f"matmul single-row batches {case}")
    g = wl.rng(904, *case[:5])
    a = full_range(g, (batch - 1) * a_bs + k)
    b = full_range(g, k * m)
    c_len = (batch - 1) * c_bs + m
    add = None if mode is None else full_range(g, m if mode == "column" else c_len)
    fill = np.full(c_len, 0x5A5A, np.int16)
    c = dev(fill)
    K.MatmulKernel(dev(a), dev(b), c, 1, k, m, batch, a_bs, 0, c_bs,
                   add=None if add is None else dev(add), add_column=mode == "column", act=act)
    y = fill.copy()
    oracle.set_threads(oracle_threads())
    oracle.matmul(a, b, y, 1, k, m, batch, a_bs, 0, c_bs, threads=True)
    want = y.copy()
    for r in range(batch):
        row = y[r * c_bs: r * c_bs + m].copy()
        radd = None if add is None else (add if mode == "column" else add[r * c_bs: r * c_bs + m])
        want[r * c_bs: r * c_bs + m] = apply_epilogue(row, radd, False, act, 1, m)
    np.testing.assert_array_equal(host(c), want)
