"""Pins the CPU oracle (oracle/cm_oracle.c) before it is trusted as the parity reference.

Checks, per kernel:
  * the reference's own known-answer tables (copied as data into refcases.py);
  * agreement with the independent float64 numpy model of the scheduler
    (oracle/numpy_sim.py) wherever the two reference oracles agree;
  * closed forms the mathematics fixes (floor vs trunc directions, exact
    rational AVG, integer square root for LP p=2, modular wrap of big sums
    computed with Python integers on tiny inputs).
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from oracle import numpy_sim as ns
from cormorant_amd import workloads as wl
from tests import refcases as rc


def q(v: float) -> int:
    """Data_t(double) for on-grid values (the table entries are all on-grid)."""
    r = math.floor(v * 256.0)
    assert r == v * 256.0
    return int(r)


# ------------------------------------------------------------------ VectorOP --

@pytest.mark.parametrize("row", rc.VECOP_SAT_TABLE, ids=[r[3] for r in rc.VECOP_SAT_TABLE])
def test_vectorop_saturation_table(row):
    op, av, bv, _ = row
    n = 8                                   # TestSimulation.cpp:129 kSize = 8
    a = np.full(n, q(av), np.int16)
    b = np.full(n, q(bv), np.int16)
    c = np.zeros(n, np.int16)
    oracle.vectorop(a, b, c, n, op)
    want = rc.vecop_table_expected(op, av, bv)
    assert np.all(c.astype(np.float64) / 256.0 == want)


@pytest.mark.parametrize("op", range(6))
@pytest.mark.parametrize("size", rc.VECOP_RANDOM_SIZES)
def test_vectorop_random_vs_numpy_sim(op, size):
    lo, hi = rc.VECOP_RANDOM_RANGES[op]
    g = wl.rng(900, op, size)
    a = wl.quantize_trn(g.uniform(lo, hi, size))
    b = wl.quantize_trn(g.uniform(*((1.0, 10.0) if op == rc.DIV else (lo, hi)), size))
    c = np.zeros(size, np.int16)
    oracle.vectorop(a, b, c, size, op)
    want = ns.to_raw(ns.elementwise(op, ns.to_float(a), ns.to_float(b)))
    np.testing.assert_array_equal(c, want)
    # the reference's own double-precision check: within 1 LSB (TestSimulation.cpp:89)
    ref = np.array([rc.vecop_table_expected(op, x / 256.0, y / 256.0) for x, y in zip(a, b)])
    assert np.all(np.abs(c / 256.0 - ref) <= 1.0 / 256.0)


def test_vectorop_broadcast_cases():
    # TestSimulation.cpp:274-339
    a = np.array([q(v) for v in (1, 2, 3, 4, 5, 6, 7, 8)], np.int16)
    b = np.array([q(1)] * 4, np.int16)
    c = np.zeros(8, np.int16)
    oracle.vectorop(a, b, c, 4, rc.ADD, outer=2, a_inc=4, b_inc=0)
    np.testing.assert_array_equal(c, [q(v) for v in (2, 3, 4, 5, 6, 7, 8, 9)])
    a = np.array([q(2)] * 4, np.int16)
    b = np.array([q(i + 1) for i in range(12)], np.int16)
    c = np.zeros(12, np.int16)
    oracle.vectorop(a, b, c, 4, rc.MUL, outer=3, a_inc=0, b_inc=4)
    np.testing.assert_array_equal(c, [q(2 * (i + 1)) for i in range(12)])


def test_vectorop_rounding_directions():
    # MUL floors (AP_TRN): -1 LSB * +1 LSB = -2^-16 -> -1 LSB, not 0.
    assert oracle.q88_mul(-1, 1) == -1
    assert oracle.q88_mul(1, 1) == 0
    # DIV truncates toward zero: (-1/256) / (3/256) = -1/3 -> -85 LSB, not -86.
    assert oracle.q88_div(-1, 3) == -85
    assert oracle.q88_div(1, 3) == 85
    assert oracle.q88_div(123, 0) == 0          # VectorOP.cpp:22-23
    assert oracle.q88_div(-32768, -1) == 32767  # saturates
    assert oracle.q88_div(-32768, 1) == -32768


def test_div_against_exact_rationals_sampled():
    """DIV for every a against a sample of b (all edge b and every 61st b),
    compared with numpy's float64 trunc model and with exact integer math."""
    a = np.arange(-32768, 32768, dtype=np.int64)
    bs = sorted(set(list(range(-40, 41)) + list(range(-32768, 32768, 61)) + [32767, -32768]))
    for bv in bs:
        got = np.array([0], np.int16)
        aa = a.astype(np.int16)
        bb = np.full(a.size, bv, np.int16)
        c = np.zeros(a.size, np.int16)
        oracle.vectorop(aa, bb, c, a.size, rc.DIV)
        if bv == 0:
            assert not c.any()
            continue
        num = a * 256
        exact = np.abs(num) // abs(bv) * np.sign(num) * np.sign(bv)   # trunc toward zero
        np.testing.assert_array_equal(c, np.clip(exact, -32768, 32767))
        sim = ns.to_raw(ns.elementwise(rc.DIV, ns.to_float(aa), ns.to_float(bb)))
        np.testing.assert_array_equal(c, sim)
        del got


def test_vectorop_ramp_kats():
    """test_saturation.py closed-form ramp models: X[i] = i/256, i < 256."""
    x = np.arange(256, dtype=np.int16)

    def run(op, a, bval):
        b = np.full(256, q(bval), np.int16)
        c = np.zeros(256, np.int16)
        oracle.vectorop(a, b, c, 256, op)
        return c

    y = run(rc.ADD, x, 127.5)                         # TestSatAddPos
    assert y[0] == q(127.5) and y[127] == 32767 and y[128] == 32767
    assert int(np.sum(y == 32767)) == 129
    y = run(rc.ADD, run(rc.ADD, x, -63.0), -65.5)     # TestSatAddNeg
    assert int(np.sum(y == -32768)) == 129 and y[129] == q(129 / 256 - 128.5)
    y = run(rc.MUL, run(rc.ADD, x, 1.0), 90.0)        # TestSatMulPos
    assert y[0] == q(90.0) and y[108] == q(127.96875) and int(np.sum(y == 32767)) == 147
    y = run(rc.MUL, run(rc.SUB, x, 2.0), 90.0)        # TestSatMulNeg
    assert y[148] == q(-127.96875) and int(np.sum(y == -32768)) == 148
    y = run(rc.SUB, x, -127.5)                        # TestSatSubPos
    assert int(np.sum(y == 32767)) == 129
    y = run(rc.SUB, run(rc.SUB, x, 63.0), 65.5)       # TestSatSubNeg
    assert int(np.sum(y == -32768)) == 129
    y = run(rc.DIV, x, 1 / 256)                       # TestSatDivPos
    assert y[127] == q(127.0) and int(np.sum(y == 32767)) == 128
    y = run(rc.DIV, x, -1 / 256)                      # TestSatDivNeg
    assert y[127] == q(-127.0) and y[128] == -32768 and int(np.sum(y == -32768)) == 128


def test_vectorop_overlapping_outer_keeps_last_step():
    # c_inc = a_inc + b_inc = 2 < size = 4: outer steps overwrite each other.
    a = np.arange(1, 11, dtype=np.int16) * 256
    b = np.zeros(10, np.int16)
    c = np.full(12, 7, np.int16)
    oracle.vectorop(a, b, c, 4, rc.ADD, outer=3, a_inc=2, b_inc=0)
    want = np.full(12, 7, np.int16)
    for o in range(3):
        want[2 * o:2 * o + 4] = a[2 * o:2 * o + 4]
    np.testing.assert_array_equal(c, want)


# ------------------------------------------------------------------- MatMul --

@pytest.mark.parametrize("shape", rc.MATMUL_2D, ids=[s[0] for s in rc.MATMUL_2D])
def test_matmul_reference_shapes_vs_numpy_sim(shape):
    _, n, k, m = shape
    g = wl.rng(901, n, k, m)
    a = wl.uniform_q88(g, (n, k), -1.0, 1.0)
    b = wl.uniform_q88(g, (k, m), -1.0, 1.0)
    c = np.zeros((n, m), np.int16)
    oracle.matmul(a, b, c, n, k, m)
    np.testing.assert_array_equal(c, ns.to_raw(ns.matmul(ns.to_float(a), ns.to_float(b))))
    c2 = np.zeros((n, m), np.int16)
    oracle.matmul(a, b, c2, n, k, m, threads=True)
    np.testing.assert_array_equal(c, c2)


@pytest.mark.parametrize("case", rc.MATMUL_BATCH, ids=[s[0] for s in rc.MATMUL_BATCH])
def test_matmul_batch_strides(case):
    _, n, k, m, batch, a_bs, b_bs = case
    g = wl.rng(902, batch, a_bs, b_bs)
    a = wl.uniform_q88(g, max(a_bs * (batch - 1) + n * k, n * k), -1.0, 1.0)
    b = wl.uniform_q88(g, max(b_bs * (batch - 1) + k * m, k * m), -1.0, 1.0)
    c = np.zeros(batch * n * m, np.int16)
    oracle.matmul(a, b, c, n, k, m, batch, a_bs, b_bs, n * m)
    for bi in range(batch):
        A = ns.to_float(a[bi * a_bs: bi * a_bs + n * k].reshape(n, k))
        B = ns.to_float(b[bi * b_bs: bi * b_bs + k * m].reshape(k, m))
        np.testing.assert_array_equal(c[bi * n * m:(bi + 1) * n * m].reshape(n, m),
                                      ns.to_raw(ns.matmul(A, B)))


@pytest.mark.parametrize("case", rc.MATMUL_SAT, ids=[s[0] for s in rc.MATMUL_SAT])
def test_matmul_saturation_kats(case):
    _, av, bv, k, want = case
    n, m = rc.TN + 1, rc.TM + 1
    a = np.full((n, k), q(av), np.int16)
    b = np.full((k, m), q(bv), np.int16)
    c = np.zeros((n, m), np.int16)
    oracle.matmul(a, b, c, n, k, m)
    assert np.all(c / 256.0 == want)


def test_matmul_accumulator_wraps_mod_2_32():
    """Sum of products beyond 2^31 (raw) must wrap like ap_fixed<32,16> AP_WRAP."""
    g = wl.rng(903)
    n, k, m = 3, 300, 5
    a = g.integers(-32768, 32768, size=(n, k)).astype(np.int16)
    b = g.integers(-32768, 32768, size=(k, m)).astype(np.int16)
    a[0, :] = 32767
    b[:, 0] = 32767                       # row 0 x col 0 = 300 * 32767^2 >> 2^31
    c = np.zeros((n, m), np.int16)
    oracle.matmul(a, b, c, n, k, m)
    for i in range(n):
        for j in range(m):
            s = sum(int(a[i, t]) * int(b[t, j]) for t in range(k))
            w = ((s + 2**31) % 2**32) - 2**31      # two's complement 32-bit
            assert c[i, j] == max(-32768, min(32767, w >> 8)), (i, j)


@pytest.mark.parametrize("n,k,m,batch,c_bs", [(4, 32, 8, 5, 8), (16, 300, 40, 3, 1),
                                               (2, 64, 130, 4, 129), (8, 16, 8, 4, 0)])
def test_matmul_overlapping_outputs_sequential(n, k, m, batch, c_bs):
    """Batches whose outputs overlap: each shared element holds the last writing
    batch's value (MatmulKernel.cpp:108-111 runs batches in order), one thread and
    OpenMP alike; checked against per-batch products written in order."""
    g = wl.rng(907, n, c_bs)
    a = g.integers(-32768, 32768, batch * n * k, dtype=np.int16)
    b = g.integers(-32768, 32768, batch * k * m, dtype=np.int16)
    size = (batch - 1) * c_bs + n * m
    want = np.full(size, 77, np.int16)
    for bi in range(batch):
        A = a[bi * n * k:(bi + 1) * n * k].reshape(n, k)
        B = b[bi * k * m:(bi + 1) * k * m].reshape(k, m)
        want[bi * c_bs: bi * c_bs + n * m] = _closed_form_matmul(A, B).reshape(-1)
    for threads in (False, True):
        c = np.full(size, 77, np.int16)
        oracle.matmul(a, b, c, n, k, m, batch, n * k, k * m, c_bs, threads=threads)
        np.testing.assert_array_equal(c, want)


def _closed_form_matmul(a, b):
    """sat16(wrap32(sum a*b) >> 8) with Python integers (no fixed-width arithmetic)."""
    s = a.astype(object) @ b.astype(object)
    w = (s + 2**31) % 2**32 - 2**31
    return np.vectorize(lambda v: max(-32768, min(32767, v >> 8)), otypes=[np.int64])(w)


@pytest.mark.parametrize("shape", [(1, 1, 1), (3, 300, 5), (7, 257, 33), (4, 2049, 17)])
def test_matmul_row_closed_form(shape):
    """The naive row loop (TestMatmulSim.cpp:65-82 order) against Python big integers
    on full-range operands whose sums wrap, row by row."""
    n, k, m = shape
    g = wl.rng(905, n, k, m)
    a = g.integers(-32768, 32768, size=(n, k)).astype(np.int16)
    b = g.integers(-32768, 32768, size=(k, m)).astype(np.int16)
    a[0, :] = -32768
    b[:, 0] = -32768                     # row 0 x col 0 = k * 2^30: wraps for k >= 2
    want = _closed_form_matmul(a, b)
    for r in range(n):
        np.testing.assert_array_equal(oracle.matmul_row(a[r], b, k, m), want[r], err_msg=f"row {r}")


@pytest.mark.parametrize("shape", [(5, 17, 3), (64, 784, 256), (33, 4096, 70), (9, 300, 1000)])
def test_matmul_tiled_equals_naive_rows(shape):
    """The reference's own invariant (TestMatmulSim.cpp:111-122): the tiled kernel
    equals the naive product exactly; here ora_matmul (tile loops of the HLS kernel,
    one thread and OpenMP) against ora_matmul_row on every row, full-range values."""
    n, k, m = shape
    g = wl.rng(906, n, k, m)
    a = g.integers(-32768, 32768, size=(n, k)).astype(np.int16)
    b = g.integers(-32768, 32768, size=(k, m)).astype(np.int16)
    c1 = np.zeros((n, m), np.int16)
    c2 = np.zeros((n, m), np.int16)
    oracle.matmul(a, b, c1, n, k, m)
    oracle.matmul(a, b, c2, n, k, m, threads=True)
    rows = np.stack([oracle.matmul_row(a[r], b, k, m) for r in range(n)])
    np.testing.assert_array_equal(c1, rows)
    np.testing.assert_array_equal(c2, rows)


# --------------------------------------------------------------------- Conv --

def _conv_case(geom, seed):
    (_, N, C, H, W, M, kh, kw, sh, sw, dh, dw, pt, pl, pb, pr, bias, dwise, xs, ws, bs) = geom
    g = wl.rng(904, seed)
    x = wl.uniform_q88(g, (N, C, H, W), -xs, xs)
    w = wl.uniform_q88(g, (M, 1 if dwise else C, kh, kw), -ws, ws)
    b = wl.uniform_q88(g, (M,), -bs, bs)
    oh = rc.conv_out_size(H, kh, sh, dh, pt, pb)
    ow = rc.conv_out_size(W, kw, sw, dw, pl, pr)
    return x, w, b, oh, ow


@pytest.mark.parametrize("i", range(len(rc.CONV_GEOMS)), ids=[g[0] for g in rc.CONV_GEOMS])
def test_conv_reference_geometries_vs_numpy_sim(i):
    geom = rc.CONV_GEOMS[i]
    (_, N, C, H, W, M, kh, kw, sh, sw, dh, dw, pt, pl, pb, pr, bias, dwise, *_s) = geom
    x, w, b, oh, ow = _conv_case(geom, i)
    y = np.zeros((N, M, oh, ow), np.int16)
    oracle.conv(x, w, b, y, N, C, H, W, M, oh, ow, kh, kw, sh, sw, dh, dw, pt, pl, bias, dwise)
    want = ns.to_raw(ns.conv2d(ns.to_float(x), ns.to_float(w), ns.to_float(b) if bias else None,
                               sh, sw, pt, pl, dh, dw, oh, ow, is_depthwise=bool(dwise)))
    np.testing.assert_array_equal(y, want)
    y2 = np.zeros_like(y)
    oracle.conv(x, w, b, y2, N, C, H, W, M, oh, ow, kh, kw, sh, sw, dh, dw, pt, pl, bias, dwise,
                threads=True)
    np.testing.assert_array_equal(y, y2)


def _closed_form_conv(x, w, bias, oh_n, ow_n, sh, sw, dh, dw, pt, pl, has_bias, dwise):
    """sat16(wrap32((has_bias ? bias << 8 : 0) + sum of in-bounds x*w) >> 8) with Python
    integers, straight from the definition (ConvKernel.cpp:160-169, 235-237, 308-310, 333):
    ih = oh*sh + i*dh - pt, iw = ow*sw + j*dw - pl; bottom/right padding is what the
    output size leaves past the input."""
    N, C, H, W = x.shape
    M, _, KH, KW = w.shape
    out = np.zeros((N, M, oh_n, ow_n), np.int64)
    wrapped = 0
    for n in range(N):
        for m in range(M):
            chans = [m] if dwise else range(C)
            for oh in range(oh_n):
                for ow in range(ow_n):
                    s = (int(bias[m]) << 8) if has_bias else 0
                    for c in chans:
                        wc = 0 if dwise else c
                        for i in range(KH):
                            ih = oh * sh + i * dh - pt
                            if not 0 <= ih < H:
                                continue
                            for j in range(KW):
                                iw = ow * sw + j * dw - pl
                                if 0 <= iw < W:
                                    s += int(x[n, c, ih, iw]) * int(w[m, wc, i, j])
                    wrapped += not -2**31 <= s < 2**31
                    s = (s + 2**31) % 2**32 - 2**31
                    out[n, m, oh, ow] = max(-32768, min(32767, s >> 8))
    return out, wrapped


# N, C, H, W, M, kh, kw, sh, sw, dh, dw, pad top, left, bottom, right, bias, depthwise
CONV_WRAP_GEOMS = [
    (2, 5, 7, 6, 3, 3, 2, 2, 1, 1, 2, 2, 1, 0, 2, 1, 0),     # asymmetric pads, mixed stride/dilation
    (1, 3, 6, 9, 4, 3, 3, 1, 2, 2, 1, 1, 0, 2, 1, 1, 0),
    (2, 4, 5, 5, 4, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1),     # depthwise, bias
    (1, 6, 8, 7, 4, 2, 3, 2, 1, 1, 2, 0, 2, 1, 0, 1, 1),     # depthwise, out_ch < in_ch
    (1, 9, 4, 4, 2, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 1, 0),     # 1x1
    (1, 2, 3, 3, 2, 5, 5, 1, 1, 1, 1, 2, 2, 2, 2, 0, 0),     # window wider than the input
]


@pytest.mark.parametrize("geom", CONV_WRAP_GEOMS, ids=[str(g) for g in CONV_WRAP_GEOMS])
def test_conv_closed_form_full_range(geom):
    """ora_conv (one thread and OpenMP) against Python big integers on tiny full-range
    shapes: standard and depthwise, bias, asymmetric padding, stride and dilation.  A
    planted block of -32768 inputs and weights makes sums of k * 2^30 that wrap."""
    N, C, H, W, M, kh, kw, sh, sw, dh, dw, pt, pl, pb, pr, hb, dwise = geom
    g = wl.rng(912, *geom)
    x = g.integers(-32768, 32768, size=(N, C, H, W)).astype(np.int16)
    w = g.integers(-32768, 32768, size=(M, 1 if dwise else C, kh, kw)).astype(np.int16)
    b = g.integers(-32768, 32768, size=(M,)).astype(np.int16)
    x[0, :, : min(H, 3), : min(W, 3)] = -32768
    w[0] = -32768
    oh = rc.conv_out_size(H, kh, sh, dh, pt, pb)
    ow = rc.conv_out_size(W, kw, sw, dw, pl, pr)
    want, wrapped = _closed_form_conv(x, w, b, oh, ow, sh, sw, dh, dw, pt, pl, hb, dwise)
    assert wrapped > 0      # some accumulators left the int32 range: the wrap is exercised
    for threads in (False, True):
        y = np.full((N, M, oh, ow), 55, np.int16)
        oracle.conv(x, w, b, y, N, C, H, W, M, oh, ow, kh, kw, sh, sw, dh, dw, pt, pl, hb, dwise,
                    threads=threads)
        np.testing.assert_array_equal(y, want)


def test_conv_bias_wraps_with_sum():
    """A bias whose <<8 joins a sum near 2^31 wraps with it: 1 input channel, 1x1,
    x = w = -32768 gives 2^30 per product; two channels give 2^31, which wraps to
    -2^31, and bias 0x7FFF << 8 moves it back up (ConvKernel.cpp:160-169, 333)."""
    x = np.full((1, 2, 1, 1), -32768, np.int16)
    w = np.full((1, 2, 1, 1), -32768, np.int16)
    for bias, hb in ((0, 0), (32767, 1), (-32768, 1), (-1, 1)):
        y = np.zeros((1, 1, 1, 1), np.int16)
        b = np.array([bias], np.int16)
        oracle.conv(x, w, b, y, 1, 2, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 0, 0, hb, 0)
        s = 2 * 2**30 + ((bias << 8) if hb else 0)
        s = (s + 2**31) % 2**32 - 2**31
        assert int(y[0, 0, 0, 0]) == max(-32768, min(32767, s >> 8)), bias


@pytest.mark.parametrize("case", rc.CONV_SAT, ids=[c[0] for c in rc.CONV_SAT])
def test_conv_saturation_kats(case):
    _, wv, bv, want = case
    x = np.full((1, 1, 3, 3), q(rc.SAT_MAX), np.int16)
    w = np.full((1, 1, 1, 1), q(wv), np.int16)
    b = np.full((1,), q(bv), np.int16)
    y = np.zeros((1, 1, 3, 3), np.int16)
    oracle.conv(x, w, b, y, 1, 1, 3, 3, 1, 3, 3, 1, 1, 1, 1, 1, 1, 0, 0, 1, 0)
    assert np.all(y / 256.0 == want)


# --------------------------------------------------------------------- Pool --

@pytest.mark.parametrize("case", rc.POOL_TESTS, ids=[c[0] for c in rc.POOL_TESTS])
def test_pool_reference_cases(case):
    (_, N, C, H, W, OH, OW, ph, pw, sh, sw, pt, pl, dh, dw, pt_, lp, cip) = case
    x = rc.pool_test_fill(N * C * H * W)
    y = np.zeros(N * C * OH * OW, np.int16)
    oracle.pool(x, y, N, C, H, W, OH, OW, ph, pw, sh, sw, pt, pl, dh, dw, pt_, lp, cip)
    # the reference's own check: float reference within 0.02 (TestPoolingSim.cpp:22)
    for n in range(N):
        for c in range(C):
            for oh in range(OH):
                for ow in range(OW):
                    r = rc.pool_ref_elem(x, C, H, W, n, c, oh, ow, ph, pw, sh, sw, pt, pl, dh, dw,
                                         pt_, lp, cip)
                    got = y[((n * C + c) * OH + oh) * OW + ow] / 256.0
                    assert abs(r - got) <= rc.POOL_TOL
    # bit-exact against the scheduler's numpy model (no wrap, LP2 outputs < 16 here)
    want = ns.to_raw(ns.pool2d(ns.to_float(x).reshape(N, C, H, W), ph, pw, sh, sw, pt, pl, dh, dw,
                               OH, OW, pt_, lp, cip))
    np.testing.assert_array_equal(y.reshape(N, C, OH, OW), want)


AVG_DENOMS = [1, 2, 3, 4, 6, 8, 9, 25, 49, 196, 784, 3136]


@pytest.mark.parametrize("d", AVG_DENOMS)
def test_avg_finalizer_is_floor_division_exhaustive(d):
    """AVG's float32 path (PoolingKernel.cpp:137, 259) equals floor(S / d) for every
    accumulator state: acc = v << 8 for v in [0, 2^24) covers all of them, and
    (int32)acc / 65536 = S / 256 with S the 24-bit sign extension of v."""
    v = np.arange(1 << 24, dtype=np.int64)
    s = np.where(v >= (1 << 23), v - (1 << 24), v)
    want = np.clip(np.floor_divide(s, d), -32768, 32767)
    assert oracle.avg_checksum(0, 1 << 24, d) == oracle.checksum_of(want, v)
    for sv in (-(1 << 23), -1, 0, 1, (1 << 23) - 1, 12345, -12345):   # spot values
        assert oracle.avg_finalize((sv & 0xFFFFFF) << 8, d) == max(-32768, min(32767, sv // d))


def test_lp2_finalizer_is_integer_sqrt_below_2_24():
    """For A < 2^24, floor(sqrtf(A/65536) * 256) == isqrt(A) exactly (all A)."""
    a = np.arange(1 << 24, dtype=np.int64)
    isq = np.floor(np.sqrt(a.astype(np.float64))).astype(np.int64)
    isq -= (isq * isq > a)                      # guard the float64 root
    isq += ((isq + 1) * (isq + 1) <= a)
    assert oracle.lp2_checksum(0, 1 << 24) == oracle.checksum_of(isq, a)


def test_lp2_finalizer_float32_path_above_2_24():
    """Above 2^24 the C-simulation path rounds A to float32 first: emulate it in
    numpy float32 (independent implementation of the same IEEE operations)."""
    g = wl.rng(905)
    a = np.unique(np.concatenate([g.integers(1 << 24, 1 << 31, size=200000),
                                  np.arange((1 << 24), (1 << 24) + 20000),
                                  np.arange((1 << 31) - 20000, 1 << 31)])).astype(np.int64)
    f = np.sqrt(a.astype(np.float32) * np.float32(1.0 / 65536.0))   # float32 RN ops
    want = np.clip(np.floor(f.astype(np.float64) * 256.0), -32768, 32767).astype(np.int64)
    f_lp2 = oracle.lib().ora_lp2_finalize
    got = np.fromiter((f_lp2(int(x)) for x in a), dtype=np.int64, count=a.size)
    np.testing.assert_array_equal(got, want)
    # the first float32-vs-float64 divergence above 2^24: A = 16785407 -> 16.0039 (not 16.0)
    assert oracle.lp2_finalize(16785407) == 4097 and math.isqrt(16785407) == 4096
    assert oracle.lp2_finalize(-5) == 0         # wrapped accumulator: NaN -> 0 (unpinned)


def test_pool_wrap_and_edges():
    """MAX of an all-padded window is -32768; LP1/AVG sums wrap modulo 2^32."""
    x = np.full((1, 1, 1, 1), 100, np.int16)
    y = np.zeros(9, np.int16)
    # 3x3 window stride 1 pad 2 over a 1x1 input: corner windows see no valid pixel
    oracle.pool(x, y, 1, 1, 1, 1, 3, 3, 3, 3, 1, 1, 2, 2, 1, 1, 0, 0, 0)
    assert y[0] == 100 and y.min() == 100   # every 3x3 window overlaps the pixel
    y = np.zeros(1, np.int16)
    oracle.pool(x, y, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 5, 5, 1, 1, 0, 0, 0)
    assert y[0] == -32768                   # window entirely in padding
    # LP1 over a plane of 300 x -32768: sum |x| << 8 = 300 * 2^23 wraps mod 2^32
    x = np.full((1, 1, 1, 300), -32768, np.int16)
    y = np.zeros(1, np.int16)
    oracle.pool(x, y, 1, 1, 1, 300, 1, 1, 1, 300, 1, 1, 0, 0, 1, 1, 2, 1, 0)
    s = (300 * 32768 * 256) % 2**32
    s = s - 2**32 if s >= 2**31 else s
    assert y[0] == max(-32768, min(32767, s >> 8))


def _closed_form_lp(x, OH, OW, ph, pw, sh, sw, pt, pl, dh, dw, p):
    """LpPool from the definition with Python integers: p = 1 gives
    sat16(wrap32(sum |x| << 8) >> 8); p = 2 gives isqrt(sum x^2), exact when the sum
    of squares stays below 2^24 (PoolingKernel.cpp:222-224, 262-265)."""
    N, C, H, W = x.shape
    out = np.zeros((N, C, OH, OW), np.int64)
    for n in range(N):
        for c in range(C):
            for oh in range(OH):
                for ow in range(OW):
                    s = 0
                    for i in range(ph):
                        ih = oh * sh + i * dh - pt
                        for j in range(pw):
                            iw = ow * sw + j * dw - pl
                            if 0 <= ih < H and 0 <= iw < W:
                                v = int(x[n, c, ih, iw])
                                s += (abs(v) << 8) if p == 1 else v * v
                    if p == 1:
                        s = (s + 2**31) % 2**32 - 2**31
                        out[n, c, oh, ow] = max(-32768, min(32767, s >> 8))
                    else:
                        assert s < 1 << 24
                        out[n, c, oh, ow] = math.isqrt(s)
    return out


@pytest.mark.parametrize("pool_type", [2, 3, 7, 255])
@pytest.mark.parametrize("lp_order", [0, 1, 2, 3, 9])
def test_pool_out_of_range_codes_closed_form(pool_type, lp_order):
    """Any pool_type other than 0 (MAX) and 1 (AVG) is LpPool, and any lp_order other
    than 1 is p = 2 (PoolingKernel.cpp:214-224, 256-263): each code against the
    definition.  p = 2 on values whose window sums of squares stay below 2^24; p = 1
    on full-range values whose sums wrap."""
    N, C, H, W, ph, pw, sh, sw, pt, pl, dh, dw = 2, 3, 9, 8, 3, 2, 2, 1, 1, 0, 1, 2
    OH = (H + 2 * pt - dh * (ph - 1) - 1) // sh + 1
    OW = (W + 2 * pl - dw * (pw - 1) - 1) // sw + 1
    p = 1 if lp_order == 1 else 2
    g = wl.rng(913, pool_type, lp_order)
    if p == 1:
        x = g.integers(-32768, 32768, size=(N, C, H, W)).astype(np.int16)
    else:
        x = g.integers(-1365, 1366, size=(N, C, H, W)).astype(np.int16)   # 6 * 1365^2 < 2^24
    want = _closed_form_lp(x, OH, OW, ph, pw, sh, sw, pt, pl, dh, dw, p)
    for threads in (False, True):
        y = np.full(N * C * OH * OW, 99, np.int16)
        oracle.pool(x.reshape(-1), y, N, C, H, W, OH, OW, ph, pw, sh, sw, pt, pl, dh, dw,
                    pool_type, lp_order, 0, threads=threads)
        np.testing.assert_array_equal(y.reshape(N, C, OH, OW), want)
