"""GPU parity: PoolingKernel through the C ABI vs the CPU oracle (bit-exact)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from cormorant_amd import kernels as K
from cormorant_amd import workloads as wl
from tests import refcases as rc
from tests.gpu_util import dev, empty_dev, host, oracle_threads, say

pytestmark = pytest.mark.gpu


def pool_both(x, N, C, H, W, OH, OW, ph, pw, sh, sw, pt, pl, dh, dw, ptype, lp, cip):
    y = empty_dev(N * C * OH * OW)
    K.PoolingKernel(dev(x), y, N, C, H, W, OH, OW, ph, pw, sh, sw, pt, pl, dh, dw, ptype, lp, cip)
    want = np.zeros(N * C * OH * OW, np.int16)
    oracle.set_threads(oracle_threads())
    oracle.pool(np.ascontiguousarray(x.reshape(-1)), want, N, C, H, W, OH, OW, ph, pw, sh, sw, pt,
                pl, dh, dw, ptype, lp, cip, threads=True)
    return host(y), want


@pytest.mark.parametrize("case", rc.POOL_TESTS, ids=[c[0] for c in rc.POOL_TESTS])
def test_reference_cases(case):
    name, N, C, H, W, OH, OW, ph, pw, sh, sw, pt, pl, dh, dw, ptype, lp, cip = case
    say(f"pool reference case: {name}")
    x = rc.pool_test_fill(N * C * H * W)
    got, want = pool_both(x, N, C, H, W, OH, OW, ph, pw, sh, sw, pt, pl, dh, dw, ptype, lp, cip)
    np.testing.assert_array_equal(got, want)


EDGE_CASES = [
    # N, C, H, W, ph, pw, sh, sw, pt, pl, dh, dw  (out size computed with symmetric pads)
    (2, 3, 9, 11, 3, 3, 2, 2, 1, 1, 1, 1),
    (1, 5, 17, 13, 2, 3, 1, 2, 0, 1, 2, 1),
    (1, 2, 7, 7, 5, 5, 3, 3, 2, 2, 1, 1),
    (1, 1, 3, 3, 3, 3, 1, 1, 3, 3, 1, 1),       # windows entirely in padding at the corners
    (1, 2, 5, 20000, 3, 3, 1, 1, 1, 1, 1, 1),   # rows too wide for LDS -> direct path
    (2, 4, 56, 56, 56, 56, 1, 1, 0, 0, 1, 1),   # global (wave reduction path)
    (1, 3, 7, 9, 7, 9, 1, 1, 0, 0, 1, 1),       # global, plane not a multiple of 8
    (3, 2, 33, 31, 4, 4, 4, 4, 0, 0, 1, 1),
    # widths a multiple of 8 with 2x2 / 3x3 windows and row stride 1 or 2: the
    # one-strip-per-thread path (pair reads at even / odd offsets, several bands
    # per plane, a 255-wide output, and more items than twice the grid)
    (2, 3, 16, 16, 3, 3, 2, 2, 1, 1, 1, 1),
    (1, 4, 24, 32, 2, 2, 2, 2, 0, 0, 1, 1),
    (1, 3, 40, 128, 3, 3, 1, 1, 1, 1, 1, 1),
    (2, 2, 21, 64, 2, 2, 1, 2, 0, 1, 1, 1),
    (1, 2, 9, 512, 3, 3, 2, 2, 0, 0, 1, 1),
    (1, 1, 8, 8, 3, 3, 1, 1, 1, 1, 1, 1),
    (1, 2, 12, 16, 3, 3, 2, 3, 1, 1, 1, 1),
    (32, 128, 8, 16, 2, 2, 2, 2, 0, 0, 1, 1),
    (16, 512, 8, 8, 3, 3, 1, 1, 1, 1, 1, 1),
]


@pytest.mark.parametrize("ptype,lp,cip", [(0, 0, 0), (1, 0, 0), (1, 0, 1), (2, 1, 0), (2, 2, 0)])
@pytest.mark.parametrize("geom", EDGE_CASES, ids=[str(g) for g in EDGE_CASES])
def test_geometries_full_range_values(ptype, lp, cip, geom):
    N, C, H, W, ph, pw, sh, sw, pt, pl, dh, dw = geom
    OH = (H + 2 * pt - dh * (ph - 1) - 1) // sh + 1
    OW = (W + 2 * pl - dw * (pw - 1) - 1) // sw + 1
    say(f"pool geometry {geom} type={ptype} lp={lp} cip={cip}")
    g = wl.rng(810, ptype, lp, cip, *geom)
    x = g.integers(-32768, 32768, N * C * H * W, dtype=np.int16)   # full range: sums wrap
    got, want = pool_both(x, N, C, H, W, OH, OW, ph, pw, sh, sw, pt, pl, dh, dw, ptype, lp, cip)
    np.testing.assert_array_equal(got, want)


def test_lp2_finalizer_all_accumulators():
    """LP p=2 finaliser (float32 convert + sqrt) for every A in [0, 2^31): checksums
    of GPU and host float32 paths agree, chunk by chunk."""
    oracle.set_threads(oracle_threads())
    step = 1 << 27
    for lo in range(0, 1 << 31, step):
        say(f"lp2 sweep chunk {lo >> 27}")
        assert K.selftest_finalize(0, lo, step) == oracle.lp2_checksum(lo, lo + step), lo
    # negative (wrapped) accumulators map to 0 on both sides
    assert K.selftest_finalize(0, 0x80000000, 1 << 20) == oracle.lp2_checksum(0x80000000, 0x80100000)


@pytest.mark.parametrize("d", [0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 12, 16, 25, 49, 196, 784, 3136, 50176])
def test_avg_finalizer_all_accumulators(d):
    """AVG finaliser for every accumulator state (v << 8, v < 2^24) and denominator d."""
    say(f"avg sweep d={d}")
    oracle.set_threads(oracle_threads())
    assert K.selftest_finalize(1, 0, 1 << 24, d) == oracle.avg_checksum(0, 1 << 24, d)


@pytest.mark.parametrize("seed", range(16))
def test_strip_path_random(seed):
    """Random shapes on the one-strip-per-thread path (2x2 / 3x3 window, row
    stride 1 or 2, rows a multiple of 8 elements, output width <= 256): every
    pool type, padding, column stride and count_include_pad, full-range values."""
    g = wl.rng(811, seed)
    k = int(g.choice([2, 3]))
    sh, sw = int(g.choice([1, 2])), int(g.choice([1, 2, 3]))
    pt, pl = int(g.integers(0, k)), int(g.integers(0, k))
    H, W = int(g.integers(k, 40)), 8 * int(g.integers(1, 24))
    N, C = int(g.integers(1, 4)), int(g.integers(1, 40))
    ptype, lp = [(0, 0), (1, 0), (2, 1), (2, 2)][int(g.integers(0, 4))]
    cip = int(g.integers(0, 2)) if ptype == 1 else 0
    OH = (H + 2 * pt - k) // sh + 1
    OW = (W + 2 * pl - k) // sw + 1
    say(f"pool strip random seed {seed}: {(N, C, H, W, k, sh, sw, pt, pl, ptype, lp, cip)}")
    x = g.integers(-32768, 32768, N * C * H * W, dtype=np.int16)
    got, want = pool_both(x, N, C, H, W, OH, OW, k, k, sh, sw, pt, pl, 1, 1, ptype, lp, cip)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("seed", range(24))
def test_plane_path_random(seed):
    """Random shapes on the wave-per-plane path (planes of at most 2048 elements):
    2x2 / 3x3 windows (interior rectangle + border ring) and other windows,
    independent row / column strides and pads (some windows wholly in padding),
    plane sizes that are and are not multiples of 8, plane counts not a multiple
    of 4, every pool type, full-range values."""
    g = wl.rng(812, seed)
    k = int(g.choice([2, 3, 3, 4]))
    kw = k if g.integers(0, 4) else int(g.choice([1, 2, 3]))
    sh, sw = int(g.integers(1, 4)), int(g.integers(1, 4))
    pt, pl = int(g.integers(0, k + 1)), int(g.integers(0, kw + 1))
    H = int(g.integers(1, 45))
    W = int(g.integers(1, max(2, min(64, 2048 // H))))
    H, W = max(H, k - 2 * pt, 1), max(W, kw - 2 * pl, 1)
    N, C = int(g.integers(1, 4)), int(g.integers(1, 23))
    ptype, lp = [(0, 0), (1, 0), (2, 1), (2, 2)][int(g.integers(0, 4))]
    cip = int(g.integers(0, 2)) if ptype == 1 else 0
    OH = (H + 2 * pt - k) // sh + 1
    OW = (W + 2 * pl - kw) // sw + 1
    say(f"pool plane random seed {seed}: {(N, C, H, W, k, kw, sh, sw, pt, pl, ptype, lp, cip)}")
    assert H * W <= 2048 and OH >= 1 and OW >= 1
    x = g.integers(-32768, 32768, N * C * H * W, dtype=np.int16)
    got, want = pool_both(x, N, C, H, W, OH, OW, k, kw, sh, sw, pt, pl, 1, 1, ptype, lp, cip)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("ptype,lp", [(3, 0), (3, 1), (7, 3), (7, 1), (2, 0), (2, 3)])
@pytest.mark.parametrize("geom", EDGE_CASES, ids=[str(g) for g in EDGE_CASES])
def test_out_of_range_type_and_order_codes(ptype, lp, geom):
    """pool_type outside {0, 1} selects LpPool and lp_order other than 1 selects p = 2
    (PoolingKernel.cpp:214-224, 256-263), on every kernel path (strip, band, plane,
    global, direct), full-range values."""
    N, C, H, W, ph, pw, sh, sw, pt, pl, dh, dw = geom
    OH = (H + 2 * pt - dh * (ph - 1) - 1) // sh + 1
    OW = (W + 2 * pl - dw * (pw - 1) - 1) // sw + 1
    say(f"pool geometry {geom} out-of-range codes type={ptype} lp={lp}")
    g = wl.rng(812, ptype, lp, *geom)
    x = g.integers(-32768, 32768, N * C * H * W, dtype=np.int16)
    got, want = pool_both(x, N, C, H, W, OH, OW, ph, pw, sh, sw, pt, pl, dh, dw, ptype, lp, 0)
    np.testing.assert_array_equal(got, want)


GLOBAL_PLANES = [(8, 64), (8, 65), (28, 28), (10, 160), (60, 80), (56, 56), (7, 9), (1, 3)]


@pytest.mark.parametrize("ptype,lp", [(0, 0), (1, 0), (2, 1), (2, 2)])
@pytest.mark.parametrize("hw", GLOBAL_PLANES, ids=[f"{h}x{w}" for h, w in GLOBAL_PLANES])
def test_global_pool_load_counts(ptype, lp, hw):
    """Global pools on planes whose 16-byte vectors take 1, 2, 4 or 8 loads per lane
    (one and two passes of the 8-load loop), and on planes that are no whole number
    of vectors (the element path), every reduction kind, full-range values (sums
    that wrap, negative maxima against the zero reads past a plane)."""
    H, W = hw
    N, C = 3, 5
    say(f"global pool {H}x{W} type={ptype} lp={lp}")
    g = wl.rng(813, ptype, lp, H, W)
    x = g.integers(-32768, 32768, N * C * H * W, dtype=np.int16)
    x[: H * W] = -(np.arange(H * W) % 7000) - 100          # an all-negative plane
    got, want = pool_both(x, N, C, H, W, 1, 1, H, W, 1, 1, 0, 0, 1, 1, ptype, lp, 1)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("seed", range(32))
def test_colpair_path_random(seed):
    """Random shapes on the sixteen-lanes-per-plane path (2x2 / 3x3 window, stride 2
    both ways, top / left padding 0 or 1, even rows of at most 32 elements, at most
    16 x 16 outputs): plane counts that are not a multiple of 16, some output
    sizes past the natural ones (windows wholly in the bottom / right padding),
    every pool type and count_include_pad, full-range values."""
    g = wl.rng(813, seed)
    k = int(g.choice([2, 3]))
    p = int(g.integers(0, 2))
    W = 2 * int(g.integers(1, 17))
    H = int(g.integers(1, 36))
    OH = min((H + 2 * p - k) // 2 + 1 if H + 2 * p >= k else 1, 16)
    OW = min((W + 2 * p - k) // 2 + 1 if W + 2 * p >= k else 1, 16)
    if g.integers(0, 3) == 0:   # outputs past the natural size: windows in the padding
        OH, OW = min(OH + int(g.integers(0, 3)), 16), min(OW + int(g.integers(0, 3)), 16)
    OH, OW = max(OH, 1), max(OW, 1)
    N, C = int(g.integers(1, 5)), int(g.integers(1, 40))
    ptype, lp = [(0, 0), (1, 0), (2, 1), (2, 2), (3, 0), (2, 0)][int(g.integers(0, 6))]
    cip = int(g.integers(0, 2)) if ptype == 1 else 0
    say(f"pool colpair random seed {seed}: {(N, C, H, W, OH, OW, k, p, ptype, lp, cip)}")
    x = g.integers(-32768, 32768, N * C * H * W, dtype=np.int16)
    got, want = pool_both(x, N, C, H, W, OH, OW, k, k, 2, 2, p, p, 1, 1, ptype, lp, cip)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("ptype,lp,cip", [(0, 0, 0), (1, 0, 1), (1, 0, 0), (2, 2, 0), (2, 1, 0)])
@pytest.mark.parametrize("k,p", [(3, 0), (3, 1), (2, 0), (2, 1)])
def test_colpair_path_conv_b_size(ptype, lp, cip, k, p):
    """The conv + pool block's 28x28 pools at full size ([32, 128, 28, 28], 4096
    planes) on the sixteen-lanes-per-plane path, full-range values."""
    N, C, H = 32, 128, 28
    OH = (H + 2 * p - k) // 2 + 1
    say(f"pool colpair 28x28 k={k} p={p} type={ptype} lp={lp} cip={cip}")
    x = wl.rng(814, k, p, ptype, lp, cip).integers(-32768, 32768, N * C * H * H, dtype=np.int16)
    got, want = pool_both(x, N, C, H, H, OH, OH, k, k, 2, 2, p, p, 1, 1, ptype, lp, cip)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("seed", range(24))
def test_colpair32_path_random(seed):
    """Random shapes on the 32-lanes-per-row-group path (rows of 34-64 elements,
    planes of at most 4096 elements a multiple of 8, at most 28 output rows and 32
    columns): 2x2 / 3x3 windows at stride 2, padding 0 or 1, some output sizes past
    the natural ones, plane counts not a multiple of 4, every pool type, full-range
    values.  Shapes outside the path (a plane size not a multiple of 8) check the
    path they take instead."""
    g = wl.rng(815, seed)
    k = int(g.choice([2, 3]))
    p = int(g.integers(0, 2))
    W = 2 * int(g.integers(17, 33))
    H = int(g.integers(1, min(57, 4096 // W + 1)))
    if g.integers(0, 4):
        H -= H % 4   # plane size a multiple of 8 (W even)
        H = max(H, 4)
    OH = min((H + 2 * p - k) // 2 + 1 if H + 2 * p >= k else 1, 28)
    OW = min((W + 2 * p - k) // 2 + 1, 32)
    if g.integers(0, 3) == 0:
        OH, OW = min(OH + int(g.integers(0, 3)), 28), min(OW + int(g.integers(0, 3)), 32)
    OH, OW = max(OH, 1), max(OW, 1)
    N, C = int(g.integers(1, 4)), int(g.integers(1, 20))
    ptype, lp = [(0, 0), (1, 0), (2, 1), (2, 2), (3, 0), (2, 0)][int(g.integers(0, 6))]
    cip = int(g.integers(0, 2)) if ptype == 1 else 0
    say(f"pool colpair32 random seed {seed}: {(N, C, H, W, OH, OW, k, p, ptype, lp, cip)}")
    x = g.integers(-32768, 32768, N * C * H * W, dtype=np.int16)
    got, want = pool_both(x, N, C, H, W, OH, OW, k, k, 2, 2, p, p, 1, 1, ptype, lp, cip)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("ptype,lp,cip", [(0, 0, 0), (1, 0, 1), (1, 0, 0), (2, 2, 0), (2, 1, 0)])
@pytest.mark.parametrize("k,p", [(3, 0), (3, 1), (2, 0), (2, 1)])
def test_colpair32_path_conv_a_size(ptype, lp, cip, k, p):
    """The conv + pool block's 56x56 pools at full size ([32, 128, 56, 56], 4096
    planes) on the 32-lanes-per-row-group path, full-range values."""
    N, C, H = 32, 128, 56
    OH = (H + 2 * p - k) // 2 + 1
    say(f"pool colpair32 56x56 k={k} p={p} type={ptype} lp={lp} cip={cip}")
    x = wl.rng(816, k, p, ptype, lp, cip).integers(-32768, 32768, N * C * H * H, dtype=np.int16)
    got, want = pool_both(x, N, C, H, H, OH, OH, k, k, 2, 2, p, p, 1, 1, ptype, lp, cip)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("seed", range(20))
def test_global_pool_random(seed):
    """Global pools (window = plane) over random plane sizes: the sixteen-lanes-per-
    plane kernel (at most 128 elements) and the wave-per-plane kernel (planes that
    are and are not multiples of 8), plane counts not a multiple of 16, every pool
    type, full-range values."""
    g = wl.rng(817, seed)
    H = int(g.integers(1, 12 if seed < 12 else 40))
    W = int(g.integers(1, 12 if seed < 12 else 40))
    N, C = int(g.integers(1, 5)), int(g.integers(1, 70))
    ptype, lp = [(0, 0), (1, 0), (2, 1), (2, 2), (3, 0), (2, 0)][int(g.integers(0, 6))]
    cip = int(g.integers(0, 2)) if ptype == 1 else 0
    say(f"global pool random seed {seed}: {(N, C, H, W, ptype, lp, cip)}")
    x = g.integers(-32768, 32768, N * C * H * W, dtype=np.int16)
    got, want = pool_both(x, N, C, H, W, 1, 1, H, W, 1, 1, 0, 0, 1, 1, ptype, lp, cip)
    np.testing.assert_array_equal(got, want)
