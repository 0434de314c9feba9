"""GPU parity: MatmulKernel (int8-limb MFMA) through the C ABI vs the CPU oracle."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from cormorant_amd import kernels as K
from cormorant_amd import workloads as wl
from tests import refcases as rc
from tests.gpu_util import dev, empty_dev, host, oracle_threads, say

pytestmark = pytest.mark.gpu


def mm_both(a, b, n, k, m, batch=1, a_bs=0, b_bs=0, c_bs=None, c_len=None):
    c_bs = n * m if c_bs is None else c_bs
    c_len = c_len or ((batch - 1) * c_bs + n * m)
    c = empty_dev(c_len)
    K.MatmulKernel(dev(a), dev(b), c, n, k, m, batch, a_bs, b_bs, c_bs)
    want = np.full(c_len, 0x5A5A, np.int16)
    oracle.set_threads(oracle_threads())
    oracle.matmul(np.ascontiguousarray(a.reshape(-1)), np.ascontiguousarray(b.reshape(-1)), want,
                  n, k, m, batch, a_bs, b_bs, c_bs, threads=True)
    return host(c), want


@pytest.mark.parametrize("shape", rc.MATMUL_2D, ids=[s[0] for s in rc.MATMUL_2D])
def test_reference_shapes(shape):
    name, n, k, m = shape
    say(f"matmul reference shape {name}")
    g = wl.rng(820, n, k, m)
    a = wl.uniform_q88(g, (n, k), -1.0, 1.0)
    b = wl.uniform_q88(g, (k, m), -1.0, 1.0)
    got, want = mm_both(a, b, n, k, m)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("case", rc.MATMUL_BATCH, ids=[s[0] for s in rc.MATMUL_BATCH])
def test_reference_batches(case):
    name, n, k, m, batch, a_bs, b_bs = case
    say(f"matmul reference batch {name}")
    g = wl.rng(821, batch, a_bs, b_bs)
    a = wl.uniform_q88(g, max((batch - 1) * a_bs + n * k, n * k), -1.0, 1.0)
    b = wl.uniform_q88(g, max((batch - 1) * b_bs + k * m, k * m), -1.0, 1.0)
    got, want = mm_both(a, b, n, k, m, batch, a_bs, b_bs)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("case", rc.MATMUL_SAT, ids=[s[0] for s in rc.MATMUL_SAT])
def test_saturation_kats(case):
    name, av, bv, k, expect = case
    say(f"matmul saturation {name}")
    n, m = 5, 17
    a = np.full((n, k), int(av * 256), np.int16)
    b = np.full((k, m), int(bv * 256), np.int16)
    got, want = mm_both(a, b, n, k, m)
    np.testing.assert_array_equal(got, want)
    assert np.all(got / 256.0 == expect)


SHAPES = [
    # n, k, m -- vector and scalar load paths, partial tiles, many k tiles
    (128, 64, 128), (129, 65, 127), (1, 1, 1), (3, 7, 5), (64, 784, 256), (64, 256, 10),
    (16, 1280, 1000), (200, 520, 72), (256, 8, 8), (17, 2048, 33), (130, 1000, 260),
]


@pytest.mark.parametrize("shape", SHAPES, ids=[str(s) for s in SHAPES])
def test_full_range_values_wrap(shape):
    """Uniform int16 over the whole range: sums overflow 2^31 and must wrap."""
    n, k, m = shape
    say(f"matmul full-range {shape}")
    g = wl.rng(822, n, k, m)
    a = g.integers(-32768, 32768, (n, k), dtype=np.int16)
    b = g.integers(-32768, 32768, (k, m), dtype=np.int16)
    got, want = mm_both(a, b, n, k, m)
    np.testing.assert_array_equal(got, want)


def test_extreme_values():
    """All-(-32768) and all-32767 operands: the limb offsets and corrections at the edges."""
    for av, bv in [(-32768, -32768), (32767, 32767), (-32768, 32767), (0, 0), (-1, 255), (255, -1)]:
        say(f"matmul extremes a={av} b={bv}")
        n, k, m = 70, 300, 90
        a = np.full((n, k), av, np.int16)
        b = np.full((k, m), bv, np.int16)
        got, want = mm_both(a, b, n, k, m)
        np.testing.assert_array_equal(got, want)


def test_misaligned_and_broadcast_batches():
    import torch
    say("matmul misaligned views")
    g = wl.rng(823)
    n, k, m, batch = 33, 96, 40, 3
    a = g.integers(-2000, 2000, batch * n * k + 1, dtype=np.int16)
    b = g.integers(-2000, 2000, k * m + 1, dtype=np.int16)
    da, db = dev(a), dev(b)
    c = torch.zeros(batch * n * m + 1, dtype=torch.int16, device="cuda")
    K.MatmulKernel(da[1:], db[1:], c[1:], n, k, m, batch, n * k, 0, n * m)   # B broadcasts
    want = np.zeros(batch * n * m, np.int16)
    oracle.matmul(a[1:].copy(), b[1:].copy(), want, n, k, m, batch, n * k, 0, n * m)
    np.testing.assert_array_equal(host(c)[1:], want)


def test_same_output_every_batch_keeps_last():
    say("matmul c_stride = 0")
    g = wl.rng(824)
    n, k, m, batch = 8, 16, 8, 4
    a = g.integers(-3000, 3000, batch * n * k, dtype=np.int16)
    b = g.integers(-3000, 3000, batch * k * m, dtype=np.int16)
    got, want = mm_both(a, b, n, k, m, batch, n * k, k * m, 0, c_len=n * m)
    np.testing.assert_array_equal(got, want)


def test_overlapping_batch_outputs_keep_the_last_batch():
    """0 < c_stride < n*m: batch outputs overlap; the reference's sequential batch
    loop leaves each shared element with the last writing batch's value."""
    g = wl.rng(827)
    for n, k, m, batch, c_bs in [(4, 32, 8, 5, 8), (16, 300, 40, 3, 1), (2, 64, 130, 4, 129)]:
        say(f"matmul overlapping outputs {(n, k, m, batch, c_bs)}")
        a = g.integers(-32768, 32768, batch * n * k, dtype=np.int16)
        b = g.integers(-32768, 32768, batch * k * m, dtype=np.int16)
        got, want = mm_both(a, b, n, k, m, batch, n * k, k * m, c_bs)
        np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("n,m,batch", [(5, 7, 1), (130, 260, 3), (1, 1000, 1)])
def test_k_zero_gives_zero(n, m, batch):
    """k = 0: the reference's k loop is empty, every output is 0 (and the fused
    column Add then gives the added row)."""
    import torch
    say(f"matmul k=0 {(n, m, batch)}")
    c = empty_dev(batch * n * m)
    K.MatmulKernel(None, None, c, n, 0, m, batch, 0, 0, n * m)
    np.testing.assert_array_equal(host(c), np.zeros(batch * n * m, np.int16))
    want = np.zeros(batch * n * m, np.int16)
    oracle.matmul(np.zeros(1, np.int16), np.zeros(1, np.int16), want, n, 0, m, batch, 0, 0, n * m)
    np.testing.assert_array_equal(want, 0)
    add = wl.rng(828, n, m).integers(-32768, 32768, m, dtype=np.int16)
    c2 = empty_dev(batch * n * m)
    K.MatmulKernel(torch.zeros(1, dtype=torch.int16, device="cuda"), None, c2, n, 0, m, batch,
                   0, 0, n * m, add=dev(add), add_column=True, act=K.ACT_RELU6)
    np.testing.assert_array_equal(host(c2).reshape(-1, m), np.tile(np.clip(add, 0, 1536), (batch * n, 1)))


def test_long_k_folds_partials():
    """K > 32768 takes the path that folds MFMA partials into a uint32 total."""
    n, k, m = 20, 70000, 24
    say(f"matmul long k={k}")
    g = wl.rng(825)
    a = g.integers(-32768, 32768, (n, k), dtype=np.int16)
    b = g.integers(-32768, 32768, (k, m), dtype=np.int16)
    got, want = mm_both(a, b, n, k, m)
    np.testing.assert_array_equal(got, want)


def test_config3a_full():
    case = wl.GEMM_CASES[0]
    say(f"matmul full-size {case.name}")
    a, b = wl.gemm_operands(case, 0)
    n, k, m = case.n, case.k, case.m
    got, want = mm_both(a, b, n, k, m, case.batch, n * k, k * m, n * m)
    np.testing.assert_array_equal(got, want)


def test_config3b_full():
    """4096^3 (K above the reference's kMaxK): the whole output against the oracle's
    tiled kernel with OpenMP (itself pinned to the naive row loop and to Python
    integers in test_oracle.py)."""
    case = wl.GEMM_CASES[1]
    say(f"matmul full-size {case.name}")
    a, b = wl.gemm_operands(case, 1)
    n, k, m = case.n, case.k, case.m
    got, want = mm_both(a.reshape(n, k), b.reshape(k, m), n, k, m)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("seed", range(16))
def test_small_products_register_kernel(seed):
    """Small single products (<= 2^18 outputs, K <= 4096) on the register-only
    kernel (the reduction split over a block's waves): row / column counts around
    the 32-wide tile, K with and without whole 16-byte rows, full-range values that
    wrap, unaligned A, and the fused epilogue (same-shaped Add, column Add, Relu6)."""
    g = wl.rng(823, seed)
    n = int(g.choice([1, 7, 16, 31, 32, 33, 64, 100, 200]))
    m = int(g.choice([1, 10, 31, 33, 96, 256, 1000]))
    k = int(g.choice([1, 5, 8, 64, 65, 256, 784, 1280, 2047, 4096]))
    if n * m > (1 << 18):
        m = (1 << 18) // n
    say(f"matmul register kernel seed {seed}: {n} x {k} x {m}")
    assert K.matmul_workspace_size(n, k, m) == 0
    a = g.integers(-32768, 32768, n * k + 1, dtype=np.int16)
    b = g.integers(-32768, 32768, k * m, dtype=np.int16)
    off = int(seed % 2)   # odd seeds: A one element past a 16-byte boundary
    want = np.zeros(n * m, np.int16)
    oracle.set_threads(oracle_threads())
    oracle.matmul(np.ascontiguousarray(a[off:off + n * k]), b, want, n, k, m, threads=True)
    da = dev(a)[off:off + n * k]
    c = empty_dev(n * m)
    K.MatmulKernel(da, dev(b), c, n, k, m)
    np.testing.assert_array_equal(host(c), want)
    same = g.integers(-32768, 32768, n * m, dtype=np.int16)
    col = g.integers(-32768, 32768, m, dtype=np.int16)
    for add, column, act in ((same, False, K.ACT_NONE), (col, True, K.ACT_RELU6)):
        c2 = empty_dev(n * m)
        K.MatmulKernel(da, dev(b), c2, n, k, m, add=dev(add), add_column=column, act=act)
        addv = np.tile(col, n) if column else same
        exp = np.clip(want.astype(np.int32) + addv, -32768, 32767)
        if act == K.ACT_RELU6:
            exp = np.clip(exp, 0, 1536)
        np.testing.assert_array_equal(host(c2).astype(np.int32), exp)
