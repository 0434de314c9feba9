"""GPU parity: VectorOPKernel through the C ABI vs the CPU oracle (bit-exact)."""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from cormorant_amd import kernels as K
from cormorant_amd import workloads as wl
from tests import refcases as rc
from tests.gpu_util import dev, empty_dev, host, oracle_threads, say

pytestmark = pytest.mark.gpu


def run_gpu(a, b, size, op, outer=1, a_inc=0, b_inc=0, c_len=None, c_init=None):
    c_len = c_len or (outer - 1) * (a_inc + b_inc) + size
    c = dev(c_init) if c_init is not None else empty_dev(c_len)
    K.VectorOPKernel(dev(a), dev(b) if b is not None else None, c, size, op, outer, a_inc, b_inc)
    return host(c)


def run_cpu(a, b, size, op, outer=1, a_inc=0, b_inc=0, c_init=None, c_len=None):
    c_len = c_len or (outer - 1) * (a_inc + b_inc) + size
    c = c_init.copy() if c_init is not None else np.full(c_len, 0x5A5A, np.int16)
    oracle.vectorop(a, b if b is not None else np.zeros(1, np.int16), c, size, op, outer, a_inc, b_inc)
    return c


@pytest.mark.parametrize("row", rc.VECOP_SAT_TABLE, ids=[r[3] for r in rc.VECOP_SAT_TABLE])
def test_saturation_table(row):
    op, av, bv, desc = row
    say(f"vectorop table: {desc}")
    a = np.full(8, int(av * 256), np.int16)
    b = np.full(8, int(bv * 256), np.int16)
    c = run_gpu(a, b, 8, op)
    assert np.all(c / 256.0 == rc.vecop_table_expected(op, av, bv))


@pytest.mark.parametrize("op", list(range(7)) + [42])
@pytest.mark.parametrize("size", [1, 7, 8, 64, 256, 1000, 1024, 4099, 1_000_003])
def test_random_flat(op, size):
    say(f"vectorop flat op={op} size={size}")
    g = wl.rng(800, op, size)
    a = g.integers(-32768, 32768, size, dtype=np.int16)
    b = g.integers(-32768, 32768, size, dtype=np.int16)
    got = run_gpu(a, b if op < 4 else None, size, op)
    np.testing.assert_array_equal(got, run_cpu(a, b, size, op))


@pytest.mark.parametrize("op", range(6))
def test_unaligned_pointers(op):
    """Operands starting 1 element past a 16-byte boundary use the scalar path."""
    say(f"vectorop unaligned op={op}")
    import torch
    g = wl.rng(801, op)
    n = 5000
    a = g.integers(-32768, 32768, n + 1, dtype=np.int16)
    b = g.integers(-32768, 32768, n + 1, dtype=np.int16)
    da, db = dev(a), dev(b)
    dc = torch.zeros(n + 1, dtype=torch.int16, device="cuda")
    K.VectorOPKernel(da[1:], db[1:], dc[1:], n, op)
    want = run_cpu(a[1:].copy(), b[1:].copy(), n, op)
    np.testing.assert_array_equal(host(dc)[1:], want)


BROADCASTS = [
    # (size, outer, a_inc, b_inc)   a advancing / b advancing, aligned and not
    (4, 2, 4, 0), (4, 3, 0, 4),
    (256, 64, 256, 0), (10, 64, 16, 0), (1000, 16, 0, 1000), (16, 64, 0, 16),
    (24, 7, 24, 0), (8, 300, 0, 8), (13, 9, 13, 0),
    (4, 5, 2, 0), (6, 4, 1, 2), (5, 3, 0, 0),          # overlapping outer steps
]


@pytest.mark.parametrize("op", range(6))
@pytest.mark.parametrize("bc", BROADCASTS, ids=[str(b) for b in BROADCASTS])
def test_broadcast(op, bc):
    size, outer, a_inc, b_inc = bc
    say(f"vectorop broadcast op={op} {bc}")
    g = wl.rng(802, op, *bc)
    a = g.integers(-32768, 32768, (outer - 1) * a_inc + size, dtype=np.int16)
    b = g.integers(-32768, 32768, (outer - 1) * b_inc + size, dtype=np.int16)
    c_len = (outer - 1) * (a_inc + b_inc) + size + 16
    init = g.integers(-32768, 32768, c_len, dtype=np.int16)   # gap slots must stay untouched
    got = run_gpu(a, b, size, op, outer, a_inc, b_inc, c_init=init)
    np.testing.assert_array_equal(got, run_cpu(a, b, size, op, outer, a_inc, b_inc, c_init=init))


def test_div_exhaustive_all_pairs():
    """The DIV estimate-and-correct path equals integer trunc division for all 2^32 pairs."""
    say("vectorop DIV exhaustive sweep")
    n, example = K.selftest_div(0, 65536)
    assert n == 0, f"{n} mismatches, e.g. (a, b, got, want) = {example}"


@pytest.mark.parametrize("name,op", wl.VECOP_OPS)
def test_config2_full_size(name, op):
    """64Mi-element sweep of the benchmark configuration, bit-exact vs the oracle."""
    say(f"vectorop full-size {name}")
    n = wl.VECOP_N
    a = wl.vecop_operand(n, op, 0)
    b = wl.vecop_operand(n, op, 1)
    got = run_gpu(a, b if op < 4 else None, n, op)
    oracle.set_threads(oracle_threads())
    want = run_cpu(a, b, n, op)
    np.testing.assert_array_equal(got, want)
    if op == 3:
        assert not np.any(b == 0)
    edge = np.isin(a, wl.EDGE_VALUES).mean()
    assert math.isclose(edge, 0.3, abs_tol=0.01)
