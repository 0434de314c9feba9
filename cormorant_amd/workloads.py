"""Seeded synthetic workloads for the five benchmark configurations.

All tensors are raw int16 ap_fixed<16,8>.  Real values are quantised with
AP_TRN + AP_SAT (floor to 1/256, then clamp), the reference's conversion rule.
Every tensor has its own numpy PCG64 sub-stream keyed by
(master seed 42, config id, tensor id), so a tensor never depends on the
size or order of the others (kSeed = 42: kernels/*/include/Config.h.in).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

SEED = 42
EDGE_VALUES = np.array([32767, 32766, -32768, -32767], dtype=np.int16)


def rng(*ids: int) -> np.random.Generator:
    return np.random.default_rng([SEED, *ids])


def quantize_trn(x: np.ndarray) -> np.ndarray:
    """AP_TRN + AP_SAT: raw = clamp(floor(x * 256), -32768, 32767)."""
    r = np.floor(np.asarray(x, dtype=np.float64) * 256.0)
    return np.clip(r, -32768, 32767).astype(np.int16)


def uniform_q88(g: np.random.Generator, shape, lo: float, hi: float) -> np.ndarray:
    return quantize_trn(g.uniform(lo, hi, size=shape))


def normal_q88(g: np.random.Generator, shape, sigma: float) -> np.ndarray:
    return quantize_trn(g.normal(0.0, sigma, size=shape))


# ---------------------------------------------------------------- config 2 --
VECOP_N = 64 * 1024 * 1024
VECOP_OPS = (("Add", 0), ("Sub", 1), ("Mul", 2), ("Div", 3), ("Relu", 4), ("Clip06", 5))


def vecop_operand(n: int, op: int, which: int) -> np.ndarray:
    """70% uniform over [-8, 8), 30% pinned at the saturation edges.

    For Div the divisor never holds raw 0 (magnitude >= 1/256)."""
    g = rng(2, op, which)
    x = uniform_q88(g, n, -8.0, 8.0)
    edge = g.random(n) < 0.3
    x[edge] = EDGE_VALUES[g.integers(0, len(EDGE_VALUES), size=int(edge.sum()))]
    if op == 3 and which == 1:
        zero = x == 0
        while zero.any():
            x[zero] = uniform_q88(g, int(zero.sum()), -8.0, 8.0)
            zero = x == 0
    return x


# ---------------------------------------------------------------- config 3 --
@dataclass(frozen=True)
class GemmCase:
    name: str
    batch: int
    n: int
    k: int
    m: int
    lo: float
    hi: float

    @property
    def macs(self) -> int:
        return self.batch * self.n * self.k * self.m


GEMM_CASES = (
    GemmCase("gemm_b32_1024", 32, 1024, 1024, 1024, -4.0, 4.0),
    GemmCase("gemm_b1_4096", 1, 4096, 4096, 4096, -1.0, 1.0),
)


def gemm_operands(case: GemmCase, case_id: int):
    a = uniform_q88(rng(3, case_id, 0), (case.batch, case.n, case.k), case.lo, case.hi)
    b = uniform_q88(rng(3, case_id, 1), (case.batch, case.k, case.m), case.lo, case.hi)
    return a, b


# ---------------------------------------------------------------- config 4 --
def conv_out(n: int, k: int, s: int, d: int, p: int) -> int:
    """(in + 2*pad - dil*(k-1) - 1) / stride + 1 (bench_src/bench_conv.c:74-75)."""
    return (n + 2 * p - d * (k - 1) - 1) // s + 1


@dataclass(frozen=True)
class ConvCase:
    name: str
    batch: int
    in_ch: int
    hw: int
    out_ch: int
    k: int
    stride: int
    dil: int
    pad: int

    @property
    def out_hw(self) -> int:
        return conv_out(self.hw, self.k, self.stride, self.dil, self.pad)

    @property
    def macs(self) -> int:
        return self.batch * self.out_ch * self.out_hw ** 2 * self.in_ch * self.k * self.k


# Conv B shares conv A's input and weight tensors (64 -> 128 channels on 56x56).
CONV_CASES = (
    ConvCase("conv_a_3x3_s1_p1", 32, 64, 56, 128, 3, 1, 1, 1),
    ConvCase("conv_b_3x3_s2_d2_p2", 32, 64, 56, 128, 3, 2, 2, 2),
)


def conv_operands(case: ConvCase):
    x = uniform_q88(rng(4, 0), (case.batch, case.in_ch, case.hw, case.hw), -2.0, 2.0)
    w = normal_q88(rng(4, 1), (case.out_ch, case.in_ch, case.k, case.k), 0.05)
    b = normal_q88(rng(4, 2), (case.out_ch,), 0.1)
    return x, w, b


@dataclass(frozen=True)
class PoolCase:
    name: str
    pool_type: int      # 0 MAX, 1 AVG, 2 LP
    k: int              # window (0 = global)
    stride: int
    pad: int
    lp_order: int = 2
    cip: int = 0

    def out_hw(self, hw: int) -> int:
        if self.k == 0:
            return 1
        return conv_out(hw, self.k, self.stride, 1, self.pad)


# Pools run on conv A's output [32, 128, 56, 56].  AvgPool takes pad 1 so that
# count_include_pad matters; MaxPool and LpPool use no padding.
POOL_CASES = (
    PoolCase("maxpool_3x3_s2", 0, 3, 2, 0),
    PoolCase("avgpool_3x3_s2_p1_cip", 1, 3, 2, 1, cip=1),
    PoolCase("lppool_p2_2x2_s2", 2, 2, 2, 0, lp_order=2),
    PoolCase("globalavgpool", 1, 0, 1, 0),
)


def pool_args(case: PoolCase, n: int, c: int, hw: int):
    """Arguments of PoolingKernel after the scheduler's Global rewrite (nodes.py:1275-1284)."""
    if case.k == 0:
        k, s, p = hw, 1, 0
    else:
        k, s, p = case.k, case.stride, case.pad
    o = case.out_hw(hw)
    return dict(batch=n, channels=c, in_h=hw, in_w=hw, out_h=o, out_w=o, pool_h=k, pool_w=k,
                stride_h=s, stride_w=s, pad_top=p, pad_left=p, dil_h=1, dil_w=1,
                pool_type=case.pool_type, lp_order=case.lp_order, count_include_pad=case.cip)
