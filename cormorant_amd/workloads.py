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


# The pools run on each convolution's output: conv A's [32, 128, 56, 56] and
# conv B's [32, 128, 28, 28].  AvgPool takes pad 1 so that count_include_pad
# matters; MaxPool and LpPool use no padding.
POOL_CASES = (
    PoolCase("maxpool_3x3_s2", 0, 3, 2, 0),
    PoolCase("avgpool_3x3_s2_p1_cip", 1, 3, 2, 1, cip=1),
    PoolCase("lppool_p2_2x2_s2", 2, 2, 2, 0, lp_order=2),
    PoolCase("globalavgpool", 1, 0, 1, 0),
)


def block_pools():
    """(conv case, pool case) pairs of the conv + pool block: the four pools after each
    convolution, named '<pool>_on_<conv>'."""
    return [(cv, pc, f"{pc.name}_on_{cv.name[:6]}") for cv in CONV_CASES for pc in POOL_CASES]


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


# ---------------------------------------------------------------- ONNX graphs --
def _q88_initializer(name: str, raw: np.ndarray):
    """An ONNX float32 initializer holding on-grid Q8.8 values (raw / 256, exact)."""
    from .scheduler import onnx_io as ox
    return ox.from_array((raw.astype(np.float32) / np.float32(256.0)), name)


# config 1: 2-layer MLP, batch 64: Gemm 784->256, Relu, Gemm 256->10
MLP_BATCH, MLP_IN, MLP_HIDDEN, MLP_OUT = 64, 784, 256, 10


def mlp_model(batch: int = MLP_BATCH):
    """X[b,784] -> Gemm(W1,b1) -> Relu -> Gemm(W2,b2) -> Y[b,10]; weights N(0,0.1),
    biases N(0,0.05), quantised AP_TRN+AP_SAT."""
    from .scheduler import onnx_io as ox
    w1 = normal_q88(rng(1, 1), (MLP_IN, MLP_HIDDEN), 0.1)
    b1 = normal_q88(rng(1, 2), (MLP_HIDDEN,), 0.05)
    w2 = normal_q88(rng(1, 3), (MLP_HIDDEN, MLP_OUT), 0.1)
    b2 = normal_q88(rng(1, 4), (MLP_OUT,), 0.05)
    nodes = [
        ox.make_node("Gemm", ["X", "W1", "B1"], ["H"], name="fc1"),
        ox.make_node("Relu", ["H"], ["R"], name="relu1"),
        ox.make_node("Gemm", ["R", "W2", "B2"], ["Y"], name="fc2"),
    ]
    g = ox.make_graph(nodes, "mlp_784_256_10", [ox.value_info("X", [batch, MLP_IN])],
                      [ox.value_info("Y", [batch, MLP_OUT])],
                      [_q88_initializer("W1", w1), _q88_initializer("B1", b1),
                       _q88_initializer("W2", w2), _q88_initializer("B2", b2)])
    return ox.make_model(g, opset=13)


def mlp_input(batch: int = MLP_BATCH) -> np.ndarray:
    return uniform_q88(rng(1, 0), (batch, MLP_IN), -1.0, 1.0)


# config 5: MobileNetV2-like graph without grouped convolutions.
# The MobileNetV2 stage schedule (channels, repeats, first stride) with expansion
# 1: every block is Conv3x3(c_in -> c_in, stride) + Clip(0,6), then a linear
# Conv1x1(c_in -> c_out); a block with stride 1 and c_in == c_out adds its input
# back.  Stem Conv3x3 s2 3->32 + Clip; head Conv1x1 -> 1280 + Clip,
# GlobalAveragePool, Reshape, Gemm 1280 -> 1000.
MOBILENET_STAGES = ((16, 1, 1), (24, 2, 2), (32, 3, 2), (64, 4, 2), (96, 3, 1), (160, 3, 2),
                    (320, 1, 1))
MOBILENET_BATCH, MOBILENET_HW, MOBILENET_HEAD, MOBILENET_CLASSES = 16, 224, 1280, 1000


def mobilenet_model(batch: int = MOBILENET_BATCH, hw: int = MOBILENET_HW,
                    stages=MOBILENET_STAGES, head: int = MOBILENET_HEAD,
                    classes: int = MOBILENET_CLASSES):
    """The MobileNetV2-like graph; weights and biases N(0, 0.05), AP_TRN+AP_SAT."""
    from .scheduler import onnx_io as ox
    nodes, inits = [], []
    counter = [0]

    def conv(x, cin, cout, k, stride, clip):
        i = counter[0]
        counter[0] += 1
        w = normal_q88(rng(5, i, 0), (cout, cin, k, k), 0.05)
        b = normal_q88(rng(5, i, 1), (cout,), 0.05)
        inits.extend([_q88_initializer(f"conv{i}_w", w), _q88_initializer(f"conv{i}_b", b)])
        y = f"conv{i}_y"
        p = k // 2
        nodes.append(ox.make_node("Conv", [x, f"conv{i}_w", f"conv{i}_b"], [y], name=f"conv{i}",
                                  kernel_shape=[k, k], strides=[stride, stride],
                                  pads=[p, p, p, p]))
        if clip:
            nodes.append(ox.make_node("Clip", [y, "clip_lo", "clip_hi"], [f"{y}_r6"],
                                      name=f"clip{i}"))
            y = f"{y}_r6"
        return y

    inits.append(ox.from_array(np.array(0.0, np.float32), "clip_lo"))
    inits.append(ox.from_array(np.array(6.0, np.float32), "clip_hi"))
    x = conv("X", 3, 32, 3, 2, True)
    cin = 32
    for cout, reps, s in stages:
        for r in range(reps):
            stride = s if r == 0 else 1
            h = conv(x, cin, cin, 3, stride, True)
            y = conv(h, cin, cout, 1, 1, False)
            if stride == 1 and cin == cout:
                nodes.append(ox.make_node("Add", [y, x], [f"{y}_res"], name=f"res_{y}"))
                y = f"{y}_res"
            x, cin = y, cout
    x = conv(x, cin, head, 1, 1, True)
    nodes.append(ox.make_node("GlobalAveragePool", [x], ["gap"], name="gap"))
    inits.append(ox.from_array(np.array([batch, head], np.int64), "flat_shape"))
    nodes.append(ox.make_node("Reshape", ["gap", "flat_shape"], ["flat"], name="flatten"))
    fw = normal_q88(rng(5, 1000, 0), (head, classes), 0.05)
    fb = normal_q88(rng(5, 1000, 1), (classes,), 0.05)
    inits.extend([_q88_initializer("fc_w", fw), _q88_initializer("fc_b", fb)])
    nodes.append(ox.make_node("Gemm", ["flat", "fc_w", "fc_b"], ["Y"], name="fc"))
    g = ox.make_graph(nodes, "mobilenetv2_like", [ox.value_info("X", [batch, 3, hw, hw])],
                      [ox.value_info("Y", [batch, classes])], inits)
    return ox.make_model(g, opset=13)


def mobilenet_input(batch: int = MOBILENET_BATCH, hw: int = MOBILENET_HW) -> np.ndarray:
    return uniform_q88(rng(5, 9999), (batch, 3, hw, hw), -1.0, 1.0)
