"""Case tables taken from the reference's own C-simulation tests (data only).

Each table cites the reference test it reproduces.  Geometry and known-answer
values are copied as data; the random fills of the reference (std::mt19937 /
default_random_engine) are replaced by this repository's seeded generators
with the same value scales.
"""
from __future__ import annotations

# --------------------------------------------------------------------------
# kernels/vectorop/test/TestSimulation.cpp:192-248 -- saturation / boundary
# table, exact comparison for ap_fixed (kTol = 0).  (op, a, b, description)
# --------------------------------------------------------------------------
ADD, SUB, MUL, DIV, RELU, RELU6 = range(6)
LSB = 1.0 / 256.0
VECOP_SAT_TABLE = [
    (ADD, 100.0, 100.0, "ADD 100+100=200 -> sat_max"),
    (ADD, 64.0, 64.0, "ADD 64+64=128 -> sat_max"),
    (ADD, 127.99609375, 0.00390625, "ADD max+1LSB -> sat_max"),
    (ADD, -100.0, -100.0, "ADD -100-100 -> sat_min"),
    (ADD, -128.0, -0.00390625, "ADD min-1LSB -> sat_min"),
    (ADD, 64.0, 63.99609375, "ADD 64+63.996=max (no clip)"),
    (ADD, -64.0, -64.0, "ADD -64-64=-128=min (no clip)"),
    (SUB, 100.0, -100.0, "SUB 100-(-100) -> sat_max"),
    (SUB, 127.99609375, -0.00390625, "SUB max-(-1LSB) -> sat_max"),
    (SUB, -100.0, 100.0, "SUB -100-100 -> sat_min"),
    (SUB, -128.0, 0.00390625, "SUB min-1LSB -> sat_min"),
    (MUL, 16.0, 16.0, "MUL 16x16=256 -> sat_max"),
    (MUL, 12.0, 12.0, "MUL 12x12=144 -> sat_max"),
    (MUL, -16.0, -16.0, "MUL -16x-16 -> sat_max"),
    (MUL, -16.0, 16.0, "MUL -16x16 -> sat_min"),
    (MUL, 11.0, 11.0, "MUL 11x11=121 (no clip)"),
    (RELU, -0.00390625, 0.0, "RELU -1LSB -> 0"),
    (RELU, -1.0, 0.0, "RELU -1.0 -> 0"),
    (RELU, 0.0, 0.0, "RELU 0 -> 0"),
    (RELU, 0.00390625, 0.0, "RELU +1LSB -> +1LSB"),
    (RELU, 3.5, 0.0, "RELU 3.5 -> 3.5"),
    (RELU6, -1.0, 0.0, "RELU6 -1 -> 0"),
    (RELU6, -0.00390625, 0.0, "RELU6 -1LSB -> 0"),
    (RELU6, 0.0, 0.0, "RELU6 0 -> 0"),
    (RELU6, 0.00390625, 0.0, "RELU6 +1LSB -> +1LSB"),
    (RELU6, 3.0, 0.0, "RELU6 3.0 -> 3.0"),
    (RELU6, 5.99609375, 0.0, "RELU6 6-1LSB -> 6-1LSB"),
    (RELU6, 6.0, 0.0, "RELU6 6.0 -> 6.0"),
    (RELU6, 6.00390625, 0.0, "RELU6 6+1LSB -> 6"),
    (RELU6, 8.0, 0.0, "RELU6 8 -> 6"),
    (RELU6, 20.0, 0.0, "RELU6 20 -> 6"),
]
SAT_MAX = 127.99609375
SAT_MIN = -128.0


def vecop_table_expected(op: int, a: float, b: float) -> float:
    """ref_op / ref_sat of TestSimulation.cpp:36-50 (double arithmetic, clamp)."""
    sat = lambda v: max(SAT_MIN, min(SAT_MAX, v))
    if op == ADD:
        return sat(a + b)
    if op == SUB:
        return sat(a - b)
    if op == MUL:
        return sat(a * b)
    if op == DIV:
        return 0.0 if b == 0.0 else sat(a / b)
    if op == RELU:
        return max(0.0, a)
    if op == RELU6:
        return min(max(0.0, a), 6.0)
    return a


# TestSimulation.cpp:60-69 -- value ranges of the random tests per op (b for DIV: [1, 10]).
VECOP_RANDOM_RANGES = {ADD: (-80.0, 80.0), SUB: (-80.0, 80.0), MUL: (-15.0, 15.0),
                       DIV: (1.0, 10.0), RELU: (-10.0, 10.0), RELU6: (-10.0, 10.0)}
VECOP_RANDOM_SIZES = (1, 8, 64, 256, 1024)   # TestSimulation.cpp:346

# --------------------------------------------------------------------------
# kernels/matmul/test/TestMatmulSim.cpp:276-367 with kTileN=4, kTileK=256,
# kTileM=16 (kernels/matmul/CMakeLists.txt:50-57).  Values U[-1, 1).
# --------------------------------------------------------------------------
TN, TK, TM = 4, 256, 16
MATMUL_2D = [
    ("1x1x1", 1, 1, 1),
    ("TileN x TileK x TileM", TN, TK, TM),
    ("2*TileN x TileK x TileM", 2 * TN, TK, TM),
    ("TileN x 2*TileK x TileM", TN, 2 * TK, TM),
    ("TileN x TileK x 2*TileM", TN, TK, 2 * TM),
    ("partial N", TN + 2, TK, TM),
    ("partial K", TN, TK + 5, TM),
    ("partial M", TN, TK, TM + 3),
    ("all partial", TN + 2, TK + 5, TM + 3),
    ("7 x 13 x 5", 7, 13, 5),
    ("K=1 outer product", TN + 1, 1, TM + 1),
    ("N=1 row vector", 1, TK, TM),
    ("M=1 column vector", TN, TK, 1),
    ("multi-tile all", 3 * TN, 2 * TK + 7, 2 * TM + 1),
]
_BN, _BK, _BM = TN + 1, TK // 4, TM + 3
# (name, n, k, m, batch, a_stride, b_stride); c_stride = n*m
MATMUL_BATCH = [
    ("batch=3, no broadcast", _BN, _BK, _BM, 3, _BN * _BK, _BK * _BM),
    ("batch=4, A broadcasts", _BN, _BK, _BM, 4, 0, _BK * _BM),
    ("batch=4, B broadcasts", _BN, _BK, _BM, 4, _BN * _BK, 0),
    ("batch=6, both strided", _BN, _BK, _BM, 6, _BN * _BK, _BK * _BM),
]
# (name, a value, b value, K, expected output) -- TestMatmulSim.cpp:364-367
MATMUL_SAT = [
    ("sat_pos", 100.0, 100.0, 3, SAT_MAX),
    ("sat_neg", 100.0, -100.0, 3, SAT_MIN),
]

# --------------------------------------------------------------------------
# kernels/conv/test/TestConvSim.cpp:283-629 with kTileM=8, kTileIC=16.
# (name, batch, C, H, W, M, kh, kw, sh, sw, dh, dw, pt, pl, pb, pr, bias, dw,
#  x_scale, w_scale, b_scale)
# --------------------------------------------------------------------------
CONV_GEOMS = [
    ("1x1 kernel, 1ch, no bias", 1, 1, 5, 5, 1, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 0, 0, 2.0, 2.0, 1.0),
    ("3x3, no pad, no bias", 1, 1, 5, 5, 1, 3, 3, 1, 1, 1, 1, 0, 0, 0, 0, 0, 0, 1.0, 1.0, 1.0),
    ("3x3, pad=1 (same)", 1, 1, 5, 5, 1, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1, 0, 0, 1.0, 1.0, 1.0),
    ("3x3, stride=2", 1, 1, 6, 6, 1, 3, 3, 2, 2, 1, 1, 0, 0, 0, 0, 0, 0, 1.0, 1.0, 1.0),
    ("3x3, pad=1, has_bias, 2 out_ch", 1, 1, 5, 5, 2, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1, 1, 0, 1.0, 1.0, 0.5),
    ("batch=2, 3x3, pad=1", 2, 1, 5, 5, 1, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1, 0, 0, 1.0, 1.0, 1.0),
    ("partial IC tile", 1, 21, 5, 5, 1, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1, 0, 0, 0.5, 0.5, 1.0),
    ("partial M tile", 1, 1, 5, 5, 11, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1, 1, 0, 0.5, 0.5, 0.5),
    ("3x3 dilation=2", 1, 1, 9, 9, 1, 3, 3, 1, 1, 2, 2, 0, 0, 0, 0, 0, 0, 1.0, 1.0, 1.0),
    ("5x5 kernel", 1, 1, 7, 7, 1, 5, 5, 1, 1, 1, 1, 0, 0, 0, 0, 0, 0, 1.0, 0.5, 1.0),
    ("14x14, multi-tile M and IC, bias", 1, 35, 14, 14, 17, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1, 1, 0,
     0.25, 0.25, 0.25),
    ("non-square 6x8 input, 3x5 kernel", 1, 1, 6, 8, 2, 3, 5, 1, 1, 1, 1, 0, 0, 0, 0, 0, 0, 1.0, 0.5, 1.0),
    ("7x7, stride=2, asymmetric pad", 1, 1, 7, 7, 1, 3, 3, 2, 2, 1, 1, 1, 1, 0, 0, 0, 0, 1.0, 0.5, 1.0),
    ("DW 3x3, 4ch, no pad, no bias", 1, 4, 8, 8, 4, 3, 3, 1, 1, 1, 1, 0, 0, 0, 0, 0, 1, 1.0, 1.0, 0.5),
    ("DW 3x3, 4ch, pad=1, has_bias", 1, 4, 8, 8, 4, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1.0, 0.5, 0.5),
    ("DW partial M tile", 1, 11, 6, 6, 11, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1, 0, 1, 0.5, 0.5, 0.5),
    ("DW 3x3 dilation=2, 4ch", 1, 4, 9, 9, 4, 3, 3, 1, 1, 2, 2, 0, 0, 0, 0, 0, 1, 0.5, 0.5, 0.5),
    ("DW stride=2, 8ch, pad=1", 1, 8, 8, 8, 8, 3, 3, 2, 2, 1, 1, 1, 1, 1, 1, 0, 1, 0.5, 0.5, 0.5),
]
# TestConvSim.cpp:592-629: 1x1 conv on 3x3, x = kSatMax everywhere,
# (w, bias, expected) = (+1, kSatMax, AP_MAX) and (-1, kSatMin, AP_MIN).
CONV_SAT = [
    ("saturation: positive overflow", 1.0, SAT_MAX, SAT_MAX),
    ("saturation: negative overflow", -1.0, SAT_MIN, SAT_MIN),
]


def conv_out_size(n, k, s, d, p0, p1):
    """out_size of TestConvSim.cpp (ONNX output size with explicit pads)."""
    return (n + p0 + p1 - d * (k - 1) - 1) // s + 1


# --------------------------------------------------------------------------
# kernels/pool/test/TestPoolingSim.cpp:161-229
# (name, N, C, H, W, out_h, out_w, ph, pw, sh, sw, pt, pl, dh, dw, type, lp, cip)
# --------------------------------------------------------------------------
POOL_TESTS = [
    ("MaxPool 2x2 stride2", 1, 4, 8, 8, 4, 4, 2, 2, 2, 2, 0, 0, 1, 1, 0, 0, 0),
    ("MaxPool 3x3 stride1 pad1", 1, 4, 8, 8, 8, 8, 3, 3, 1, 1, 1, 1, 1, 1, 0, 0, 0),
    ("MaxPool 2x2 stride2 rect 6x10", 1, 8, 6, 10, 3, 5, 2, 2, 2, 2, 0, 0, 1, 1, 0, 0, 0),
    ("MaxPool batch=3 2x2 stride2", 3, 4, 6, 6, 3, 3, 2, 2, 2, 2, 0, 0, 1, 1, 0, 0, 0),
    ("MaxPool channels>kTileC (C=16)", 1, 16, 8, 8, 4, 4, 2, 2, 2, 2, 0, 0, 1, 1, 0, 0, 0),
    ("MaxPool dilation=2 pool2x2", 1, 4, 8, 8, 6, 6, 2, 2, 1, 1, 0, 0, 2, 2, 0, 0, 0),
    ("GlobalMaxPool 4x4", 1, 8, 4, 4, 1, 1, 4, 4, 1, 1, 0, 0, 1, 1, 0, 0, 0),
    ("GlobalMaxPool batch=2 C=12 6x6", 2, 12, 6, 6, 1, 1, 6, 6, 1, 1, 0, 0, 1, 1, 0, 0, 0),
    ("AvgPool 2x2 stride2 no_pad", 1, 4, 8, 8, 4, 4, 2, 2, 2, 2, 0, 0, 1, 1, 1, 0, 0),
    ("AvgPool 3x3 stride1 pad1 no_include", 1, 4, 8, 8, 8, 8, 3, 3, 1, 1, 1, 1, 1, 1, 1, 0, 0),
    ("AvgPool 3x3 stride1 pad1 include_pad", 1, 4, 8, 8, 8, 8, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1, 0),
    ("AvgPool channels>kTileC (C=12)", 1, 12, 8, 8, 4, 4, 2, 2, 2, 2, 0, 0, 1, 1, 1, 0, 0),
    ("GlobalAvgPool 4x4 C=8", 1, 8, 4, 4, 1, 1, 4, 4, 1, 1, 0, 0, 1, 1, 1, 0, 0),
    ("GlobalAvgPool batch=2 C=16 6x6", 2, 16, 6, 6, 1, 1, 6, 6, 1, 1, 0, 0, 1, 1, 1, 0, 0),
    ("AvgPool rect 6x10 2x2 stride2", 1, 4, 6, 10, 3, 5, 2, 2, 2, 2, 0, 0, 1, 1, 1, 0, 0),
    ("LpPool p=1 2x2 stride2", 1, 4, 8, 8, 4, 4, 2, 2, 2, 2, 0, 0, 1, 1, 2, 1, 0),
    ("LpPool p=2 2x2 stride2", 1, 4, 8, 8, 4, 4, 2, 2, 2, 2, 0, 0, 1, 1, 2, 2, 0),
    ("LpPool p=1 3x3 pad1", 1, 4, 8, 8, 8, 8, 3, 3, 1, 1, 1, 1, 1, 1, 2, 1, 0),
    ("LpPool p=2 3x3 pad1", 1, 4, 8, 8, 8, 8, 3, 3, 1, 1, 1, 1, 1, 1, 2, 2, 0),
    ("GlobalLpPool p=1 4x4 C=8", 1, 8, 4, 4, 1, 1, 4, 4, 1, 1, 0, 0, 1, 1, 2, 1, 0),
    ("GlobalLpPool p=2 4x4 C=8", 1, 8, 4, 4, 1, 1, 4, 4, 1, 1, 0, 0, 1, 1, 2, 2, 0),
    ("GlobalLpPool p=2 batch=2 C=16 6x6", 2, 16, 6, 6, 1, 1, 6, 6, 1, 1, 0, 0, 1, 1, 2, 2, 0),
    ("MaxPool 1x1 pool full 5x5", 1, 4, 5, 5, 1, 1, 5, 5, 1, 1, 0, 0, 1, 1, 0, 0, 0),
    ("AvgPool corner padding 3x3 pad1 on 2x2", 1, 2, 2, 2, 2, 2, 3, 3, 1, 1, 1, 1, 1, 1, 1, 0, 0),
    ("MaxPool C=32 2x2 stride2", 1, 32, 8, 8, 4, 4, 2, 2, 2, 2, 0, 0, 1, 1, 0, 0, 0),
]
POOL_TOL = 0.02   # TestPoolingSim.cpp:22


def pool_test_fill(n: int):
    """Deterministic fill of TestPoolingSim.cpp:103-106: values (v - 40) * 0.1f,
    v = ((42 * 1103515245 + i * 12345) mod 2^32 >> 16) % 81, stored with
    Data_t(float) = floor to 1/256 (AP_TRN)."""
    import numpy as np
    i = np.arange(n, dtype=np.uint64)
    v = (((np.uint64(42) * np.uint64(1103515245) + i * np.uint64(12345)) & np.uint64(0xFFFFFFFF))
         >> np.uint64(16)) % np.uint64(81)
    f = (v.astype(np.int64) - 40).astype(np.float32) * np.float32(0.1)
    return np.floor(f.astype(np.float64) * 256.0).astype(np.int16)


def pool_ref_elem(x, C, H, W, n, c, oh, ow, ph, pw, sh, sw, pt, pl, dh, dw, ptype, lp, cip):
    """Float reference ref_pool_elem of TestPoolingSim.cpp:30-76 (tolerance check only)."""
    import math
    acc = -1.0e30 if ptype == 0 else 0.0
    valid = 0
    for khi in range(ph):
        for kwi in range(pw):
            ih = oh * sh + khi * dh - pt
            iw = ow * sw + kwi * dw - pl
            if 0 <= ih < H and 0 <= iw < W:
                v = float(x[((n * C + c) * H + ih) * W + iw]) / 256.0
                if ptype == 0:
                    acc = max(acc, v)
                elif ptype == 1:
                    acc += v
                else:
                    acc += abs(v) if lp == 1 else v * v
                valid += 1
    if ptype == 0:
        r = acc
    elif ptype == 1:
        d = ph * pw if cip else valid
        r = acc / d if d > 0 else 0.0
    else:
        r = acc if lp == 1 else math.sqrt(acc)
    return max(-128.0, min(127.996, r))
