"""The reference's per-kernel benchmark case list, for cm_bench.

Every case of inference-scheduler/perf_config.json.example:66-133 (14 VectorOP,
10 MatMul, 9 Conv, 8 Pool), plus the rows of the published KV260 report that
the example file does not list (inference-scheduler/doc/REMOTE_TESTING.md:662-740:
MUL-bcast-dw-12544x16, the five op-6 "SOFTMAX" rows, dw-12544x16x1/x3).  Their
arguments follow from the report's parameters and the bench programs'
formulas: MUL-bcast-dw moves 12544 x 16 elements (a advancing by 16, b
repeating), SOFTMAX-*-N rows advance a by the row size, and the
dw-12544x16xB MatMuls use independent batches.  Opcode 6 is not an operation
of the reference VectorOPKernel source (kernels/vectorop/include/VectorOP.h:50-57);
its kernel copies a for any opcode >= 6 (VectorOP.cpp:112), and so does this
library, so those rows time a copy.

`kv260` holds the published KV260 figures (lat_ms and gbs / gops) where the
report has the row; the other perf_config cases have none (the report's Conv
table lists one case).
"""
from __future__ import annotations

# (kind, label, args in the bench program's order (after instance, label), iters, warmup, kv260)
# vectorop args: op size outer a_inc b_inc
# matmul args:   n k m batch a_stride b_stride
# conv args:     batch in_ch in_h in_w out_ch kh kw sh sw dh dw pt pl has_bias is_dw
# pool args:     batch channels in_h in_w pool_h pool_w sh sw pt pl dh dw pool_type lp_order cip
CASES = [
    ("vectorop", "ADD-1K", (0, 1024, 1, 0, 0), 200, 10, (0.0207, 0.297)),
    ("vectorop", "ADD-4K", (0, 4096, 1, 0, 0), 200, 10, (0.0516, 0.476)),
    ("vectorop", "ADD-16K", (0, 16384, 1, 0, 0), 200, 10, (0.1754, 0.561)),
    ("vectorop", "ADD-64K", (0, 65536, 1, 0, 0), 100, 10, (0.6709, 0.586)),
    ("vectorop", "ADD-256K", (0, 262144, 1, 0, 0), 50, 10, (2.6528, 0.593)),
    ("vectorop", "MUL-16K", (2, 16384, 1, 0, 0), 200, 10, (0.1756, 0.560)),
    ("vectorop", "MUL-64K", (2, 65536, 1, 0, 0), 100, 10, (0.6712, 0.586)),
    ("vectorop", "DIV-4K", (3, 4096, 1, 0, 0), 50, 10, (0.0520, 0.473)),
    ("vectorop", "RELU-16K", (4, 16384, 1, 0, 0), 200, 10, (0.1728, 0.379)),
    ("vectorop", "RELU-64K", (4, 65536, 1, 0, 0), 100, 10, (0.6683, 0.392)),
    ("vectorop", "RELU6-16K", (5, 16384, 1, 0, 0), 200, 10, (0.1729, 0.379)),
    ("vectorop", "ADD-bcast-8x16K", (0, 16384, 8, 16384, 0), 100, 10, (1.3813, 0.569)),
    ("vectorop", "MUL-bcast-8x16K", (2, 16384, 8, 16384, 0), 100, 10, (1.3813, 0.569)),
    ("vectorop", "RELU-bcast-8x16K", (4, 16384, 8, 16384, 0), 100, 10, (1.3484, 0.389)),
    ("vectorop", "MUL-bcast-dw-12544x16", (2, 16, 12544, 16, 0), 100, 10, (5.8274, 0.207)),
    ("vectorop", "SOFTMAX-1K-1row", (6, 1024, 1, 0, 0), 200, 10, (0.0181, 0.226)),
    ("vectorop", "SOFTMAX-4K-1row", (6, 4096, 1, 0, 0), 200, 10, (0.0491, 0.334)),
    ("vectorop", "SOFTMAX-16K-1row", (6, 16384, 1, 0, 0), 200, 10, (0.1728, 0.379)),
    ("vectorop", "SOFTMAX-1K-8rows", (6, 1024, 8, 1024, 0), 200, 10, (0.1100, 0.298)),
    ("vectorop", "SOFTMAX-4K-4rows", (6, 4096, 4, 4096, 0), 200, 10, (0.1811, 0.362)),
    ("matmul", "8x8x8", (8, 8, 8, 1, 0, 0), 500, 10, (0.0176, 0.058)),
    ("matmul", "16x16x16", (16, 16, 16, 1, 0, 0), 500, 10, (0.0520, 0.157)),
    ("matmul", "32x32x32", (32, 32, 32, 1, 0, 0), 200, 10, (0.3039, 0.216)),
    ("matmul", "64x64x64", (64, 64, 64, 1, 0, 0), 100, 10, (2.1416, 0.245)),
    ("matmul", "128x128x128", (128, 128, 128, 1, 0, 0), 50, 10, (16.1860, 0.259)),
    ("matmul", "256x256x256", (256, 256, 256, 1, 0, 0), 20, 10, (126.2730, 0.266)),
    ("matmul", "FC-1x256x256", (1, 256, 256, 1, 0, 0), 500, 10, (1.9489, 0.067)),
    ("matmul", "FC-4x256x256", (4, 256, 256, 1, 0, 0), 200, 10, (1.9778, 0.265)),
    ("matmul", "batch4-64x64x64", (64, 64, 64, 4, 4096, 4096), 50, 10, (8.5376, 0.246)),
    ("matmul", "batch4-A-bcast", (64, 64, 64, 4, 0, 4096), 50, 10, (8.5382, 0.246)),
    ("matmul", "dw-12544x16x1", (12544, 16, 1, 1, 0, 0), 100, 10, (13.3935, 0.030)),
    ("matmul", "dw-12544x16x3", (12544, 16, 1, 3, 12544 * 16, 16), 100, 10, (40.1768, 0.030)),
    ("conv", "3x3-1ch-28x28-32out", (1, 1, 28, 28, 32, 3, 3, 1, 1, 1, 1, 1, 1, 0, 0), 200, 10,
     (14.5811, 0.031)),
    ("conv", "3x3-64ch-56x56", (1, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1, 1, 0, 0), 50, 10, None),
    ("conv", "3x3-64ch-56x56-s2", (1, 64, 56, 56, 64, 3, 3, 2, 2, 1, 1, 1, 1, 0, 0), 50, 10, None),
    ("conv", "3x3-64ch-28x28", (1, 64, 28, 28, 64, 3, 3, 1, 1, 1, 1, 1, 1, 0, 0), 100, 10, None),
    ("conv", "1x1-64to128-56x56", (1, 64, 56, 56, 128, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0), 50, 10, None),
    ("conv", "1x1-128to256-28x28", (1, 128, 28, 28, 256, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0), 50, 10, None),
    ("conv", "5x5-16ch-28x28", (1, 16, 28, 28, 16, 5, 5, 1, 1, 1, 1, 2, 2, 0, 0), 100, 10, None),
    ("conv", "dw-3x3-32ch-28x28", (1, 32, 28, 28, 32, 3, 3, 1, 1, 1, 1, 1, 1, 0, 1), 200, 10, None),
    ("conv", "dw-3x3-64ch-56x56", (1, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1, 1, 0, 1), 50, 10, None),
    ("pool", "MaxPool-2x2-56x56", (1, 64, 56, 56, 2, 2, 2, 2, 0, 0, 1, 1, 0, 1, 0), 200, 10,
     (21.6922, 0.023)),
    ("pool", "MaxPool-2x2-28x28", (1, 64, 28, 28, 2, 2, 2, 2, 0, 0, 1, 1, 0, 1, 0), 200, 10,
     (5.3711, 0.023)),
    ("pool", "MaxPool-3x3-56x56", (1, 64, 56, 56, 3, 3, 2, 2, 1, 1, 1, 1, 0, 1, 0), 100, 10,
     (36.2833, 0.014)),
    ("pool", "MaxPool-3x3-14x14", (1, 64, 14, 14, 3, 3, 2, 2, 1, 1, 1, 1, 0, 1, 0), 200, 10,
     (2.1684, 0.014)),
    ("pool", "AvgPool-2x2-56x56", (1, 64, 56, 56, 2, 2, 2, 2, 0, 0, 1, 1, 1, 1, 0), 200, 10,
     (21.6922, 0.023)),
    ("pool", "AvgPool-3x3-28x28", (1, 64, 28, 28, 3, 3, 2, 2, 1, 1, 1, 1, 1, 1, 0), 200, 10,
     (8.8810, 0.014)),
    ("pool", "GlobalMaxPool-14x14", (1, 64, 14, 14, 14, 14, 1, 1, 0, 0, 1, 1, 0, 1, 0), 200, 10,
     (0.7044, 0.036)),
    ("pool", "GlobalAvgPool-7x7", (1, 64, 7, 7, 7, 7, 1, 1, 0, 0, 1, 1, 1, 1, 0), 200, 10,
     (0.1908, 0.034)),
]


def case_line(case, instance: str = "0") -> str:
    """The cm_bench argument line of one case (the reference program's arguments)."""
    kind, label, args, iters, warmup, _ = case
    return " ".join([kind, instance, label, *map(str, args), str(iters), str(warmup)])


def buffer_sizes(kind: str, args):
    """Element counts of the case's buffers in cm_bench's order (inputs..., output),
    as the reference programs allocate them (bench_src/bench_*.c)."""
    if kind == "vectorop":
        op, sz, outer, ai, bi = args
        return [outer * sz if ai else sz, outer * sz if bi else sz, outer * sz]
    if kind == "matmul":
        n, k, m, batch, a_s, b_s = args
        return [batch * n * k if a_s else n * k, batch * k * m if b_s else k * m, batch * n * m]
    if kind == "conv":
        b, ic, ih, iw, oc, kh, kw, sh, sw, dh, dw, pt, pl, hb, idw = args
        oh = (ih + 2 * pt - dh * (kh - 1) - 1) // sh + 1
        ow = (iw + 2 * pl - dw * (kw - 1) - 1) // sw + 1
        return [b * ic * ih * iw, oc * kh * kw if idw else oc * ic * kh * kw, oc if hb else 1,
                b * oc * oh * ow]
    b, ch, ih, iw, ph, pw, sh, sw, pt, pl, dh, dw, *_ = args
    oh = (ih + 2 * pt - dh * (ph - 1) - 1) // sh + 1
    ow = (iw + 2 * pl - dw * (pw - 1) - 1) // sw + 1
    return [b * ch * ih * iw, b * ch * oh * ow]


_GOLDEN = 0x9E3779B97F4A7C15


def fill(seed: int, which: int, n: int):
    """The input cm_bench writes into buffer `which` of a case (cm_bench.c fill()):
    element i = low 16 bits of splitmix64(seed * 0x100000001B3 + which + i * golden)."""
    import numpy as np
    mask = (1 << 64) - 1
    base = (seed * 0x100000001B3 + which) & mask
    with np.errstate(over="ignore"):
        x = np.uint64(base) + np.arange(n, dtype=np.uint64) * np.uint64(_GOLDEN)
        z = x + np.uint64(_GOLDEN)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return (z & np.uint64(0xFFFF)).astype(np.uint16).view(np.int16)


def fnv1a(raw) -> str:
    """FNV-1a 64 of an int16 array's little-endian bytes, as cm_bench prints it."""
    h = 0xCBF29CE484222325
    for byte in raw.astype("<i2").tobytes():
        h = ((h ^ byte) * 0x100000001B3) & ((1 << 64) - 1)
    return f"{h:016x}"
