"""Expected outputs of cm_bench cases -- TEST INFRASTRUCTURE ONLY.

cm_bench fills a case's input buffers from a seeded splitmix64 stream
(cormorant_amd/bench_src/perf_cases.fill) and runs the reference program's call
(bench_src/bench_*.c: run_op / run_matmul with c_stride = n*m / run_conv /
run_pool).  `expected` recomputes that call with the C oracle on the same
inputs; `check_dump` compares an output cm_bench wrote with CM_BENCH_DUMP.
"""
from __future__ import annotations

import os

import numpy as np

from . import conv, matmul, pool, vectorop


def expected(case, seed: int = 42, threads: bool = True) -> np.ndarray:
    from cormorant_amd.bench_src import perf_cases as pc
    kind, _label, args, *_ = case
    sizes = pc.buffer_sizes(kind, args)
    ins = [pc.fill(seed, i, n) for i, n in enumerate(sizes[:-1])]
    out = np.zeros(sizes[-1], np.int16)
    if kind == "vectorop":
        op, sz, outer, ai, bi = args
        vectorop(ins[0], ins[1], out, sz, op, outer, ai, bi, threads=threads)
    elif kind == "matmul":
        n, k, m, batch, a_s, b_s = args
        matmul(ins[0], ins[1], out, n, k, m, batch, a_s, b_s, n * m, threads=threads)
    elif kind == "conv":
        b, ic, ih, iw, oc, kh, kw, sh, sw, dh, dw, pt, pl, hb, idw = args
        oh = (ih + 2 * pt - dh * (kh - 1) - 1) // sh + 1
        ow = (iw + 2 * pl - dw * (kw - 1) - 1) // sw + 1
        conv(ins[0], ins[1], ins[2], out, b, ic, ih, iw, oc, oh, ow, kh, kw, sh, sw, dh, dw, pt,
             pl, hb, idw, threads=threads)
    else:
        b, ch, ih, iw, ph, pw, sh, sw, pt, pl, dh, dw, ptype, lpo, cip = args
        oh = (ih + 2 * pt - dh * (ph - 1) - 1) // sh + 1
        ow = (iw + 2 * pl - dw * (pw - 1) - 1) // sw + 1
        pool(ins[0], out, b, ch, ih, iw, oh, ow, ph, pw, sh, sw, pt, pl, dh, dw, ptype, lpo, cip,
             threads=threads)
    return out


def check_dump(case, dump_dir: str, seed: int = 42) -> int:
    """Number of output elements that differ between cm_bench's dump and the oracle."""
    got = np.fromfile(os.path.join(dump_dir, case[1] + ".bin"), dtype="<i2")
    want = expected(case, seed)
    if got.size != want.size:
        return max(got.size, want.size)
    return int(np.count_nonzero(got != want))
