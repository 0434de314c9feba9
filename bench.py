"""Benchmark of the MI355X Q8.8 kernels.

Output: one JSON line per result record ({"record": name, ...}) and per
reference case ({"record": "perf_case", ...}), as the reference's bench
programs print one line per case, then the headline line LAST: the contract's
fields, `roofline`, `cpu_baseline`, `host` and a `summary` of every
configuration, kept under 4,000 bytes.

Headline workload (the headline metric's vector-op configuration): one step is
the six-op VectorOP sweep -- Add, Sub, Mul, Div, Relu, Clip(0,6) -- over
67,108,864-element int16 Q8.8 tensors (70% uniform over [-8, 8), 30% pinned at
the saturation edges), every op with its own operand buffers (2.3 GB touched
per step, far beyond the 256 MB Infinity Cache).  `value` is the aggregate
GB/s of the step with the reference formula ports * elements * 2 B / time,
ports = 3 for binary and 2 for unary ops (bench_src/bench_vectorop.c:93-95).

The same run also reports, as record lines:
* the GEMM configurations and the conv + pool block: Q8.8 GOP/s = 2*MAC / t
  (bench_matmul.c:95, bench_conv.c:129-132) with the int8-MFMA utilisation of
  the four limb products; conv A and conv B, then MaxPool / AvgPool / LpPool /
  GlobalAveragePool on each convolution's own output, pool GB/s = (x + y) * 2 B
  / t (bench_pool.c:116-117) with rotating inputs larger than the Infinity
  Cache, next to two copies of the same byte count timed the same way -- VectorOP's
  copy opcode and a device-to-device hipMemcpyAsync -- the faster of which is the
  streaming ceiling at that size (`frac_of_copy_ceiling`);
* the two ONNX graphs run by the scheduler's HIP backend: the MLP's batch-64
  latency and the MobileNetV2-like graph's images/s at batch 16, each with its
  roofline fraction: the sum over the launches that run of each launch's bound
  (bytes it moves at 8 TB/s, or its MACs' four limb products at 5 POP/s) over the
  measured time, beside the per-op form (every ONNX node's call alone);
* `perf_cases`: the reference's per-kernel case list (perf_config.json.example
  and the published KV260 report's rows) through cm_bench, the C counterpart
  of bench_src/bench_*.c, one record per case with the reference's fields and
  the published KV260 figures beside it, every output checked against the
  oracle.
CPU figures (the oracle, a C restatement of the reference C-simulation loops, on
this host): one thread (the faithful C-simulation path, `cpu_baseline.value` and
each result's `cpu.gops` / `cpu.gbs`, the whole product) and OpenMP over the
independent outer loop (`*_mt`); both check the GPU output bit for bit; `host`
records lscpu's CPU model and the thread count.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
                       [--workloads vecop,gemm,conv,pool,graphs,cases] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "Q8.8 GOP/s (conv/GEMM), GB/s (vecop/pool); images/s MobileNet-like b16"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, 8 TB/s
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA, 5.0 POP/s
LIMB_PRODUCTS = 4              # int8 MFMA products per exact Q8.8 product
SETTLE_MS = 30.0               # untimed back-to-back runs ahead of each measurement


HEADLINE_MAX = 4000            # bytes of the last stdout line


def log(msg: str) -> None:
    sys.stderr.write(f"[bench] {msg}\n")
    sys.stderr.flush()


def emit(record: dict) -> None:
    """One result record as its own stdout line (ahead of the headline line)."""
    print(json.dumps(record, separators=(",", ":")), flush=True)


def summarize(results: dict, cases: list, cpu_res: dict) -> dict:
    """The headline line's digest of every configuration: one rate and its roofline
    fraction each (the full figures are in the record lines printed before it)."""
    s = {}
    ops = results.get("vecop", {}).get("ops", {})
    if ops:
        s["vecop_hbm_frac"] = {k: v["hbm_frac"] for k, v in ops.items()}
    for name, e in results.items():
        if name.startswith("gemm_"):
            s[name] = dict(gops=e["gops"], mfma_frac=e["mfma_frac"])
            lib = e.get("library_int8", {})
            if "mfma_frac" in lib:
                s[name]["library_int8_mfma_frac"] = lib["mfma_frac"]
        elif name.startswith("conv_"):
            s[name] = dict(gops=e["gops"], mfma_frac_issued=e["mfma_frac"],
                           frac_4product=e["frac_of_4product_roofline"])
            if e.get("packed_weights"):
                s[name]["packed_gops"] = e["packed_weights"]["gops"]
        elif "_on_conv" in name:
            s[name] = dict(gbs=e["gbs"], hbm_frac=e["hbm_frac"], of_copy=e["frac_of_copy_ceiling"])
        elif name.startswith("pool_copy_ceiling"):
            s[name] = dict(gbs=e["gbs"], hbm_frac=e["hbm_frac"])
        elif name in ("mlp_b64", "mobilenet_like_b16"):
            s[name] = dict(ms=e["ms_hip_graph"], images_s=e["images_s_hip_graph"],
                           roofline_frac=e["roofline_frac"], per_op_frac=e["per_op_frac"])
            if "cpu" in e:
                s[name]["cpu_images_s"] = e["cpu"]["images_s"]
        if name in cpu_res and "gops" in cpu_res[name]:
            s[name]["cpu_gops_1t"] = round(cpu_res[name]["gops"], 2)
    if cases:
        s["perf_cases"] = dict(n=len(cases), checked_vs_oracle=all(r.get("checked_vs_oracle")
                                                                   for r in cases))
    return s


def settle(run_once, min_ms: float = SETTLE_MS, max_runs: int = 100000) -> None:
    """Run `run_once` back to back, untimed, for at least `min_ms` of wall time
    (synchronising every few runs, so that the time is the GPU's): the engine clock
    climbs for a few milliseconds after an idle stretch (host-side checks between
    the measurements), and a measurement taken on the ramp reads 5-10 % slow."""
    import torch
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    runs = 0
    while (time.perf_counter() - t0) * 1e3 < min_ms and runs < max_runs:
        run_once()
        runs += 1
        if runs % 4 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def time_launches(calls, steps: int) -> float:
    """Mean duration (ms) of one launch: HIP events on the launch stream (torch's
    current stream, which the C-ABI wrappers use) bracket `steps` back-to-back
    launches, cycling through `calls`, after the clock has settled under the same
    launches."""
    import torch

    def once():
        for c in calls:
            c()
    settle(once)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        calls[i % len(calls)]()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def time_graph(calls, steps: int) -> float:
    """Mean duration (ms) of one launch with host overhead removed: `steps`
    launches (cycling through `calls`) are captured into one HIP graph, which is
    replayed untimed until the clock has settled and then once between HIP events.  The calls run once
    eagerly on the capture stream first."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for c in calls:
            c()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for i in range(steps):
            calls[i % len(calls)]()
    settle(graph.replay)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


# ------------------------------------------------------------------ vecop --
def setup_vecop():
    from cormorant_amd import workloads as wl
    import torch
    bufs = []
    for name, op in wl.VECOP_OPS:
        a = wl.vecop_operand(wl.VECOP_N, op, 0)
        b = wl.vecop_operand(wl.VECOP_N, op, 1) if op < 4 else None
        bufs.append(dict(name=name, op=op, a=dev(a), b=dev(b) if b is not None else None,
                         c=torch.empty(wl.VECOP_N, dtype=torch.int16, device="cuda"),
                         a_host=a, b_host=b))
    return bufs


def vecop_bytes(op: int, n: int) -> int:
    return (3 if op < 4 else 2) * n * 2


def vecop_call(bf):
    from cormorant_amd import kernels as K
    return lambda: K.VectorOPKernel(bf["a"], bf["b"], bf["c"], bf["a"].numel(), bf["op"])


def run_vecop_step(bufs):
    for bf in bufs:
        vecop_call(bf)()


# ------------------------------------------------------------------- gemm --
def bench_gemm(steps: int, warmup: int):
    import torch
    from cormorant_amd import kernels as K
    from cormorant_amd import workloads as wl
    out = {}
    for cid, case in enumerate(wl.GEMM_CASES):
        a, b = wl.gemm_operands(case, cid)
        da, db = dev(a), dev(b)
        dc = torch.empty(case.batch * case.n * case.m, dtype=torch.int16, device="cuda")
        # the caller-owned workspace the call uses (the packed B of the direct-to-LDS path)
        need = K.matmul_workspace_size(case.n, case.k, case.m, case.batch, case.n * case.k,
                                       case.k * case.m, case.n * case.m)
        ws = torch.empty(max(need, 4) // 4, dtype=torch.int32, device="cuda")
        fn = lambda: K.MatmulKernel(da, db, dc, case.n, case.k, case.m, case.batch,
                                    case.n * case.k, case.k * case.m, case.n * case.m, workspace=ws)
        for _ in range(warmup):
            fn()
        ms = time_launches([fn], steps)
        gops = 2.0 * case.macs / (ms * 1e-3) / 1e9
        out[case.name] = dict(
            shape=f"batch {case.batch}, {case.n}x{case.k}x{case.m}, U[{case.lo},{case.hi})",
            ms=round(ms, 5), gops=round(gops, 1),
            mfma_int8_tops=round(LIMB_PRODUCTS * gops / 1e3, 2),
            mfma_frac=round(LIMB_PRODUCTS * gops / 1e3 / INT8_PEAK_TOPS, 4),
            workspace_bytes=need,
            kernel="gemm_bpack + gemm_dma (B packed per call, A streamed into LDS)" if need
            else "q88_gemm (dense)")
        out[case.name]["library_int8"] = library_int8_gemm(case, steps)
        out[case.name]["_dev"] = (da, db, dc, a, b)
    return out


def library_int8_gemm(case, steps: int):
    """The platform's own int8 GEMM rate at the case's shape: torch._int_mm
    (hipBLASLt) on random int8 operands, B column-major (its faster layout), one
    call per batch.  It computes ONE int8 product per MAC where the exact Q8.8
    kernel issues four, so its MFMA fraction is the practical ceiling for an
    MFMA fraction at this shape."""
    import torch
    try:
        g = torch.Generator(device="cuda").manual_seed(7)
        a8 = torch.randint(-128, 128, (case.n, case.k), dtype=torch.int8, device="cuda", generator=g)
        b8 = torch.randint(-128, 128, (case.m, case.k), dtype=torch.int8, device="cuda", generator=g).t()
        fn = lambda: torch._int_mm(a8, b8)
        for _ in range(3):
            fn()
        # as a HIP graph: a 1024^3 call is short enough for host launch costs to dominate
        ms = time_graph([fn], steps * case.batch) * case.batch
    except (RuntimeError, AttributeError) as ex:   # no int8 GEMM in this torch build
        return dict(kernel="torch._int_mm", error=str(ex)[:200])
    tops = 2.0 * case.macs / (ms * 1e-3) / 1e12
    return dict(kernel="torch._int_mm (hipBLASLt), int8 x int8 -> int32, B column-major, "
                       "one call per batch in a HIP graph",
                ms=round(ms, 5), int8_tops=round(tops, 1), mfma_frac=round(tops / INT8_PEAK_TOPS, 4))


# ------------------------------------------------------- conv + pool block --
MALL_BYTES = 256 << 20      # MI355X Infinity Cache: rotating inputs must exceed it
POOL_ROTATE_MIN = 12


def bench_block(steps: int, warmup: int):
    """Conv A and conv B (each timed as a HIP graph of back-to-back calls on one
    input: per call with the weight pack, with weights packed once, and with
    full-range weights), then the four pools on
    each convolution's own device output.  Pool inputs rotate over copies of that
    output totalling more than the Infinity Cache, timed as a HIP graph of
    back-to-back launches, next to a VectorOP copy of the same byte count timed
    the same way (the streaming ceiling at that size)."""
    import torch
    from cormorant_amd import kernels as K
    from cormorant_amd import workloads as wl
    out = {}
    x, w, b = wl.conv_operands(wl.CONV_CASES[0])
    dx, dw_, db = dev(x), dev(w), dev(b)
    conv_out = {}
    for case in wl.CONV_CASES:
        o = case.out_hw
        dy = torch.empty(case.batch * case.out_ch * o * o, dtype=torch.int16, device="cuda")
        args = (case.batch, case.in_ch, case.hw, case.hw, case.out_ch, o, o, case.k, case.k,
                case.stride, case.stride, case.dil, case.dil, case.pad, case.pad, 1, 0)
        need = K.conv_workspace_size(*args)   # the caller-owned scratch the call uses
        ws = torch.empty(max(need, 4) // 4, dtype=torch.int32, device="cuda")
        fn = lambda args=args, dy=dy, ws=ws: K.ConvKernel(dx, dw_, db, dy, *args, workspace=ws)
        for _ in range(warmup):
            fn()
        # a HIP graph of back-to-back calls: a conv call is shorter than the
        # host's issue time for it through the Python wrapper
        ms = time_graph([fn], steps)
        gops = 2.0 * case.macs / (ms * 1e-3) / 1e9
        # weights N(0, 0.05) all lie in [-128, 127] raw: the exact two-product path
        products = 2 if int(w.min()) >= -128 and int(w.max()) <= 127 else LIMB_PRODUCTS
        # the same call with full-range weights (every tile on the four-product path)
        wf = wl.rng(4, 7).integers(-32768, 32768, w.size, dtype=np.int16)
        dwf = dev(wf)
        dyf = torch.empty_like(dy)   # dy keeps the checked output of the N(0, 0.05) weights
        fnf = lambda args=args, dyf=dyf, ws=ws: K.ConvKernel(dx, dwf, db, dyf, *args, workspace=ws)
        for _ in range(warmup):
            fnf()
        msf = time_graph([fnf], steps)
        gopsf = 2.0 * case.macs / (msf * 1e-3) / 1e9
        # weights packed once (cm_conv_pack), then cm_conv_packed_ex per call: what the
        # inference session runs for constant weights; its output must equal the
        # per-call path's bit for bit
        packed_res = None
        psize = K.conv_packed_size(*args)
        if psize:
            packed = torch.empty(-(-psize // 4), dtype=torch.int32, device="cuda")
            K.conv_pack(dw_, packed, *args)
            dyp = torch.empty_like(dy)
            fnp = lambda args=args, dyp=dyp, packed=packed: K.ConvPackedKernel(dx, packed, db, dyp, *args)
            for _ in range(warmup):
                fnp()
            msp = time_graph([fnp], steps)
            fn()
            torch.cuda.synchronize()
            if not torch.equal(dyp, dy):
                raise RuntimeError(f"{case.name}: packed-weight output differs from the per-call output")
            gopsp = 2.0 * case.macs / (msp * 1e-3) / 1e9
            packed_res = dict(ms=round(msp, 5), gops=round(gopsp, 1), limb_products=products,
                              mfma_frac=round(products * gopsp / 1e3 / INT8_PEAK_TOPS, 4),
                              frac_of_4product_roofline=round(LIMB_PRODUCTS * gopsp / 1e3 / INT8_PEAK_TOPS, 4),
                              timing="cm_conv_pack once, then cm_conv_packed_ex per call (constant "
                                     "weights, as the inference session runs them), HIP graph of "
                                     "back-to-back calls; output equal to the per-call path's")
            del packed, dyp
        out[case.name] = dict(
            shape=f"N={case.batch} C {case.in_ch}->{case.out_ch} {case.hw}x{case.hw} {case.k}x{case.k} "
                  f"s{case.stride} d{case.dil} p{case.pad} bias -> {o}x{o}",
            ms=round(ms, 5), gops=round(gops, 1),
            limb_products=products,
            mfma_int8_tops=round(products * gops / 1e3, 2),
            mfma_frac=round(products * gops / 1e3 / INT8_PEAK_TOPS, 4),
            frac_of_4product_roofline=round(LIMB_PRODUCTS * gops / 1e3 / INT8_PEAK_TOPS, 4),
            full_range_weights=dict(ms=round(msf, 5), gops=round(gopsf, 1), limb_products=LIMB_PRODUCTS,
                                    mfma_frac=round(LIMB_PRODUCTS * gopsf / 1e3 / INT8_PEAK_TOPS, 4)),
            timing="per call, weight pack included; HIP graph of back-to-back calls",
            packed_weights=packed_res,
            workspace_bytes=need)
        del dwf, dyf
        out[case.name]["_dev"] = (dx, dw_, db, dy, x, w, b)
        conv_out[case.name] = (dy, o)
    ceilings = {}
    for cv, pc, name in wl.block_pools():
        dy, o = conv_out[cv.name]
        n, c = cv.batch, cv.out_ch
        rot = max(POOL_ROTATE_MIN, -(-MALL_BYTES // (dy.numel() * 2)) + 1)
        xs = [dy] + [dy.clone() for _ in range(rot - 1)]
        a = wl.pool_args(pc, n, c, o)
        ny = n * c * a["out_h"] * a["out_w"]
        ys = [torch.empty(ny, dtype=torch.int16, device="cuda") for _ in range(rot)]
        calls = [lambda i=i: K.PoolingKernel(xs[i], ys[i], **a) for i in range(rot)]
        for i in range(warmup):
            calls[i % rot]()
        ms = time_graph(calls, max(steps, 4 * rot))
        nbytes = (dy.numel() + ny) * 2
        gbs = nbytes / (ms * 1e-3) / 1e9
        if o not in ceilings:
            # two copies of the largest pool's byte count, timed the same way: VectorOP's
            # copy opcode and the runtime's device-to-device hipMemcpyAsync (torch's copy_
            # of a contiguous same-dtype tensor); the faster one is the streaming ceiling
            ncopy = (dy.numel() + n * c * (o // 2) ** 2) // 2
            src = [t[:ncopy] for t in xs]
            dst = [torch.empty(ncopy, dtype=torch.int16, device="cuda") for _ in range(rot)]
            ccalls = [lambda i=i: K.VectorOPKernel(src[i], None, dst[i], ncopy, 6) for i in range(rot)]
            cms = time_graph(ccalls, max(steps, 4 * rot))
            mcalls = [lambda i=i: dst[i].copy_(src[i]) for i in range(rot)]
            mms = time_graph(mcalls, max(steps, 4 * rot))
            cgbs, mgbs = 4 * ncopy / (cms * 1e-3) / 1e9, 4 * ncopy / (mms * 1e-3) / 1e9
            ceilings[o] = dict(bytes=4 * ncopy, rotating_inputs=rot,
                               vecop_copy=dict(ms=round(cms, 5), gbs=round(cgbs, 1),
                                               hbm_frac=round(cgbs / HBM_PEAK_GBS, 4),
                                               kernel="vecop_flat<6>"),
                               hip_memcpy_d2d=dict(ms=round(mms, 5), gbs=round(mgbs, 1),
                                                   hbm_frac=round(mgbs / HBM_PEAK_GBS, 4)),
                               gbs=round(max(cgbs, mgbs), 1),
                               hbm_frac=round(max(cgbs, mgbs) / HBM_PEAK_GBS, 4))
            del dst
        out[name] = dict(input=f"{cv.name} output [{n},{c},{o},{o}]", ms=round(ms, 5),
                         gbs=round(gbs, 1), hbm_frac=round(gbs / HBM_PEAK_GBS, 4), bytes=nbytes,
                         frac_of_copy_ceiling=round(gbs / ceilings[o]["gbs"], 4),
                         rotating_inputs=rot, timing="HIP graph of back-to-back launches")
        out[name]["_dev"] = (dy, ys[0], a)
        del xs
    for o, cl in ceilings.items():
        out[f"pool_copy_ceiling_{o}x{o}"] = cl
    return out


# ----------------------------------------------------------------- graphs --
def call_macs(call) -> int:
    a = call.args
    if call.kernel in ("matmul", "matmul_at"):
        return a[0] * a[1] * a[2] * a[3]
    if call.kernel == "conv":
        nb, c, _, _, mo, oh, ow, kh, kw = a[:9]
        return nb * mo * oh * ow * (1 if a[16] else c) * kh * kw
    return 0


def bound_s(nbytes: int, macs: int) -> float:
    """max(HBM time of the bytes, int8-MFMA time of the four limb products per MAC)."""
    return max(nbytes / (HBM_PEAK_GBS * 1e9), LIMB_PRODUCTS * 2 * macs / (INT8_PEAK_TOPS * 1e12))


def graph_lower_bound_s(plan) -> float:
    """Per-op bound: the sum over the reference's kernel calls (one per ONNX node, every
    intermediate through memory) of each call's bound."""
    return sum(bound_s(2 * sum(c.extents().values()), call_macs(c)) for _, c in plan.calls)


def launch_members(item):
    """The kernel calls one launch of the session runs, in order."""
    from cormorant_amd.scheduler import fuse
    if isinstance(item, (fuse.FusedCall, fuse.PairCall, fuse.GapCall)):
        return (item.call,) + tuple(item.absorbed)
    return (item,)


def launch_lower_bound_s(launch_list) -> float:
    """Fused bound: the sum over the launches that actually run of max(HBM time of the
    bytes the launch must move, MFMA time of its MACs).  A launch's bytes are the
    tensors its member calls read that no member writes, plus the tensor it leaves in
    memory; intermediates kept on chip (fused epilogues, a convolution pair's middle
    tensor, the output a fused GlobalAveragePool reduces) count for nothing."""
    from cormorant_amd.scheduler import fuse
    total = 0.0
    for item in launch_list:
        members = launch_members(item)
        written = {fuse._writes(c) for c in members}
        out = item.out if isinstance(item, (fuse.FusedCall, fuse.PairCall, fuse.GapCall)) else fuse._writes(item)
        need = {}
        for c in members:
            ext = c.extents()
            for name in fuse._reads(c):
                if name not in written:
                    need[name] = max(need.get(name, 0), ext[name])
        need[out] = members[-1].extents()[out]
        total += bound_s(2 * sum(need.values()), sum(call_macs(c) for c in members))
    return total


def bench_graphs(steps: int, warmup: int, check: bool):
    """Config 1 (MLP b64 latency) and config 5 (MobileNetV2-like b16 images/s) through
    the scheduler's HIP backend, inputs resident on the device."""
    import torch
    from cormorant_amd import workloads as wl
    from cormorant_amd.scheduler import InferenceSession, OnnxGraph, onnx_io as ox
    out = {}
    cases = (("mlp_b64", wl.mlp_model(), wl.mlp_input(), wl.MLP_BATCH),
             ("mobilenet_like_b16", wl.mobilenet_model(), wl.mobilenet_input(),
              wl.MOBILENET_BATCH))
    for name, model, x, batch in cases:
        g = OnnxGraph(ox.encode_model(model))
        sess = InferenceSession(g)
        sess.write_input("X", x)
        cur = lambda: torch.cuda.current_stream().cuda_stream
        launch = lambda: sess.launch(cur())
        for _ in range(warmup):
            launch()
        torch.cuda.synchronize()
        ms = time_launches([launch], steps)
        ms_graph = time_graph([launch], max(steps, 4))
        macs = sum(call_macs(c) for _, c in sess.plan.calls)
        lb = graph_lower_bound_s(sess.plan)
        lbf = launch_lower_bound_s(sess.launch_list)
        e = dict(kernel_calls=len(sess.plan.calls), launches=len(sess.launch_list),
                 gmac=round(macs / 1e9, 4),
                 ms=round(ms, 4), ms_hip_graph=round(ms_graph, 4),
                 images_s=round(batch / (ms * 1e-3), 1),
                 images_s_hip_graph=round(batch / (ms_graph * 1e-3), 1),
                 gops=round(2 * macs / (ms_graph * 1e-3) / 1e9, 1),
                 roofline_lower_bound_ms=round(lbf * 1e3, 4),
                 roofline_frac=round(lbf * 1e3 / ms_graph, 4),
                 roofline_bound="sum over the launches that run of max(bytes each moves / 8 TB/s, "
                                "4 limb products x 2 x MACs / 5 POP/s)",
                 per_op_lower_bound_ms=round(lb * 1e3, 4),
                 per_op_frac=round(lb * 1e3 / ms_graph, 4),
                 pool_bytes=2 * sess.plan.pool_elems)
        y = sess.read_output("Y")
        if check:
            import oracle
            from oracle import graph_sim as gs
            threads = host_threads()
            oracle.set_threads(threads)
            t0 = time.perf_counter()
            want = gs.run_plan(sess.plan, {"X": x}, threads=True)["Y"]
            dt = time.perf_counter() - t0
            if not np.array_equal(y, want):
                raise SystemExit(f"bench: GPU {name} output differs from the oracle")
            e["cpu"] = dict(ms=round(dt * 1e3, 2), images_s=round(batch / dt, 2), cores=threads,
                            kind="port", sample="whole graph, kernel-call list on the oracle, "
                                                "OpenMP over each kernel's outer loop")
        sess.close()
        out[name] = e
    return out


# ------------------------------------------------------------ cpu baseline --
def host_threads() -> int:
    """OpenMP threads for the multi-thread CPU figures: the CPUs this process may
    run on, at most 16."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def host_info() -> dict:
    """CPU identity: `lscpu`'s model name, with the x86 family / model / stepping
    numbers (a virtual machine may report only a vendor string as the name)."""
    import subprocess
    info = {}
    try:
        r = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10,
                           env=dict(os.environ, LC_ALL="C"))
        for line in r.stdout.splitlines():
            key, _, val = line.partition(":")
            info[key.strip()] = val.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    if "Model name" not in info:
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        info["Model name"] = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
    return dict(cpu_model=info.get("Model name"), cpu_family=info.get("CPU family"),
                cpu_model_number=info.get("Model"), stepping=info.get("Stepping"),
                logical_cpus=os.cpu_count(), omp_threads=host_threads())


def cpu_baseline(vec_bufs, extras: dict):
    """The oracle (C restatement of the reference C-simulation loops, -O2) timed
    on this host on a bounded sample: single thread (the faithful C-simulation
    path; this run also checks the GPU outputs of that sample bit-for-bit), and
    with OpenMP over the independent outer loop (`*_mt`, host_threads() threads)."""
    import oracle
    mt = host_threads()
    oracle.set_threads(1)
    res = {}
    # VectorOP: the whole 64Mi sweep, one thread
    t_total, bytes_total = 0.0, 0
    for bf in vec_bufs:
        want = np.empty(bf["a_host"].size, np.int16)
        b = bf["b_host"] if bf["b_host"] is not None else np.zeros(1, np.int16)
        t0 = time.perf_counter()
        oracle.vectorop(bf["a_host"], b, want, want.size, bf["op"])
        t_total += time.perf_counter() - t0
        bytes_total += vecop_bytes(bf["op"], want.size)
        got = bf["c"].cpu().numpy()
        if not np.array_equal(got, want):
            raise SystemExit(f"bench: GPU {bf['name']} output differs from the oracle")
    res["vecop"] = dict(gbs=bytes_total / t_total / 1e9, seconds=t_total)
    oracle.set_threads(mt)
    t_mt = 0.0
    for bf in vec_bufs:
        want = np.empty(bf["a_host"].size, np.int16)
        b = bf["b_host"] if bf["b_host"] is not None else np.zeros(1, np.int16)
        t0 = time.perf_counter()
        oracle.vectorop(bf["a_host"], b, want, want.size, bf["op"], threads=True)
        t_mt += time.perf_counter() - t0
    res["vecop"].update(gbs_mt=bytes_total / t_mt / 1e9, seconds_mt=t_mt, threads_mt=mt)
    oracle.set_threads(1)
    # GEMM / conv: the whole product on one thread (the faithful C-simulation path,
    # ~45 s over the four products) and with OpenMP; both check the GPU output bit
    # for bit
    from cormorant_amd import workloads as wl

    def timed(fn, threads):
        oracle.set_threads(threads)
        t0 = time.perf_counter()
        fn()
        dt = time.perf_counter() - t0
        oracle.set_threads(1)
        return dt

    for cid, case in enumerate(wl.GEMM_CASES):
        if case.name not in extras:
            continue
        da, db, dc, a, b = extras[case.name].pop("_dev")
        n, k, m, bt = case.n, case.k, case.m, case.batch
        a1, b1 = np.ascontiguousarray(a).reshape(-1), np.ascontiguousarray(b).reshape(-1)
        want = np.empty(bt * n * m, np.int16)
        dt_mt = timed(lambda: oracle.matmul(a1, b1, want, n, k, m, bt, n * k, k * m, n * m,
                                            threads=True), mt)
        if not np.array_equal(dc.cpu().numpy(), want):
            raise SystemExit(f"bench: GPU {case.name} differs from the oracle")
        log(f"CPU baseline: {case.name} on one thread (whole product)")
        one = np.empty_like(want)
        dt_1 = timed(lambda: oracle.matmul(a1, b1, one, n, k, m, bt, n * k, k * m, n * m), 1)
        if not np.array_equal(one, want):
            raise SystemExit(f"bench: {case.name} one-thread oracle run differs")
        res[case.name] = dict(gops=2.0 * case.macs / dt_1 / 1e9, seconds=dt_1,
                              sample="the whole product, one thread, checked bit for bit",
                              gops_mt=2.0 * case.macs / dt_mt / 1e9, seconds_mt=dt_mt,
                              threads_mt=mt, sample_mt="the whole product, checked bit for bit")
    for case in wl.CONV_CASES:
        if case.name not in extras:
            continue
        dx, dw_, db_, dy, x, w, b = extras[case.name].pop("_dev")
        o = case.out_hw
        args = (case.in_ch, case.hw, case.hw, case.out_ch, o, o, case.k, case.k, case.stride,
                case.stride, case.dil, case.dil, case.pad, case.pad, 1, 0)
        x1, w1 = np.ascontiguousarray(x).reshape(-1), w.reshape(-1)
        want = np.empty(case.batch * case.out_ch * o * o, np.int16)
        dt_mt = timed(lambda: oracle.conv(x1, w1, b, want, case.batch, *args, threads=True), mt)
        if not np.array_equal(dy.cpu().numpy(), want):
            raise SystemExit(f"bench: GPU {case.name} differs from the oracle")
        log(f"CPU baseline: {case.name} on one thread (all 32 images)")
        one = np.empty_like(want)
        dt_1 = timed(lambda: oracle.conv(x1, w1, b, one, case.batch, *args), 1)
        if not np.array_equal(one, want):
            raise SystemExit(f"bench: {case.name} one-thread oracle run differs")
        res[case.name] = dict(gops=2.0 * case.macs / dt_1 / 1e9, seconds=dt_1,
                              sample="all 32 images, one thread, checked bit for bit",
                              gops_mt=2.0 * case.macs / dt_mt / 1e9, seconds_mt=dt_mt,
                              threads_mt=mt, sample_mt="all 32 images, checked bit for bit")
    for name, e in list(extras.items()):
        if "_on_conv" not in name:
            continue
        x, y, a = e.pop("_dev")
        xh = x.cpu().numpy()
        want = np.empty(y.numel(), np.int16)
        pargs = tuple(a.values())
        dt_1 = timed(lambda: oracle.pool(xh, want, *pargs), 1)
        if not np.array_equal(y.cpu().numpy(), want):
            raise SystemExit(f"bench: GPU {name} differs from the oracle")
        dt_mt = timed(lambda: oracle.pool(xh, want, *pargs, threads=True), mt)
        res[name] = dict(gbs=(xh.size + want.size) * 2 / dt_1 / 1e9, seconds=dt_1,
                         sample="full tensor, one thread",
                         gbs_mt=(xh.size + want.size) * 2 / dt_mt / 1e9, seconds_mt=dt_mt,
                         threads_mt=mt)
    return res


# ------------------------------------------------------ per-case harness --
def bench_cases(dump_dir: str | None):
    """The reference's per-kernel case list (perf_config.json.example plus the published
    report's rows) through cm_bench, the C counterpart of bench_src/bench_*.c: one JSON
    line per case with the reference's fields, the published KV260 figures beside it."""
    import subprocess
    from cormorant_amd import build as hipbuild
    from cormorant_amd.bench_src import perf_cases as pc
    if not os.path.exists(hipbuild.BENCH_BIN):
        raise SystemExit(f"bench: {hipbuild.BENCH_BIN} is missing (run the build)")
    lines = "\n".join(pc.case_line(c) for c in pc.CASES) + "\n"
    env = dict(os.environ)
    if dump_dir:
        env["CM_BENCH_DUMP"] = dump_dir
    r = subprocess.run([hipbuild.BENCH_BIN, "-"], input=lines, capture_output=True, text=True,
                       timeout=600, env=env)
    if r.returncode != 0:
        raise SystemExit(f"bench: cm_bench failed ({r.returncode}): {r.stderr[-2000:]}")
    rows = [json.loads(l) for l in r.stdout.splitlines() if l.startswith("{")]
    for case, row in zip(pc.CASES, rows):
        kv = case[5]
        if kv is not None:
            metric = "gbs" if case[0] in ("vectorop", "pool") else "gops"
            row["kv260"] = {"lat_ms": kv[0], metric: kv[1]}
            row["speedup_vs_kv260"] = round(kv[0] / row["lat_ms"], 1)
    return rows


def load_traffic(kernel: str):
    """Calibrated HBM bytes per launch of `kernel` (FETCH_SIZE + WRITE_SIZE, each scaled by
    the factor the same counter reads for the copy kernel) from the committed PMC summary."""
    p = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(p) as f:
            entry = json.load(f)["kernels"].get(kernel)
    except (OSError, ValueError, KeyError):
        return None
    return None if entry is None else entry.get("traffic_bytes")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--quick", action="store_true", help="headline workload only, no CPU baseline")
    ap.add_argument("--workloads", default="vecop,gemm,conv,pool,graphs,cases",
                    help="comma list of vecop (always run: the headline), gemm, conv, pool "
                         "(conv and pool: the conv + pool block), graphs, cases (the "
                         "reference's per-kernel case list through cm_bench)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()
    work = set(args.workloads.split(","))
    if args.quick:
        work, args.no_cpu = {"vecop"}, True
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X; multi-GPU runs are not part of it "
              "(--gpus must be 1).", file=sys.stderr)
        return 2

    import torch
    from cormorant_amd import _native
    _native.load()
    torch.cuda.set_device(0)

    log("generating the 64Mi-element VectorOP operands")
    bufs = setup_vecop()
    for _ in range(args.warmup):
        run_vecop_step(bufs)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run_vecop_step(bufs)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    from cormorant_amd import workloads as wl
    step_bytes = sum(vecop_bytes(op, wl.VECOP_N) for _, op in wl.VECOP_OPS)
    per_op = {}
    for bf in bufs:   # each op alone: its average launch duration
        ms = time_launches([vecop_call(bf)], max(args.steps, 10))
        gbs = vecop_bytes(bf["op"], wl.VECOP_N) / (ms * 1e-3) / 1e9
        per_op[bf["name"]] = dict(ms=round(ms, 5), gbs=round(gbs, 1), hbm_frac=round(gbs / HBM_PEAK_GBS, 4))
    # copy calibration: VectorOP's copy opcode (op >= 6 copies a) over the same 64 Mi
    # elements -- the streaming ceiling at this size, and the PMC byte-count reference
    from cormorant_amd import kernels as K
    src = bufs[0]["a"]
    dst = torch.empty_like(src)       # its own output: the sweep's outputs are checked later
    copy_ms = time_launches([lambda: K.VectorOPKernel(src, None, dst, src.numel(), 6)],
                            max(args.steps, 10))
    del dst
    copy_gbs = vecop_bytes(6, wl.VECOP_N) / (copy_ms * 1e-3) / 1e9
    kernel_ms = sum(v["ms"] for v in per_op.values())
    ms_per_step = wall * 1e3 / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    dom_name = max(per_op, key=lambda k: per_op[k]["ms"])
    dom_op = dict(wl.VECOP_OPS)[dom_name]
    dom_kernel = f"vecop_flat<{dom_op}>"
    traffic = load_traffic(dom_kernel)
    roofline = dict(bound="hbm", achieved=per_op[dom_name]["gbs"], peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=per_op[dom_name]["hbm_frac"], traffic=traffic,
                    kernel=dom_kernel, op=dom_name,
                    bytes_per_launch=vecop_bytes(dom_op, wl.VECOP_N))

    results = dict(vecop=dict(ops=per_op, kernel_ms_per_step=round(kernel_ms, 5),
                              copy_ceiling=dict(ms=round(copy_ms, 5), gbs=round(copy_gbs, 1),
                                                hbm_frac=round(copy_gbs / HBM_PEAK_GBS, 4),
                                                kernel="vecop_flat<6>",
                                                bytes_per_launch=vecop_bytes(6, wl.VECOP_N))))
    cpu = None
    extras, graphs = {}, {}
    if "gemm" in work:
        log("GEMM configurations")
        extras.update(bench_gemm(max(5, args.steps // 2), 2))
    if "conv" in work or "pool" in work:
        log("conv + pool block: conv A, conv B, four pools on each output")
        extras.update(bench_block(max(5, args.steps // 2), 2))
    cases = []
    dump_dir = None
    if "cases" in work:
        import tempfile
        log("reference per-case list through cm_bench")
        dump_dir = None if args.no_cpu else tempfile.mkdtemp(prefix="cm_bench_")
        cases = bench_cases(dump_dir)
    if "graphs" in work:
        log("scheduler graphs: MLP b64, MobileNetV2-like b16")
        graphs = bench_graphs(max(5, args.steps // 2), 2, check=not args.no_cpu)
    cpu_res = {}
    if not args.no_cpu:
        log("CPU baseline (oracle, 1 thread and OpenMP) and sample check")
        cpu_res = cpu_baseline(bufs, extras)
        v = cpu_res["vecop"]
        cpu = dict(value=round(v["gbs"], 3), unit="GB/s", cores=1, kind="port",
                   sample="the full six-op 64Mi-element sweep, oracle C restatement -O2, one thread",
                   seconds=round(v["seconds"], 3),
                   value_mt=round(v["gbs_mt"], 3), cores_mt=v["threads_mt"],
                   seconds_mt=round(v["seconds_mt"], 3))
    if cases and dump_dir:
        from cormorant_amd.bench_src import perf_cases as pc
        from oracle import bench_cases as bc
        oracle_threads = host_threads()
        import oracle
        oracle.set_threads(oracle_threads)
        for case, row in zip(pc.CASES, cases):
            n_bad = bc.check_dump(case, dump_dir, seed=row["seed"])
            if n_bad:
                raise SystemExit(f"bench: cm_bench case {case[1]} differs from the oracle "
                                 f"in {n_bad} elements")
            row["checked_vs_oracle"] = True
        import shutil
        shutil.rmtree(dump_dir, ignore_errors=True)
    for name, e in extras.items():
        e.pop("_dev", None)
        if name in cpu_res:
            e["cpu"] = {k: (round(v, 4) if isinstance(v, float) else v)
                        for k, v in cpu_res[name].items()}
        results[name] = e
    results.update(graphs)

    # one JSON line per result and per reference case first (the reference's bench
    # programs print one line per case), then the compact headline line last
    for name, e in results.items():
        emit(dict(record=name, **e))
    for row in cases:
        emit(dict(record="perf_case", **row))
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int16",
        "data": "synthetic",
        "config": {
            "workload": "vecop_sweep_64Mi: Add, Sub, Mul, Div, Relu, Clip(0,6) on 67108864-element "
                        "int16 Q8.8 tensors, 70% U[-8,8) + 30% saturation edges, own buffers per op",
            "elements": wl.VECOP_N,
            "bytes_per_step": step_bytes,
            "parallelism": "single GPU",
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "host": host_info(),
        "summary": summarize(results, cases, cpu_res),
    }
    text = json.dumps(line, separators=(",", ":"))
    if len(text) > HEADLINE_MAX:     # keep the headline readable by line-tail parsers
        line["summary"] = {"dropped": f"summary over {HEADLINE_MAX} bytes; see the records above"}
        text = json.dumps(line, separators=(",", ":"))
    print(text, flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
