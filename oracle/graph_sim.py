"""Graph-level oracles for the scheduler -- TEST INFRASTRUCTURE ONLY.

Two checkers for a scheduled ONNX graph (``cormorant_amd.scheduler.OnnxGraph``):

* ``forward_pass`` restates the reference scheduler's float64 simulation
  (inference-scheduler/src/codegen/_simulate.py:271-383): weights quantised
  with round-to-nearest (dtype.py:266-268), every node computed in float64 and
  narrowed with ``truncate`` (``truncate_div`` for Div), Reshape as a view.  It
  walks the graph's nodes and ignores the buffer plan entirely, so it checks
  layouts, strides, aliases and the kernels at once.  It agrees with the
  kernels wherever no 32-bit accumulator wraps (see numpy_sim).

* ``run_plan`` executes the scheduler's kernel-call list with the C-simulation
  kernels of ``libcm_oracle.so`` on host buffers laid out exactly like the
  device pool, inputs and outputs: the bit-exact expectation for the HIP
  backend, including accumulator wrap.
"""
from __future__ import annotations

from typing import Dict

import numpy as np

from . import numpy_sim as ns
import oracle as _ora


def forward_pass(graph, inputs: Dict[str, np.ndarray]) -> Dict[str, np.ndarray]:
    """{tensor: float64 array} for every tensor visited; inputs are float64 values."""
    from cormorant_amd.scheduler.nodes import (ConvNode, MatmulNode, PoolNode, ReshapeNode)
    arrays: Dict[str, np.ndarray] = {}
    for t in graph.weight_tensors:
        arrays[t.onnx_name] = ns.quantize(t.data.reshape(t.shape).astype(np.float64))
    arrays.update({k: np.asarray(v, dtype=np.float64) for k, v in inputs.items()})
    for sn in graph.nodes:
        out = sn.output
        if isinstance(sn, MatmulNode):
            a = arrays[sn.inputs[0].onnx_name]
            b = arrays[sn.inputs[1].onnx_name]
            arrays[out.onnx_name] = ns.matmul(a, b).reshape(out.shape)
        elif isinstance(sn, ConvNode):
            bias = arrays[sn.inputs[2].onnx_name] if sn.has_bias else None
            arrays[out.onnx_name] = ns.conv2d(
                arrays[sn.inputs[0].onnx_name], arrays[sn.inputs[1].onnx_name], bias,
                sn.stride_h, sn.stride_w, sn.pad_top, sn.pad_left, sn.dilation_h,
                sn.dilation_w, sn.out_h, sn.out_w, sn.is_depthwise).reshape(out.shape)
        elif isinstance(sn, ReshapeNode):
            arrays[out.onnx_name] = arrays[sn.inputs[0].onnx_name].reshape(out.shape)
        elif isinstance(sn, PoolNode):
            arrays[out.onnx_name] = ns.pool2d(
                arrays[sn.inputs[0].onnx_name], sn.pool_h, sn.pool_w, sn.stride_h, sn.stride_w,
                sn.pad_top, sn.pad_left, sn.dil_h, sn.dil_w, sn.out_h, sn.out_w, sn.pool_type,
                sn.lp_order, sn.count_include_pad).reshape(out.shape)
        else:
            a = arrays[sn.inputs[0].onnx_name]
            b = arrays[sn.inputs[1].onnx_name] if sn.arity == 2 else None
            arrays[out.onnx_name] = ns.elementwise(sn.op_code, a, b).reshape(out.shape)
    return arrays


def simulate_raw(graph, feeds_raw: Dict[str, np.ndarray]) -> Dict[str, np.ndarray]:
    """forward_pass on raw int16 inputs; graph outputs returned as raw int16."""
    arrays = forward_pass(graph, {k: ns.to_float(v) for k, v in feeds_raw.items()})
    return {t.onnx_name: ns.to_raw(arrays[t.onnx_name]) for t in graph.output_tensors}


def run_plan(plan, feeds_raw: Dict[str, np.ndarray], threads: bool = True,
             launches=None) -> Dict[str, np.ndarray]:
    """Execute plan.calls with the C-simulation kernels; graph outputs as raw int16.

    ``launches`` (a backend launch list: calls and fused groups) is executed
    instead when given: a fused group runs its calls in order with every
    intermediate of the group in a private scratch array, i.e. never in the
    plan's storage -- what the fused GPU epilogue does."""
    bufs = {("pool", ""): plan.pool_image() if plan.pool_elems else np.zeros(1, np.int16)}
    for t in plan.graph.input_tensors:
        b = np.zeros(plan.layouts[t.onnx_name].alloc, dtype=np.int16)
        plan.scatter(t.onnx_name, feeds_raw[t.onnx_name], b)
        bufs[("input", t.onnx_name)] = b
    for t in plan.graph.output_tensors:
        bufs[("output", t.onnx_name)] = np.zeros(plan.layouts[t.onnx_name].alloc, np.int16)

    def view(name, extra=0):
        if name is None:
            return None
        st = plan.storage[name]
        base = bufs[(st.kind, st.key)]
        start = st.offset + extra
        return base[start:start + max(st.capacity - extra, 0)]

    def execute(call, view):
        offs = call.offsets or (0,) * len(call.tensors)
        v = [view(n, o) for n, o in zip(call.tensors, offs)]
        a = call.args
        if call.kernel == "op":
            _ora.vectorop(v[0], v[1], v[2], *a, threads=threads)
        elif call.kernel in ("matmul", "matmul_at"):
            _ora.matmul(v[0], v[1], v[2], *a, threads=threads)
        elif call.kernel == "conv":
            _ora.conv(v[0], v[1], v[2], v[3], *a, threads=threads)
        elif call.kernel == "pool":
            _ora.pool(v[0], v[1], *a, threads=threads)
        else:
            raise ValueError(call.kernel)

    for item in ([c for _, c in plan.calls] if launches is None else launches):
        if not hasattr(item, "absorbed"):
            execute(item, view)
            continue
        chain = (item.call,) + tuple(item.absorbed)
        scratch = {}
        for c in chain[:-1]:
            out = c.tensors[3] if c.kernel == "conv" else c.tensors[-1]
            scratch[out] = np.full(plan.storage[out].capacity, 0x5A5A, np.int16)

        def fused_view(name, extra=0, scratch=scratch):
            return scratch[name][extra:] if name in scratch else view(name, extra)
        for c in chain:
            execute(c, fused_view)
    return {t.onnx_name: plan.gather(t.onnx_name, bufs[("output", t.onnx_name)])
            for t in plan.graph.output_tensors}
