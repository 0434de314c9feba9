"""ONNX graph loading, Gemm decomposition and node dispatch.

Mirrors OnnxGraph of inference-scheduler/src/graph.py:79-346:

1. load the model and infer every intermediate shape;
2. split each Gemm (alpha = beta = 1, no transposes) into MatMul -> tmp and
   Add(tmp, C), the temporary named ``_gemm_mm_out_<n>`` (graph.py:100-176);
3. register every tensor (initializers with float32 data, graph inputs,
   value_info, graph outputs);
4. map each node onto its node class, in graph order.
"""
from __future__ import annotations

from typing import Dict, List, Union

import numpy as np

from . import onnx_io as ox
from .nodes import (POOL_OP_TYPES, RESHAPE_OP_TYPES, VECTOROP_OP_TYPES, ConvNode, MatmulNode,
                    PoolNode, ReshapeNode, ScheduledNode, SchedulerError)
from .shapes import ShapeError, infer_shapes
from .tensor import ALIGN_ELEMS, TensorInfo

ALL_SUPPORTED_OP_TYPES = frozenset({"MatMul", "Conv", "Gemm"}) | POOL_OP_TYPES | \
    VECTOROP_OP_TYPES | RESHAPE_OP_TYPES

_DTYPE_NAMES = {ox.FLOAT: "float32", ox.DOUBLE: "float64", ox.INT8: "int8", ox.INT16: "int16",
                ox.INT32: "int32", ox.INT64: "int64", ox.UINT8: "uint8", ox.UINT16: "uint16",
                ox.UINT32: "uint32", ox.UINT64: "uint64", ox.FLOAT16: "float16",
                ox.BOOL: "bool"}

AnyNode = Union[ScheduledNode, MatmulNode, ConvNode, PoolNode, ReshapeNode]


def _dtype_name(code: int) -> str:
    return _DTYPE_NAMES.get(code, f"onnx_dtype_{code}")


def _check_model(model: ox.Model) -> None:
    """Structural checks: every node input exists before it is used, names are unique."""
    g = model.graph
    known = {t.name for t in g.initializer} | {v.name for v in g.input}
    produced = set()
    for node in g.node:
        if node.op_type not in ALL_SUPPORTED_OP_TYPES:
            raise SchedulerError(f"{node.op_type} node '{node.name or node.op_type}' is not "
                                 f"supported; supported ops: {sorted(ALL_SUPPORTED_OP_TYPES)}")
        for x in node.input:
            if x and x not in known:
                raise SchedulerError(
                    f"{node.op_type} node '{node.name}' reads '{x}', which is neither a graph "
                    f"input, an initializer nor an earlier node's output")
        for y in node.output:
            if not y:
                continue
            if y in produced or y in known:
                raise SchedulerError(f"tensor '{y}' is produced twice")
            produced.add(y)
            known.add(y)
    for v in g.output:
        if v.name not in known:
            raise SchedulerError(f"graph output '{v.name}' is never produced")


def split_gemms(model: ox.Model) -> ox.Model:
    """Gemm(A, B[, C]) -> MatMul(A, B) [-> Add(., C)] (graph.py:100-176)."""
    g = model.graph
    shapes: Dict[str, List[int]] = {t.name: list(t.dims) for t in g.initializer}
    for vi in list(g.input) + list(g.value_info) + list(g.output):
        if vi.shape is not None:
            shapes[vi.name] = [d if d >= 0 else 0 for d in vi.shape]
    count = 0
    nodes: List[ox.Node] = []
    for node in g.node:
        if node.op_type != "Gemm":
            nodes.append(node)
            continue
        at = node.attribute
        alpha = at["alpha"].f if "alpha" in at else 1.0
        beta = at["beta"].f if "beta" in at else 1.0
        ta = at["transA"].i if "transA" in at else 0
        tb = at["transB"].i if "transB" in at else 0
        if abs(alpha - 1.0) > 1e-6 or abs(beta - 1.0) > 1e-6:
            raise SchedulerError(f"Gemm node '{node.name}': alpha={alpha}, beta={beta}; only "
                                 f"alpha = beta = 1 is supported")
        if ta or tb:
            raise SchedulerError(f"Gemm node '{node.name}': transA={ta}, transB={tb}; "
                                 f"transposed operands are not supported")
        count += 1
        a, b = node.input[0], node.input[1]
        c = node.input[2] if len(node.input) >= 3 and node.input[2] else None
        y = node.output[0]
        if c:
            tmp = f"_gemm_mm_out_{count}"
            sa, sb = shapes.get(a, []), shapes.get(b, [])
            if len(sa) >= 2 and len(sb) >= 2:
                g.value_info.append(ox.value_info(tmp, sa[:-1] + [sb[-1]]))
            nodes.append(ox.make_node("MatMul", [a, b], [tmp], name=f"_gemm_matmul_{count}"))
            nodes.append(ox.make_node("Add", [tmp, c], [y], name=f"_gemm_add_{count}"))
        else:
            nodes.append(ox.make_node("MatMul", [a, b], [y], name=f"_gemm_matmul_{count}"))
    g.node = nodes
    return model


class OnnxGraph:
    """Parsed, shape-resolved, scheduled graph (graph.py:79-346)."""

    def __init__(self, model, align_elems: int = ALIGN_ELEMS) -> None:
        if isinstance(model, ox.Model):
            m = model
        else:
            m = ox.load(model)
        _check_model(m)
        try:
            infer_shapes(m)
        except ShapeError as e:
            raise SchedulerError(f"shape inference failed: {e}") from e
        split_gemms(m)
        self.model = m
        g = m.graph
        self._tensors: Dict[str, TensorInfo] = {}
        for t in g.initializer:
            self._tensors[t.name] = TensorInfo(t.name, list(t.dims), _dtype_name(t.data_type),
                                               np.asarray(t.array, dtype=np.float32).copy())
        for group in (g.input, g.value_info, g.output):
            for vi in group:
                if vi.name in self._tensors:
                    continue
                shape = [d if d >= 0 else 0 for d in (vi.shape or [])]
                self._tensors[vi.name] = TensorInfo(vi.name, shape, _dtype_name(vi.elem_type))
        inits = {t.name for t in g.initializer}
        self._input_names = [vi.name for vi in g.input if vi.name not in inits]
        self._output_names = [vi.name for vi in g.output]

        self._nodes: List[AnyNode] = []
        for idx, node in enumerate(g.node):
            op = node.op_type
            if op == "MatMul":
                sn = MatmulNode.from_onnx_node(node, self._tensors, idx, align_elems)
            elif op == "Conv":
                sn = ConvNode.from_onnx_node(node, self._tensors, idx, align_elems)
            elif op in POOL_OP_TYPES:
                sn = PoolNode.from_onnx_node(node, self._tensors, idx, align_elems)
            elif op in RESHAPE_OP_TYPES:
                sn = ReshapeNode.from_onnx_node(node, self._tensors, idx, align_elems)
            elif op in VECTOROP_OP_TYPES:
                sn = ScheduledNode.from_onnx_node(node, self._tensors, idx, align_elems)
            else:
                raise SchedulerError(f"{op} node '{node.name or op}' is not supported; "
                                     f"supported ops: {sorted(ALL_SUPPORTED_OP_TYPES)}")
            self._nodes.append(sn)

    @property
    def nodes(self) -> List[AnyNode]:
        return self._nodes

    @property
    def input_tensors(self) -> List[TensorInfo]:
        return [self._tensors[n] for n in self._input_names]

    @property
    def output_tensors(self) -> List[TensorInfo]:
        return [self._tensors[n] for n in self._output_names]

    @property
    def weight_tensors(self) -> List[TensorInfo]:
        """Initializers read by a scheduled node, in first-use order."""
        seen, out = set(), []
        for sn in self._nodes:
            for t in sn.inputs:
                if t.is_weight and t.onnx_name not in seen:
                    seen.add(t.onnx_name)
                    out.append(t)
        return out

    @property
    def intermediate_tensors(self) -> List[TensorInfo]:
        """Node outputs and inputs that are neither graph inputs, outputs nor weights."""
        boundary = ({t.onnx_name for t in self.input_tensors}
                    | {t.onnx_name for t in self.output_tensors}
                    | {t.onnx_name for t in self.weight_tensors})
        seen, out = set(), []
        for sn in self._nodes:
            for t in [sn.output] + list(sn.inputs):
                if t.onnx_name not in boundary and t.onnx_name not in seen:
                    seen.add(t.onnx_name)
                    out.append(t)
        return out

    def get_tensor(self, name: str) -> TensorInfo:
        return self._tensors[name]
