"""Static shape inference for the operators the scheduler accepts.

The reference runs ``onnx.shape_inference.infer_shapes`` before scheduling
(inference-scheduler/src/graph.py:202) so that every intermediate tensor has a
value_info entry with concrete dims.  This module does the same for the
supported op set (graph.py:30-32): element-wise ops with multidirectional
broadcasting, MatMul, Gemm, Conv, the pools and their Global forms, and the
view ops Reshape / Squeeze / Unsqueeze / Dropout.  Shapes already declared in
the model are kept, and a declared shape that disagrees with the inferred one
is an error.
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional

import numpy as np

from . import onnx_io as ox


class ShapeError(ValueError):
    pass


def _bcast(a: List[int], b: List[int], what: str) -> List[int]:
    n = max(len(a), len(b))
    a = [1] * (n - len(a)) + list(a)
    b = [1] * (n - len(b)) + list(b)
    out = []
    for x, y in zip(a, b):
        if x == y or y == 1:
            out.append(x)
        elif x == 1:
            out.append(y)
        else:
            raise ShapeError(f"{what}: shapes {a} and {b} do not broadcast")
    return out


def _ints(node: ox.Node, name: str, default):
    a = node.attribute.get(name)
    return list(a.ints) if a is not None else default


def _int(node: ox.Node, name: str, default: int) -> int:
    a = node.attribute.get(name)
    return a.i if a is not None else default


def _spatial_out(node: ox.Node, in_hw: List[int], kernel: List[int], ceil_mode: bool) -> List[int]:
    nd = len(in_hw)
    strides = _ints(node, "strides", [1] * nd)
    dil = _ints(node, "dilations", [1] * nd)
    pads = _ints(node, "pads", [0] * (2 * nd))
    auto_pad = node.attribute["auto_pad"].s.decode() if "auto_pad" in node.attribute else "NOTSET"
    out = []
    for i in range(nd):
        eff = dil[i] * (kernel[i] - 1) + 1
        if auto_pad in ("SAME_UPPER", "SAME_LOWER"):
            out.append(-(-in_hw[i] // strides[i]))
        elif auto_pad == "VALID":
            out.append(-(-(in_hw[i] - eff + 1) // strides[i]))
        elif auto_pad in ("NOTSET", ""):
            span = in_hw[i] + pads[i] + pads[i + nd] - eff
            q = span / strides[i]
            out.append((math.ceil(q) if ceil_mode else span // strides[i]) + 1)
        else:
            raise ShapeError(f"{node.op_type} '{node.name}': unknown auto_pad '{auto_pad}'")
    return out


def _const(name: str, consts: Dict[str, np.ndarray]) -> Optional[np.ndarray]:
    return consts.get(name)


def infer_node(node: ox.Node, shapes: Dict[str, List[int]],
               consts: Dict[str, np.ndarray]) -> List[Optional[List[int]]]:
    """Output shapes of one node from its input shapes (None where unknown)."""
    op = node.op_type
    ins = [shapes.get(x) if x else None for x in node.input]

    def need(i: int) -> List[int]:
        if i >= len(ins) or ins[i] is None:
            raise ShapeError(f"{op} '{node.name}': shape of input {i} is unknown")
        return ins[i]

    if op in ("Add", "Sub", "Mul", "Div"):
        return [_bcast(need(0), need(1), f"{op} '{node.name}'")]
    if op in ("Relu", "Clip", "Dropout"):
        return [list(need(0))] + [list(need(0))] * (len(node.output) - 1)
    if op == "MatMul":
        a, b = need(0), need(1)
        if len(a) == 1 and len(b) == 1:
            return [[]]
        a2 = [1] + a if len(a) == 1 else a
        b2 = b + [1] if len(b) == 1 else b
        if a2[-1] != b2[-2]:
            raise ShapeError(f"MatMul '{node.name}': inner dims {a} x {b}")
        out = _bcast(a2[:-2], b2[:-2], f"MatMul '{node.name}'") + [a2[-2], b2[-1]]
        if len(a) == 1:
            out.pop(-2)
        if len(b) == 1:
            out.pop(-1)
        return [out]
    if op == "Gemm":
        a, b = need(0), need(1)
        if len(a) != 2 or len(b) != 2:
            raise ShapeError(f"Gemm '{node.name}': operands must be 2-D")
        m = a[1] if _int(node, "transA", 0) else a[0]
        n = b[0] if _int(node, "transB", 0) else b[1]
        return [[m, n]]
    if op == "Conv":
        x, w = need(0), need(1)
        if len(x) < 3:
            raise ShapeError(f"Conv '{node.name}': input rank {len(x)}")
        k = _ints(node, "kernel_shape", w[2:])
        return [[x[0], w[0]] + _spatial_out(node, x[2:], k, False)]
    if op in ("MaxPool", "AveragePool", "LpPool"):
        x = need(0)
        k = _ints(node, "kernel_shape", None)
        if not k:
            raise ShapeError(f"{op} '{node.name}': kernel_shape missing")
        return [[x[0], x[1]] + _spatial_out(node, x[2:], k, bool(_int(node, "ceil_mode", 0)))]
    if op in ("GlobalMaxPool", "GlobalAveragePool", "GlobalLpPool"):
        x = need(0)
        return [[x[0], x[1]] + [1] * (len(x) - 2)]
    if op == "Reshape":
        x = need(0)
        target = _const(node.input[1], consts) if len(node.input) > 1 else None
        if target is None:
            sa = node.attribute.get("shape")
            if sa is None:
                raise ShapeError(f"Reshape '{node.name}': target shape is not a constant")
            target = np.asarray(sa.ints)
        target = [int(v) for v in np.asarray(target).reshape(-1)]
        allowzero = _int(node, "allowzero", 0)
        out = []
        for i, d in enumerate(target):
            out.append(x[i] if (d == 0 and not allowzero) else d)
        total = int(np.prod(x)) if x else 1
        if out.count(-1) > 1:
            raise ShapeError(f"Reshape '{node.name}': more than one -1")
        if -1 in out:
            rest = int(np.prod([d for d in out if d != -1])) if len(out) > 1 else 1
            if rest == 0 or total % rest:
                raise ShapeError(f"Reshape '{node.name}': cannot infer -1 for {x} -> {target}")
            out[out.index(-1)] = total // rest
        if int(np.prod(out)) != total:
            raise ShapeError(f"Reshape '{node.name}': {x} -> {out} changes the element count")
        return [out]
    if op in ("Squeeze", "Unsqueeze"):
        x = need(0)
        axes = _ints(node, "axes", None)
        if axes is None and len(node.input) > 1 and node.input[1]:
            c = _const(node.input[1], consts)
            if c is None:
                raise ShapeError(f"{op} '{node.name}': axes are not a constant")
            axes = [int(v) for v in np.asarray(c).reshape(-1)]
        if op == "Squeeze":
            if not axes:
                return [[d for d in x if d != 1]]
            ax = sorted({a + len(x) if a < 0 else a for a in axes})
            for a in ax:
                if a >= len(x) or x[a] != 1:
                    raise ShapeError(f"Squeeze '{node.name}': axis {a} of {x} is not 1")
            return [[d for i, d in enumerate(x) if i not in ax]]
        if not axes:
            raise ShapeError(f"Unsqueeze '{node.name}': axes missing")
        r = len(x) + len(axes)
        ax = sorted({a + r if a < 0 else a for a in axes})
        out, src = [], iter(x)
        for i in range(r):
            out.append(1 if i in ax else next(src))
        return [out]
    raise ShapeError(f"no shape rule for op_type '{op}' (node '{node.name}')")


def infer_shapes(model: ox.Model) -> ox.Model:
    """Fill graph.value_info with the shape of every node output, in place."""
    g = model.graph
    shapes: Dict[str, List[int]] = {}
    consts: Dict[str, np.ndarray] = {}
    for t in g.initializer:
        shapes[t.name] = list(t.dims)
        consts[t.name] = t.array
    declared: Dict[str, ox.ValueInfo] = {}
    for vi in list(g.input) + list(g.value_info) + list(g.output):
        if vi.shape is not None and all(d >= 0 for d in vi.shape):
            shapes.setdefault(vi.name, list(vi.shape))
        declared.setdefault(vi.name, vi)
    for node in g.node:
        if node.op_type == "Constant":
            raise ShapeError("Constant nodes are not supported; use initializers")
        outs = infer_node(node, shapes, consts)
        for name, shp in zip(node.output, outs):
            if not name or shp is None:
                continue
            have = shapes.get(name)
            if have is not None and name in declared and list(have) != list(shp):
                raise ShapeError(
                    f"tensor '{name}': declared shape {have} but {node.op_type} "
                    f"'{node.name}' produces {shp}")
            shapes[name] = shp
    known = {vi.name for vi in list(g.input) + list(g.output)}
    have_vi = {vi.name: vi for vi in g.value_info}
    for node in g.node:
        for name in node.output:
            if not name or name in known:
                continue
            if name in have_vi:
                have_vi[name].shape = shapes[name]
            else:
                vi = ox.value_info(name, shapes[name])
                g.value_info.append(vi)
                have_vi[name] = vi
    for vi in g.output:
        if vi.name in shapes:
            vi.shape = shapes[vi.name]
    return model
