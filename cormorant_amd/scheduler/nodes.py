"""Scheduled nodes: one ONNX operator -> the kernel calls that implement it.

Each class mirrors one node class of the reference scheduler
(inference-scheduler/src/nodes.py) and derives the same kernel arguments from
the ONNX node, its attributes and the inferred shapes.  Where the reference
emits a line of C (``run_op(...)``, ``run_matmul(...)``, ...), these classes
return ``KernelCall`` records with the same argument values; the HIP backend
executes them through the C ABI and the CPU oracle can execute the same list.

    ScheduledNode  VectorOPKernel  nodes.py:227-453   Add Sub Mul Div Relu Clip(0,6)
    MatmulNode     MatmulKernel    nodes.py:460-821   MatMul (rank 2-5, broadcast batch)
    ConvNode       ConvKernel      nodes.py:828-1119  Conv (group 1 or depthwise)
    PoolNode       PoolingKernel   nodes.py:1143-1418 Max/Average/Lp pools + Global forms
    ReshapeNode    (no kernel)     nodes.py:1425-1493 Reshape Squeeze Unsqueeze Dropout
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import ClassVar, Dict, List, Optional, Tuple

from . import onnx_io as ox
from .tensor import ALIGN_ELEMS, TensorInfo


class SchedulerError(Exception):
    """The ONNX graph cannot be mapped onto the four kernels."""


OP_ADD, OP_SUB, OP_MUL, OP_DIV, OP_RELU, OP_RELU6 = range(6)
OP_COPY = 6  # VectorOPKernel copies a for op >= 6
OP_NAMES = {OP_ADD: "ADD", OP_SUB: "SUB", OP_MUL: "MUL", OP_DIV: "DIV", OP_RELU: "RELU",
            OP_RELU6: "RELU6", OP_COPY: "COPY"}

# op_type -> (op code, arity); Clip is accepted only as Clip(0, 6)
_VECTOR_OPS = {"Add": (OP_ADD, 2), "Sub": (OP_SUB, 2), "Mul": (OP_MUL, 2), "Div": (OP_DIV, 2),
               "Relu": (OP_RELU, 1), "Clip": (OP_RELU6, 1)}
VECTOROP_OP_TYPES = frozenset(_VECTOR_OPS)
RESHAPE_OP_TYPES = frozenset({"Reshape", "Squeeze", "Unsqueeze", "Dropout"})

POOL_MAX, POOL_AVG, POOL_LP = 0, 1, 2
GLOBAL_POOL_OP_TYPES = frozenset({"GlobalMaxPool", "GlobalAveragePool", "GlobalLpPool"})
POOL_OP_TYPES = frozenset({"MaxPool", "AveragePool", "LpPool"}) | GLOBAL_POOL_OP_TYPES


def align_up(n: int, a: int) -> int:
    return (n + a - 1) // a * a


# --------------------------------------------------------------------------- kernel calls

@dataclass(frozen=True)
class KernelCall:
    """One kernel invocation, in the argument order of the reference's run_* helpers.

    kernel   "op" | "matmul" | "matmul_at" | "conv" | "pool"
    tensors  tensor names bound to the pointer arguments (None = NULL)
    args     the uint32 scalar arguments
    offsets  element offsets of the tensors (matmul_at only)
    """
    kernel: str
    tensors: Tuple[Optional[str], ...]
    args: Tuple[int, ...]
    offsets: Tuple[int, ...] = ()

    def extents(self) -> Dict[str, int]:
        """Elements (from the tensor's base) each tensor must hold for this call."""
        need: Dict[str, int] = {}

        def put(name, n):
            if name is not None and n > 0:
                need[name] = max(need.get(name, 0), n)

        t, a = self.tensors, self.args
        if self.kernel == "op":
            size, op, outer, a_inc, b_inc = a
            if size and outer:
                put(t[0], (outer - 1) * a_inc + size)
                if op < OP_RELU:
                    put(t[1], (outer - 1) * b_inc + size)
                put(t[2], (outer - 1) * (a_inc + b_inc) + size)
        elif self.kernel in ("matmul", "matmul_at"):
            n, k, m, batch, a_bs, b_bs, c_bs = a
            off = self.offsets or (0, 0, 0)
            if n and m and batch:
                put(t[0], off[0] + (batch - 1) * a_bs + n * k)
                put(t[1], off[1] + (batch - 1) * b_bs + k * m)
                put(t[2], off[2] + (batch - 1) * c_bs + n * m)
        elif self.kernel == "conv":
            (nb, c, h, w, mo, oh, ow, kh, kw, _sh, _sw, _dh, _dw, _pt, _pl, hb, dw) = a
            if nb * mo * oh * ow:
                put(t[0], nb * c * h * w)
                put(t[1], mo * (1 if dw else c) * kh * kw)
                if hb:
                    put(t[2], mo)
                put(t[3], nb * mo * oh * ow)
        elif self.kernel == "pool":
            nb, c, h, w, oh, ow = a[:6]
            if nb * c * oh * ow:
                put(t[0], nb * c * h * w)
                put(t[1], nb * c * oh * ow)
        else:
            raise ValueError(f"unknown kernel '{self.kernel}'")
        return need

    def __str__(self) -> str:
        names = ["NULL" if x is None else x for x in self.tensors]
        if self.kernel == "op":
            size, op, outer, a_inc, b_inc = self.args
            return (f"run_op({names[0]}, {names[1]}, {names[2]}, {size}, "
                    f"{OP_NAMES.get(op, op)}, {outer}, {a_inc}, {b_inc})")
        if self.kernel == "matmul_at":
            head = ", ".join(f"{n}+{o}" for n, o in zip(names, self.offsets))
            return f"run_matmul_at({head}, {', '.join(map(str, self.args))})"
        return f"run_{self.kernel}({', '.join(names)}, {', '.join(map(str, self.args))})"


# --------------------------------------------------------------------------- helpers

def _resolve(tensors: Dict[str, TensorInfo], name: str, what: str) -> TensorInfo:
    if name not in tensors:
        raise SchedulerError(f"tensor '{name}' used by {what} is not in the graph")
    return tensors[name]


def _output(node: ox.Node, tensors, what: str) -> TensorInfo:
    if not node.output or node.output[0] == "":
        raise SchedulerError(f"{what} has no output")
    return _resolve(tensors, node.output[0], what)


def _label(node: ox.Node) -> str:
    return f"{node.op_type} node '{node.name or node.op_type}'"


def broadcast_info(t: TensorInfo, out: TensorInfo,
                   align_elems: int = ALIGN_ELEMS) -> Tuple[int, int, int, bool]:
    """How input t maps onto output out: (outer_count, chunk, aligned_chunk, advances).

    Same rule as nodes.py:151-224: a tensor as large as the output advances
    through it in one pass; a smaller one must right-align to the output with
    its size-1 (broadcast) dimensions forming one leading block, and then
    repeats at offset 0 once per chunk of t.numel elements."""
    if t.numel == out.numel:
        return 1, out.numel, out.numel, True
    if out.numel % t.numel:
        raise SchedulerError(
            f"'{t.onnx_name}' ({t.numel} elements) does not divide output "
            f"'{out.onnx_name}' ({out.numel} elements)")
    shape = [1] * (len(out.shape) - len(t.shape)) + list(t.shape)
    if len(shape) > len(out.shape):
        raise SchedulerError(f"'{t.onnx_name}' {t.shape} has higher rank than {out.shape}")
    matched = False
    for td, od in zip(shape, out.shape):
        if td == od:
            matched = True
        elif td == 1:
            if matched:
                raise SchedulerError(
                    f"'{t.onnx_name}' {t.shape} -> {out.shape}: a broadcast dimension "
                    f"follows a matching one; broadcast dims must lead")
        else:
            raise SchedulerError(
                f"'{t.onnx_name}' {t.shape} does not broadcast to {out.shape}")
    chunk = t.numel
    return out.numel // chunk, chunk, align_up(chunk, align_elems), False


# --------------------------------------------------------------------------- VectorOP

@dataclass
class ScheduledNode:
    """Element-wise op on VectorOPKernel (nodes.py:227-453)."""

    kernel_name: ClassVar[str] = "VectorOPKernel"

    onnx_node: ox.Node
    op_code: int
    arity: int
    inputs: List[TensorInfo]
    output: TensorInfo
    index: int = 0
    align_elems: int = ALIGN_ELEMS

    outer_count: int = field(default=1, init=False)
    chunk_size: int = field(default=0, init=False)
    aligned_chunk_size: int = field(default=0, init=False)
    a_advances: bool = field(default=True, init=False)
    b_advances: bool = field(default=True, init=False)

    @classmethod
    def from_onnx_node(cls, node: ox.Node, tensors: Dict[str, TensorInfo], index: int,
                       align_elems: int = ALIGN_ELEMS) -> "ScheduledNode":
        if node.op_type not in _VECTOR_OPS:
            raise SchedulerError(
                f"{_label(node)} is not supported by VectorOPKernel; supported: "
                f"{sorted(_VECTOR_OPS)}")
        op, arity = _VECTOR_OPS[node.op_type]
        ins = [_resolve(tensors, x, _label(node)) for x in node.input if x != ""]
        sn = cls(onnx_node=node, op_code=op, arity=arity, inputs=ins,
                 output=_output(node, tensors, _label(node)), index=index,
                 align_elems=align_elems)
        sn.validate()
        return sn

    def _clip_bounds(self) -> Tuple[Optional[float], Optional[float]]:
        """Clip bounds from attributes (opset < 11) or constant inputs (opset >= 11)."""
        attrs = self.onnx_node.attribute
        if "min" in attrs or "max" in attrs:
            lo = attrs["min"].f if "min" in attrs else None
            hi = attrs["max"].f if "max" in attrs else None
            return lo, hi
        lo = hi = None
        if len(self.inputs) > 1 and self.inputs[1].is_weight:
            lo = float(self.inputs[1].data.reshape(-1)[0])
        if len(self.inputs) > 2 and self.inputs[2].is_weight:
            hi = float(self.inputs[2].data.reshape(-1)[0])
        return lo, hi

    def validate(self) -> None:
        node = self.onnx_node
        if node.op_type == "Clip":
            lo, hi = self._clip_bounds()
            if lo != 0.0 or hi != 6.0:
                raise SchedulerError(
                    f"{_label(node)} has bounds ({lo}, {hi}); only Clip(0, 6) maps to RELU6")
            self.inputs = [self.inputs[0]]
            self.arity = 1
        if len(self.inputs) != self.arity:
            raise SchedulerError(
                f"{_label(node)} needs {self.arity} input(s), got {len(self.inputs)}")
        if self.arity == 1:
            if self.inputs[0].numel != self.output.numel:
                raise SchedulerError(
                    f"{_label(node)}: input has {self.inputs[0].numel} elements, output "
                    f"{self.output.numel}")
            self.outer_count = 1
            self.chunk_size = self.aligned_chunk_size = self.output.numel
            self.a_advances = self.b_advances = True
            return
        ae = self.align_elems
        a_outer, _, _, a_adv = broadcast_info(self.inputs[0], self.output, ae)
        b_outer, _, _, b_adv = broadcast_info(self.inputs[1], self.output, ae)
        if not a_adv and not b_adv:
            raise SchedulerError(
                f"{_label(node)}: both inputs are smaller than the output; only one "
                f"input may broadcast")
        self.outer_count = max(a_outer, b_outer)
        self.chunk_size = self.output.numel // self.outer_count
        self.aligned_chunk_size = align_up(self.chunk_size, ae)
        self.a_advances, self.b_advances = a_adv, b_adv

    def calls(self, layouts) -> List[KernelCall]:
        a = self.inputs[0].onnx_name
        b = self.inputs[1].onnx_name if self.arity == 2 else None
        c = self.output.onnx_name
        if self.outer_count == 1:
            lay = layouts.get(c)
            size = lay.alloc if lay is not None else self.chunk_size
            return [KernelCall("op", (a, b, c), (size, self.op_code, 1, 0, 0))]
        stride = self.aligned_chunk_size
        a_inc = stride if self.a_advances else 0
        b_inc = (stride if self.b_advances else 0) if self.arity == 2 else 0
        return [KernelCall("op", (a, b, c),
                           (self.chunk_size, self.op_code, self.outer_count, a_inc, b_inc))]


# --------------------------------------------------------------------------- MatMul

@dataclass
class MatmulNode:
    """MatMul on MatmulKernel (nodes.py:460-821).

    A[..., n, k] @ B[..., k, m].  Shared trailing batch dims run in one kernel
    call (batch strides; a 2-D operand gets stride 0); a leading block of batch
    dims present on one side only becomes an outer loop of offset calls."""

    kernel_name: ClassVar[str] = "MatmulKernel"

    onnx_node: ox.Node
    inputs: List[TensorInfo]
    output: TensorInfo
    index: int = 0
    align_elems: int = ALIGN_ELEMS
    n: int = 0
    k: int = 0
    m: int = 0
    batch: int = 1
    a_batch_stride: int = 0
    b_batch_stride: int = 0
    c_batch_stride: int = 0
    outer_count: int = 1
    a_outer_stride: int = 0
    b_outer_stride: int = 0
    c_outer_stride: int = 0

    # neutral broadcast fields so layout passes can treat every node alike
    chunk_size: int = field(default=0, init=False)
    aligned_chunk_size: int = field(default=0, init=False)
    a_advances: bool = field(default=True, init=False)
    b_advances: bool = field(default=True, init=False)
    arity: int = field(default=2, init=False)

    @classmethod
    def from_onnx_node(cls, node: ox.Node, tensors: Dict[str, TensorInfo], index: int,
                       align_elems: int = ALIGN_ELEMS) -> "MatmulNode":
        what = _label(node)
        if node.op_type != "MatMul":
            raise SchedulerError(f"MatmulNode cannot take {what}")
        if len(node.input) != 2:
            raise SchedulerError(f"{what} needs 2 inputs, got {len(node.input)}")
        a = _resolve(tensors, node.input[0], what)
        b = _resolve(tensors, node.input[1], what)
        y = _output(node, tensors, what)
        sa, sb = tuple(a.shape), tuple(b.shape)
        if not (2 <= len(sa) <= 5 and 2 <= len(sb) <= 5):
            raise SchedulerError(f"{what}: ranks 2-5 supported, got {list(sa)} @ {list(sb)}")
        n, k, m = sa[-2], sa[-1], sb[-1]
        if sb[-2] != k:
            raise SchedulerError(f"{what}: inner dims differ in {list(sa)} @ {list(sb)}")
        ab, bb = sa[:-2], sb[:-2]
        base = dict(onnx_node=node, inputs=[a, b], output=y, index=index,
                    align_elems=align_elems, n=n, k=k, m=m)

        def prod(dims):
            p = 1
            for d in dims:
                p *= d
            return p

        if not ab and not bb:
            return cls(**base)
        if not bb:
            return cls(**base, batch=prod(ab), a_batch_stride=n * k, b_batch_stride=0,
                       c_batch_stride=n * m)
        if not ab:
            return cls(**base, batch=prod(bb), a_batch_stride=0, b_batch_stride=k * m,
                       c_batch_stride=n * m)

        r = max(len(ab), len(bb))
        ae = (1,) * (r - len(ab)) + ab
        be = (1,) * (r - len(bb)) + bb
        out_b = []
        for x, z in zip(ae, be):
            if x == z or z == 1:
                out_b.append(x)
            elif x == 1:
                out_b.append(z)
            else:
                raise SchedulerError(f"{what}: batch dims {list(ab)} and {list(bb)} do not "
                                     f"broadcast")
        # leading dims where exactly one side is 1 form the outer loop; all of them must
        # come from the same side
        split, a_drives = r, None
        for i, (x, z) in enumerate(zip(ae, be)):
            if (x > 1 and z > 1) or (x == 1 and z == 1):
                split = i
                break
            drives = x > 1
            if a_drives is None:
                a_drives = drives
            elif a_drives != drives:
                raise SchedulerError(f"{what}: outer broadcast runs in both directions "
                                     f"({list(ab)} vs {list(bb)})")
        outer, batch = prod(out_b[:split]), prod(out_b[split:])
        if batch <= 1:
            a_bs = b_bs = c_bs = 0
        else:
            a_bs = n * k if any(ae[i] > 1 for i in range(split, r)) else 0
            b_bs = k * m if any(be[i] > 1 for i in range(split, r)) else 0
            c_bs = n * m
        if outer <= 1:
            return cls(**base, batch=batch, a_batch_stride=a_bs, b_batch_stride=b_bs,
                       c_batch_stride=c_bs)
        return cls(**base, batch=batch, a_batch_stride=a_bs, b_batch_stride=b_bs,
                   c_batch_stride=c_bs, outer_count=outer,
                   a_outer_stride=batch * n * k if a_drives else 0,
                   b_outer_stride=0 if a_drives else batch * k * m,
                   c_outer_stride=batch * n * m)

    def calls(self, layouts) -> List[KernelCall]:
        a, b, c = (self.inputs[0].onnx_name, self.inputs[1].onnx_name, self.output.onnx_name)
        if self.outer_count == 1:
            a_lay, y_lay = layouts.get(a), layouts.get(c)
            a_rs = a_lay.stride if (a_lay is not None and a_lay.gap > 0) else 0
            c_rs = y_lay.stride if (y_lay is not None and y_lay.gap > 0) else 0
            if a_rs or c_rs:
                # rows of A or Y sit at a padded stride: one kernel batch entry per row
                # (nodes.py:785-801).  That only holds for a plain 2-D product whose
                # padded chunks are exactly the rows.
                if self.batch > 1 or (a_rs and a_lay.chunk != self.k) or (
                        c_rs and y_lay.chunk != self.m):
                    raise SchedulerError(
                        f"{_label(self.onnx_node)}: padded layout of A or Y does not "
                        f"match its rows; a row-strided MatMul needs a 2-D product")
                return [KernelCall("matmul", (a, b, c),
                                   (1, self.k, self.m, self.n, a_rs or self.k,
                                    self.b_batch_stride, c_rs or self.m))]
            return [KernelCall("matmul", (a, b, c),
                               (self.n, self.k, self.m, self.batch, self.a_batch_stride,
                                self.b_batch_stride, self.c_batch_stride))]
        args = (self.n, self.k, self.m, self.batch, self.a_batch_stride, self.b_batch_stride,
                self.c_batch_stride)
        return [KernelCall("matmul_at", (a, b, c), args,
                           (i * self.a_outer_stride, i * self.b_outer_stride,
                            i * self.c_outer_stride))
                for i in range(self.outer_count)]


# --------------------------------------------------------------------------- Conv

def _pads(node: ox.Node, what: str, in_hw, out_hw, kernel, strides, dil) -> Tuple[int, int]:
    """(pad_top, pad_left) from pads / auto_pad (nodes.py:1025-1047, 1306-1325)."""
    attrs = node.attribute
    auto = attrs["auto_pad"].s.decode("utf-8") if "auto_pad" in attrs else "NOTSET"
    if auto == "NOTSET":
        pads = list(attrs["pads"].ints) if "pads" in attrs else [0, 0, 0, 0]
        return (int(pads[0]) if len(pads) > 0 else 0, int(pads[1]) if len(pads) > 1 else 0)
    if auto == "VALID":
        return 0, 0
    if auto in ("SAME_UPPER", "SAME_LOWER"):
        out = []
        for i in range(2):
            eff = dil[i] * (kernel[i] - 1) + 1
            total = max(0, (out_hw[i] - 1) * strides[i] + eff - in_hw[i])
            out.append(total // 2 if auto == "SAME_UPPER" else (total + 1) // 2)
        return out[0], out[1]
    raise SchedulerError(f"{what}: unsupported auto_pad '{auto}'")


@dataclass
class ConvNode:
    """2-D Conv on ConvKernel, group 1 or depthwise (nodes.py:828-1119)."""

    kernel_name: ClassVar[str] = "ConvKernel"

    onnx_node: ox.Node
    inputs: List[TensorInfo]
    output: TensorInfo
    index: int = 0
    align_elems: int = ALIGN_ELEMS
    batch: int = 1
    in_ch: int = 0
    in_h: int = 0
    in_w: int = 0
    out_ch: int = 0
    out_h: int = 0
    out_w: int = 0
    kh: int = 1
    kw: int = 1
    stride_h: int = 1
    stride_w: int = 1
    dilation_h: int = 1
    dilation_w: int = 1
    pad_top: int = 0
    pad_left: int = 0
    has_bias: bool = False
    is_depthwise: bool = False

    outer_count: int = field(default=1, init=False)
    chunk_size: int = field(default=0, init=False)
    aligned_chunk_size: int = field(default=0, init=False)
    a_advances: bool = field(default=True, init=False)
    b_advances: bool = field(default=True, init=False)
    arity: int = field(default=2, init=False)

    @classmethod
    def from_onnx_node(cls, node: ox.Node, tensors: Dict[str, TensorInfo], index: int,
                       align_elems: int = ALIGN_ELEMS) -> "ConvNode":
        what = _label(node)
        if node.op_type != "Conv":
            raise SchedulerError(f"ConvNode cannot take {what}")
        n_in = len([x for x in node.input if x != ""])
        if n_in not in (2, 3):
            raise SchedulerError(f"{what} needs 2 or 3 inputs, got {n_in}")
        x = _resolve(tensors, node.input[0], what)
        w = _resolve(tensors, node.input[1], what)
        has_b = n_in == 3 and node.input[2] != ""
        bias = _resolve(tensors, node.input[2], what) if has_b else None
        y = _output(node, tensors, what)
        for t, role in ((x, "input"), (w, "weight"), (y, "output")):
            if len(t.shape) != 4:
                raise SchedulerError(f"{what}: {role} must be 4-D, got {t.shape}")
        nb, c, h, wd = x.shape
        mo, cw, kh, kw = w.shape
        oh, ow = y.shape[2], y.shape[3]
        attrs = node.attribute
        group = attrs["group"].i if "group" in attrs else 1
        if group == 1:
            dw = False
            if cw != c:
                raise SchedulerError(f"{what}: weight has {cw} input channels, input has {c}")
        elif group == c:
            dw = True
            if cw != 1:
                raise SchedulerError(f"{what}: depthwise weight needs 1 channel per filter, "
                                     f"got {cw}")
            if mo != c:
                raise SchedulerError(f"{what}: depthwise conv needs out_ch ({mo}) == "
                                     f"in_ch ({c})")
        else:
            raise SchedulerError(f"{what}: group={group} is not supported (only 1 or in_ch)")
        if mo != y.shape[1]:
            raise SchedulerError(f"{what}: weight has {mo} filters, output {y.shape[1]} "
                                 f"channels")
        strides = list(attrs["strides"].ints) if "strides" in attrs else [1, 1]
        dil = list(attrs["dilations"].ints) if "dilations" in attrs else [1, 1]
        if len(strides) != 2:
            raise SchedulerError(f"{what}: only 2-D strides are supported, got {strides}")
        if len(dil) != 2:
            raise SchedulerError(f"{what}: only 2-D dilations are supported, got {dil}")
        pt, pl = _pads(node, what, (h, wd), (oh, ow), (kh, kw), strides, dil)
        ins = [x, w] + ([bias] if has_b else [])
        return cls(onnx_node=node, inputs=ins, output=y, index=index, align_elems=align_elems,
                   batch=nb, in_ch=c, in_h=h, in_w=wd, out_ch=mo, out_h=oh, out_w=ow, kh=kh,
                   kw=kw, stride_h=strides[0], stride_w=strides[1], dilation_h=dil[0],
                   dilation_w=dil[1], pad_top=pt, pad_left=pl, has_bias=has_b,
                   is_depthwise=dw)

    def calls(self, layouts) -> List[KernelCall]:
        names = (self.inputs[0].onnx_name, self.inputs[1].onnx_name,
                 self.inputs[2].onnx_name if self.has_bias else None, self.output.onnx_name)
        return [KernelCall("conv", names, (
            self.batch, self.in_ch, self.in_h, self.in_w, self.out_ch, self.out_h, self.out_w,
            self.kh, self.kw, self.stride_h, self.stride_w, self.dilation_h, self.dilation_w,
            self.pad_top, self.pad_left, int(self.has_bias), int(self.is_depthwise)))]


# --------------------------------------------------------------------------- Pool

@dataclass
class PoolNode:
    """2-D pooling on PoolingKernel (nodes.py:1143-1418)."""

    kernel_name: ClassVar[str] = "PoolKernel"

    onnx_node: ox.Node
    inputs: List[TensorInfo]
    output: TensorInfo
    index: int = 0
    align_elems: int = ALIGN_ELEMS
    batch: int = 1
    channels: int = 0
    in_h: int = 0
    in_w: int = 0
    out_h: int = 0
    out_w: int = 0
    pool_h: int = 1
    pool_w: int = 1
    stride_h: int = 1
    stride_w: int = 1
    pad_top: int = 0
    pad_left: int = 0
    dil_h: int = 1
    dil_w: int = 1
    pool_type: int = POOL_MAX
    lp_order: int = 2
    count_include_pad: int = 0

    outer_count: int = field(default=1, init=False)
    chunk_size: int = field(default=0, init=False)
    aligned_chunk_size: int = field(default=0, init=False)
    a_advances: bool = field(default=True, init=False)
    b_advances: bool = field(default=True, init=False)
    arity: int = field(default=1, init=False)

    @classmethod
    def from_onnx_node(cls, node: ox.Node, tensors: Dict[str, TensorInfo], index: int,
                       align_elems: int = ALIGN_ELEMS) -> "PoolNode":
        op = node.op_type
        what = _label(node)
        if op not in POOL_OP_TYPES:
            raise SchedulerError(f"PoolNode cannot take {what}")
        if not node.input or node.input[0] == "":
            raise SchedulerError(f"{what} has no input")
        x = _resolve(tensors, node.input[0], what)
        y = _output(node, tensors, what)
        for t, role in ((x, "input"), (y, "output")):
            if len(t.shape) != 4:
                raise SchedulerError(f"{what}: {role} must be 4-D (NCHW), got {t.shape}")
        nb, c, h, w = x.shape
        oh, ow = y.shape[2], y.shape[3]
        ptype = (POOL_MAX if op in ("MaxPool", "GlobalMaxPool") else
                 POOL_AVG if op in ("AveragePool", "GlobalAveragePool") else POOL_LP)
        attrs = node.attribute

        def ints(name, default):
            return list(attrs[name].ints) if name in attrs else default

        def one(name, default):
            return attrs[name].i if name in attrs else default

        if op in GLOBAL_POOL_OP_TYPES:
            ph, pw, sh, sw, pt, pl, dh, dw = h, w, 1, 1, 0, 0, 1, 1
        else:
            ks = ints("kernel_shape", [])
            if len(ks) != 2:
                raise SchedulerError(f"{what}: kernel_shape must have 2 values, got {ks}")
            ph, pw = int(ks[0]), int(ks[1])
            st = ints("strides", [1, 1])
            if len(st) != 2:
                raise SchedulerError(f"{what}: only 2-D strides are supported, got {st}")
            sh, sw = int(st[0]), int(st[1])
            dl = ints("dilations", [1, 1])
            dh = int(dl[0]) if len(dl) >= 1 else 1
            dw = int(dl[1]) if len(dl) >= 2 else 1
            pt, pl = _pads(node, what, (h, w), (oh, ow), (ph, pw), (sh, sw), (dh, dw))
            if one("ceil_mode", 0) != 0:
                raise SchedulerError(f"{what}: ceil_mode=1 is not supported")
        p = one("p", 2) if ptype == POOL_LP else 2
        if ptype == POOL_LP and p not in (1, 2):
            raise SchedulerError(f"{what}: p={p} is not supported (p = 1 or 2)")
        cip = one("count_include_pad", 0) if ptype == POOL_AVG else 0
        return cls(onnx_node=node, inputs=[x], output=y, index=index, align_elems=align_elems,
                   batch=nb, channels=c, in_h=h, in_w=w, out_h=oh, out_w=ow, pool_h=ph,
                   pool_w=pw, stride_h=sh, stride_w=sw, pad_top=pt, pad_left=pl, dil_h=dh,
                   dil_w=dw, pool_type=ptype, lp_order=p, count_include_pad=cip)

    def calls(self, layouts) -> List[KernelCall]:
        return [KernelCall("pool", (self.inputs[0].onnx_name, self.output.onnx_name), (
            self.batch, self.channels, self.in_h, self.in_w, self.out_h, self.out_w,
            self.pool_h, self.pool_w, self.stride_h, self.stride_w, self.pad_top,
            self.pad_left, self.dil_h, self.dil_w, self.pool_type, self.lp_order,
            self.count_include_pad))]


# --------------------------------------------------------------------------- views

@dataclass
class ReshapeNode:
    """Reshape / Squeeze / Unsqueeze / Dropout: the output aliases the input's
    buffer, no kernel runs (nodes.py:1425-1493)."""

    kernel_name: ClassVar[str] = ""

    onnx_node: ox.Node
    inputs: List[TensorInfo]
    output: TensorInfo
    index: int = 0
    align_elems: int = ALIGN_ELEMS

    outer_count: int = field(default=1, init=False)
    chunk_size: int = field(default=0, init=False)
    aligned_chunk_size: int = field(default=0, init=False)
    a_advances: bool = field(default=True, init=False)
    b_advances: bool = field(default=True, init=False)
    arity: int = field(default=1, init=False)

    @classmethod
    def from_onnx_node(cls, node: ox.Node, tensors: Dict[str, TensorInfo], index: int,
                       align_elems: int = ALIGN_ELEMS) -> "ReshapeNode":
        what = _label(node)
        src = _resolve(tensors, node.input[0], what)
        out = _output(node, tensors, what)
        if src.numel != out.numel:
            raise SchedulerError(f"{what}: {src.shape} -> {out.shape} changes the element "
                                 f"count; only views are supported")
        return cls(onnx_node=node, inputs=[src], output=out, index=index,
                   align_elems=align_elems)

    def calls(self, layouts) -> List[KernelCall]:
        return []
