"""Buffer plan: tensor layouts, live intervals, the single pool allocation and
where every tensor's storage lives.

Follows the reference code generator's core (inference-scheduler/src/codegen/_core.py):

* ``compute_tensor_layouts``  _core.py:75-249   flat / advancing / repeating layouts,
  propagated so that one VectorOP call covers every padded buffer it touches;
* ``live_intervals``          _core.py:270-296  (first producer, last consumer) per
  intermediate;
* ``pool_layout``             _core.py:298-373  weights first, then intermediates packed
  into 64-byte aligned slots by greedy interval colouring;
* reshape aliases and output alias chains  _core.py:429-534.

``BufferPlan`` adds what the generated C expressed with pointer assignments:
a storage map (which allocation and element offset backs each tensor), the
flat kernel-call list, and a host-side check that every call stays inside the
storage it touches.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

from .graph import OnnxGraph
from .nodes import (OP_COPY, ConvNode, KernelCall, MatmulNode, PoolNode, ReshapeNode,
                    SchedulerError)
from .tensor import BYTES_PER_ELEM, POOL_ALIGN_BYTES


@dataclass(frozen=True)
class TensorLayout:
    """How a tensor's elements sit in its buffer (inference-scheduler/src/layout.py).

    n_chunks == 1, stride == chunk == numel: flat.
    n_chunks == 1, stride > chunk: one data block then padding (repeating input).
    n_chunks > 1: n_chunks blocks of `chunk` data elements at `stride` spacing."""
    numel: int
    alloc: int
    n_chunks: int
    chunk: int
    stride: int

    @property
    def gap(self) -> int:
        return self.stride - self.chunk

    @property
    def is_strided(self) -> bool:
        return self.stride > self.chunk

    @staticmethod
    def flat(numel: int) -> "TensorLayout":
        return TensorLayout(numel, numel, 1, numel, numel)

    @staticmethod
    def advancing(numel: int, n_chunks: int, stride: int) -> "TensorLayout":
        return TensorLayout(numel, n_chunks * stride, n_chunks, numel // n_chunks, stride)

    @staticmethod
    def repeating(numel: int, alloc: int) -> "TensorLayout":
        return TensorLayout(numel, alloc, 1, numel, alloc)

    def positions(self):
        """Buffer position of every logical element, in logical order."""
        import numpy as np
        idx = np.arange(self.numel, dtype=np.int64)
        if self.n_chunks > 1:
            return (idx // self.chunk) * self.stride + idx % self.chunk
        return idx


_SPECIAL = (MatmulNode, ConvNode, PoolNode, ReshapeNode)


def compute_tensor_layouts(graph: OnnxGraph) -> Dict[str, TensorLayout]:
    """Layout of every tensor (_core.py:75-249).

    1. every tensor starts flat;
    2. a broadcasting VectorOP gives its output and advancing input an
       advancing layout (outer_count chunks at the aligned stride) and its
       repeating input one padded block;
    3. in graph order, a non-broadcast VectorOP output inherits the largest
       input allocation (and its chunking), and smaller co-inputs are raised to
       the output's, so that one call over `alloc` elements is valid for all.
    Conv and Pool outputs must stay flat: they write plain NCHW."""
    tensors = (graph.weight_tensors + graph.intermediate_tensors + graph.input_tensors
               + graph.output_tensors)
    lay: Dict[str, TensorLayout] = {t.onnx_name: TensorLayout.flat(t.numel) for t in tensors}

    for sn in graph.nodes:
        if sn.outer_count <= 1 or isinstance(sn, _SPECIAL):
            continue
        n, stride = sn.outer_count, sn.aligned_chunk_size
        alloc = n * stride

        def set_advancing(t):
            cur = lay[t.onnx_name]
            if cur.n_chunks == 1 or alloc > cur.alloc:
                lay[t.onnx_name] = TensorLayout.advancing(t.numel, n, stride)

        def set_repeating(t):
            cur = lay[t.onnx_name]
            if stride > cur.alloc:
                lay[t.onnx_name] = TensorLayout.repeating(t.numel, stride)

        set_advancing(sn.output)
        (set_advancing if sn.a_advances else set_repeating)(sn.inputs[0])
        if sn.arity == 2:
            (set_advancing if sn.b_advances else set_repeating)(sn.inputs[1])

    for sn in graph.nodes:
        if sn.outer_count > 1 or isinstance(sn, _SPECIAL):
            continue
        ins = [lay[t.onnx_name] for t in sn.inputs]
        out_name = sn.output.onnx_name
        out = lay[out_name]
        dominant = None
        for li in ins:
            if li.n_chunks > 1 and (dominant is None or li.alloc > dominant.alloc):
                dominant = li
        biggest = max(li.alloc for li in ins)
        if biggest > out.alloc:
            if dominant is not None:
                lay[out_name] = TensorLayout.advancing(out.numel, dominant.n_chunks,
                                                       dominant.stride)
            else:
                lay[out_name] = TensorLayout(out.numel, biggest, 1, out.numel, biggest)
        out = lay[out_name]
        for t in sn.inputs:
            cur = lay[t.onnx_name]
            if cur.alloc >= out.alloc:
                continue
            if out.n_chunks > 1:
                lay[t.onnx_name] = TensorLayout.advancing(cur.numel, out.n_chunks, out.stride)
            else:
                lay[t.onnx_name] = TensorLayout(cur.numel, out.alloc, 1, cur.numel, out.alloc)

    for sn in graph.nodes:
        if isinstance(sn, (ConvNode, PoolNode)) and lay[sn.output.onnx_name].n_chunks > 1:
            kind = "Conv" if isinstance(sn, ConvNode) else "Pool"
            raise SchedulerError(
                f"{kind} node [{sn.index}] output '{sn.output.onnx_name}' feeds a broadcasting "
                f"element-wise op that needs a padded layout, but the kernel writes plain "
                f"NCHW; use the Conv bias input or put a non-broadcast op in between")
    return lay


def reshape_aliases(graph: OnnxGraph) -> Dict[str, str]:
    """{reshape output: reshape source} for every ReshapeNode."""
    return {sn.output.onnx_name: sn.inputs[0].onnx_name
            for sn in graph.nodes if isinstance(sn, ReshapeNode)}


def live_intervals(graph: OnnxGraph, live_from: Optional[Dict[str, int]] = None
                   ) -> Dict[str, Tuple[int, int]]:
    """(producing node index, last consuming node index) of each non-alias intermediate.

    A read of a reshape alias (Reshape / Squeeze / Unsqueeze / Dropout output)
    counts as a read of the tensor it aliases: the alias IS that storage.  The
    reference's interval (_core.py:270-296) counts only direct readers, so a
    tensor produced between the reshape and the alias's reader may be given the
    source's slot and overwrite it; extending the interval keeps that from
    happening (it only changes slot offsets, never a kernel argument).

    ``live_from`` moves the start of some intermediates earlier (a backend that
    writes a tensor from an earlier node, e.g. a fused epilogue)."""
    aliases = reshape_aliases(graph)
    names = {t.onnx_name for t in graph.intermediate_tensors if t.onnx_name not in aliases}

    def root(n: str) -> str:
        seen = 0
        while n in aliases and seen <= len(aliases):
            n, seen = aliases[n], seen + 1
        return n

    first: Dict[str, int] = {}
    last: Dict[str, int] = {}
    for i, sn in enumerate(graph.nodes):
        if sn.output.onnx_name in names:
            first[sn.output.onnx_name] = i
        for t in sn.inputs:
            r = root(t.onnx_name)
            if r in names:
                last[r] = i
    if live_from:
        for n, i in live_from.items():
            if n in first:
                first[n] = min(first[n], i)
    return {n: (first[n], last.get(n, first[n])) for n in names if n in first}


def pool_layout(graph: OnnxGraph, layouts: Dict[str, TensorLayout],
                live_from: Optional[Dict[str, int]] = None) -> Tuple[List[Tuple[str, int, int]], int]:
    """([(tensor, offset, alloc)], total elements) of the one pool allocation.

    Weights come first, each in its own slot.  Intermediates are sorted by
    start (ties: largest first) and each takes the first slot whose last
    tenant has already died, growing it if needed."""
    unit = POOL_ALIGN_BYTES // BYTES_PER_ELEM

    def up(n):
        return (n + unit - 1) // unit * unit

    aliases = reshape_aliases(graph)
    entries: List[Tuple[str, int, int]] = []
    off = 0
    for t in graph.weight_tensors:
        a = layouts[t.onnx_name].alloc
        entries.append((t.onnx_name, off, a))
        off += up(a)
    iv = live_intervals(graph, live_from)
    cands = [t.onnx_name for t in graph.intermediate_tensors if t.onnx_name not in aliases]
    timed = sorted(((n, iv[n]) for n in cands if n in iv),
                   key=lambda kv: (kv[1][0], -layouts[kv[0]].alloc))
    slots: List[list] = []  # [end, size, [names]]
    for name, (start, end) in timed:
        a = layouts[name].alloc
        for s in slots:
            if s[0] < start:
                s[0] = end
                s[1] = max(s[1], up(a))
                s[2].append(name)
                break
        else:
            slots.append([end, up(a), [name]])
    for _, size, names in slots:
        for n in names:
            entries.append((n, off, layouts[n].alloc))
        off += size
    for n in cands:
        if n not in iv:
            a = layouts[n].alloc
            entries.append((n, off, a))
            off += up(a)
    return entries, off


@dataclass(frozen=True)
class Storage:
    """Where a tensor's elements live: allocation kind ("pool", "input" or
    "output"), the allocation's key (tensor name for inputs/outputs), element
    offset and the number of elements available from there."""
    kind: str
    key: str
    offset: int
    capacity: int


class BufferPlan:
    """Everything the backend needs to run the graph on one device."""

    def __init__(self, graph: OnnxGraph, live_from: Optional[Dict[str, int]] = None) -> None:
        self.graph = graph
        self.layouts = compute_tensor_layouts(graph)
        self.pool_entries, self.pool_elems = pool_layout(graph, self.layouts, live_from)
        self.aliases = reshape_aliases(graph)
        inputs = {t.onnx_name for t in graph.input_tensors}
        outputs = {t.onnx_name for t in graph.output_tensors}
        inter = {t.onnx_name for t in graph.intermediate_tensors}

        # graph outputs produced by a reshape chain over kernel outputs: the kernel writes
        # straight into the caller's buffer (_core.py:498-534)
        self.redirect: Dict[str, str] = {}
        for o in graph.output_tensors:
            cur = self.aliases.get(o.onnx_name)
            while cur is not None and cur in inter:
                self.redirect[cur] = o.onnx_name
                cur = self.aliases.get(cur)
        # graph outputs that are reshapes of graph inputs: copied after the kernels
        # (_core.py:462-496)
        self.input_copies: List[Tuple[str, str]] = []
        for o in graph.output_tensors:
            cur = o.onnx_name
            while cur in self.aliases:
                src = self.aliases[cur]
                if src in inputs:
                    self.input_copies.append((o.onnx_name, src))
                    break
                if src not in inter:
                    break
                cur = src

        pool = {n: (off, a) for n, off, a in self.pool_entries}
        self.storage: Dict[str, Storage] = {}

        def resolve(name: str, depth: int = 0) -> Storage:
            if name in self.storage:
                return self.storage[name]
            if depth > len(self.aliases) + 1:
                raise SchedulerError(f"reshape alias cycle at '{name}'")
            if name in self.redirect:
                st = resolve(self.redirect[name], depth + 1)
            elif name in outputs:
                st = Storage("output", name, 0, self.layouts[name].alloc)
            elif name in self.aliases:
                st = resolve(self.aliases[name], depth + 1)
            elif name in pool:
                off, a = pool[name]
                st = Storage("pool", "", off, a)
            elif name in inputs:
                st = Storage("input", name, 0, self.layouts[name].alloc)
            else:
                raise SchedulerError(f"tensor '{name}' has no storage")
            self.storage[name] = st
            return st

        for name in self.layouts:
            resolve(name)

        self.calls: List[Tuple[int, KernelCall]] = []
        for sn in graph.nodes:
            for call in sn.calls(self.layouts):
                self.calls.append((sn.index, call))
        for out, src in self.input_copies:
            n = graph.get_tensor(out).numel
            self.calls.append((len(graph.nodes), KernelCall("op", (src, None, out),
                                                            (n, OP_COPY, 1, 0, 0))))
        self.check_extents()

    def check_extents(self) -> None:
        """Every call stays inside the storage of every tensor it touches."""
        for idx, call in self.calls:
            for name, need in call.extents().items():
                st = self.storage[name]
                if need > st.capacity:
                    raise SchedulerError(
                        f"node [{idx}] {call}: touches {need} elements of '{name}', whose "
                        f"buffer holds {st.capacity}")

    # ------------------------------------------------------------- host images

    def pool_image(self):
        """Initial contents of the pool: every weight at its offset (padded layouts
        get their data at the chunk positions, zeros in the gaps), the rest zero."""
        import numpy as np
        img = np.zeros(self.pool_elems, dtype=np.int16)
        for t in self.graph.weight_tensors:
            st = self.storage[t.onnx_name]
            lay = self.layouts[t.onnx_name]
            img[st.offset + lay.positions()] = t.storage()
        return img

    def scatter(self, name: str, raw, buf) -> None:
        """Write a tensor's logical raw int16 values into its buffer (padded layout aware)."""
        import numpy as np
        lay = self.layouts[name]
        raw = np.asarray(raw, dtype=np.int16).reshape(-1)
        if raw.size != lay.numel:
            raise ValueError(f"'{name}' needs {lay.numel} values, got {raw.size}")
        buf[lay.positions()] = raw

    def gather(self, name: str, buf):
        """A tensor's logical raw int16 values, in its shape, read from its buffer."""
        import numpy as np
        lay = self.layouts[name]
        shape = self.graph.get_tensor(name).shape
        return np.asarray(buf)[lay.positions()].astype(np.int16).reshape(shape or [1])

    def summary(self) -> str:
        lines = [f"pool: {self.pool_elems} elements ({self.pool_elems * BYTES_PER_ELEM} B)"]
        for n, off, a in self.pool_entries:
            lines.append(f"  {n:<32} offset {off:>10}  alloc {a}")
        for idx, call in self.calls:
            lines.append(f"  [{idx}] {call}")
        return "\n".join(lines)
