"""Epilogue fusion for the GPU backend.

The reference scheduler emits one kernel call per ONNX node, so a Conv followed
by Clip(0,6) is a run_conv writing an intermediate and a run_op reading it back
(inference-scheduler/src/nodes.py:227-453, 828-1119).  On the GPU the second
call costs a launch and a round trip of the intermediate through memory.  This
pass finds, in a buffer plan's call list, a MatMul / Conv call whose output is
read by nothing but the immediately following VectorOP call(s) and folds those
into the MatMul / Conv epilogue (``cm_matmul_ex`` / ``cm_conv_ex``):

    conv | matmul  ->  Add (same-shaped tensor)           [-> Relu | Clip(0,6)]
    matmul         ->  Add (bias row broadcast per column) [-> Relu | Clip(0,6)]
    conv | matmul  ->  Relu | Clip(0,6)

The fused epilogue computes exactly what the unfused calls compute (the same
saturating Add and clamp applied to the same saturated value), so the graph's
outputs are bit-identical; only the intermediate is never materialised.

A fused call writes its final output while it still reads its inputs, so that
output must not share memory with them.  ``live_from`` gives each fused
output's new first-use node (the MatMul / Conv node) for the pool layout, which
then never places it in a slot its inputs occupy; ``fusions`` re-checks the
actual storage of every fused group and drops any group that overlaps.

Convolution pairs: a Conv (with its Relu / Clip(0,6)) whose output nothing but
a 1x1 Conv (with its Add / activation) reads can run as one launch
(``cm_conv_pair_packed_ex``) that keeps the middle tensor on chip:

    conv [-> Relu | Clip(0,6)] -> conv 1x1 [-> Add (same-shaped)] [-> Relu | Clip(0,6)]

``launch_list(plan, pair_ok)`` forms them where ``pair_ok`` (the backend's
shape check) accepts the pair; the result is the same bit for bit.

Pooled heads: a 1x1 Conv (with its Relu / Clip(0,6)) whose output nothing but a
GlobalAveragePool reads runs as one launch (``cm_conv_gap``) that averages the
activated outputs without storing them:

    conv 1x1 [-> Relu | Clip(0,6)] -> GlobalAveragePool

``launch_list(plan, pair_ok, gap_ok)`` forms them where ``gap_ok`` accepts the
shape.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Dict, List, Optional, Set, Tuple

from .nodes import OP_ADD, OP_RELU, OP_RELU6, KernelCall

ADD_NONE, ADD_SAME, ADD_COLUMN = 0, 1, 2
ACT_NONE, ACT_RELU, ACT_RELU6 = 0, 1, 2
_ACT_OF_OP = {OP_RELU: ACT_RELU, OP_RELU6: ACT_RELU6}


@dataclass(frozen=True)
class FusedCall:
    """A MatMul / Conv call with the VectorOP calls folded into its epilogue."""
    call: KernelCall                 # the MatMul / Conv call (its output tensor is bypassed)
    absorbed: Tuple[KernelCall, ...]  # the VectorOP calls it replaces, in order
    out: str                         # tensor the fused call writes (last absorbed call's output)
    add: Optional[str]               # tensor added in the epilogue
    add_mode: int
    act: int

    def __str__(self) -> str:
        return " + ".join(str(c) for c in (self.call,) + self.absorbed)


def _call_of(item) -> KernelCall:
    return item.call if isinstance(item, FusedCall) else item


def _absorbed(item) -> Tuple[KernelCall, ...]:
    return item.absorbed if isinstance(item, FusedCall) else ()


def _out_of(item) -> str:
    return item.out if isinstance(item, FusedCall) else _writes(item)


@dataclass(frozen=True)
class PairCall:
    """A convolution group and the 1x1 convolution group that alone reads its
    output, as one launch.  ``call`` / ``absorbed`` list the member calls in
    order (the first convolution, its activation, the 1x1 convolution, its Add
    and activation), like a fused group's."""
    first: object    # KernelCall or FusedCall: the convolution (activation only)
    second: object   # KernelCall or FusedCall: the 1x1 convolution (same-shaped Add, activation)

    @property
    def call(self) -> KernelCall:
        return _call_of(self.first)

    @property
    def absorbed(self) -> Tuple[KernelCall, ...]:
        return _absorbed(self.first) + (_call_of(self.second),) + _absorbed(self.second)

    @property
    def out(self) -> str:
        return _out_of(self.second)

    @property
    def act1(self) -> int:
        return self.first.act if isinstance(self.first, FusedCall) else ACT_NONE

    def __str__(self) -> str:
        return " + ".join(str(c) for c in (self.call,) + self.absorbed)


@dataclass(frozen=True)
class GapCall:
    """A 1x1 convolution group and the GlobalAveragePool that alone reads its
    output, as one launch (``call`` / ``absorbed``: the convolution, its
    activation, the pool)."""
    first: object     # KernelCall or FusedCall: the 1x1 convolution (activation only)
    pool: KernelCall  # the GlobalAveragePool

    @property
    def call(self) -> KernelCall:
        return _call_of(self.first)

    @property
    def absorbed(self) -> Tuple[KernelCall, ...]:
        return _absorbed(self.first) + (self.pool,)

    @property
    def out(self) -> str:
        return _writes(self.pool)

    @property
    def act(self) -> int:
        return self.first.act if isinstance(self.first, FusedCall) else ACT_NONE

    def __str__(self) -> str:
        return " + ".join(str(c) for c in (self.call,) + self.absorbed)


def _reads(call: KernelCall) -> List[str]:
    t = call.tensors
    if call.kernel == "op":
        names = [t[0], t[1]] if call.args[1] < OP_RELU else [t[0]]
    elif call.kernel in ("matmul", "matmul_at"):
        names = [t[0], t[1]]
    elif call.kernel == "conv":
        names = [t[0], t[1], t[2]]
    elif call.kernel == "pool":
        names = [t[0]]
    else:
        raise ValueError(f"unknown kernel '{call.kernel}'")
    return [n for n in names if n is not None]


def _writes(call: KernelCall) -> str:
    return call.tensors[3] if call.kernel == "conv" else call.tensors[-1]


def _written_count(call: KernelCall) -> Optional[int]:
    """Elements of one contiguous block the call writes from its output base, or
    None when the output has gaps (strided batches) or an element offset."""
    if call.kernel == "conv":
        nb, _c, _h, _w, mo, oh, ow = call.args[:7]
        return nb * mo * oh * ow
    n, _k, m, batch, _a, _b, c_bs = call.args
    if call.offsets and call.offsets[2]:
        return None
    if batch == 1 or c_bs == 0:
        return n * m
    return batch * n * m if c_bs == n * m else None


class _Graph:
    """Readers / writers of every tensor root (reshape aliases resolved)."""

    def __init__(self, plan) -> None:
        self.plan = plan
        self.calls = [c for _, c in plan.calls]
        self.readers: Dict[str, Set[int]] = {}
        self.writers: Dict[str, Set[int]] = {}
        for i, c in enumerate(self.calls):
            for n in _reads(c):
                self.readers.setdefault(self.root(n), set()).add(i)
            self.writers.setdefault(self.root(_writes(c)), set()).add(i)
        self.outputs = {self.root(t.onnx_name) for t in plan.graph.output_tensors}

    def root(self, name: str) -> str:
        seen = 0
        while name in self.plan.aliases and seen <= len(self.plan.aliases):
            name = self.plan.aliases[name]
            seen += 1
        return name

    def private(self, name: str, writer: int, reader: int) -> bool:
        """`name` is written only by call `writer`, read only by call `reader`,
        and is not (a view of) a graph output."""
        r = self.root(name)
        return (name not in self.plan.redirect and r not in self.outputs and
                self.writers.get(r) == {writer} and self.readers.get(r) == {reader})


def _match(g: _Graph, k: int) -> Optional[FusedCall]:
    calls = g.calls
    c = calls[k]
    if c.kernel not in ("matmul", "matmul_at", "conv") or k + 1 >= len(calls):
        return None
    count = _written_count(c)
    t = _writes(c)
    nxt = calls[k + 1]
    if nxt.kernel != "op" or not g.private(t, k, k + 1):
        return None
    size, op, outer, a_inc, b_inc = nxt.args
    a, b, y = nxt.tensors
    if op in _ACT_OF_OP:
        if a != t or outer != 1 or size != count:
            return None
        return FusedCall(c, (nxt,), y, None, ADD_NONE, _ACT_OF_OP[op])
    if op != OP_ADD or (a == t) == (b == t):
        return None
    other = b if a == t else a
    if count is not None and outer == 1 and size == count:
        mode = ADD_SAME
    elif c.kernel != "conv" and _column_add(c, size, outer, a_inc if a == t else b_inc,
                                            b_inc if a == t else a_inc):
        mode = ADD_COLUMN   # MatMul rows + bias[m] broadcast over them
        count = outer * size if (a_inc if a == t else b_inc) == size else None
    else:
        return None
    fused = FusedCall(c, (nxt,), y, other, mode, ACT_NONE)
    if k + 2 < len(calls) and count is not None:
        act = calls[k + 2]
        if act.kernel == "op":
            size2, op2, outer2, _, _ = act.args
            if (op2 in _ACT_OF_OP and act.tensors[0] == y and outer2 == 1 and
                    size2 == count and g.private(y, k + 1, k + 2)):
                fused = FusedCall(c, (nxt, act), act.tensors[2], other, mode, _ACT_OF_OP[op2])
    return fused


def _column_add(c: KernelCall, size: int, outer: int, t_inc: int, o_inc: int) -> bool:
    """The broadcast Add walks the MatMul's output rows in order (row stride
    t_inc, the same stride for its own output) adding one row vector: each
    output row r of batch z sits at z*c_stride + r*m."""
    n, _k, m, batch, _a, _b, c_bs = c.args
    if o_inc != 0 or size != m or (c.offsets and c.offsets[2]):
        return False
    if batch == 1:
        return outer == n and t_inc == m
    return n == 1 and outer == batch and t_inc == c_bs


def candidates(plan) -> List[Tuple[int, FusedCall]]:
    """(index of the MatMul / Conv call in plan.calls, fused group) for every
    group the call structure allows, without looking at storage."""
    g = _Graph(plan)
    out: List[Tuple[int, FusedCall]] = []
    k = 0
    while k < len(g.calls):
        f = _match(g, k)
        if f is not None:
            out.append((k, f))
            k += 1 + len(f.absorbed)
        else:
            k += 1
    return out


def _indexed(plan, groups: Dict[int, FusedCall]) -> List[Tuple[int, object]]:
    """(index in plan.calls of the item's first call, item) with `groups` in place."""
    seq: List[Tuple[int, object]] = []
    calls = [c for _, c in plan.calls]
    k = 0
    while k < len(calls):
        if k in groups:
            seq.append((k, groups[k]))
            k += 1 + len(groups[k].absorbed)
        else:
            seq.append((k, calls[k]))
            k += 1
    return seq


def _pair_match(g: _Graph, ka: int, a, kb: int, b) -> Optional[PairCall]:
    """The pair of items a (plan index ka) and b (plan index kb), or None."""
    ca, cb = _call_of(a), _call_of(b)
    if ca.kernel != "conv" or cb.kernel != "conv" or any(ca.offsets or ()) or any(cb.offsets or ()):
        return None
    n, _c, _h, _w, m, oh, ow, kh, kw, sh, sw, dh, dw, _pt, _pl, _hb, dwise = ca.args
    if dwise or kh * kw < 2 or sh != sw or dh != dw:
        return None
    if isinstance(a, FusedCall) and a.add is not None:
        return None
    n2, c2, h2, w2, _m2, oh2, ow2, kh2, kw2, sh2, sw2, dh2, dw2, pt2, pl2, _hb2, dwise2 = cb.args
    if dwise2 or (kh2, kw2, sh2, sw2, dh2, dw2, pt2, pl2) != (1, 1, 1, 1, 1, 1, 0, 0):
        return None
    if (n2, c2, h2, w2, oh2, ow2) != (n, m, oh, ow, oh, ow):
        return None
    if isinstance(b, FusedCall) and b.add_mode not in (ADD_NONE, ADD_SAME):
        return None
    mid = _out_of(a)
    if cb.tensors[0] != mid or not g.private(mid, ka + len(_absorbed(a)), kb):
        return None
    return PairCall(a, b)


def _pairs(plan, seq: List[Tuple[int, object]]) -> List[Tuple[int, PairCall]]:
    """Every pair the call structure allows in seq (no storage or shape check)."""
    g = _Graph(plan)
    out: List[Tuple[int, PairCall]] = []
    i = 0
    while i + 1 < len(seq):
        pc = _pair_match(g, seq[i][0], seq[i][1], seq[i + 1][0], seq[i + 1][1])
        if pc is not None:
            out.append((i, pc))
            i += 2
        else:
            i += 1
    return out


def _gap_match(g: _Graph, ka: int, a, kb: int, b) -> Optional[GapCall]:
    """The pooled head of items a (plan index ka) and b (plan index kb), or None."""
    if isinstance(b, (FusedCall, PairCall)) or isinstance(a, PairCall):
        return None
    ca = _call_of(a)
    if ca.kernel != "conv" or b.kernel != "pool" or any(ca.offsets or ()) or any(b.offsets or ()):
        return None
    n, _c, h, w, m, oh, ow, kh, kw, sh, sw, dh, dw, pt, pl, _hb, dwise = ca.args
    if dwise or (kh, kw, sh, sw, dh, dw, pt, pl) != (1, 1, 1, 1, 1, 1, 0, 0) or (oh, ow) != (h, w):
        return None
    if isinstance(a, FusedCall) and a.add is not None:
        return None
    pb, pc, ph, pw, poh, pow_, kph, kpw, _psh, _psw, ppt, ppl, pdh, pdw, ptype = b.args[:15]
    if (pb, pc, ph, pw) != (n, m, oh, ow) or (poh, pow_, kph, kpw) != (1, 1, oh, ow):
        return None
    if (ppt, ppl, pdh, pdw, ptype) != (0, 0, 1, 1, 1):
        return None
    mid = _out_of(a)
    if b.tensors[0] != mid or not g.private(mid, ka + len(_absorbed(a)), kb):
        return None
    return GapCall(a, b)


def _gaps(plan, seq: List[Tuple[int, object]]) -> List[Tuple[int, GapCall]]:
    """Every pooled head the call structure allows in seq (no storage or shape check)."""
    g = _Graph(plan)
    out: List[Tuple[int, GapCall]] = []
    for i in range(len(seq) - 1):
        gc = _gap_match(g, seq[i][0], seq[i][1], seq[i + 1][0], seq[i + 1][1])
        if gc is not None:
            out.append((i, gc))
    return out


def live_from(plan) -> Dict[str, int]:
    """{fused or paired output tensor: node index of its first MatMul / Conv} for
    the pool layout."""
    node_of = [idx for idx, _ in plan.calls]
    cands = candidates(plan)
    starts = {f.out: node_of[k] for k, f in cands}
    seq = _indexed(plan, dict(cands))
    for i, pc in _pairs(plan, seq):
        starts[pc.out] = node_of[seq[i][0]]
    for i, gc in _gaps(plan, seq):
        starts[gc.out] = node_of[seq[i][0]]
    return starts


def _span(plan, call: KernelCall, name: str) -> Tuple[str, str, int, int]:
    """(allocation kind, key, first element, end element) a call touches of `name`."""
    st = plan.storage[name]
    i = call.tensors.index(name)
    off = st.offset + (call.offsets[i] if call.offsets else 0)
    return st.kind, st.key, off, st.offset + call.extents()[name]


def _overlap(x, y) -> bool:
    return x[0] == y[0] and x[1] == y[1] and x[2] < y[3] and y[2] < x[3]


def fusions(plan) -> List[Tuple[int, FusedCall]]:
    """The candidate groups whose fused output does not overlap anything the
    fused call reads (an Add operand may coincide with it exactly: in place)."""
    ok = []
    for k, f in candidates(plan):
        last = f.absorbed[-1]
        out = _span(plan, last, f.out)
        inputs = [_span(plan, f.call, n) for n in _reads(f.call)]
        if any(_overlap(out, s) for s in inputs):
            continue
        if f.add is not None:
            add = _span(plan, f.absorbed[0], f.add)
            if _overlap(out, add) and not (f.add_mode == ADD_SAME and add[2] == out[2]):
                continue
        ok.append((k, f))
    return ok


def _pair_storage_ok(plan, pc: PairCall) -> bool:
    """The pair's output overlaps nothing the launch reads (its Add operand may
    coincide with it exactly: in place)."""
    cb = _call_of(pc.second)
    out = _span(plan, pc.absorbed[-1], pc.out)
    ins = [_span(plan, pc.call, n) for n in _reads(pc.call)]
    ins += [_span(plan, cb, n) for n in _reads(cb) if n != cb.tensors[0]]
    if any(_overlap(out, s) for s in ins):
        return False
    b = pc.second
    if isinstance(b, FusedCall) and b.add is not None:
        add = _span(plan, b.absorbed[0], b.add)
        if _overlap(out, add) and add[2] != out[2]:
            return False
    return True


def _gap_storage_ok(plan, gc: GapCall) -> bool:
    """The pooled output overlaps nothing the convolution reads."""
    out = _span(plan, gc.pool, gc.out)
    return not any(_overlap(out, _span(plan, gc.call, n)) for n in _reads(gc.call))


def launch_list(plan, pair_ok: Optional[Callable[[PairCall], bool]] = None,
                gap_ok: Optional[Callable[[GapCall], bool]] = None) -> List[object]:
    """plan.calls with every fusable group replaced by its FusedCall and, when
    ``pair_ok`` is given, every convolution pair it accepts by a PairCall; when
    ``gap_ok`` is given, every pooled head it accepts by a GapCall."""
    seq = _indexed(plan, dict(fusions(plan)))
    pairs = {} if pair_ok is None else {
        i: pc for i, pc in _pairs(plan, seq) if _pair_storage_ok(plan, pc) and pair_ok(pc)}
    gaps = {} if gap_ok is None else {
        i: gc for i, gc in _gaps(plan, seq) if _gap_storage_ok(plan, gc) and gap_ok(gc)}
    out: List[object] = []
    i = 0
    while i < len(seq):
        if i in pairs:
            out.append(pairs[i])
            i += 2
        elif i in gaps:
            out.append(gaps[i])
            i += 2
        else:
            out.append(seq[i][1])
            i += 1
    return out
