"""HIP backend of the scheduler: run a scheduled ONNX graph on one GPU.

Replaces the generated KV260 runtime (inference_init / inference_run,
inference-scheduler/src/codegen/_source.py:475-791) with calls into
libcormorant_amd.so:

* init: one ``cm_buf_alloc`` for the pool (weights + intermediates, 64-byte
  aligned slots, intermediates with disjoint lifetimes sharing a slot, then
  the split-K workspace the MatMul / Conv calls share, then each patch-GEMM
  convolution's packed weights), one buffer per graph input and output,
  weights copied in once and packed once (``cm_conv_pack``);
* run: graph inputs copied to the device, every kernel call enqueued in graph
  order on one in-order stream, graph outputs copied back (the only host
  synchronisation, as in the reference's sync_from_device).

Reshape / Squeeze / Unsqueeze / Dropout outputs are the same device address
as their source; a graph output at the end of a reshape chain is written
directly by the producing kernel.  With ``fuse=True`` (default) an Add /
Relu / Clip(0,6) call that is the sole reader of a MatMul / Conv output runs
in that call's epilogue, and a convolution whose output only a 1x1
convolution reads runs with it as one launch (``cm_conv_pair_packed_ex``,
weights packed at init; ``fuse.py``), and a 1x1 convolution whose output only a
GlobalAveragePool reads runs with it as one launch (``cm_conv_gap``); results
are bit-identical either way.
There is no CPU execution path: without the native library the constructor
raises.
"""
from __future__ import annotations

import ctypes
from typing import Dict, List, Optional, Tuple

import numpy as np

from .. import _native
from . import fuse as _fuse
from .graph import OnnxGraph
from .nodes import KernelCall
from .plan import BufferPlan

_FUNCS = {"op": "cm_vectorop", "matmul": "cm_matmul", "matmul_at": "cm_matmul",
          "conv": "cm_conv", "pool": "cm_pool"}
_EX_FUNCS = {"matmul": "cm_matmul_ex", "matmul_at": "cm_matmul_ex", "conv": "cm_conv_ex"}


class InferenceSession:
    """Device-resident instance of one model (weights loaded, buffers allocated)."""

    def __init__(self, model, stream: int = 0, fuse: bool = True) -> None:
        self.graph = model if isinstance(model, OnnxGraph) else OnnxGraph(model)
        self.plan = BufferPlan(self.graph)
        self._lib = _native.load()
        if fuse:
            starts = _fuse.live_from(self.plan)
            if starts:
                self.plan = BufferPlan(self.graph, starts)
            self.launch_list = _fuse.launch_list(self.plan, pair_ok=lambda pc: self._packed_size(pc) > 0,
                                                 gap_ok=self._gap_ok)
        else:
            self.launch_list = [c for _, c in self.plan.calls]
        self.stream = int(stream)
        _native.call("cm_buf_pool_init")
        self._bufs: Dict[Tuple[str, str], object] = {}
        self.workspace_bytes = 0
        self._ws_ptr: Optional[int] = None
        self._packed: Dict[int, Tuple[int, int]] = {}   # launch index -> (pool byte offset, bytes)
        try:
            # convolutions on the patch-GEMM path get their weights packed once
            packed_sizes = [self._packed_size(c) for c in self.launch_list]
            # split-K workspace: one region after the pool's tensors, as large as
            # the largest need over the other calls (the calls run one after
            # another on one stream, so they share it)
            self.workspace_bytes = max((self._workspace_need(c) for c, ps in
                                        zip(self.launch_list, packed_sizes) if not ps), default=0)
            ws_off = -(-self.plan.pool_elems // 128) * 128   # 256-byte aligned
            end = 2 * ws_off + self.workspace_bytes
            for i, ps in enumerate(packed_sizes):
                if ps:
                    end = -(-end // 256) * 256
                    self._packed[i] = (end, ps)
                    end += ps
            total = -(-end // 2) if (self.workspace_bytes or self._packed) else self.plan.pool_elems
            if total:
                pool = self._alloc(("pool", ""), total)
                self._host(pool, total)[:self.plan.pool_elems] = self.plan.pool_image()
                _native.call("cm_buf_sync_to_device", pool)
                base = int(pool.contents.dev)
                if self.workspace_bytes:
                    self._ws_ptr = base + 2 * ws_off
                for i, (off, ps) in self._packed.items():
                    item = self.launch_list[i]
                    call = self._call_of(item)
                    wptr = self.device_ptr(call.tensors[1]) + (2 * call.offsets[1] if call.offsets else 0)
                    if isinstance(item, _fuse.PairCall):
                        w2ptr = self.device_ptr(self._call_of(item.second).tensors[1])
                        _native.call("cm_conv_pair_pack", wptr, w2ptr, *self._pair_args(item), base + off,
                                     ps, None)
                    else:
                        _native.call("cm_conv_pack", wptr, *call.args, base + off, ps, None)
            for t in self.graph.input_tensors:
                self._alloc(("input", t.onnx_name), self.plan.layouts[t.onnx_name].alloc)
            for t in self.graph.output_tensors:
                self._alloc(("output", t.onnx_name), self.plan.layouts[t.onnx_name].alloc)
            _native.call("cm_sync", None)
            self._launches = [self._prepare(c, i) for i, c in enumerate(self.launch_list)]
        except Exception:
            self.close()
            raise

    # ------------------------------------------------------------------ buffers

    def _alloc(self, key, n: int):
        if n >= 1 << 32:
            raise ValueError(f"buffer {key} of {n} elements exceeds the uint32 element count")
        b = self._lib.cm_buf_alloc(n)
        if not b:
            raise _native.CmError("cm_buf_alloc", _native.CM_ERR_NOMEM, _native.last_error())
        self._bufs[key] = b
        return b

    @staticmethod
    def _host(buf, n: int) -> np.ndarray:
        p = buf.contents.host
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_int16)), shape=(n,))

    def device_ptr(self, name: str) -> int:
        """Device address of a tensor's storage (graph inputs/outputs, weights, intermediates)."""
        st = self.plan.storage[name]
        buf = self._bufs[(st.kind, st.key)]
        return int(buf.contents.dev) + 2 * st.offset

    def _pointers(self, call: KernelCall):
        ptrs = []
        for i, name in enumerate(call.tensors):
            if name is None:
                ptrs.append(None)
                continue
            p = self.device_ptr(name)
            if call.offsets:
                p += 2 * call.offsets[i]
            ptrs.append(p)
        return ptrs

    @staticmethod
    def _call_of(item) -> KernelCall:
        return item.call if isinstance(item, (_fuse.FusedCall, _fuse.PairCall, _fuse.GapCall)) else item

    def _gap_ok(self, gc) -> bool:
        a = gc.call.args
        return bool(self._lib.cm_conv_gap_supported(a[0], a[1], a[2] * a[3], a[4]))

    @classmethod
    def _pair_args(cls, pc) -> Tuple[int, ...]:
        """cm_conv_pair_* shape arguments: batch, in_ch, in_h, in_w, mid_ch, out_h,
        out_w, kh, kw, stride, dilation, pad_top, pad_left, out_ch."""
        a = pc.call.args
        return (a[0], a[1], a[2], a[3], a[4], a[5], a[6], a[7], a[8], a[9], a[11], a[13], a[14],
                cls._call_of(pc.second).args[4])

    def _packed_size(self, item) -> int:
        if isinstance(item, _fuse.GapCall):
            return 0
        if isinstance(item, _fuse.PairCall):
            return int(self._lib.cm_conv_pair_packed_size(*self._pair_args(item)))
        call = self._call_of(item)
        if call.kernel != "conv":
            return 0
        return int(self._lib.cm_conv_packed_size(*call.args))

    def _workspace_need(self, item) -> int:
        if isinstance(item, (_fuse.PairCall, _fuse.GapCall)):
            return 0
        call = item.call if isinstance(item, _fuse.FusedCall) else item
        if call.kernel in ("matmul", "matmul_at"):
            return int(self._lib.cm_matmul_workspace_size(*call.args))
        if call.kernel == "conv":
            return int(self._lib.cm_conv_workspace_size(*call.args))
        return 0

    def _prepare(self, item, index: int):
        ws = (self._ws_ptr, self.workspace_bytes) if self._ws_ptr else (None, 0)
        packed = self._packed.get(index)
        if packed is not None:   # packed weights in place of the weight tensor, no workspace
            ws = ()
        if isinstance(item, _fuse.GapCall):
            ca = item.call
            a = ca.args
            name = "cm_conv_gap"
            args = (self.device_ptr(ca.tensors[0]), self.device_ptr(ca.tensors[1]),
                    self.device_ptr(ca.tensors[2]) if a[15] else None, self.device_ptr(item.out),
                    a[0], a[1], a[2] * a[3], a[4], item.act)
            return getattr(self._lib, name), name, args, None
        if isinstance(item, _fuse.PairCall):
            ca, cb = item.call, self._call_of(item.second)
            epi = None
            if isinstance(item.second, _fuse.FusedCall):
                epi = _native.CmEpilogue()
                epi.add = self.device_ptr(item.second.add) if item.second.add is not None else None
                epi.add_mode = item.second.add_mode
                epi.act = item.second.act
            name = "cm_conv_pair_packed_ex"
            args = (self.device_ptr(ca.tensors[0]),
                    int(self._bufs[("pool", "")].contents.dev) + packed[0],
                    self.device_ptr(ca.tensors[2]) if ca.args[15] else None,
                    self.device_ptr(cb.tensors[2]) if cb.args[15] else None,
                    self.device_ptr(item.out)) + self._pair_args(item) + (
                        item.act1, ctypes.byref(epi) if epi is not None else None)
            return getattr(self._lib, name), name, args, epi
        if isinstance(item, _fuse.FusedCall):
            call = item.call
            name = "cm_conv_ex" if call.kernel == "conv" else "cm_matmul_ex"
            ptrs = self._pointers(call)
            ptrs[-1] = self.device_ptr(item.out)   # the output of the last absorbed call
            epi = _native.CmEpilogue()
            epi.add = self.device_ptr(item.add) if item.add is not None else None
            epi.add_mode = item.add_mode
            epi.act = item.act
            if packed is not None:
                name = "cm_conv_packed_ex"
                ptrs[1] = int(self._bufs[("pool", "")].contents.dev) + packed[0]
            # the epilogue object rides along in the tuple so it outlives the pointer
            return getattr(self._lib, name), name, tuple(ptrs) + tuple(call.args) + (
                ctypes.byref(epi),) + ws, epi
        if packed is not None:
            name = "cm_conv_packed_ex"
            ptrs = self._pointers(item)
            ptrs[1] = int(self._bufs[("pool", "")].contents.dev) + packed[0]
            return getattr(self._lib, name), name, tuple(ptrs) + tuple(item.args) + (None,), None
        if item.kernel in _EX_FUNCS:   # MatMul / Conv: the _ex form carries the workspace
            name = _EX_FUNCS[item.kernel]
            return (getattr(self._lib, name), name,
                    tuple(self._pointers(item)) + tuple(item.args) + (None,) + ws, None)
        fn = getattr(self._lib, _FUNCS[item.kernel])
        return fn, _FUNCS[item.kernel], tuple(self._pointers(item)) + tuple(item.args), None

    # ------------------------------------------------------------------ running

    def launch(self, stream: Optional[int] = None) -> None:
        """Enqueue every kernel of the graph (inputs must already be on the device)."""
        s = self.stream if stream is None else int(stream)
        s = s or None
        for fn, name, args, _keep in self._launches:
            rc = fn(*args, s)
            if rc:
                raise _native.CmError(name, rc, _native.last_error())

    def write_input(self, name: str, raw) -> None:
        """Copy one graph input (raw int16 Q8.8, logical shape) to the device."""
        buf = self._bufs[("input", name)]
        host = self._host(buf, self.plan.layouts[name].alloc)
        self.plan.scatter(name, raw, host)
        _native.call("cm_buf_sync_to_device", buf)

    def read_output(self, name: str) -> np.ndarray:
        """Wait for the stream and return one graph output (raw int16, logical shape)."""
        buf = self._bufs[("output", name)]
        _native.call("cm_buf_sync_from_device", buf)
        return self.plan.gather(name, self._host(buf, self.plan.layouts[name].alloc))

    def run(self, feeds: Dict[str, np.ndarray]) -> Dict[str, np.ndarray]:
        """inference_run: raw int16 inputs -> raw int16 outputs, by tensor name."""
        missing = [t.onnx_name for t in self.graph.input_tensors if t.onnx_name not in feeds]
        if missing:
            raise KeyError(f"missing graph inputs: {missing}")
        prev = self._lib.cm_get_stream()
        if self.stream:
            self._lib.cm_set_stream(self.stream)
        try:
            for t in self.graph.input_tensors:
                self.write_input(t.onnx_name, feeds[t.onnx_name])
            self.launch()
            return {t.onnx_name: self.read_output(t.onnx_name) for t in self.graph.output_tensors}
        finally:
            if self.stream:
                self._lib.cm_set_stream(prev)

    @property
    def kernel_calls(self) -> List[KernelCall]:
        return [c for _, c in self.plan.calls]

    def close(self) -> None:
        for b in self._bufs.values():
            self._lib.cm_buf_free(b)
        self._bufs = {}

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
