"""Python mirror of the four Cormorant kernel entry points, on device tensors.

Each function takes int16 tensors resident on the GPU (raw ap_fixed<16,8>
bits) plus the reference kernel's scalar arguments in the reference's order,
checks on the host that every tensor covers the elements the kernel will
touch (so a bad call is an exception, never an out-of-bounds access), and
enqueues the gfx950 kernel through the C ABI on the current torch stream.

    VectorOPKernel  kernels/vectorop/include/VectorOP.h:86-95
    MatmulKernel    kernels/matmul/include/MatmulKernel.h:68-79
    ConvKernel      kernels/conv/include/ConvKernel.h:79-101
    PoolingKernel   kernels/pool/include/PoolingKernel.h:63-83
"""
from __future__ import annotations

import ctypes

from . import _native

OP_ADD, OP_SUB, OP_MUL, OP_DIV, OP_RELU, OP_RELU6 = range(6)
POOL_MAX, POOL_AVG, POOL_LP = 0, 1, 2


def _stream(stream=None) -> int:
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return int(stream.cuda_stream) if hasattr(stream, "cuda_stream") else int(stream)


def _dev_ptr(t, need: int, name: str) -> int:
    """Device address of int16 tensor t after checking it holds `need` elements."""
    import torch
    if t is None:
        raise ValueError(f"{name} is None")
    if t.dtype != torch.int16:
        raise TypeError(f"{name} must be int16 (raw Q8.8), got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.numel() < need:
        raise ValueError(f"{name} has {t.numel()} elements, the kernel reads/writes {need}")
    return int(t.data_ptr())


def _u32(name: str, v: int) -> int:
    v = int(v)
    if v < 0 or v > 0xFFFFFFFF:
        raise ValueError(f"{name}={v} is not a uint32")
    return v


def VectorOPKernel(a, b, c, size, op, outer=1, a_inc=0, b_inc=0, stream=None) -> None:
    """c[o*(a_inc+b_inc)+i] = op(a[o*a_inc+i], b[o*b_inc+i]) for o < outer, i < size."""
    size, op, outer = _u32("size", size), _u32("op", op), _u32("outer", outer)
    a_inc, b_inc = _u32("a_inc", a_inc), _u32("b_inc", b_inc)
    if size == 0 or outer == 0:
        return
    pa = _dev_ptr(a, (outer - 1) * a_inc + size, "a")
    pb = _dev_ptr(b, (outer - 1) * b_inc + size, "b") if op < OP_RELU else (
        int(b.data_ptr()) if b is not None else None)
    pc = _dev_ptr(c, (outer - 1) * (a_inc + b_inc) + size, "c")
    _native.call("cm_vectorop", pa, pb, pc, size, op, outer, a_inc, b_inc, _stream(stream))


ACT_NONE, ACT_RELU, ACT_RELU6 = 0, 1, 2


def _epilogue(add, column: bool, act: int, need: int):
    """cm_epilogue_t for a fused Add (same layout as the output, or one value per
    output column) and activation; None when neither is requested."""
    if add is None and not act:
        return None
    if act not in (ACT_NONE, ACT_RELU, ACT_RELU6):
        raise ValueError(f"act={act} is not ACT_NONE / ACT_RELU / ACT_RELU6")
    e = _native.CmEpilogue()
    e.act = act
    if add is not None:
        e.add = _dev_ptr(add, need, "add")
        e.add_mode = _native.CM_EPI_ADD_COLUMN if column else _native.CM_EPI_ADD_SAME
    return e


def _workspace(ws):
    """(device address, bytes) of a split-K workspace tensor (any dtype), or (None, 0)."""
    if ws is None:
        return None, 0
    if not ws.is_cuda or not ws.is_contiguous():
        raise ValueError("workspace must be a contiguous device tensor")
    return int(ws.data_ptr()), int(ws.numel() * ws.element_size())


def matmul_workspace_size(n, k, m, batch=1, a_batch_stride=0, b_batch_stride=0,
                          c_batch_stride=0) -> int:
    """Bytes of split-K workspace MatmulKernel(..., workspace=) uses for this shape."""
    return int(_native.load().cm_matmul_workspace_size(
        *(_u32("matmul arg", v) for v in (n, k, m, batch, a_batch_stride, b_batch_stride,
                                           c_batch_stride))))


def conv_workspace_size(batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, stride_h=1,
                        stride_w=1, dilation_h=1, dilation_w=1, pad_top=0, pad_left=0,
                        has_bias=0, is_depthwise=0) -> int:
    """Bytes of split-K workspace ConvKernel(..., workspace=) uses for this shape."""
    args = [batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, stride_h, stride_w,
            dilation_h, dilation_w, pad_top, pad_left, int(bool(has_bias)), int(bool(is_depthwise))]
    return int(_native.load().cm_conv_workspace_size(*(_u32("conv arg", v) for v in args)))


def MatmulKernel(a, b, c, n, k, m, batch=1, a_batch_stride=0, b_batch_stride=0,
                 c_batch_stride=0, stream=None, add=None, add_column=False, act=ACT_NONE,
                 workspace=None) -> None:
    """C_bi = sat16(wrap32(A_bi @ B_bi) >> 8), A_bi = a + bi*a_batch_stride, ...

    Optional fused epilogue: C = act(sat16(C + add)) with `add` laid out like C
    (or, with add_column, one value per column j), act = ACT_RELU / ACT_RELU6.
    `workspace`: a device tensor for split-K partial sums (see
    matmul_workspace_size); without one the call does not split."""
    n, k, m, batch = (_u32(x, v) for x, v in (("n", n), ("k", k), ("m", m), ("batch", batch)))
    a_bs, b_bs, c_bs = (_u32(x, v) for x, v in (("a_batch_stride", a_batch_stride),
                                                  ("b_batch_stride", b_batch_stride),
                                                  ("c_batch_stride", c_batch_stride)))
    if batch == 0 or n == 0 or m == 0:
        return
    pa = _dev_ptr(a, (batch - 1) * a_bs + n * k, "a") if k else None
    pb = _dev_ptr(b, (batch - 1) * b_bs + k * m, "b") if k else None
    pc = _dev_ptr(c, (batch - 1) * c_bs + n * m, "c")
    epi = _epilogue(add, add_column, act, m if add_column else (batch - 1) * c_bs + n * m)
    ws, ws_bytes = _workspace(workspace)
    _native.call("cm_matmul_ex", pa, pb, pc, n, k, m, batch, a_bs, b_bs, c_bs,
                 ctypes.byref(epi) if epi is not None else None, ws, ws_bytes, _stream(stream))


def ConvKernel(x, weight, bias, y, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw,
               stride_h=1, stride_w=1, dilation_h=1, dilation_w=1, pad_top=0, pad_left=0,
               has_bias=0, is_depthwise=0, stream=None, add=None, act=ACT_NONE,
               workspace=None) -> None:
    """ONNX Conv (group 1 or depthwise), NCHW, implicit bottom/right padding.

    Optional fused epilogue: y = act(sat16(y + add)), add shaped like y.
    `workspace`: a device tensor for split-K partial sums (see
    conv_workspace_size); without one the call does not split."""
    args = [batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, stride_h, stride_w,
            dilation_h, dilation_w, pad_top, pad_left, int(bool(has_bias)), int(bool(is_depthwise))]
    args = [_u32("conv arg", v) for v in args]
    if batch * out_ch * out_h * out_w == 0:
        return
    if is_depthwise and out_ch > in_ch:
        raise ValueError("depthwise conv needs out_ch <= in_ch")
    px = _dev_ptr(x, batch * in_ch * in_h * in_w, "x")
    pw = _dev_ptr(weight, out_ch * (1 if is_depthwise else in_ch) * kh * kw, "weight")
    pbias = _dev_ptr(bias, out_ch, "bias") if has_bias else None
    py = _dev_ptr(y, batch * out_ch * out_h * out_w, "y")
    epi = _epilogue(add, False, act, batch * out_ch * out_h * out_w)
    ws, ws_bytes = _workspace(workspace)
    _native.call("cm_conv_ex", px, pw, pbias, py, *args,
                 ctypes.byref(epi) if epi is not None else None, ws, ws_bytes, _stream(stream))


def conv_packed_size(batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, stride_h=1,
                     stride_w=1, dilation_h=1, dilation_w=1, pad_top=0, pad_left=0,
                     has_bias=0, is_depthwise=0) -> int:
    """Bytes of packed weights for ConvPackedKernel on this shape (0: the shape runs
    on another path and cannot use packed weights)."""
    args = [batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, stride_h, stride_w,
            dilation_h, dilation_w, pad_top, pad_left, int(bool(has_bias)), int(bool(is_depthwise))]
    return int(_native.load().cm_conv_packed_size(*(_u32("conv arg", v) for v in args)))


def conv_pack(weight, packed, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw,
              stride_h=1, stride_w=1, dilation_h=1, dilation_w=1, pad_top=0, pad_left=0,
              has_bias=0, is_depthwise=0, stream=None) -> None:
    """Pack `weight` (the ConvKernel layout) into the device tensor `packed` once."""
    args = [batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, stride_h, stride_w,
            dilation_h, dilation_w, pad_top, pad_left, int(bool(has_bias)), int(bool(is_depthwise))]
    args = [_u32("conv arg", v) for v in args]
    pw = _dev_ptr(weight, out_ch * in_ch * kh * kw, "weight")
    pp, nbytes = _workspace(packed)
    _native.call("cm_conv_pack", pw, *args, pp, nbytes, _stream(stream))


def ConvPackedKernel(x, packed, bias, y, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw,
                     stride_h=1, stride_w=1, dilation_h=1, dilation_w=1, pad_top=0, pad_left=0,
                     has_bias=0, is_depthwise=0, stream=None, add=None, act=ACT_NONE) -> None:
    """ConvKernel with weights packed earlier by conv_pack (same result bit for bit)."""
    args = [batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, stride_h, stride_w,
            dilation_h, dilation_w, pad_top, pad_left, int(bool(has_bias)), int(bool(is_depthwise))]
    args = [_u32("conv arg", v) for v in args]
    if batch * out_ch * out_h * out_w == 0:
        return
    px = _dev_ptr(x, batch * in_ch * in_h * in_w, "x")
    pp, _ = _workspace(packed)
    pbias = _dev_ptr(bias, out_ch, "bias") if has_bias else None
    py = _dev_ptr(y, batch * out_ch * out_h * out_w, "y")
    epi = _epilogue(add, False, act, batch * out_ch * out_h * out_w)
    _native.call("cm_conv_packed_ex", px, pp, pbias, py, *args,
                 ctypes.byref(epi) if epi is not None else None, _stream(stream))


def conv_gap_supported(batch, in_ch, hw, out_ch) -> bool:
    """Whether ConvGapKernel takes the shape (planes of at most 64 pixels, at most
    512 input channels)."""
    args = [_u32("conv gap arg", v) for v in (batch, in_ch, hw, out_ch)]
    return bool(_native.load().cm_conv_gap_supported(*args))


def ConvGapKernel(x, weight, bias, y, batch, in_ch, hw, out_ch, has_bias=1, act=ACT_NONE,
                  stream=None) -> None:
    """A 1x1 convolution (stride 1, no padding), its activation and a
    GlobalAveragePool of every output plane as one launch: y [batch][out_ch] equals
    ConvKernel(..., act) followed by PoolingKernel's global average, bit for bit."""
    args = [_u32("conv gap arg", v) for v in (batch, in_ch, hw, out_ch, act)]
    if batch * out_ch == 0:
        return
    px = _dev_ptr(x, batch * in_ch * hw, "x")
    pw = _dev_ptr(weight, out_ch * in_ch, "weight")
    pbias = _dev_ptr(bias, out_ch, "bias") if has_bias else None
    py = _dev_ptr(y, batch * out_ch, "y")
    _native.call("cm_conv_gap", px, pw, pbias, py, *args, _stream(stream))


def conv_pair_packed_size(batch, in_ch, in_h, in_w, mid_ch, out_h, out_w, kh, kw, stride,
                          dilation, pad_top, pad_left, out_ch) -> int:
    """Bytes of packed weights for ConvPairKernel: a kh x kw convolution in_ch -> mid_ch
    (stride and dilation the same on both axes) and a 1x1 convolution mid_ch -> out_ch
    of its output, in one launch (0: the shapes do not take that path)."""
    args = [batch, in_ch, in_h, in_w, mid_ch, out_h, out_w, kh, kw, stride, dilation, pad_top,
            pad_left, out_ch]
    return int(_native.load().cm_conv_pair_packed_size(*(_u32("conv pair arg", v) for v in args)))


def conv_pair_pack(w1, w2, packed, batch, in_ch, in_h, in_w, mid_ch, out_h, out_w, kh, kw, stride,
                   dilation, pad_top, pad_left, out_ch, stream=None) -> None:
    """Pack both convolutions' weights (ConvKernel layouts: [mid_ch][in_ch][kh][kw] and
    [out_ch][mid_ch]) into the device tensor `packed` once."""
    args = [batch, in_ch, in_h, in_w, mid_ch, out_h, out_w, kh, kw, stride, dilation, pad_top,
            pad_left, out_ch]
    args = [_u32("conv pair arg", v) for v in args]
    p1 = _dev_ptr(w1, mid_ch * in_ch * kh * kw, "w1")
    p2 = _dev_ptr(w2, out_ch * mid_ch, "w2")
    pp, nbytes = _workspace(packed)
    _native.call("cm_conv_pair_pack", p1, p2, *args, pp, nbytes, _stream(stream))


def ConvPairKernel(x, packed, bias1, bias2, y, batch, in_ch, in_h, in_w, mid_ch, out_h, out_w, kh,
                   kw, stride, dilation, pad_top, pad_left, out_ch, act1=ACT_NONE, add=None,
                   act=ACT_NONE, stream=None) -> None:
    """y = act(Add(Conv1x1(act1(Conv(x, w1, bias1)), w2, bias2), add)), with the weights
    packed by conv_pair_pack; the middle tensor never leaves the GPU's LDS.  The same
    result, bit for bit, as the two ConvKernel calls with their fused epilogues."""
    args = [batch, in_ch, in_h, in_w, mid_ch, out_h, out_w, kh, kw, stride, dilation, pad_top,
            pad_left, out_ch]
    args = [_u32("conv pair arg", v) for v in args]
    if batch * out_ch * out_h * out_w == 0:
        return
    px = _dev_ptr(x, batch * in_ch * in_h * in_w, "x")
    pp, _ = _workspace(packed)
    pb1 = _dev_ptr(bias1, mid_ch, "bias1") if bias1 is not None else None
    pb2 = _dev_ptr(bias2, out_ch, "bias2") if bias2 is not None else None
    py = _dev_ptr(y, batch * out_ch * out_h * out_w, "y")
    epi = _epilogue(add, False, act, batch * out_ch * out_h * out_w)
    _native.call("cm_conv_pair_packed_ex", px, pp, pb1, pb2, py, *args, _u32("act1", act1),
                 ctypes.byref(epi) if epi is not None else None, _stream(stream))


def PoolingKernel(x, y, batch, channels, in_h, in_w, out_h, out_w, pool_h, pool_w,
                  stride_h=1, stride_w=1, pad_top=0, pad_left=0, dil_h=1, dil_w=1,
                  pool_type=POOL_MAX, lp_order=2, count_include_pad=0, stream=None) -> None:
    """ONNX MaxPool / AveragePool / LpPool (and Global*) over NCHW planes."""
    args = [batch, channels, in_h, in_w, out_h, out_w, pool_h, pool_w, stride_h, stride_w,
            pad_top, pad_left, dil_h, dil_w, pool_type, lp_order, count_include_pad]
    args = [_u32("pool arg", v) for v in args]
    if batch * channels * out_h * out_w == 0:
        return
    px = _dev_ptr(x, batch * channels * in_h * in_w, "x")
    py = _dev_ptr(y, batch * channels * out_h * out_w, "y")
    _native.call("cm_pool", px, py, *args, _stream(stream))


def selftest_div(b_lo: int = 0, b_count: int = 65536, stream=None):
    """(mismatches, example) of the DIV path against exact integer division for
    every a and b in [b_lo, b_lo + b_count); example = (a, b, got, want) raw or None."""
    out = ctypes.c_uint64(0)
    ex = ctypes.c_uint64(0)
    _native.call("cm_selftest_div", b_lo, b_count, ctypes.byref(out), ctypes.byref(ex),
                 _stream(stream))
    n = int(out.value)
    if n == 0:
        return 0, None
    v = int(ex.value)
    s16 = lambda x: x - 65536 if x >= 32768 else x
    return n, (s16(v >> 48), s16((v >> 32) & 0xFFFF), s16((v >> 16) & 0xFFFF), s16(v & 0xFFFF))


def selftest_finalize(mode: int, lo: int, count: int, d: int = 0, stream=None) -> int:
    """Checksum of the LP2 (mode 0) or AVG (mode 1) finaliser over an accumulator range."""
    out = ctypes.c_uint64(0)
    _native.call("cm_selftest_finalize", mode, lo, count, d, ctypes.byref(out), _stream(stream))
    return int(out.value)


def sync(stream=None) -> None:
    _native.call("cm_sync", _stream(stream))
