"""Scheduler counterpart on the CPU: ONNX codec, shape inference, node argument
derivation, layouts and buffer plan, and graph-level agreement of the two
oracles (C-simulation kernels executing the kernel-call list vs the float64
numpy simulation).

Expected values come from the reference scheduler's tests
(inference-scheduler/test/test_broadcast*.py, test_chunk_one.py,
test_live_intervals.py, test_conv.py, test_pool.py, test_reshape_gemm.py,
gen_matmul_models.py docstrings) for the same graph structures.
"""
from __future__ import annotations

import os
from collections import Counter

import numpy as np
import pytest

import oracle
from oracle import graph_sim as gs
from cormorant_amd import workloads as wl
from cormorant_amd.scheduler import (BufferPlan, OnnxGraph, SchedulerError, fuse, live_intervals,
                                     onnx_io as ox)
from cormorant_amd.scheduler.nodes import (OP_ADD, OP_RELU6, ConvNode, MatmulNode, PoolNode,
                                           ReshapeNode, ScheduledNode)
from cormorant_amd.scheduler.shapes import ShapeError, infer_node
from cormorant_amd.scheduler.tensor import ramp_to_storage
from tests import onnx_models as om

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def graph(model):
    """Round-trip through the wire format, as a file on disk would be."""
    return OnnxGraph(ox.encode_model(model))


def calls(g):
    return [str(c) for _, c in BufferPlan(g).calls]


# --------------------------------------------------------------------------- codec


def test_decode_libtorch_export():
    """A model serialised by libtorch's exporter decodes to what torch recorded."""
    m = ox.load(os.path.join(GOLDEN, "torch_export_small.onnx"))
    ref = np.load(os.path.join(GOLDEN, "torch_export_small.npz"))
    assert m.opset("") == 13 and m.producer_name == "pytorch"
    ops = [n.op_type for n in m.graph.node]
    assert ops == ["Conv", "Constant", "Constant", "Clip", "MaxPool", "GlobalAveragePool",
                   "Constant", "Reshape", "MatMul", "Add"]
    conv = m.graph.node[0]
    assert conv.attribute["kernel_shape"].ints == [3, 3]
    assert conv.attribute["strides"].ints == [2, 2]
    assert conv.attribute["pads"].ints == [1, 1, 1, 1]
    assert conv.attribute["group"].i == 1
    assert m.graph.node[4].attribute["ceil_mode"].i == 0
    consts = [n.attribute["value"].value for n in m.graph.node if n.op_type == "Constant"]
    assert float(consts[0].array) == 0.0 and float(consts[1].array) == 6.0
    assert consts[2].array.tolist() == [2, 8] and consts[2].data_type == ox.INT64
    inits = {t.name: t.array for t in m.graph.initializer}
    np.testing.assert_array_equal(inits["c.weight"], ref["conv_weight"])
    np.testing.assert_array_equal(inits["c.bias"], ref["conv_bias"])
    np.testing.assert_array_equal(inits["w"], ref["w"])
    np.testing.assert_array_equal(inits["b"], ref["b"])
    assert [(v.name, v.shape) for v in m.graph.input] == [("X", [2, 3, 16, 16])]
    assert [(v.name, v.shape) for v in m.graph.output] == [("Y", [2, 4])]


def test_libtorch_export_runs_after_constant_folding():
    """The reference scheduler rejects Constant nodes; folded into initializers, the
    exported graph schedules, both oracles agree bit for bit, and the Q8.8 result
    stays within the quantisation error of torch's float32 output."""
    m = ox.load(os.path.join(GOLDEN, "torch_export_small.onnx"))
    with pytest.raises(SchedulerError, match="Constant"):
        OnnxGraph(m)
    ref = np.load(os.path.join(GOLDEN, "torch_export_small.npz"))
    m = ox.load(os.path.join(GOLDEN, "torch_export_small.onnx"))
    keep = []
    for n in m.graph.node:
        if n.op_type == "Constant":
            t = n.attribute["value"].value
            m.graph.initializer.append(ox.Tensor(n.output[0], t.data_type, t.dims, t.array))
        else:
            keep.append(n)
    m.graph.node = keep
    g = OnnxGraph(m)
    assert [type(sn).__name__ for sn in g.nodes] == [
        "ConvNode", "ScheduledNode", "PoolNode", "PoolNode", "ReshapeNode", "MatmulNode",
        "ScheduledNode"]
    x = np.clip(np.round(ref["x"] * 256), -32768, 32767).astype(np.int16)
    got = gs.run_plan(BufferPlan(g), {"X": x})["Y"]
    np.testing.assert_array_equal(got, gs.simulate_raw(g, {"X": x})["Y"])
    assert np.abs(got / 256.0 - ref["y"]).max() < 0.1


def test_encode_decode_round_trip():
    m = wl.mlp_model(batch=4)
    m2 = ox.decode_model(ox.encode_model(m))
    assert [n.op_type for n in m2.graph.node] == ["Gemm", "Relu", "Gemm"]
    for a, b in zip(m.graph.initializer, m2.graph.initializer):
        assert a.name == b.name and a.dims == b.dims
        np.testing.assert_array_equal(a.array, b.array)
    assert ox.encode_model(m2) == ox.encode_model(m)


def test_wire_packed_and_unpacked_ints_agree():
    # AttributeProto{name="ints", ints=[1,-2,300], type=INTS}: unpacked and packed forms
    def attr(payload):
        return ox._read_attribute(memoryview(payload))
    name = b"\x0a\x04ints"
    unpacked = name + b"\x40\x01" + b"\x40" + ox._enc_varint(-2) + b"\x40\xac\x02" + b"\xa0\x01\x07"
    body = b"\x01" + ox._enc_varint(-2) + b"\xac\x02"
    packed = name + b"\x42" + bytes([len(body)]) + body + b"\xa0\x01\x07"
    assert attr(unpacked).ints == [1, -2, 300]
    assert attr(packed).ints == [1, -2, 300]


def test_truncated_model_is_an_error():
    data = ox.encode_model(om.single_add())
    with pytest.raises(ox.OnnxFormatError):
        ox.decode_model(data[:-3])


# --------------------------------------------------------------------------- shapes


@pytest.mark.parametrize("attrs,expect", [
    (dict(kernel_shape=[3, 3]), [1, 8, 6, 6]),                                   # conv_with_bias
    (dict(kernel_shape=[3, 3], strides=[2, 2]), [1, 8, 3, 3]),                   # conv_stride2
    (dict(kernel_shape=[3, 3], pads=[1, 1, 1, 1]), [1, 8, 8, 8]),                # conv_padded
    (dict(kernel_shape=[3, 3], dilations=[2, 2]), [1, 8, 4, 4]),                 # conv_dilation
    (dict(kernel_shape=[3, 3], auto_pad="VALID"), [1, 8, 6, 6]),                 # auto_pad VALID
    (dict(kernel_shape=[3, 3], auto_pad="SAME_UPPER", strides=[2, 2]), [1, 8, 4, 4]),
])
def test_conv_output_shapes(attrs, expect):
    node = ox.make_node("Conv", ["X", "W"], ["Y"], **attrs)
    assert infer_node(node, {"X": [1, 4, 8, 8], "W": [8, 4, 3, 3]}, {}) == [expect]


def test_view_op_shapes():
    c = {"s": np.array([0, -1], np.int64)}
    assert infer_node(ox.make_node("Reshape", ["X", "s"], ["Y"]), {"X": [2, 3, 4]}, c) == [[2, 12]]
    assert infer_node(ox.make_node("Squeeze", ["X"], ["Y"], axes=[2, 3]),
                      {"X": [1, 4, 1, 1]}, {}) == [[1, 4]]
    assert infer_node(ox.make_node("Unsqueeze", ["X"], ["Y"], axes=[2, 3]),
                      {"X": [1, 4]}, {}) == [[1, 4, 1, 1]]
    assert infer_node(ox.make_node("MatMul", ["A", "B"], ["Y"]),
                      {"A": [2, 3, 4, 16], "B": [3, 16, 8]}, {}) == [[2, 3, 4, 8]]
    with pytest.raises(ShapeError):
        infer_node(ox.make_node("Add", ["A", "B"], ["Y"]), {"A": [2, 3], "B": [4]}, {})


def test_declared_shape_mismatch_is_an_error():
    m = om.single_add()
    m.graph.output[0].shape = [1, 128]
    with pytest.raises(SchedulerError):
        graph(m)


# --------------------------------------------------------------------------- VectorOP nodes


def test_broadcast_aligned():
    g = graph(om.broadcast_aligned())
    sn = g.nodes[0]
    assert (sn.outer_count, sn.chunk_size, sn.aligned_chunk_size) == (8, 16, 16)
    assert sn.a_advances and not sn.b_advances
    p = BufferPlan(g)
    assert p.layouts["X"].alloc == 128 and p.layouts["Y"].alloc == 128
    assert p.layouts["bias"].alloc == 16
    assert calls(g) == ["run_op(X, bias, Y, 16, ADD, 8, 16, 0)"]


def test_broadcast_unaligned():
    g = graph(om.broadcast_unaligned())
    sn = g.nodes[0]
    assert (sn.outer_count, sn.chunk_size, sn.aligned_chunk_size) == (4, 6, 8)
    p = BufferPlan(g)
    assert p.layouts["X"].alloc == 32 > g.input_tensors[0].numel
    assert calls(g) == ["run_op(X, bias, Y, 6, ADD, 4, 8, 0)"]


def test_chunk_one():
    g = graph(om.chunk_one())
    sn = g.nodes[0]
    assert (sn.outer_count, sn.chunk_size, sn.aligned_chunk_size) == (16, 1, 8)
    p = BufferPlan(g)
    assert p.layouts["X"].gap == 7
    assert (p.layouts["X"].alloc, p.layouts["Y"].alloc, p.layouts["bias"].alloc) == (128, 128, 8)


def test_broadcast_3d():
    g = graph(om.broadcast_3d())
    sn = g.nodes[0]
    assert (sn.outer_count, sn.chunk_size, sn.aligned_chunk_size) == (6, 4, 8)
    p = BufferPlan(g)
    assert (p.layouts["X"].alloc, p.layouts["Y"].alloc, p.layouts["bias"].alloc) == (48, 48, 8)


def test_broadcast_mixed_relu_inherits_padding():
    g = graph(om.broadcast_mixed())
    p = BufferPlan(g)
    assert [sn.outer_count for sn in g.nodes] == [4, 1]
    assert p.layouts["add_Y"].alloc == 32 and p.layouts["X"].alloc == 32
    assert p.layouts["Y"].alloc == 32
    assert calls(g)[1] == "run_op(add_Y, NULL, Y, 32, RELU, 1, 0, 0)"


def test_broadcast_chain_all_buffers_padded():
    g = graph(om.broadcast_chain())
    p = BufferPlan(g)
    for name in ("X", "add_Y", "relu_Y", "Y"):
        assert p.layouts[name].alloc == 32, name
    assert calls(g)[2] == "run_op(relu_Y, X, Y, 32, ADD, 1, 0, 0)"


def test_broadcast_chain_bias_weight_is_strided():
    g = graph(om.broadcast_chain_bias())
    p = BufferPlan(g)
    assert g.get_tensor("bias2").numel == 24
    lay = p.layouts["bias2"]
    assert (lay.alloc, lay.n_chunks, lay.stride) == (32, 4, 8)
    assert p.layouts["bias"].alloc == 8
    img = p.pool_image()
    off = p.storage["bias2"].offset
    block = img[off:off + 32].reshape(4, 8)
    np.testing.assert_array_equal(block[:, 6:], 0)
    np.testing.assert_array_equal(block[:, :6].reshape(-1), g.get_tensor("bias2").storage())


def test_broadcast_tapped_output():
    g = graph(om.broadcast_tapped())
    assert len(g.output_tensors) == 2 and len(g.intermediate_tensors) == 0
    p = BufferPlan(g)
    assert (p.layouts["X"].alloc, p.layouts["add_Y"].alloc, p.layouts["Y"].alloc) == (32, 32, 32)


def test_clip_forms():
    assert graph(om.clip_opset10()).nodes[0].op_code == OP_RELU6
    sn = graph(om.clip_opset13()).nodes[0]
    assert sn.op_code == OP_RELU6 and sn.arity == 1 and len(sn.inputs) == 1
    with pytest.raises(SchedulerError, match="Clip"):
        graph(om.clip_opset13(0.0, 5.0))


def test_broadcast_errors():
    bad = om._model([ox.make_node("Add", ["X", "bias"], ["Y"])], "bad", [("X", [2, 3, 4, 4])],
                    [("Y", [2, 3, 4, 4])], [om._w("bias", np.ones((2, 1, 4, 4)))])
    with pytest.raises(SchedulerError):
        graph(bad)
    both = om._model([ox.make_node("Add", ["A", "B"], ["Y"])], "both", [("A", [1, 4]), ("B", [2, 1])],
                     [("Y", [2, 4])])
    with pytest.raises(SchedulerError):
        graph(both)


def test_unsupported_op():
    with pytest.raises(SchedulerError, match="not supported"):
        graph(om.unsupported())


# --------------------------------------------------------------------------- MatMul nodes

MATMUL_EXPECT = {
    "mm_2d": ["run_matmul(X, W, Y, 4, 16, 8, 1, 0, 0, 0)"],
    "mm_batch_broadcast": ["run_matmul(X, W, Y, 4, 4, 16, 2, 16, 0, 64)"],
    "mm_3d_3d": ["run_matmul(X, W, Y, 4, 16, 8, 3, 64, 128, 32)"],
    "mm_4d_4d": ["run_matmul(X, W, Y, 4, 16, 8, 6, 64, 128, 32)"],
    "mm_4d_3d": [f"run_matmul_at(X+{i * 192}, W+0, Y+{i * 96}, 4, 16, 8, 3, 64, 128, 32)"
                 for i in range(2)],
    "mm_3d_4d": [f"run_matmul_at(X+0, W+{i * 384}, Y+{i * 96}, 4, 16, 8, 3, 64, 128, 32)"
                 for i in range(2)],
    "mm_5d_3d": [f"run_matmul_at(X+{i * 128}, W+0, Y+{i * 64}, 4, 16, 8, 2, 64, 128, 32)"
                 for i in range(4)],
    "mm_3d_5d": [f"run_matmul_at(X+0, W+{i * 256}, Y+{i * 64}, 4, 16, 8, 2, 64, 128, 32)"
                 for i in range(4)],
    "mm_5d_4d": [f"run_matmul_at(X+{i * 256}, W+0, Y+{i * 128}, 4, 16, 8, 4, 64, 128, 32)"
                 for i in range(2)],
    "mm_4d_5d": [f"run_matmul_at(X+0, W+{i * 512}, Y+{i * 128}, 4, 16, 8, 4, 64, 128, 32)"
                 for i in range(2)],
    "mm_5d_2d": ["run_matmul(X, W, Y, 4, 16, 8, 8, 64, 0, 32)"],
    "mm_2d_5d": ["run_matmul(X, W, Y, 4, 16, 8, 8, 0, 128, 32)"],
}


@pytest.mark.parametrize("name", sorted(om.MATMUL_CASES))
def test_matmul_argument_derivation(name):
    a, w = om.MATMUL_CASES[name]
    g = graph(om.matmul(a, w, name))
    assert calls(g) == MATMUL_EXPECT[name]
    x = wl.uniform_q88(wl.rng(60, len(name)), a, -2.0, 2.0)
    np.testing.assert_array_equal(gs.run_plan(BufferPlan(g), {"X": x}, threads=False)["Y"],
                                  gs.simulate_raw(g, {"X": x})["Y"])


def test_gemm_split():
    g = graph(om.gemm_with_bias())
    assert [type(sn).__name__ for sn in g.nodes] == ["MatmulNode", "ScheduledNode"]
    assert g.nodes[0].output.onnx_name == "_gemm_mm_out_1"
    assert g.nodes[0].onnx_node.name == "_gemm_matmul_1"
    assert g.nodes[1].onnx_node.name == "_gemm_add_1"
    g2 = graph(om.gemm_no_bias())
    assert len(g2.nodes) == 1 and g2.nodes[0].output.onnx_name == "Y"
    with pytest.raises(SchedulerError, match="trans"):
        graph(om.gemm_trans_b())


def test_mlp_plan_matches_reference_decomposition():
    """64x256x10 Gemm: Y's rows sit at stride 16, so the MatMul runs as 64 batch entries
    of 1x256x10 with c_stride 16; b2 broadcasts with chunk 10 / stride 16."""
    g = graph(wl.mlp_model())
    assert calls(g) == [
        "run_matmul(X, W1, _gemm_mm_out_1, 64, 784, 256, 1, 0, 0, 0)",
        "run_op(_gemm_mm_out_1, B1, H, 256, ADD, 64, 256, 0)",
        "run_op(H, NULL, R, 16384, RELU, 1, 0, 0)",
        "run_matmul(R, W2, _gemm_mm_out_2, 1, 256, 10, 64, 256, 0, 16)",
        "run_op(_gemm_mm_out_2, B2, Y, 10, ADD, 64, 16, 0)",
    ]


# --------------------------------------------------------------------------- Conv / Pool nodes


def test_conv_fields():
    sn = graph(om.conv([1, 4, 8, 8], [8, 4, 3, 3], kernel_shape=[3, 3], strides=[2, 2])).nodes[0]
    assert isinstance(sn, ConvNode) and (sn.stride_h, sn.stride_w, sn.out_h) == (2, 2, 3)
    sn = graph(om.conv([1, 4, 8, 8], [8, 4, 3, 3], pads=[1, 1, 1, 1])).nodes[0]
    assert (sn.pad_top, sn.pad_left, sn.out_h, sn.in_h) == (1, 1, 8, 8)
    sn = graph(om.conv([1, 4, 8, 8], [8, 4, 3, 3], auto_pad="VALID")).nodes[0]
    assert (sn.pad_top, sn.pad_left) == (0, 0)
    sn = graph(om.conv([1, 4, 9, 9], [8, 4, 4, 4], auto_pad="SAME_UPPER", strides=[2, 2])).nodes[0]
    # pad total = (5-1)*2 + 4 - 9 = 3: SAME_UPPER puts 1 first, SAME_LOWER 2
    assert (sn.out_h, sn.pad_top) == (5, 1)
    sn = graph(om.conv([1, 4, 9, 9], [8, 4, 4, 4], auto_pad="SAME_LOWER", strides=[2, 2])).nodes[0]
    assert (sn.out_h, sn.pad_top) == (5, 2)
    sn = graph(om.conv([1, 4, 8, 8], [4, 1, 3, 3], group=4)).nodes[0]
    assert sn.is_depthwise and sn.out_h == 6
    with pytest.raises(SchedulerError, match="group"):
        graph(om.conv([1, 4, 8, 8], [4, 2, 3, 3], group=2))
    sn = graph(om.conv([1, 3, 224, 224], [64, 3, 3, 3], bias=False)).nodes[0]
    assert (sn.out_h, sn.has_bias) == (222, False)
    assert calls(graph(om.conv([1, 4, 8, 8], [8, 4, 3, 3])))[0].endswith("1, 0)")


def test_conv_feeding_broadcast_is_rejected():
    m = om._model([ox.make_node("Conv", ["X", "W"], ["Z"]), ox.make_node("Add", ["Z", "b"], ["Y"])],
                  "conv_bias_add", [("X", [2, 4, 8, 8])], [("Y", [2, 8, 6, 6])],
                  [om._w("W", np.zeros((8, 4, 3, 3))), om._w("b", np.zeros((6, 6)))])
    with pytest.raises(SchedulerError, match="NCHW"):
        BufferPlan(graph(m))


@pytest.mark.parametrize("op,attrs,fields", [
    ("MaxPool", dict(kernel_shape=[2, 2], strides=[2, 2]), (0, 2, 2, 2, 0, 2, 0, 4)),
    ("AveragePool", dict(kernel_shape=[3, 3], strides=[2, 2], pads=[1, 1, 1, 1],
                         count_include_pad=1), (1, 3, 3, 2, 1, 2, 1, 4)),
    ("LpPool", dict(kernel_shape=[2, 2], strides=[2, 2], p=1), (2, 2, 2, 2, 0, 1, 0, 4)),
    ("GlobalAveragePool", {}, (1, 8, 8, 1, 0, 2, 0, 1)),
    ("GlobalMaxPool", {}, (0, 8, 8, 1, 0, 2, 0, 1)),
    ("GlobalLpPool", dict(p=2), (2, 8, 8, 1, 0, 2, 0, 1)),
])
def test_pool_fields(op, attrs, fields):
    sn = graph(om.pool(op, **attrs)).nodes[0]
    assert isinstance(sn, PoolNode)
    assert (sn.pool_type, sn.pool_h, sn.pool_w, sn.stride_h, sn.pad_top, sn.lp_order,
            sn.count_include_pad, sn.out_h) == fields


def test_pool_rejections():
    with pytest.raises(SchedulerError, match="ceil_mode"):
        graph(om.pool("MaxPool", kernel_shape=[3, 3], strides=[2, 2], ceil_mode=1))
    with pytest.raises(SchedulerError, match="p=3"):
        graph(om.pool("LpPool", kernel_shape=[2, 2], p=3))


# --------------------------------------------------------------------------- plan


def test_live_intervals_and_slot_reuse():
    g = graph(om.gemm_chain())
    iv = live_intervals(g)
    assert all(a <= b for a, b in iv.values())
    starts = sorted(a for a, _ in iv.values())
    assert len(set(starts)) == len(starts)
    p = BufferPlan(g)
    inter = [(n, off) for n, off, _ in p.pool_entries if n in iv]
    offsets = [off for _, off in inter]
    assert len(set(offsets)) < len(offsets), "a 4-node chain must reuse a slot"
    for i, (n1, o1) in enumerate(inter):
        for n2, o2 in inter[i + 1:]:
            if o1 == o2:
                a, b = iv[n1], iv[n2]
                assert not (a[0] <= b[1] and b[0] <= a[1]), (n1, n2)
    assert all(off % 32 == 0 for _, off, _ in p.pool_entries)  # 64-byte aligned views
    single = BufferPlan(graph(om.gemm_with_bias()))
    offs = [off for _, off, _ in single.pool_entries]
    assert len(set(offs)) == len(offs)


def test_reshape_aliases_share_storage():
    g = graph(om.mixed_all_kernels())
    p = BufferPlan(g)
    assert isinstance(g.nodes[4], ReshapeNode)
    assert p.storage["f"] == p.storage["g"]
    assert "f" not in live_intervals(g)
    assert all("run_" in c for c in calls(g))


def test_output_alias_chain_is_redirected():
    g = graph(om.reshape_output_alias())
    p = BufferPlan(g)
    assert p.storage["c"].kind == "output" and p.storage["c"].key == "Y"
    assert p.storage["r"] == p.storage["c"]


def test_input_to_output_reshape_is_copied():
    g = graph(om.reshape_input_to_output())
    p = BufferPlan(g)
    assert p.input_copies == [("Z", "X")]
    assert str(p.calls[-1][1]) == "run_op(X, NULL, Z, 16, COPY, 1, 0, 0)"
    x = wl.uniform_q88(wl.rng(61), (2, 8), -4, 4)
    out = gs.run_plan(p, {"X": x}, threads=False)
    np.testing.assert_array_equal(out["Z"], x.reshape(16))


# --------------------------------------------------------------------------- graph oracles agree

GRAPH_CASES = {
    "single_add": om.single_add, "relu_chain": om.relu_chain, "mixed_ops": om.mixed_ops,
    "two_input_add": om.two_input_add, "two_output_tap": om.two_output_tap,
    "residual_chain": om.residual_chain, "broadcast_aligned": om.broadcast_aligned,
    "broadcast_unaligned": om.broadcast_unaligned, "chunk_one": om.chunk_one,
    "broadcast_3d": om.broadcast_3d, "broadcast_mixed": om.broadcast_mixed,
    "broadcast_chain": om.broadcast_chain, "broadcast_chain_bias": om.broadcast_chain_bias,
    "broadcast_tapped": om.broadcast_tapped, "broadcast_lhs": om.broadcast_lhs,
    "clip_opset10": om.clip_opset10, "clip_opset13": om.clip_opset13,
    "gemm_with_bias": om.gemm_with_bias, "gemm_chain": om.gemm_chain,
    "conv_relu_chain": om.conv_relu_chain, "mixed_all_kernels": om.mixed_all_kernels,
    "squeeze_then_matmul_v13": lambda: om.squeeze_then_matmul(13),
    "squeeze_then_matmul_v11": lambda: om.squeeze_then_matmul(11),
    "unsqueeze_then_relu": om.unsqueeze_then_relu, "reshape_then_matmul": om.reshape_then_matmul,
    "reshape_output_alias": om.reshape_output_alias,
    "depthwise": lambda: om.conv([2, 6, 9, 9], [6, 1, 3, 3], group=6, pads=[1, 1, 1, 1]),
    "conv_dilated": lambda: om.conv([1, 5, 12, 12], [7, 5, 3, 3], dilations=[2, 2],
                                    strides=[2, 1]),
    "avgpool_cip": lambda: om.pool("AveragePool", (2, 3, 9, 9), kernel_shape=[3, 3],
                                   strides=[2, 2], pads=[1, 1, 1, 1], count_include_pad=1),
    "lppool": lambda: om.pool("LpPool", (2, 3, 8, 8), kernel_shape=[2, 2], strides=[2, 2]),
    "maxpool": lambda: om.pool("MaxPool", (2, 3, 9, 9), kernel_shape=[3, 3], strides=[2, 2]),
}


def feeds_for(g, seed):
    out = {}
    for i, t in enumerate(g.input_tensors):
        out[t.onnx_name] = wl.uniform_q88(wl.rng(62, seed, i), t.shape, -4.0, 4.0)
    return out


@pytest.mark.parametrize("name", sorted(GRAPH_CASES))
def test_graph_oracles_agree(name):
    g = graph(GRAPH_CASES[name]())
    feeds = feeds_for(g, len(name))
    got = gs.run_plan(BufferPlan(g), feeds, threads=False)
    want = gs.simulate_raw(g, feeds)
    for k in want:
        np.testing.assert_array_equal(got[k], want[k], err_msg=k)


SAT_EXPECT = {   # test_saturation.py: value at index, count of saturated outputs
    "add_pos": (lambda y: int(np.sum(y == 32767)) == 129),
    "add_neg": (lambda y: int(np.sum(y == -32768)) == 129),
    "mul_pos": (lambda y: y[0] == 90 * 256 and y[108] == int(127.96875 * 256)
                and int(np.sum(y == 32767)) == 147),
    "mul_neg": (lambda y: y[148] == int(-127.96875 * 256) and int(np.sum(y == -32768)) == 148),
    "sub_pos": (lambda y: int(np.sum(y == 32767)) == 129),
    "sub_neg": (lambda y: int(np.sum(y == -32768)) == 129),
    "div_pos": (lambda y: y[0] == 0 and int(np.sum(y == 32767)) == 128),
    "div_neg": (lambda y: y[0] == 0 and int(np.sum(y == -32768)) == 128),
}


@pytest.mark.parametrize("kind", om.SAT_KINDS)
def test_saturation_models_on_ramp(kind):
    g = graph(om.sat_model(kind))
    x = ramp_to_storage(np.arange(256)).reshape(1, 256)
    y = gs.run_plan(BufferPlan(g), {"X": x}, threads=False)["Y"].reshape(-1)
    assert SAT_EXPECT[kind](y), y[:8]
    np.testing.assert_array_equal(y, gs.simulate_raw(g, {"X": x})["Y"].reshape(-1))


def test_mobilenet_like_small_oracles_agree():
    g = graph(wl.mobilenet_model(batch=2, hw=32))
    x = wl.mobilenet_input(2, 32)
    oracle.set_threads(min(os.cpu_count() or 1, 8))
    got = gs.run_plan(BufferPlan(g), {"X": x})["Y"]
    np.testing.assert_array_equal(got, gs.simulate_raw(g, {"X": x})["Y"])
    assert np.count_nonzero(got) > 0.9 * got.size


# --------------------------------------------------------------------------- epilogue fusion

def fused_plan(g):
    plan = BufferPlan(g, fuse.live_from(BufferPlan(g)))
    return plan, fuse.launch_list(plan)


def test_fusion_mobilenet_groups():
    """Every Clip(0,6) and residual Add of the MobileNetV2-like graph, and the
    classifier's bias Add, run in a convolution / MatMul epilogue."""
    g = graph(wl.mobilenet_model(batch=2, hw=32))
    plan, seq = fused_plan(g)
    assert len(plan.calls) == 68 and len(seq) == 38
    groups = [x for x in seq if isinstance(x, fuse.FusedCall)]
    kinds = Counter((x.add_mode, x.act) for x in groups)
    assert kinds == {(fuse.ADD_NONE, fuse.ACT_RELU6): 19, (fuse.ADD_SAME, fuse.ACT_NONE): 10,
                     (fuse.ADD_COLUMN, fuse.ACT_NONE): 1}
    assert not any(getattr(x, "kernel", None) == "op" for x in seq)
    # the group's string form keeps the reference call syntax of every member
    assert str(groups[0]).startswith("run_conv(X, conv0_w, conv0_b, conv0_y, 2, 3, 32, 32, 32,")
    assert str(groups[0]).endswith("+ run_op(conv0_y, NULL, conv0_y_r6, 16384, RELU6, 1, 0, 0)")


def test_fusion_mlp_chains_bias_and_relu():
    plan, seq = fused_plan(graph(wl.mlp_model()))
    assert [type(x).__name__ for x in seq] == ["FusedCall", "FusedCall"]
    assert (seq[0].add, seq[0].add_mode, seq[0].act, seq[0].out) == \
        ("B1", fuse.ADD_COLUMN, fuse.ACT_RELU, "R")
    # second layer: batch-64 single-row MatMul with 16-element row stride + bias
    assert seq[1].call.args == (1, 256, 10, 64, 256, 0, 16)
    assert (seq[1].add, seq[1].add_mode, seq[1].act, seq[1].out) == \
        ("B2", fuse.ADD_COLUMN, fuse.ACT_NONE, "Y")


def _conv_then(nodes_after, outputs, extra_inputs=()):
    N = ox.make_node
    inits = [ox.from_array(np.full((4, 3, 1, 1), 0.25, np.float32), "W")]
    nodes = [N("Conv", ["X", "W"], ["c"], kernel_shape=[1, 1])] + nodes_after
    ins = [ox.value_info("X", [1, 3, 4, 4])] + [ox.value_info(n, s) for n, s in extra_inputs]
    g = ox.make_graph(nodes, "conv_then", ins, [ox.value_info(n, s) for n, s in outputs], inits)
    return graph(ox.make_model(g))


def test_fusion_rejections():
    N = ox.make_node
    shape = [1, 4, 4, 4]
    # the conv output has a second reader
    g = _conv_then([N("Relu", ["c"], ["r"]), N("Add", ["c", "r"], ["Y"])], [("Y", shape)])
    assert not fuse.candidates(BufferPlan(g))
    # the conv output is itself a graph output
    g = _conv_then([N("Relu", ["c"], ["Y"])], [("c", shape), ("Y", shape)])
    assert not fuse.candidates(BufferPlan(g))
    # Sub is not an epilogue operation
    g = _conv_then([N("Sub", ["c", "Z"], ["Y"])], [("Y", shape)], [("Z", shape)])
    assert not fuse.candidates(BufferPlan(g))
    # a broadcast Add repeating a [2, 8] block over MatMul batches is not a column add
    mm = ox.make_graph([N("MatMul", ["X", "W"], ["m"]), N("Add", ["m", "Z"], ["Y"])], "mm_bcast",
                       [ox.value_info("X", [2, 2, 4]), ox.value_info("Z", [2, 8])],
                       [ox.value_info("Y", [2, 2, 8])],
                       [ox.from_array(np.full((4, 8), 0.5, np.float32), "W")])
    p = BufferPlan(graph(ox.make_model(mm)))
    assert str(p.calls[1][1]) == "run_op(m, Z, Y, 16, ADD, 2, 16, 0)"
    assert not fuse.candidates(p)
    # accepted: same-shape Add then Clip(0,6) through a reshape of the sum
    g = _conv_then([N("Add", ["c", "Z"], ["s"]), N("Relu", ["s"], ["Y"])], [("Y", shape)],
                   [("Z", shape)])
    (k, f), = fuse.candidates(BufferPlan(g))
    assert (k, f.add, f.add_mode, f.act, f.out) == (0, "Z", fuse.ADD_SAME, fuse.ACT_RELU, "Y")


def test_fusion_storage_checks():
    """With the reference pool layout a fused output may share a slot with its
    MatMul / Conv input; those groups are dropped, and ``live_from`` gives a
    layout in which none is."""
    g = graph(wl.mobilenet_model(batch=2, hw=32))
    p0 = BufferPlan(g)
    cands, ok = fuse.candidates(p0), dict(fuse.fusions(p0))
    assert 0 < len(ok) < len(cands)
    for k, f in cands:
        if k in ok:
            continue
        out = fuse._span(p0, f.absorbed[-1], f.out)
        ins = [fuse._span(p0, f.call, n) for n in fuse._reads(f.call)]
        assert any(fuse._overlap(out, s) for s in ins), str(f)
    p1, _ = fused_plan(g)
    assert len(fuse.fusions(p1)) == len(fuse.candidates(p1)) == 30


@pytest.mark.parametrize("name", ["gemm_chain", "gemm_with_bias", "conv_relu_chain",
                                  "mixed_all_kernels", "residual_chain"])
def test_fused_launches_match_simulation(name):
    """The fused launch list, executed on the oracle with every group's
    intermediates kept out of the plan's storage, gives the graph's outputs."""
    g = graph(GRAPH_CASES[name]())
    plan, seq = fused_plan(g)
    feeds = feeds_for(g, 3)
    got = gs.run_plan(plan, feeds, threads=False, launches=seq)
    want = gs.simulate_raw(g, feeds)
    for k in want:
        np.testing.assert_array_equal(got[k], want[k], err_msg=k)


def test_fused_launches_mobilenet_small():
    g = graph(wl.mobilenet_model(batch=2, hw=32))
    plan, seq = fused_plan(g)
    x = wl.mobilenet_input(2, 32)
    oracle.set_threads(min(os.cpu_count() or 1, 8))
    got = gs.run_plan(plan, {"X": x}, launches=seq)["Y"]
    np.testing.assert_array_equal(got, gs.run_plan(BufferPlan(g), {"X": x})["Y"])


def test_conv_pairs_mobilenet():
    """Each 3x3 convolution (its Clip(0,6) fused) whose output only the next 1x1
    convolution reads pairs with that convolution's group: the 14 pairs whose
    middle tensor has at most 128 channels, 38 launches -> 24; the paired launch
    list, run on the oracle with every middle tensor kept out of the plan's
    storage, gives the graph's output."""
    g = graph(wl.mobilenet_model(batch=2, hw=32))
    plan = BufferPlan(g, fuse.live_from(BufferPlan(g)))
    seq = fuse.launch_list(plan, pair_ok=lambda pc: pc.call.args[4] <= 128)
    pairs = [x for x in seq if isinstance(x, fuse.PairCall)]
    assert len(pairs) == 14 and len(seq) == 24
    assert all(p.act1 == fuse.ACT_RELU6 for p in pairs)
    assert sum(isinstance(p.second, fuse.FusedCall) and p.second.add_mode == fuse.ADD_SAME
               for p in pairs) == 8
    assert str(pairs[0]).startswith("run_conv(conv0_y_r6, conv1_w, conv1_b, conv1_y,")
    # every pair's output is live from its first convolution: it never shares a
    # slot with that convolution's input
    for p in pairs:
        out = fuse._span(plan, p.absorbed[-1], p.out)
        x = fuse._span(plan, p.call, p.call.tensors[0])
        assert not fuse._overlap(out, x), str(p)
    x = wl.mobilenet_input(2, 32)
    oracle.set_threads(min(os.cpu_count() or 1, 8))
    got = gs.run_plan(plan, {"X": x}, launches=seq)["Y"]
    np.testing.assert_array_equal(got, gs.run_plan(BufferPlan(g), {"X": x})["Y"])


def test_conv_pair_rejections():
    """No pair when the middle tensor has another reader, when the second
    convolution is not a plain 1x1 (stride 1, no padding), or when the first
    one is itself 1x1."""
    N = ox.make_node

    def model(nodes, out_shape, w2_shape=(8, 4, 1, 1)):
        inits = [ox.from_array(np.full((4, 3, 3, 3), 0.1, np.float32), "W1"),
                 ox.from_array(np.full((4, 3, 1, 1), 0.1, np.float32), "W0"),
                 ox.from_array(np.full(w2_shape, 0.1, np.float32), "W2")]
        gr = ox.make_graph(nodes, "pairs", [ox.value_info("X", [1, 3, 8, 8])],
                           [ox.value_info("Y", out_shape)], inits)
        return graph(ox.make_model(gr))

    def pairs_of(g):
        plan = BufferPlan(g, fuse.live_from(BufferPlan(g)))
        return [x for x in fuse.launch_list(plan, pair_ok=lambda pc: True) if isinstance(x, fuse.PairCall)]

    conv3 = N("Conv", ["X", "W1"], ["h"], kernel_shape=[3, 3], pads=[1, 1, 1, 1])
    # accepted: 3x3 -> 1x1
    assert len(pairs_of(model([conv3, N("Conv", ["h", "W2"], ["Y"], kernel_shape=[1, 1])],
                              [1, 8, 8, 8]))) == 1
    # the middle tensor has a second reader (a residual Add of it)
    g = model([conv3, N("Conv", ["h", "W2"], ["c"], kernel_shape=[1, 1]),
               N("Conv", ["h", "W2"], ["d"], kernel_shape=[1, 1]), N("Add", ["c", "d"], ["Y"])],
              [1, 8, 8, 8])
    assert not pairs_of(g)
    # the 1x1 convolution has stride 2
    g = model([conv3, N("Conv", ["h", "W2"], ["Y"], kernel_shape=[1, 1], strides=[2, 2])], [1, 8, 4, 4])
    assert not pairs_of(g)
    # the first convolution is 1x1
    g = model([N("Conv", ["X", "W0"], ["h"], kernel_shape=[1, 1]),
               N("Conv", ["h", "W2"], ["Y"], kernel_shape=[1, 1])], [1, 8, 8, 8])
    assert not pairs_of(g)


def test_gap_heads():
    """A 1x1 convolution (its Clip(0,6) fused) whose output only a GlobalAveragePool
    reads becomes one GapCall: the MobileNetV2-like head (24 launches -> 23 with the
    pairs of at most 128 middle channels); its pooled output is live from the
    convolution (never in the convolution's input slot); the launch list run on the
    oracle gives the graph's output.  No head when the pooled tensor has another
    reader, when the convolution is not 1x1, or when the pool is not global."""
    g = graph(wl.mobilenet_model(batch=2, hw=32))
    plan = BufferPlan(g, fuse.live_from(BufferPlan(g)))
    seq = fuse.launch_list(plan, pair_ok=lambda pc: pc.call.args[4] <= 128, gap_ok=lambda gc: True)
    gaps = [x for x in seq if isinstance(x, fuse.GapCall)]
    assert len(gaps) == 1 and len(seq) == 23
    gc = gaps[0]
    assert gc.act == fuse.ACT_RELU6 and gc.out == "gap" and gc.pool.kernel == "pool"
    assert gc.call.args[7:9] == (1, 1)
    assert not fuse._overlap(fuse._span(plan, gc.pool, gc.out), fuse._span(plan, gc.call, gc.call.tensors[0]))
    assert fuse.launch_list(plan, pair_ok=lambda pc: pc.call.args[4] <= 128, gap_ok=lambda gc: False)[-2:] != seq[-2:]
    x = wl.mobilenet_input(2, 32)
    oracle.set_threads(min(os.cpu_count() or 1, 8))
    got = gs.run_plan(plan, {"X": x}, launches=seq)["Y"]
    np.testing.assert_array_equal(got, gs.run_plan(BufferPlan(g), {"X": x})["Y"])

    N = ox.make_node

    def model(nodes, out_shape):
        inits = [ox.from_array(np.full((8, 4, 1, 1), 0.1, np.float32), "W1"),
                 ox.from_array(np.full((8, 4, 3, 3), 0.1, np.float32), "W3")]
        gr = ox.make_graph(nodes, "gaps", [ox.value_info("X", [2, 4, 6, 6])],
                           [ox.value_info("Y", out_shape)], inits)
        return graph(ox.make_model(gr))

    def gaps_of(gr):
        pl = BufferPlan(gr, fuse.live_from(BufferPlan(gr)))
        return [x for x in fuse.launch_list(pl, gap_ok=lambda gc: True) if isinstance(x, fuse.GapCall)]

    conv1 = N("Conv", ["X", "W1"], ["h"], kernel_shape=[1, 1])
    assert len(gaps_of(model([conv1, N("GlobalAveragePool", ["h"], ["Y"])], [2, 8, 1, 1]))) == 1
    # the convolution's output has a second reader
    assert not gaps_of(model([conv1, N("GlobalAveragePool", ["h"], ["p"]),
                              N("GlobalMaxPool", ["h"], ["q"]), N("Add", ["p", "q"], ["Y"])], [2, 8, 1, 1]))
    # a 3x3 convolution
    assert not gaps_of(model([N("Conv", ["X", "W3"], ["h"], kernel_shape=[3, 3], pads=[1, 1, 1, 1]),
                              N("GlobalAveragePool", ["h"], ["Y"])], [2, 8, 1, 1]))
    # a windowed average pool, and a global max pool
    assert not gaps_of(model([conv1, N("AveragePool", ["h"], ["Y"], kernel_shape=[2, 2], strides=[2, 2])],
                             [2, 8, 3, 3]))
    assert not gaps_of(model([conv1, N("GlobalMaxPool", ["h"], ["Y"])], [2, 8, 1, 1]))


def test_alias_reader_extends_source_lifetime():
    """A tensor read through a reshape alias after the reshape node stays live
    until that read: a tensor produced in between must not take its slot."""
    N = ox.make_node
    shp = ox.from_array(np.array([8], np.int64), "shp")
    nodes = [N("Relu", ["X"], ["A"]),                 # 0
             N("Reshape", ["A", "shp"], ["R"]),       # 1: R aliases A
             N("Reshape", ["X", "shp"], ["XR"]),      # 2: alias of the graph input
             N("Mul", ["XR", "XR"], ["B"]),           # 3: produced after A's last direct reader
             N("Add", ["R", "B"], ["Y"])]             # 4: reads A through R
    g = graph(ox.make_model(ox.make_graph(nodes, "alias_life", [ox.value_info("X", [2, 4])],
                                          [ox.value_info("Y", [8])], [shp])))
    iv = live_intervals(g)
    assert iv["A"] == (0, 4) and iv["B"] == (3, 4)
    plan = BufferPlan(g)
    assert plan.storage["A"].offset != plan.storage["B"].offset
    x = wl.uniform_q88(wl.rng(65), (2, 4), -4.0, 4.0)
    np.testing.assert_array_equal(gs.run_plan(plan, {"X": x}, threads=False)["Y"],
                                  gs.simulate_raw(g, {"X": x})["Y"])
