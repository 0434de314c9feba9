"""Small ONNX graphs for the scheduler tests, built with the in-repo writer.

Each builder reproduces one model family of the reference scheduler's test
suite (inference-scheduler/test/gen_test_models.py, gen_matmul_models.py,
gen_conv_models.py, gen_pool_models.py, gen_reshape_gemm_models.py): the same
graph structure and shapes, so the same node arguments and layouts are
expected.  Weight values are seeded here (the reference draws unseeded random
weights for most of them).
"""
from __future__ import annotations

import numpy as np

from cormorant_amd.scheduler import onnx_io as ox


def _w(name, data):
    return ox.from_array(np.asarray(data, dtype=np.float32), name)


def _rand(seed, shape, scale):
    g = np.random.default_rng([77, seed])
    # on the Q8.8 grid so weight quantisation is exact
    return np.floor(g.normal(0, scale, shape) * 256) / 256


def _model(nodes, name, inputs, outputs, inits=(), opset=13):
    g = ox.make_graph(nodes, name, [ox.value_info(n, s) for n, s in inputs],
                      [ox.value_info(n, s) for n, s in outputs], list(inits))
    return ox.make_model(g, opset=opset)


N = ox.make_node

# ----------------------------------------------------------------- VectorOP graphs


def single_add():
    return _model([N("Add", ["X", "bias"], ["Y"])], "single_add", [("X", [1, 256])],
                  [("Y", [1, 256])], [_w("bias", np.full((1, 256), 0.5))])


def relu_chain():
    return _model([N("Add", ["X", "bias"], ["add_Y"]), N("Relu", ["add_Y"], ["relu_Y"])],
                  "relu_chain", [("X", [1, 128])], [("relu_Y", [1, 128])],
                  [_w("bias", _rand(1, (1, 128), 0.5))])


def mixed_ops():
    return _model([N("Add", ["X", "b"], ["t1"]), N("Mul", ["t1", "s"], ["t2"]),
                   N("Sub", ["t2", "m"], ["t3"]), N("Div", ["t3", "d"], ["t4"]),
                   N("Relu", ["t4"], ["Y"])], "mixed_ops", [("X", [1, 64])], [("Y", [1, 64])],
                  [_w("b", _rand(2, (1, 64), 0.5)), _w("s", np.full((1, 64), 1.5)),
                   _w("m", _rand(3, (1, 64), 0.2)), _w("d", np.full((1, 64), 0.75))])


def two_input_add():
    return _model([N("Add", ["A", "B"], ["Y"])], "two_input_add", [("A", [1, 64]), ("B", [1, 64])],
                  [("Y", [1, 64])])


def two_output_tap():
    return _model([N("Add", ["X", "bias"], ["add_Y"]), N("Relu", ["add_Y"], ["Y"])],
                  "two_output_tap", [("X", [1, 64])], [("add_Y", [1, 64]), ("Y", [1, 64])],
                  [_w("bias", _rand(4, (1, 64), 0.5))])


def residual_chain():
    return _model([N("Add", ["X", "bias"], ["add_X"]), N("Relu", ["add_X"], ["relu_X"]),
                   N("Mul", ["relu_X", "scale"], ["mul_X"]), N("Add", ["X", "mul_X"], ["Y"])],
                  "residual_chain", [("X", [1, 64])], [("Y", [1, 64])],
                  [_w("bias", _rand(5, (1, 64), 0.1)), _w("scale", np.full((1, 64), 0.5))])


def broadcast(rows, cols, bias_shape=None, name="broadcast"):
    bias_shape = bias_shape or [cols]
    return _model([N("Add", ["X", "bias"], ["Y"])], name, [("X", [rows, cols])],
                  [("Y", [rows, cols])], [_w("bias", np.full(bias_shape, 0.25))])


def broadcast_aligned():
    return broadcast(8, 16, name="broadcast_aligned")


def broadcast_unaligned():
    return broadcast(4, 6, name="broadcast_unaligned")


def chunk_one():
    return broadcast(16, 1, [1], name="chunk_one")


def broadcast_3d():
    return _model([N("Add", ["X", "bias"], ["Y"])], "broadcast_3d", [("X", [2, 3, 4])],
                  [("Y", [2, 3, 4])], [_w("bias", [0.1, 0.2, 0.3, 0.4])])


def broadcast_mixed():
    return _model([N("Add", ["X", "bias"], ["add_Y"]), N("Relu", ["add_Y"], ["Y"])],
                  "broadcast_mixed", [("X", [4, 6])], [("Y", [4, 6])],
                  [_w("bias", np.full(6, 0.25))])


def broadcast_chain():
    return _model([N("Add", ["X", "bias"], ["add_Y"]), N("Relu", ["add_Y"], ["relu_Y"]),
                   N("Add", ["relu_Y", "X"], ["Y"])], "broadcast_chain", [("X", [4, 6])],
                  [("Y", [4, 6])], [_w("bias", np.full(6, 0.25))])


def broadcast_chain_bias():
    return _model([N("Add", ["X", "bias"], ["add_Y"]), N("Relu", ["add_Y"], ["relu_Y"]),
                   N("Add", ["relu_Y", "bias2"], ["Y"])], "broadcast_chain_bias",
                  [("X", [4, 6])], [("Y", [4, 6])],
                  [_w("bias", np.full(6, 0.25)), _w("bias2", _rand(6, (4, 6), 0.5))])


def broadcast_tapped():
    return _model([N("Add", ["X", "bias"], ["add_Y"]), N("Relu", ["add_Y"], ["Y"])],
                  "broadcast_tapped", [("X", [4, 6])], [("add_Y", [4, 6]), ("Y", [4, 6])],
                  [_w("bias", np.full(6, 0.25))])


def broadcast_lhs():
    """The smaller operand on the left: bias[6] - X[4,6]."""
    return _model([N("Sub", ["bias", "X"], ["Y"])], "broadcast_lhs", [("X", [4, 6])],
                  [("Y", [4, 6])], [_w("bias", _rand(7, (6,), 0.5))])


def clip_opset10():
    return _model([N("Clip", ["X"], ["Y"], min=0.0, max=6.0)], "clip_opset10",
                  [("X", [1, 64])], [("Y", [1, 64])], opset=10)


def clip_opset13(lo=0.0, hi=6.0):
    return _model([N("Clip", ["X", "lo", "hi"], ["Y"])], "clip_opset13", [("X", [1, 64])],
                  [("Y", [1, 64])], [_w("lo", np.float32(lo)), _w("hi", np.float32(hi))])


def sat_model(kind):
    """test_saturation.py models over a [1,256] ramp input (X[i] = i/256)."""
    n = 256
    if kind == "add_pos":
        return _model([N("Add", ["X", "b"], ["Y"])], kind, [("X", [1, n])], [("Y", [1, n])],
                      [_w("b", np.full((1, n), 127.5))])
    if kind == "add_neg":
        return _model([N("Add", ["X", "b1"], ["Z"]), N("Add", ["Z", "b2"], ["Y"])], kind,
                      [("X", [1, n])], [("Y", [1, n])],
                      [_w("b1", np.full((1, n), -63.0)), _w("b2", np.full((1, n), -65.5))])
    if kind == "mul_pos":
        return _model([N("Add", ["X", "o"], ["Z"]), N("Mul", ["Z", "s"], ["Y"])], kind,
                      [("X", [1, n])], [("Y", [1, n])],
                      [_w("o", np.full((1, n), 1.0)), _w("s", np.full((1, n), 90.0))])
    if kind == "mul_neg":
        return _model([N("Sub", ["X", "m"], ["Z"]), N("Mul", ["Z", "s"], ["Y"])], kind,
                      [("X", [1, n])], [("Y", [1, n])],
                      [_w("m", np.full((1, n), 2.0)), _w("s", np.full((1, n), 90.0))])
    if kind == "sub_pos":
        return _model([N("Sub", ["X", "b"], ["Y"])], kind, [("X", [1, n])], [("Y", [1, n])],
                      [_w("b", np.full((1, n), -127.5))])
    if kind == "sub_neg":
        return _model([N("Sub", ["X", "b1"], ["Z"]), N("Sub", ["Z", "b2"], ["Y"])], kind,
                      [("X", [1, n])], [("Y", [1, n])],
                      [_w("b1", np.full((1, n), 63.0)), _w("b2", np.full((1, n), 65.5))])
    if kind == "div_pos":
        return _model([N("Div", ["X", "d"], ["Y"])], kind, [("X", [1, n])], [("Y", [1, n])],
                      [_w("d", np.full((1, n), 1.0 / 256))])
    if kind == "div_neg":
        return _model([N("Div", ["X", "d"], ["Y"])], kind, [("X", [1, n])], [("Y", [1, n])],
                      [_w("d", np.full((1, n), -1.0 / 256))])
    raise ValueError(kind)


SAT_KINDS = ("add_pos", "add_neg", "mul_pos", "mul_neg", "sub_pos", "sub_neg", "div_pos",
             "div_neg")

# ----------------------------------------------------------------- MatMul graphs


def matmul(a_shape, w_shape, name="mm", w_input=False):
    y_shape = list(np.matmul(np.zeros(a_shape), np.zeros(w_shape)).shape)
    inits = [] if w_input else [_w("W", _rand(sum(w_shape), w_shape, 0.1))]
    inputs = [("X", list(a_shape))] + ([("W", list(w_shape))] if w_input else [])
    return _model([N("MatMul", ["X", "W"], ["Y"])], name, inputs, [("Y", y_shape)], inits)


MATMUL_CASES = {
    # name: (A shape, W shape)
    "mm_2d": ([4, 16], [16, 8]),
    "mm_batch_broadcast": ([2, 4, 4], [4, 16]),
    "mm_3d_3d": ([3, 4, 16], [3, 16, 8]),
    "mm_4d_4d": ([2, 3, 4, 16], [2, 3, 16, 8]),
    "mm_4d_3d": ([2, 3, 4, 16], [3, 16, 8]),
    "mm_3d_4d": ([3, 4, 16], [2, 3, 16, 8]),
    "mm_5d_3d": ([2, 2, 2, 4, 16], [2, 16, 8]),
    "mm_3d_5d": ([2, 4, 16], [2, 2, 2, 16, 8]),
    "mm_5d_4d": ([2, 2, 2, 4, 16], [2, 2, 16, 8]),
    "mm_4d_5d": ([2, 2, 4, 16], [2, 2, 2, 16, 8]),
    "mm_5d_2d": ([2, 2, 2, 4, 16], [16, 8]),
    "mm_2d_5d": ([4, 16], [2, 2, 2, 16, 8]),
}


def gemm_with_bias(n=4, k=16, m=8):
    return _model([N("Gemm", ["X", "W", "B"], ["Y"])], "gemm_with_bias", [("X", [n, k])],
                  [("Y", [n, m])], [_w("W", _rand(10, (k, m), 0.1)), _w("B", _rand(11, (m,), 0.1))])


def gemm_chain():
    return _model([N("Gemm", ["X", "W1", "B1"], ["H1"]), N("Relu", ["H1"], ["R1"]),
                   N("Gemm", ["R1", "W2", "B2"], ["H2"]), N("Relu", ["H2"], ["Y"])],
                  "gemm_chain", [("X", [4, 16])], [("Y", [4, 6])],
                  [_w("W1", _rand(12, (16, 12), 0.2)), _w("B1", _rand(13, (12,), 0.1)),
                   _w("W2", _rand(14, (12, 6), 0.2)), _w("B2", _rand(15, (6,), 0.1))])


def gemm_no_bias():
    return _model([N("Gemm", ["X", "W"], ["Y"])], "gemm_no_bias", [("X", [4, 16])],
                  [("Y", [4, 8])], [_w("W", _rand(16, (16, 8), 0.1))])


def gemm_trans_b():
    return _model([N("Gemm", ["X", "W", "B"], ["Y"], transB=1)], "gemm_trans_b",
                  [("X", [4, 16])], [("Y", [4, 8])],
                  [_w("W", _rand(17, (8, 16), 0.1)), _w("B", _rand(18, (8,), 0.1))])


# ----------------------------------------------------------------- Conv / Pool graphs


def conv(x_shape, w_shape, bias=True, name="conv", **attrs):
    inits = [_w("W", _rand(20 + sum(w_shape), w_shape, 0.2))]
    ins = ["X", "W"]
    if bias:
        inits.append(_w("B", _rand(21, (w_shape[0],), 0.2)))
        ins.append("B")
    g = _model([N("Conv", ins, ["Y"], **attrs)], name, [("X", list(x_shape))], [], inits)
    g.graph.output = [ox.value_info("Y", None)]
    return g


def conv_relu_chain():
    return _model([N("Conv", ["X", "W1"], ["Z1"], kernel_shape=[1, 1]), N("Relu", ["Z1"], ["Z2"]),
                   N("Conv", ["Z2", "W2", "B2"], ["Z3"], kernel_shape=[1, 1]),
                   N("Relu", ["Z3"], ["Y"])], "conv_relu_chain", [("X", [1, 4, 8, 8])],
                  [("Y", [1, 4, 8, 8])],
                  [_w("W1", _rand(30, (8, 4, 1, 1), 0.25)), _w("W2", _rand(31, (4, 8, 1, 1), 0.25)),
                   _w("B2", np.zeros(4))])


def pool(op, x_shape=(1, 4, 8, 8), name=None, **attrs):
    g = _model([N(op, ["X"], ["Y"], **attrs)], name or op, [("X", list(x_shape))], [])
    g.graph.output = [ox.value_info("Y", None)]
    return g


def mixed_all_kernels():
    """Conv -> Relu -> MaxPool -> GlobalAveragePool -> Reshape -> MatMul -> Add(bias)."""
    return _model([N("Conv", ["X", "W", "B"], ["c"], kernel_shape=[3, 3], pads=[1, 1, 1, 1]),
                   N("Relu", ["c"], ["r"]),
                   N("MaxPool", ["r"], ["p"], kernel_shape=[2, 2], strides=[2, 2]),
                   N("GlobalAveragePool", ["p"], ["g"]),
                   N("Reshape", ["g", "shp"], ["f"]),
                   N("MatMul", ["f", "FW"], ["m"]),
                   N("Add", ["m", "FB"], ["Y"])], "mixed_all_kernels", [("X", [2, 3, 8, 8])],
                  [("Y", [2, 10])],
                  [_w("W", _rand(40, (8, 3, 3, 3), 0.3)), _w("B", _rand(41, (8,), 0.1)),
                   ox.from_array(np.array([2, 8], np.int64), "shp"),
                   _w("FW", _rand(42, (8, 10), 0.3)), _w("FB", _rand(43, (10,), 0.1))])


def squeeze_then_matmul(opset=13):
    nodes = [N("GlobalAveragePool", ["X"], ["P"])]
    inits = [_w("W", np.full((4, 8), 0.25))]
    if opset >= 13:
        nodes.append(N("Squeeze", ["P", "axes"], ["F"]))
        inits.append(ox.from_array(np.array([2, 3], np.int64), "axes"))
    else:
        nodes.append(N("Squeeze", ["P"], ["F"], axes=[2, 3]))
    nodes.append(N("MatMul", ["F", "W"], ["Y"]))
    return _model(nodes, "squeeze_then_matmul", [("X", [1, 4, 4, 4])], [("Y", [1, 8])], inits,
                  opset=opset)


def unsqueeze_then_relu():
    return _model([N("Unsqueeze", ["X"], ["E"], axes=[2, 3]), N("Relu", ["E"], ["Y"])],
                  "unsqueeze_then_relu", [("X", [1, 4])], [("Y", [1, 4, 1, 1])], opset=11)


def reshape_output_alias():
    """Conv -> Reshape -> Squeeze -> graph output (the kernel writes the caller's buffer)."""
    return _model([N("Conv", ["X", "W"], ["c"], kernel_shape=[1, 1]),
                   N("Reshape", ["c", "shp"], ["r"]),
                   N("Dropout", ["r"], ["Y"])], "reshape_output_alias", [("X", [1, 4, 2, 2])],
                  [("Y", [1, 16])],
                  [_w("W", _rand(50, (4, 4, 1, 1), 0.3)),
                   ox.from_array(np.array([1, 16], np.int64), "shp")])


def reshape_input_to_output():
    """A graph output that is only a reshape of a graph input, next to a real kernel."""
    return _model([N("Reshape", ["X", "shp"], ["Z"]), N("Relu", ["X"], ["R"])],
                  "reshape_input_to_output", [("X", [2, 8])], [("Z", [16]), ("R", [2, 8])],
                  [ox.from_array(np.array([16], np.int64), "shp")])


def reshape_then_matmul():
    return _model([N("Reshape", ["X", "shp"], ["F"]), N("MatMul", ["F", "W"], ["Y"])],
                  "reshape_then_matmul", [("X", [2, 2, 4])], [("Y", [2, 3])],
                  [ox.from_array(np.array([2, 8], np.int64), "shp"), _w("W", _rand(51, (8, 3), 0.3))])


def unsupported():
    return _model([N("Softmax", ["X"], ["Y"])], "unsupported", [("X", [1, 8])], [("Y", [1, 8])])
