"""Inference scheduler: ONNX graph -> the four Q8.8 kernels on one MI355X.

The counterpart of the reference's inference-scheduler/src package: the same
op dispatch (graph.py, nodes.py), buffer plan (codegen/_core.py) and Gemm /
Reshape handling, with a HIP backend (``InferenceSession``) in place of the
generated KV260 C project.
"""
from . import fuse
from .graph import ALL_SUPPORTED_OP_TYPES, OnnxGraph, split_gemms
from .nodes import (OP_ADD, OP_DIV, OP_MUL, OP_RELU, OP_RELU6, OP_SUB, POOL_AVG, POOL_LP,
                    POOL_MAX, ConvNode, KernelCall, MatmulNode, PoolNode, ReshapeNode,
                    ScheduledNode, SchedulerError, broadcast_info)
from .plan import BufferPlan, TensorLayout, compute_tensor_layouts, live_intervals, pool_layout
from .tensor import TensorInfo, float_to_storage, ramp_to_storage, storage_to_float


def InferenceSession(*args, **kwargs):
    """HIP backend (imported lazily so graph tools work without the native library)."""
    from .session import InferenceSession as _S
    return _S(*args, **kwargs)
