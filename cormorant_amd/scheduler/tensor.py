"""Tensor metadata and the Q8.8 storage conversions the scheduler applies.

TensorInfo follows inference-scheduler/src/tensor.py:38-66 (name, shape,
dtype string, float32 data for initializers, numel >= 1, C-identifier name).

The conversions follow the reference's ApFixed(16, 8) data type
(inference-scheduler/src/dtype.py:266-296):

* weights are written to device memory with ``float_to_storage``:
  clamp to [-128, 127.99609375], then round to the nearest 1/256
  (numpy's round-half-to-even), two's-complement int16;
* the ramp fill of the generated test harness stores ``pos & 0xFFFF`` at
  buffer position ``pos`` (``ramp_to_storage``).
"""
from __future__ import annotations

import re
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

Q_SCALE = 256.0
Q_MIN = -128.0
Q_MAX = 127.99609375
ALIGN_BYTES = 16          # broadcast chunk alignment (nodes.py:117)
BYTES_PER_ELEM = 2
ALIGN_ELEMS = ALIGN_BYTES // BYTES_PER_ELEM
POOL_ALIGN_BYTES = 64     # pool slot alignment (codegen/_core.py:312-315)


def c_identifier(name: str) -> str:
    """ONNX tensor name -> C identifier (same rule as tensor.py:20-30)."""
    s = re.sub(r"[^A-Za-z0-9_]", "_", name)
    if s and s[0].isdigit():
        s = "t_" + s
    s = re.sub(r"_+", "_", s).strip("_")
    return s or "tensor"


def float_to_storage(x) -> np.ndarray:
    """Real values -> raw int16 (saturate, then round to nearest)."""
    v = np.clip(np.asarray(x, dtype=np.float64), Q_MIN, Q_MAX)
    return np.round(v * Q_SCALE).astype(np.int16)


def storage_to_float(raw) -> np.ndarray:
    return np.asarray(raw, dtype=np.int16).astype(np.float64) / Q_SCALE


def ramp_to_storage(positions) -> np.ndarray:
    """Raw bits of the test-harness ramp: element at buffer position p holds p & 0xFFFF."""
    return (np.asarray(positions, dtype=np.int64) & 0xFFFF).astype(np.uint16).view(np.int16)


@dataclass
class TensorInfo:
    onnx_name: str
    shape: List[int]
    dtype: str = "float32"
    data: Optional[np.ndarray] = field(default=None, repr=False)

    @property
    def numel(self) -> int:
        n = 1
        for d in self.shape:
            n *= int(d)
        return max(n, 1)

    @property
    def c_name(self) -> str:
        return c_identifier(self.onnx_name)

    @property
    def is_weight(self) -> bool:
        return self.data is not None

    def storage(self) -> np.ndarray:
        """Raw int16 contents of a weight, flat, in logical order."""
        if self.data is None:
            raise ValueError(f"tensor '{self.onnx_name}' has no data")
        return float_to_storage(self.data.reshape(-1))
