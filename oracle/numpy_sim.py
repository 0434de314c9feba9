"""Numpy restatement of the scheduler's float64 simulation -- TEST INFRASTRUCTURE ONLY.

Second oracle.  It follows inference-scheduler/src/codegen/_simulate.py and
inference-scheduler/src/dtype.py:

* values are float64 multiples of 1/256 (ap_fixed<16,8>);
* MatMul / Conv sum exactly in float64 (no 32-bit wrap) and then ``truncate``
  (clip to [-128, 127.99609375], floor to 1/256) -- dtype.py:270-276;
* DIV uses ``truncate_div`` (clip, trunc toward zero) -- dtype.py:278-282;
* AVG pool divides by the denominator in float64, LP p=2 takes a float64
  sqrt -- _simulate.py:126-185.

Where this model and the C-simulation differ (32-bit accumulator wrap, LP p=2
outputs >= 16.0), the C-simulation semantics (``oracle.lib``) rule; the
functions below are used where the two agree and to count where they differ.
The loops are vectorised over the spatial window instead of the reference's
per-pixel einsum; every partial sum is exactly representable in float64, so
the order of summation does not change any result.
"""
from __future__ import annotations

import numpy as np

SCALE = 256.0
MIN_VAL = -128.0
MAX_VAL = 32767.0 / 256.0

OP_ADD, OP_SUB, OP_MUL, OP_DIV, OP_RELU, OP_RELU6 = range(6)
POOL_MAX, POOL_AVG, POOL_LP = 0, 1, 2


def to_float(raw: np.ndarray) -> np.ndarray:
    """int16 raw -> float64 value (dtype.py:284-288 for the bit reinterpretation)."""
    return np.asarray(raw, dtype=np.int16).astype(np.float64) / SCALE


def to_raw(x: np.ndarray) -> np.ndarray:
    """On-grid float64 value -> int16 raw (exact for simulation outputs)."""
    return np.round(np.asarray(x, dtype=np.float64) * SCALE).astype(np.int16)


def quantize(x: np.ndarray) -> np.ndarray:
    """dtype.py:266-268: clip, round half to even."""
    c = np.clip(np.asarray(x, dtype=np.float64), MIN_VAL, MAX_VAL)
    return np.round(c * SCALE) / SCALE


def truncate(x: np.ndarray) -> np.ndarray:
    """dtype.py:270-276: clip, floor toward -inf."""
    c = np.clip(np.asarray(x, dtype=np.float64), MIN_VAL, MAX_VAL)
    return np.floor(c * SCALE) / SCALE


def truncate_div(x: np.ndarray) -> np.ndarray:
    """dtype.py:278-282: clip, truncate toward zero."""
    c = np.clip(np.asarray(x, dtype=np.float64), MIN_VAL, MAX_VAL)
    return np.trunc(c * SCALE) / SCALE


def elementwise(op: int, a: np.ndarray, b: np.ndarray | None = None) -> np.ndarray:
    """_simulate.py:332-365 (float values in, float values out)."""
    if op == OP_ADD:
        return truncate(a + b)
    if op == OP_SUB:
        return truncate(a - b)
    if op == OP_MUL:
        return truncate(a * b)
    if op == OP_DIV:
        with np.errstate(divide="ignore", invalid="ignore"):
            return truncate_div(a / b)
    if op == OP_RELU:
        return truncate(np.maximum(a, 0.0))
    if op == OP_RELU6:
        return truncate(np.minimum(np.maximum(a, 0.0), 6.0))
    raise ValueError(f"unknown op {op}")


def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """_simulate.py:300-306: np.matmul then truncate."""
    return truncate(np.matmul(a, b))


def conv2d(x, w, bias, stride_h, stride_w, pad_top, pad_left, dilation_h, dilation_w,
           out_h, out_w, is_depthwise=False):
    """_simulate.py:49-125 (exact float64 sum, bias added after), then truncate."""
    N, C, H, W = x.shape
    M, _, kH, kW = w.shape
    y = np.zeros((N, M, out_h, out_w), dtype=np.float64)
    oh = np.arange(out_h)
    ow = np.arange(out_w)
    for khi in range(kH):
        ih = oh * stride_h + khi * dilation_h - pad_top
        vh = (ih >= 0) & (ih < H)
        if not vh.any():
            continue
        for kwi in range(kW):
            iw = ow * stride_w + kwi * dilation_w - pad_left
            vw = (iw >= 0) & (iw < W)
            if not vw.any():
                continue
            xs = x[:, :, ih[vh]][:, :, :, iw[vw]]          # [N, C, h', w']
            if is_depthwise:
                contrib = xs * w[:, 0, khi, kwi].reshape(1, M, 1, 1)
            else:
                contrib = np.einsum("nchw,mc->nmhw", xs, w[:, :, khi, kwi], optimize=True)
            y[np.ix_(np.arange(N), np.arange(M), np.nonzero(vh)[0], np.nonzero(vw)[0])] += contrib
    if bias is not None:
        y += np.asarray(bias, dtype=np.float64).reshape(1, M, 1, 1)
    return truncate(y)


def pool2d(x, pool_h, pool_w, stride_h, stride_w, pad_top, pad_left, dil_h, dil_w,
           out_h, out_w, pool_type, lp_order, count_include_pad):
    """_simulate.py:126-185, then truncate."""
    N, C, H, W = x.shape
    y = np.zeros((N, C, out_h, out_w), dtype=np.float64)
    for oh in range(out_h):
        for ow in range(out_w):
            valid = 0
            acc = (np.full((N, C), -np.inf) if pool_type == POOL_MAX else np.zeros((N, C)))
            for khi in range(pool_h):
                ih = oh * stride_h + khi * dil_h - pad_top
                for kwi in range(pool_w):
                    iw = ow * stride_w + kwi * dil_w - pad_left
                    if ih < 0 or ih >= H or iw < 0 or iw >= W:
                        continue
                    valid += 1
                    v = x[:, :, ih, iw]
                    if pool_type == POOL_MAX:
                        acc = np.maximum(acc, v)
                    elif pool_type == POOL_AVG:
                        acc = acc + v
                    else:
                        acc = acc + (np.abs(v) if lp_order == 1 else v * v)
            denom = max((pool_h * pool_w) if count_include_pad else valid, 1)
            if pool_type == POOL_MAX:
                y[:, :, oh, ow] = acc
            elif pool_type == POOL_AVG:
                y[:, :, oh, ow] = acc / denom
            else:
                y[:, :, oh, ow] = acc if lp_order == 1 else np.sqrt(np.maximum(acc, 0.0))
    return truncate(y)
