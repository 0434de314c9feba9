"""GPU parity of cm_conv_gap: a 1x1 convolution, its activation and a
GlobalAveragePool in one launch equal the convolution (ConvKernel.cpp:171-249)
followed by the pool (PoolingKernel.cpp:253-266) on the CPU oracle, bit for bit,
with full-range operands whose sums wrap."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from cormorant_amd import _native
from cormorant_amd import kernels as K
from cormorant_amd import workloads as wl
from tests.gpu_util import dev, empty_dev, host, oracle_threads, say

pytestmark = pytest.mark.gpu

# batch, in_ch, hw, out_ch, bias, act
CASES = [
    (16, 320, 49, 1280, 1, K.ACT_RELU6),   # the MobileNetV2-like head
    (3, 64, 64, 96, 1, K.ACT_RELU),        # a full 64-pixel plane
    (5, 8, 1, 33, 0, K.ACT_NONE),          # one pixel, a partial second row tile
    (2, 100, 33, 31, 1, K.ACT_RELU6),      # in_ch not a multiple of 8 (element loads)
    (4, 512, 17, 65, 0, K.ACT_RELU),       # the channel limit, three row tiles
    (1, 1, 7, 1, 1, K.ACT_NONE),
]


def reference(x, w, b, batch, in_ch, hw, out_ch, has_bias, act):
    conv = np.zeros(batch * out_ch * hw, np.int16)
    oracle.set_threads(oracle_threads())
    oracle.conv(x, w, b, conv, batch, in_ch, hw, 1, out_ch, hw, 1, 1, 1, 1, 1, 1, 1, 0, 0,
                has_bias, 0, threads=True)
    if act == K.ACT_RELU:
        conv = np.maximum(conv, 0).astype(np.int16)
    elif act == K.ACT_RELU6:
        conv = np.clip(conv, 0, 1536).astype(np.int16)
    want = np.zeros(batch * out_ch, np.int16)
    oracle.pool(conv, want, batch, out_ch, hw, 1, 1, 1, hw, 1, 1, 1, 0, 0, 1, 1, 1, 2, 0)
    return want


@pytest.mark.parametrize("case", CASES, ids=[str(c) for c in CASES])
@pytest.mark.parametrize("rng_kind", ["full", "network"])
def test_conv_gap_matches_conv_then_pool(case, rng_kind):
    batch, in_ch, hw, out_ch, has_bias, act = case
    say(f"conv gap {case} {rng_kind}")
    assert K.conv_gap_supported(batch, in_ch, hw, out_ch)
    g = wl.rng(871, *case, len(rng_kind))
    if rng_kind == "full":
        x = g.integers(-32768, 32768, batch * in_ch * hw, dtype=np.int16)
        w = g.integers(-32768, 32768, out_ch * in_ch, dtype=np.int16)
        b = g.integers(-32768, 32768, out_ch, dtype=np.int16)
    else:   # activations and weights of a network: int8-range weights, small sums
        x = wl.uniform_q88(g, (batch * in_ch * hw,), -2.0, 2.0)
        w = wl.normal_q88(g, (out_ch * in_ch,), 0.05)
        b = wl.normal_q88(g, (out_ch,), 0.05)
    want = reference(x, w, b, batch, in_ch, hw, out_ch, has_bias, act)
    y = empty_dev(batch * out_ch)
    K.ConvGapKernel(dev(x), dev(w), dev(b) if has_bias else None, y, batch, in_ch, hw, out_ch,
                    has_bias=has_bias, act=act)
    np.testing.assert_array_equal(host(y), want)
    # the same through the two launches it replaces
    conv = empty_dev(batch * out_ch * hw)
    K.ConvKernel(dev(x), dev(w), dev(b) if has_bias else None, conv, batch, in_ch, hw, 1, out_ch,
                 hw, 1, 1, 1, 1, 1, 1, 1, 0, 0, has_bias, 0, act=act)
    y2 = empty_dev(batch * out_ch)
    K.PoolingKernel(conv, y2, batch, out_ch, hw, 1, 1, 1, hw, 1, 1, 1, 0, 0, 1, 1, 1, 2, 0)
    np.testing.assert_array_equal(host(y2), want)


def test_conv_gap_rejects_unsupported_shapes():
    """Planes past 64 pixels and more than 512 input channels are refused (an
    error, no launch); the query agrees."""
    x = dev(np.zeros(2 * 8 * 65, np.int16))
    w = dev(np.zeros(8 * 8, np.int16))
    y = empty_dev(16)
    assert not K.conv_gap_supported(2, 8, 65, 8)
    with pytest.raises(_native.CmError):
        K.ConvGapKernel(x, w, None, y, 2, 8, 65, 8, has_bias=0)
    assert not K.conv_gap_supported(1, 513, 4, 8)
    assert not K.conv_gap_supported(0, 8, 4, 8)
