"""GPU parity: ConvPairKernel (a convolution and a 1x1 convolution of its output in
one launch, the middle tensor kept in LDS) against the oracle running the two
convolutions one after the other, with the activation and the saturating Add
applied exactly as the fused epilogues apply them."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from cormorant_amd import _native
from cormorant_amd import kernels as K
from cormorant_amd import workloads as wl
from tests.gpu_util import dev, empty_dev, host, oracle_threads, say

pytestmark = pytest.mark.gpu

NONE, RELU, RELU6 = K.ACT_NONE, K.ACT_RELU, K.ACT_RELU6


def act_np(v, act):
    if act == RELU:
        return np.clip(v, 0, 32767)
    if act == RELU6:
        return np.clip(v, 0, 1536)
    return v


def pair_reference(x, w1, b1, w2, b2, add, N, C, H, W, M1, OH, OW, k, s, d, p, M2, act1, act2):
    oracle.set_threads(oracle_threads())
    h = np.zeros(N * M1 * OH * OW, np.int16)
    oracle.conv(x, w1, b1 if b1 is not None else np.zeros(M1, np.int16), h, N, C, H, W, M1, OH, OW,
                k, k, s, s, d, d, p, p, int(b1 is not None), 0, threads=True)
    h = act_np(h.astype(np.int32), act1).astype(np.int16)
    y = np.zeros(N * M2 * OH * OW, np.int16)
    oracle.conv(h, w2, b2 if b2 is not None else np.zeros(M2, np.int16), y, N, M1, OH, OW, M2, OH, OW,
                1, 1, 1, 1, 1, 1, 0, 0, int(b2 is not None), 0, threads=True)
    y = y.astype(np.int32)
    if add is not None:
        y = np.clip(y + add, -32768, 32767)
    return act_np(y, act2).astype(np.int16)


def run_pair(geom, seed, w1_range, w2_range, bias=(True, True), with_add=True):
    N, C, H, W, M1, k, s, d, p, M2, act1, act2 = geom
    OH, OW = (H + 2 * p - d * (k - 1) - 1) // s + 1, (W + 2 * p - d * (k - 1) - 1) // s + 1
    args = (N, C, H, W, M1, OH, OW, k, k, s, d, p, p, M2)
    size = K.conv_pair_packed_size(*args)
    assert size > 0, f"expected the pair path for {geom}"
    g = wl.rng(911, seed, *geom)
    x = g.integers(-32768, 32768, N * C * H * W, dtype=np.int16)
    w1 = g.integers(*w1_range, M1 * C * k * k, dtype=np.int16)
    w2 = g.integers(*w2_range, M2 * M1, dtype=np.int16)
    b1 = g.integers(-32768, 32768, M1, dtype=np.int16) if bias[0] else None
    b2 = g.integers(-32768, 32768, M2, dtype=np.int16) if bias[1] else None
    add = g.integers(-32768, 32768, N * M2 * OH * OW, dtype=np.int16) if with_add else None
    want = pair_reference(x, w1, b1, w2, b2, add, N, C, H, W, M1, OH, OW, k, s, d, p, M2, act1, act2)
    packed = torch.empty(-(-size // 4), dtype=torch.int32, device="cuda")
    K.conv_pair_pack(dev(w1), dev(w2), packed, *args)
    y = empty_dev(want.size)
    K.ConvPairKernel(dev(x), packed, dev(b1) if b1 is not None else None,
                     dev(b2) if b2 is not None else None, y, *args, act1=act1,
                     add=dev(add) if add is not None else None, act=act2)
    np.testing.assert_array_equal(host(y), want)


PAIRS = [
    # N, C, H, W, M1, k, s, d, p, M2, act1, act2
    (16, 64, 14, 14, 64, 3, 1, 1, 1, 64, RELU6, NONE),       # MobileNetV2-like 14x14 block
    (16, 32, 28, 28, 32, 3, 1, 1, 1, 32, RELU6, NONE),       # 28x28 block
    (8, 96, 14, 14, 96, 3, 1, 1, 1, 160, RELU6, NONE),       # two 1x1 k steps, five 1x1 row tiles
    (16, 24, 56, 56, 24, 3, 2, 1, 1, 32, RELU6, RELU6),      # stride 2, 16-byte row loads
    (2, 32, 112, 112, 32, 3, 1, 1, 1, 16, RELU6, NONE),      # 32-row tile, 256-pixel sub-tiles
    (3, 20, 17, 23, 40, 3, 1, 1, 1, 72, RELU, RELU),         # odd sizes, partial pixel tiles
    (4, 64, 28, 28, 128, 3, 2, 2, 2, 96, NONE, RELU6),       # dilation 2, 128 middle channels
    (2, 130, 9, 11, 16, 3, 1, 1, 1, 256, RELU6, NONE),       # three input chunks, 256 1x1 outputs
    (5, 8, 20, 20, 100, 5, 1, 1, 2, 48, RELU6, RELU),        # 5x5 window
]


@pytest.mark.parametrize("geom", PAIRS, ids=[str(p) for p in PAIRS])
def test_pair_int8_weights(geom):
    """Weights in [-128, 127] (both GEMMs on the two-product path), full-range
    inputs, biases, a residual Add."""
    say(f"conv pair int8 weights {geom}")
    run_pair(geom, 1, (-128, 128), (-128, 128))


@pytest.mark.parametrize("geom", PAIRS, ids=[str(p) for p in PAIRS])
def test_pair_full_range_weights(geom):
    """Full-range weights in both convolutions (four limb products each, wrapping sums)."""
    say(f"conv pair full-range weights {geom}")
    run_pair(geom, 2, (-32768, 32768), (-32768, 32768))


@pytest.mark.parametrize("which", ["first", "second"])
def test_pair_mixed_weight_paths(which):
    """One convolution on the two-product path, the other on four; no biases, no Add."""
    geom = (6, 48, 16, 16, 64, 3, 1, 1, 1, 80, RELU6, NONE)
    say(f"conv pair mixed paths ({which} full-range)")
    full, small = (-32768, 32768), (-128, 128)
    run_pair(geom, 3, full if which == "first" else small, small if which == "first" else full,
             bias=(False, False), with_add=False)


def test_pair_rejects_other_shapes():
    """Shapes outside the path report no packed size, and the packed call refuses them."""
    assert K.conv_pair_packed_size(4, 32, 14, 14, 160, 14, 14, 3, 3, 1, 1, 1, 1, 64) == 0  # 160 middle
    assert K.conv_pair_packed_size(4, 32, 14, 14, 64, 14, 14, 3, 3, 1, 1, 1, 1, 300) == 0   # 300 outputs
    assert K.conv_pair_packed_size(4, 32, 14, 14, 64, 14, 14, 1, 1, 1, 1, 0, 0, 64) == 0    # 1x1 first
    buf = torch.empty(64, dtype=torch.int32, device="cuda")
    x = torch.zeros(4 * 32 * 14 * 14, dtype=torch.int16, device="cuda")
    y = torch.zeros(4 * 64 * 14 * 14, dtype=torch.int16, device="cuda")
    with pytest.raises(_native.CmError):
        K.ConvPairKernel(x, buf, None, None, y, 4, 32, 14, 14, 160, 14, 14, 3, 3, 1, 1, 1, 1, 64)
