"""GPU parity: ConvKernel (implicit GEMM / pointwise GEMM on MFMA, direct depthwise)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from cormorant_amd import _native
from cormorant_amd import kernels as K
from cormorant_amd import workloads as wl
from tests import refcases as rc
from tests.gpu_util import dev, empty_dev, host, oracle_threads, say

pytestmark = pytest.mark.gpu


def workspace_for(*args):
    """A device workspace of the size the call asks for (None when it needs none)."""
    import torch
    need = K.conv_workspace_size(*args)
    return torch.empty(max(need, 16) // 4, dtype=torch.int32, device="cuda").fill_(0x13572468) \
        if need else None


def conv_both(x, w, b, N, C, H, W, M, OH, OW, kh, kw, sh, sw, dh, dw, pt, pl, bias, dwise,
              ws=False):
    y = empty_dev(N * M * OH * OW)
    args = (N, C, H, W, M, OH, OW, kh, kw, sh, sw, dh, dw, pt, pl, bias, dwise)
    K.ConvKernel(dev(x), dev(w), dev(b), y, *args, workspace=workspace_for(*args) if ws else None)
    want = np.zeros(N * M * OH * OW, np.int16)
    oracle.set_threads(oracle_threads())
    oracle.conv(np.ascontiguousarray(x.reshape(-1)), np.ascontiguousarray(w.reshape(-1)),
                np.ascontiguousarray(b.reshape(-1)), want, N, C, H, W, M, OH, OW, kh, kw, sh, sw,
                dh, dw, pt, pl, bias, dwise, threads=True)
    return host(y), want


@pytest.mark.parametrize("i", range(len(rc.CONV_GEOMS)), ids=[g[0] for g in rc.CONV_GEOMS])
def test_reference_geometries(i):
    geom = rc.CONV_GEOMS[i]
    (name, N, C, H, W, M, kh, kw, sh, sw, dh, dw, pt, pl, pb, pr, bias, dwise, xs, ws, bs) = geom
    say(f"conv reference geometry {name}")
    g = wl.rng(830, i)
    x = wl.uniform_q88(g, (N, C, H, W), -xs, xs)
    w = wl.uniform_q88(g, (M, 1 if dwise else C, kh, kw), -ws, ws)
    b = wl.uniform_q88(g, (M,), -bs, bs)
    OH = rc.conv_out_size(H, kh, sh, dh, pt, pb)
    OW = rc.conv_out_size(W, kw, sw, dw, pl, pr)
    got, want = conv_both(x, w, b, N, C, H, W, M, OH, OW, kh, kw, sh, sw, dh, dw, pt, pl, bias, dwise)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("case", rc.CONV_SAT, ids=[c[0] for c in rc.CONV_SAT])
def test_saturation_kats(case):
    name, wv, bv, expect = case
    say(f"conv saturation {name}")
    x = np.full((1, 1, 3, 3), 32767, np.int16)
    w = np.full((1, 1, 1, 1), int(wv * 256), np.int16)
    b = np.full((1,), int(bv * 256), np.int16)
    got, want = conv_both(x, w, b, 1, 1, 3, 3, 1, 3, 3, 1, 1, 1, 1, 1, 1, 0, 0, 1, 0)
    np.testing.assert_array_equal(got, want)
    assert np.all(got / 256.0 == expect)


GEOMS = [
    # N, C, H, W, M, kh, kw, sh, sw, dh, dw, pt, pl, bias, dw
    (2, 3, 33, 31, 32, 3, 3, 2, 2, 1, 1, 1, 1, 1, 0),     # stem-like, K = 27
    (2, 16, 14, 14, 24, 1, 1, 1, 1, 1, 1, 0, 0, 1, 0),    # pointwise, aligned plane? 196 % 8 != 0
    (2, 32, 16, 16, 40, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0),    # pointwise, 16-byte loads
    (1, 24, 7, 7, 200, 1, 1, 1, 1, 1, 1, 0, 0, 1, 0),     # pointwise on a 7x7 plane
    (1, 8, 10, 10, 8, 1, 1, 2, 2, 1, 1, 0, 0, 1, 0),      # 1x1 strided -> implicit GEMM
    (2, 20, 12, 9, 150, 3, 5, 1, 2, 2, 1, 2, 1, 1, 0),
    (1, 130, 9, 9, 7, 3, 3, 1, 1, 1, 1, 1, 1, 1, 0),      # K = 1170 (many k tiles)
    (2, 12, 10, 10, 12, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1),    # depthwise
    (1, 6, 9, 9, 4, 5, 5, 2, 2, 1, 1, 2, 2, 0, 1),        # depthwise, out_ch < in_ch
    (1, 256, 6, 6, 20, 3, 3, 1, 1, 1, 1, 1, 1, 1, 0),     # K = 2304: gather without the k table
    (1, 40, 11, 11, 9, 7, 7, 1, 1, 3, 2, 9, 6, 1, 0),     # large dilation, pad beyond the window
    # direct (vector ALU) path: <= 32 output channels, K <= 32, >= 32768 output pixels
    (4, 3, 256, 130, 32, 3, 3, 2, 2, 1, 1, 1, 1, 1, 0),   # stem, K = 27, 8 k of padding
    (3, 32, 112, 100, 16, 1, 1, 1, 1, 1, 1, 0, 0, 1, 0),  # 1x1, K = 32, 16 channels
    (3, 16, 110, 110, 20, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0),  # 20 channels in a group of 24
    (1, 7, 200, 190, 5, 2, 2, 1, 1, 2, 3, 3, 1, 1, 0),    # 2x2 dilated, padding, 5 channels
    # 3x3 patch path (channels a multiple of 8, <= 64 of them in and out, at least
    # 64 output tiles of 8 x 16): partial tiles, padding channels, dead weight
    # rows, every output access width
    (32, 32, 9, 17, 32, 3, 3, 1, 1, 1, 1, 1, 1, 1, 0),    # odd output width (1-wide stores)
    (16, 16, 30, 60, 16, 3, 3, 2, 2, 1, 1, 1, 1, 0, 0),   # stride 2, no bias, width 30
    (8, 24, 28, 28, 24, 3, 3, 1, 1, 1, 1, 1, 1, 1, 0),    # 24 of 32 channels, 24 of 32 rows
    (12, 64, 20, 24, 64, 3, 3, 1, 1, 1, 1, 1, 1, 1, 0),   # 64 x 64, nine k steps
    (64, 8, 18, 34, 5, 3, 3, 2, 2, 1, 1, 0, 0, 1, 0),     # 8 channels, 5 outputs, no padding
    (16, 40, 16, 16, 48, 3, 3, 1, 1, 1, 1, 2, 2, 1, 0),   # 48-byte positions, padding 2
    (64, 56, 9, 12, 33, 3, 3, 2, 2, 1, 1, 2, 1, 1, 0),    # 80-byte positions, pads 2 / 1
    (2, 32, 37, 45, 32, 3, 3, 1, 1, 1, 1, 1, 1, 1, 0),    # the same layer under 64 tiles: gather
    # the 3x3 patch path at sizes the register-only kernel leaves to it (> 2^21 outputs)
    (512, 32, 9, 17, 32, 3, 3, 1, 1, 1, 1, 1, 1, 1, 0),   # odd output width
    (320, 16, 30, 60, 16, 3, 3, 2, 2, 1, 1, 1, 1, 0, 0),  # stride 2, no bias
]


@pytest.mark.parametrize("geom", GEOMS, ids=[str(g) for g in GEOMS])
def test_geometries_full_range(geom):
    N, C, H, W, M, kh, kw, sh, sw, dh, dw, pt, pl, bias, dwise = geom
    OH = (H + 2 * pt - dh * (kh - 1) - 1) // sh + 1
    OW = (W + 2 * pl - dw * (kw - 1) - 1) // sw + 1
    say(f"conv geometry {geom}")
    g = wl.rng(831, *geom)
    x = g.integers(-32768, 32768, (N, C, H, W), dtype=np.int16)
    w = g.integers(-32768, 32768, (M, 1 if dwise else C, kh, kw), dtype=np.int16)
    b = g.integers(-32768, 32768, (M,), dtype=np.int16)
    got, want = conv_both(x, w, b, N, C, H, W, M, OH, OW, kh, kw, sh, sw, dh, dw, pt, pl, bias, dwise)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("geom", [
    # N, C, H, W, M, kh, kw, s, p: pointwise GEMM, implicit GEMM, direct path shapes
    (2, 0, 16, 16, 24, 1, 1, 1, 0), (1, 0, 9, 11, 40, 3, 3, 2, 1), (2, 0, 160, 160, 8, 3, 3, 1, 1)])
def test_zero_input_channels_give_bias(geom):
    """in_ch = 0: the reference's channel loop is empty and y = bias (or 0)."""
    N, C, H, W, M, kh, kw, s, p = geom
    OH, OW = (H + 2 * p - kh) // s + 1, (W + 2 * p - kw) // s + 1
    say(f"conv in_ch=0 {geom}")
    b = wl.rng(832, M).integers(-32768, 32768, M, dtype=np.int16)
    for bias in (1, 0):
        got, want = conv_both(np.zeros(1, np.int16), np.zeros(1, np.int16), b, N, C, H, W, M, OH,
                              OW, kh, kw, s, s, 1, 1, p, p, bias, 0)
        np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(got.reshape(N, M, -1), np.broadcast_to(
            (b if bias else np.zeros(M, np.int16))[None, :, None], (N, M, OH * OW)))


@pytest.mark.parametrize("ws", [False, True], ids=["no_workspace", "workspace"])
@pytest.mark.parametrize("case", wl.CONV_CASES, ids=[c.name for c in wl.CONV_CASES])
def test_config4_full_size(case, ws):
    say(f"conv full-size {case.name} workspace={ws}")
    x, w, b = wl.conv_operands(case)
    o = case.out_hw
    got, want = conv_both(x, w, b, case.batch, case.in_ch, case.hw, case.hw, case.out_ch, o, o,
                          case.k, case.k, case.stride, case.stride, case.dil, case.dil, case.pad,
                          case.pad, 1, 0, ws=ws)
    np.testing.assert_array_equal(got, want)


def pgemm_need(C, M, kh, kw):
    """Workspace sizes of the patch-GEMM path: packed weights (row tiles of TB = 32, 64
    or 128 output channels: TB x 64 k as two limb planes and one int8 plane per row
    tile and k step), and one uint32 row sum and one int8 flag per padded row.  With
    one patch of every channel chunk the step count is padded to a multiple of 3 when
    that adds at most an eighth more steps (zero-weight steps for the three-set
    pipeline); with restaged chunks it is not, so both sizes are possible."""
    taps, nch = kh * kw, -(-C // 64)
    tb = 128 if nch > 1 or M > 64 else 64 if M > 32 else 32
    mt = -(-M // tb)
    steps = (nch - 1) * taps + (taps * -(-(C - (nch - 1) * 64) // 16) + 3) // 4
    pad = (3 - steps % 3) % 3
    sizes = {mt * steps * 3 * tb * 64 + 8 * tb * mt}
    if pad and 8 * pad <= steps and (steps + pad) * 4 <= 256:
        sizes.add(mt * (steps + pad) * 3 * tb * 64 + 8 * tb * mt)
    return sizes


PGEMM = [
    # N, C, H, W, M, kh, kw, s, d, p: every shape fills >= 200 blocks and has more
    # than 2^21 outputs (smaller layers take the register-only kernel)
    (32, 64, 56, 56, 128, 3, 3, 1, 1, 1),      # conv A
    (32, 64, 56, 56, 128, 3, 3, 2, 2, 2),      # conv B
    (24, 70, 40, 36, 130, 3, 3, 1, 1, 1),      # two channel chunks, two row tiles
    (64, 24, 30, 40, 120, 3, 3, 2, 2, 2),      # stride = dilation 2, 24 channels
    (60, 16, 33, 40, 110, 5, 5, 2, 1, 2),      # 5x5, stride 2, dilation 1
    (160, 130, 11, 11, 120, 3, 3, 1, 2, 2),    # three chunks (64, 64, 2 channels), dilation 2
    (48, 8, 26, 22, 96, 3, 1, 1, 3, 1),        # 3x1 window, dilation 3
    (32, 130, 12, 100, 72, 3, 3, 1, 1, 1),     # three chunks too wide for one patch: restaged in turn
    (112, 150, 20, 24, 40, 5, 5, 1, 1, 2),     # 5x5, three chunks in one patch: 63 k steps
    (32, 96, 28, 28, 96, 3, 3, 1, 1, 1),       # 14 k steps padded to 15 (one zero-weight step)
    (96, 160, 14, 14, 160, 3, 3, 1, 1, 1),     # 23 k steps padded to 24, two row tiles
]


@pytest.mark.parametrize("geom", PGEMM, ids=[str(g) for g in PGEMM])
def test_patch_gemm_full_range(geom):
    """The patch-GEMM path (taken when a workspace holds the packed weights):
    full-range operands whose sums wrap, with bias, a fused Add and an activation."""
    N, C, H, W, M, kh, kw, s, d, p = geom
    OH, OW = (H + 2 * p - d * (kh - 1) - 1) // s + 1, (W + 2 * p - d * (kw - 1) - 1) // s + 1
    args = (N, C, H, W, M, OH, OW, kh, kw, s, s, d, d, p, p, 1, 0)
    assert K.conv_workspace_size(*args) in pgemm_need(C, M, kh, kw), "expected the patch-GEMM path"
    say(f"conv patch gemm {geom}")
    g = wl.rng(833, *geom)
    x = g.integers(-32768, 32768, N * C * H * W, dtype=np.int16)
    w = g.integers(-32768, 32768, M * C * kh * kw, dtype=np.int16)
    b = g.integers(-32768, 32768, M, dtype=np.int16)
    add = g.integers(-32768, 32768, N * M * OH * OW, dtype=np.int16)
    want = np.zeros(N * M * OH * OW, np.int16)
    oracle.set_threads(oracle_threads())
    oracle.conv(x, w, b, want, *args, threads=True)
    y = empty_dev(want.size)
    ws = workspace_for(*args)
    K.ConvKernel(dev(x), dev(w), dev(b), y, *args, workspace=ws)
    np.testing.assert_array_equal(host(y), want)
    for act in (K.ACT_RELU, K.ACT_RELU6):
        y2 = empty_dev(want.size)
        K.ConvKernel(dev(x), dev(w), dev(b), y2, *args, add=dev(add), act=act, workspace=ws)
        exp = np.clip(want.astype(np.int32) + add, -32768, 32767)
        exp = np.clip(exp, 0, 32767 if act == K.ACT_RELU else 1536)
        np.testing.assert_array_equal(host(y2).astype(np.int32), exp)


@pytest.mark.parametrize("geom", PGEMM, ids=[str(g) for g in PGEMM])
@pytest.mark.parametrize("mix", ["all", "first", "last"])
def test_patch_gemm_int8_weights(geom, mix):
    """Weights in [-128, 127] take the two-product path per 128-row tile: every
    tile ("all"), or with one out-of-range weight in the first or last output
    channel (that row's tile takes the four-product path).  Full-range inputs,
    bias, fused Add and ReLU."""
    N, C, H, W, M, kh, kw, s, d, p = geom
    OH, OW = (H + 2 * p - d * (kh - 1) - 1) // s + 1, (W + 2 * p - d * (kw - 1) - 1) // s + 1
    args = (N, C, H, W, M, OH, OW, kh, kw, s, s, d, d, p, p, 1, 0)
    assert K.conv_workspace_size(*args) in pgemm_need(C, M, kh, kw), "expected the patch-GEMM path"
    say(f"conv patch gemm int8 weights {geom} {mix}")
    g = wl.rng(834, *geom, len(mix))
    x = g.integers(-32768, 32768, N * C * H * W, dtype=np.int16)
    w = g.integers(-128, 128, M * C * kh * kw, dtype=np.int16)
    if mix == "first":
        w[int(g.integers(0, C * kh * kw))] = -129
    elif mix == "last":
        w[(M - 1) * C * kh * kw + int(g.integers(0, C * kh * kw))] = 128
    b = g.integers(-32768, 32768, M, dtype=np.int16)
    add = g.integers(-32768, 32768, N * M * OH * OW, dtype=np.int16)
    want = np.zeros(N * M * OH * OW, np.int16)
    oracle.set_threads(oracle_threads())
    oracle.conv(x, w, b, want, *args, threads=True)
    ws = workspace_for(*args)
    y = empty_dev(want.size)
    K.ConvKernel(dev(x), dev(w), dev(b), y, *args, workspace=ws)
    np.testing.assert_array_equal(host(y), want)
    y2 = empty_dev(want.size)
    K.ConvKernel(dev(x), dev(w), dev(b), y2, *args, add=dev(add), act=K.ACT_RELU, workspace=ws)
    exp = np.clip(np.clip(want.astype(np.int32) + add, -32768, 32767), 0, 32767)
    np.testing.assert_array_equal(host(y2).astype(np.int32), exp)


@pytest.mark.parametrize("seed", range(16))
def test_patch_path_random(seed):
    """Random 3x3 shapes that take the patch path (channels a multiple of 8, <= 64
    in and out, >= 64 output tiles): full-range operands, random padding, stride,
    bias, fused Add and activation."""
    g = wl.rng(977, seed)
    C = int(g.choice([8, 16, 24, 32, 40, 48, 56, 64]))
    M = int(g.integers(1, 65))
    S = int(g.choice([1, 2]))
    pt, pl = int(g.integers(0, 3)), int(g.integers(0, 3))
    H, W = int(g.integers(5, 40)), int(g.integers(5, 70))
    OH, OW = (H + 2 * pt - 3) // S + 1, (W + 2 * pl - 3) // S + 1
    tiles_img = ((OH + 7) // 8) * ((OW + 15) // 16)
    N = -(-64 // tiles_img)
    bias, act = int(g.integers(0, 2)), int(g.integers(0, 3))
    say(f"conv patch random seed {seed}: {(N, C, H, W, M, S, pt, pl, bias, act)}")
    x = g.integers(-32768, 32768, N * C * H * W, dtype=np.int16)
    w = g.integers(-32768, 32768, M * C * 9, dtype=np.int16)
    b = g.integers(-32768, 32768, M, dtype=np.int16)
    add = g.integers(-32768, 32768, N * M * OH * OW, dtype=np.int16)
    want = np.zeros(N * M * OH * OW, np.int16)
    oracle.set_threads(oracle_threads())
    oracle.conv(x, w, b, want, N, C, H, W, M, OH, OW, 3, 3, S, S, 1, 1, pt, pl, bias, 0, threads=True)
    want = np.clip(want.astype(np.int32) + add, -32768, 32767)   # fused Add: saturating
    want = np.clip(want, 0, 32767 if act == K.ACT_RELU else 1536) if act else want
    y = empty_dev(N * M * OH * OW)
    K.ConvKernel(dev(x), dev(w), dev(b), y, N, C, H, W, M, OH, OW, 3, 3, S, S, 1, 1, pt, pl, bias, 0,
                 add=dev(add), act=act)
    np.testing.assert_array_equal(host(y).astype(np.int32), want)


PACKED = [
    # N, C, H, W, M, kh, kw, s, d, p (shapes the patch-GEMM path takes: more than
    # 2^21 outputs or K > 2048)
    (80, 32, 28, 32, 32, 3, 3, 1, 1, 1),       # 32-channel row tile
    (200, 48, 20, 24, 110, 3, 3, 2, 1, 1),     # stride 2
    (2, 240, 9, 9, 150, 3, 3, 1, 2, 2),        # four channel chunks, two row tiles, K = 2160
    (192, 64, 14, 14, 96, 3, 3, 1, 1, 1),      # 14-wide rows (element staging), batch 192
]


@pytest.mark.parametrize("geom", PACKED, ids=[str(g) for g in PACKED])
def test_conv_packed_weights(geom):
    """cm_conv_pack once, then cm_conv_packed_ex on two inputs (and with a fused Add
    and ReLU6): every output equals cm_conv_ex's, for int8-range and full-range
    weights."""
    N, C, H, W, M, kh, kw, s, d, p = geom
    OH, OW = (H + 2 * p - d * (kh - 1) - 1) // s + 1, (W + 2 * p - d * (kw - 1) - 1) // s + 1
    args = (N, C, H, W, M, OH, OW, kh, kw, s, s, d, d, p, p, 1, 0)
    size = K.conv_packed_size(*args)
    assert size in pgemm_need(C, M, kh, kw)
    say(f"conv packed weights {geom}")
    g = wl.rng(835, *geom)
    for lo, hi in ((-128, 128), (-32768, 32768)):
        w = g.integers(lo, hi, M * C * kh * kw, dtype=np.int16)
        b = g.integers(-32768, 32768, M, dtype=np.int16)
        packed = torch.empty(-(-size // 4), dtype=torch.int32, device="cuda")
        K.conv_pack(dev(w), packed, *args)
        for rep in range(2):
            x = g.integers(-32768, 32768, N * C * H * W, dtype=np.int16)
            add = g.integers(-32768, 32768, N * M * OH * OW, dtype=np.int16)
            want = np.zeros(N * M * OH * OW, np.int16)
            oracle.set_threads(oracle_threads())
            oracle.conv(x, w, b, want, *args, threads=True)
            y = empty_dev(want.size)
            K.ConvPackedKernel(dev(x), packed, dev(b), y, *args)
            np.testing.assert_array_equal(host(y), want)
            y2 = empty_dev(want.size)
            K.ConvPackedKernel(dev(x), packed, dev(b), y2, *args, add=dev(add), act=K.ACT_RELU6)
            exp = np.clip(np.clip(want.astype(np.int32) + add, -32768, 32767), 0, 1536)
            np.testing.assert_array_equal(host(y2).astype(np.int32), exp)


def test_conv_packed_rejects_other_paths():
    """Shapes cm_conv runs elsewhere report no packed size, and the packed calls
    refuse them; a packed buffer that is too small is refused."""
    one = (4, 32, 14, 14, 32, 14, 14, 1, 1, 1, 1, 1, 1, 0, 0, 1, 0)      # 1x1
    dwc = (4, 32, 14, 14, 32, 14, 14, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1)      # depthwise
    aniso = (4, 32, 14, 14, 32, 14, 7, 3, 3, 1, 2, 1, 1, 1, 1, 1, 0)     # strides differ
    for a in (one, dwc, aniso):
        assert K.conv_packed_size(*a) == 0
    buf = torch.empty(16, dtype=torch.int32, device="cuda")
    w = torch.zeros(32 * 32 * 9, dtype=torch.int16, device="cuda")
    with pytest.raises(_native.CmError):
        K.conv_pack(w, buf, *aniso)
    small = (4, 32, 14, 14, 32, 7, 7, 3, 3, 2, 2, 1, 1, 1, 1, 1, 0)     # the register-only kernel
    assert K.conv_packed_size(*small) == 0
    ok = (64, 32, 28, 40, 32, 28, 40, 3, 3, 1, 1, 1, 1, 1, 1, 1, 0)
    assert K.conv_packed_size(*ok) > 64
    with pytest.raises(_native.CmError):
        K.conv_pack(w, buf, *ok)   # 64 bytes is too small


DW_CASES = [
    # N, C, H, W, M, kh, kw, sh, sw, dh, dw, pt, pl, bias
    (1, 32, 28, 28, 32, 3, 3, 1, 1, 1, 1, 1, 1, 0),      # perf case dw-3x3-32ch-28x28
    (1, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1, 1, 1, 0),      # perf case dw-3x3-64ch-56x56
    (16, 32, 112, 112, 32, 3, 3, 1, 1, 1, 1, 1, 1, 1),   # MobileNetV2's first depthwise layer
    (4, 96, 56, 56, 96, 3, 3, 2, 2, 1, 1, 1, 1, 1),      # stride 2 (16-byte staging)
    (2, 40, 15, 17, 40, 3, 3, 2, 2, 1, 1, 0, 1, 1),      # element staging, asymmetric pads
    (2, 24, 9, 40, 20, 5, 5, 1, 2, 2, 1, 3, 2, 1),       # general taps, dilation, out_ch < in_ch
    (1, 3, 4, 9000, 3, 3, 3, 1, 1, 1, 1, 1, 1, 1),       # rows too wide for the tile: per-output kernel
    (3, 5, 7, 7, 5, 7, 7, 1, 1, 1, 1, 3, 3, 0),          # a window as large as the plane
    # several channels' planes per block (small planes, many of them)
    (8, 255, 14, 14, 255, 3, 3, 1, 1, 1, 1, 1, 1, 1),    # 2 per block, a partial last group
    (16, 192, 8, 8, 192, 3, 3, 1, 1, 1, 1, 1, 1, 0),     # 16-byte staging
    (16, 400, 7, 7, 399, 3, 3, 2, 2, 1, 1, 1, 1, 1),     # stride 2, out_ch < in_ch, partial group
]


def dw_run(geom, seed, add_act=None):
    N, C, H, W, M, kh, kw, sh, sw, dh, dw, pt, pl, bias = geom
    OH = (H + 2 * pt - dh * (kh - 1) - 1) // sh + 1
    OW = (W + 2 * pl - dw * (kw - 1) - 1) // sw + 1
    g = wl.rng(835, seed, *geom)
    x = g.integers(-32768, 32768, N * C * H * W, dtype=np.int16)
    w = g.integers(-32768, 32768, M * kh * kw, dtype=np.int16)
    b = g.integers(-32768, 32768, M, dtype=np.int16)
    args = (N, C, H, W, M, OH, OW, kh, kw, sh, sw, dh, dw, pt, pl, bias, 1)
    want = np.zeros(N * M * OH * OW, np.int16)
    oracle.set_threads(oracle_threads())
    oracle.conv(x, w, b, want, *args, threads=True)
    y = empty_dev(want.size)
    if add_act is None:
        K.ConvKernel(dev(x), dev(w), dev(b), y, *args)
        return host(y), want
    add = g.integers(-32768, 32768, want.size, dtype=np.int16)
    K.ConvKernel(dev(x), dev(w), dev(b), y, *args, add=dev(add), act=add_act)
    exp = np.clip(want.astype(np.int32) + add, -32768, 32767)
    if add_act != K.ACT_NONE:
        exp = np.clip(exp, 0, 32767 if add_act == K.ACT_RELU else 1536)
    return host(y).astype(np.int32), exp


@pytest.mark.parametrize("geom", DW_CASES, ids=[str(g) for g in DW_CASES])
def test_depthwise_cases(geom):
    """Depthwise on the band kernel (3x3 taps unrolled, general taps, 16-byte and
    element staging) and the per-output kernel, full-range values that wrap."""
    say(f"depthwise {geom}")
    got, want = dw_run(geom, 0)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("act", [0, 1, 2])
def test_depthwise_fused_epilogue(act):
    """y = act(sat16(conv + add)) on the band kernel."""
    say(f"depthwise epilogue act={act}")
    got, want = dw_run((2, 32, 28, 28, 32, 3, 3, 1, 1, 1, 1, 1, 1, 1), 1, add_act=act)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("seed", range(16))
def test_depthwise_random(seed):
    """Random depthwise shapes: square and non-square filters, strides, dilations,
    pads up to and past the window, widths with and without whole 16-byte rows."""
    g = wl.rng(836, seed)
    kh, kw = int(g.integers(1, 6)), int(g.integers(1, 6))
    if g.integers(0, 2):
        kw = kh = 3
    sh, sw = int(g.integers(1, 4)), int(g.integers(1, 4))
    dh, dw = (1, 1) if g.integers(0, 2) else (int(g.integers(1, 3)), int(g.integers(1, 3)))
    pt, pl = int(g.integers(0, kh + 1)), int(g.integers(0, kw + 1))
    H = int(g.integers(max(1, dh * (kh - 1) + 1 - 2 * pt), 70))
    W = 8 * int(g.integers(1, 12)) if g.integers(0, 2) else int(g.integers(max(1, dw * (kw - 1) + 1 - 2 * pl), 90))
    C = int(g.integers(1, 40))
    M = int(g.integers(1, C + 1))
    N = int(g.integers(1, 4))
    geom = (N, C, H, W, M, kh, kw, sh, sw, dh, dw, pt, pl, int(g.integers(0, 2)))
    say(f"depthwise random seed {seed}: {geom}")
    got, want = dw_run(geom, seed)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("seed", range(20))
def test_pointwise_small_random(seed):
    """Small 1x1 convolutions (<= 2^21 outputs, in_ch <= 512) on the register-only
    MFMA kernel: channel counts that are and are not multiples of 8 / 32 / 64,
    planes of 1..900 pixels, several images per 32-column tile, bias, fused Add
    and activation, full-range values whose sums wrap."""
    g = wl.rng(837, seed)
    C = int(g.choice([1, 3, 8, 16, 24, 40, 64, 96, 100, 160, 320, 512]))
    M = int(g.choice([1, 5, 16, 24, 32, 33, 64, 96, 160, 320]))
    hw = int(g.choice([1, 3, 7, 14, 28, 30]))
    N = int(g.integers(1, 17))
    while M * N * hw * hw > (1 << 21):
        N = max(1, N // 2)
        if N == 1 and M * hw * hw > (1 << 21):
            hw //= 2
    bias, act = int(g.integers(0, 2)), int(g.integers(0, 3))
    args = (N, C, hw, hw, M, hw, hw, 1, 1, 1, 1, 1, 1, 0, 0, bias, 0)
    assert K.conv_workspace_size(*args) == 0
    say(f"pointwise small seed {seed}: N={N} C={C} M={M} hw={hw} bias={bias} act={act}")
    x = g.integers(-32768, 32768, N * C * hw * hw, dtype=np.int16)
    w = g.integers(-32768, 32768, M * C, dtype=np.int16)
    b = g.integers(-32768, 32768, M, dtype=np.int16)
    add = g.integers(-32768, 32768, N * M * hw * hw, dtype=np.int16)
    want = np.zeros(N * M * hw * hw, np.int16)
    oracle.set_threads(oracle_threads())
    oracle.conv(x, w, b, want, *args, threads=True)
    y = empty_dev(want.size)
    K.ConvKernel(dev(x), dev(w), dev(b), y, *args)
    np.testing.assert_array_equal(host(y), want)
    y2 = empty_dev(want.size)
    K.ConvKernel(dev(x), dev(w), dev(b), y2, *args, add=dev(add), act=act)
    exp = np.clip(want.astype(np.int32) + add, -32768, 32767)
    if act:
        exp = np.clip(exp, 0, 32767 if act == K.ACT_RELU else 1536)
    np.testing.assert_array_equal(host(y2).astype(np.int32), exp)


def test_pointwise_small_unaligned_weights():
    """Weights at an odd element offset (no 16-byte loads) with in_ch % 8 == 0."""
    g = wl.rng(838)
    N, C, hw, M = 4, 64, 14, 48
    args = (N, C, hw, hw, M, hw, hw, 1, 1, 1, 1, 1, 1, 0, 0, 1, 0)
    x = g.integers(-32768, 32768, N * C * hw * hw, dtype=np.int16)
    w = g.integers(-32768, 32768, M * C + 1, dtype=np.int16)
    b = g.integers(-32768, 32768, M, dtype=np.int16)
    want = np.zeros(N * M * hw * hw, np.int16)
    oracle.conv(x, w[1:].copy(), b, want, *args)
    dw_ = dev(w)[1:]
    y = empty_dev(want.size)
    K.ConvKernel(dev(x), dw_, dev(b), y, *args)
    np.testing.assert_array_equal(host(y), want)


RK_SHAPES = [
    # N, C, H, W, M, kh, kw, s, d, p: the MobileNetV2-like strided small-map layers
    (16, 24, 56, 56, 24, 3, 3, 2, 1, 1),
    (16, 32, 28, 28, 32, 3, 3, 2, 1, 1),
    (16, 96, 14, 14, 96, 3, 3, 2, 1, 1),
    (16, 160, 14, 14, 160, 3, 3, 2, 1, 1),
    (4, 227, 14, 14, 61, 3, 3, 2, 1, 1),    # K = 2043 (32 steps), K % 8 != 0
    # 1x1 layers over >= 128 channels (stride 1, no padding)
    (16, 160, 7, 7, 160, 1, 1, 1, 1, 0),
    (16, 160, 7, 7, 320, 1, 1, 1, 1, 0),
    (16, 1280, 7, 7, 256, 1, 1, 1, 1, 0),   # 20 k steps, past the 1x1 kernel's 512 channels
    (3, 130, 9, 11, 40, 1, 1, 1, 1, 0),     # K % 8 != 0, partial tiles
]


@pytest.mark.parametrize("geom", RK_SHAPES, ids=[str(g) for g in RK_SHAPES])
def test_register_conv_shapes(geom):
    """Small convolutions on the register-only kernel (the reduction split over a
    block's four waves), full-range values, bias, fused Add and Relu6."""
    N, C, H, W, M, kh, kw, s, d, p = geom
    OH, OW = (H + 2 * p - d * (kh - 1) - 1) // s + 1, (W + 2 * p - d * (kw - 1) - 1) // s + 1
    args = (N, C, H, W, M, OH, OW, kh, kw, s, s, d, d, p, p, 1, 0)
    assert K.conv_workspace_size(*args) == 0 and K.conv_packed_size(*args) == 0
    say(f"register conv {geom}")
    g = wl.rng(839, *geom)
    x = g.integers(-32768, 32768, N * C * H * W, dtype=np.int16)
    w = g.integers(-32768, 32768, M * C * kh * kw, dtype=np.int16)
    b = g.integers(-32768, 32768, M, dtype=np.int16)
    add = g.integers(-32768, 32768, N * M * OH * OW, dtype=np.int16)
    want = np.zeros(N * M * OH * OW, np.int16)
    oracle.set_threads(oracle_threads())
    oracle.conv(x, w, b, want, *args, threads=True)
    y = empty_dev(want.size)
    K.ConvKernel(dev(x), dev(w), dev(b), y, *args)
    np.testing.assert_array_equal(host(y), want)
    y2 = empty_dev(want.size)
    K.ConvKernel(dev(x), dev(w), dev(b), y2, *args, add=dev(add), act=K.ACT_RELU6)
    exp = np.clip(np.clip(want.astype(np.int32) + add, -32768, 32767), 0, 1536)
    np.testing.assert_array_equal(host(y2).astype(np.int32), exp)


@pytest.mark.parametrize("seed", range(20))
def test_register_conv_random(seed):
    """Random small strided convolutions: windows of 2..25 taps (1 x k and k x 1
    too), strides (at least one above 1) and dilations 1..3 per axis, pads up to and
    past the window, channel counts with K % 8 == 0 and not, with and without bias."""
    g = wl.rng(840, seed)
    kh, kw = int(g.integers(1, 6)), int(g.integers(1, 6))
    if kh * kw < 2:
        kw = 2
    sh, sw = int(g.integers(1, 4)), int(g.integers(1, 4))
    if sh * sw < 2:
        sw = 2   # the register-only kernel takes strided windows
    dh, dw = int(g.integers(1, 4)), int(g.integers(1, 4))
    pt, pl = int(g.integers(0, kh + 2)), int(g.integers(0, kw + 2))
    H = int(g.integers(max(1, dh * (kh - 1) + 1 - 2 * pt), 30))
    W = int(g.integers(max(1, dw * (kw - 1) + 1 - 2 * pl), 30))
    C = int(g.integers(1, max(2, min(120, 2000 // (kh * kw)))))
    M = int(g.integers(1, 70))
    N = int(g.integers(1, 5))
    OH = (H + 2 * pt - dh * (kh - 1) - 1) // sh + 1
    OW = (W + 2 * pl - dw * (kw - 1) - 1) // sw + 1
    bias = int(g.integers(0, 2))
    args = (N, C, H, W, M, OH, OW, kh, kw, sh, sw, dh, dw, pt, pl, bias, 0)
    say(f"register conv random seed {seed}: {args}")
    x = g.integers(-32768, 32768, N * C * H * W, dtype=np.int16)
    w = g.integers(-32768, 32768, M * C * kh * kw, dtype=np.int16)
    b = g.integers(-32768, 32768, M, dtype=np.int16)
    want = np.zeros(N * M * OH * OW, np.int16)
    oracle.set_threads(oracle_threads())
    oracle.conv(x, w, b, want, *args, threads=True)
    y = empty_dev(want.size)
    K.ConvKernel(dev(x), dev(w), dev(b), y, *args)
    np.testing.assert_array_equal(host(y), want)
