"""GPU parity of the scheduler's HIP backend: every graph runs through
InferenceSession (C ABI, one device pool) and must match, bit for bit, the
same kernel-call list executed by the C-simulation oracle, and the float64
numpy simulation of the graph."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import graph_sim as gs
from cormorant_amd import workloads as wl
from cormorant_amd.scheduler import BufferPlan, InferenceSession, OnnxGraph, onnx_io as ox
from cormorant_amd.scheduler.tensor import ramp_to_storage
from tests import onnx_models as om
from tests.gpu_util import oracle_threads, say
from tests.test_scheduler import GRAPH_CASES, SAT_EXPECT, feeds_for

pytestmark = pytest.mark.gpu


def check_session(g, feeds, sim=True, fuse=True):
    sess = InferenceSession(g, fuse=fuse)
    try:
        got = sess.run(feeds)
    finally:
        sess.close()
    oracle.set_threads(oracle_threads())
    want = gs.run_plan(BufferPlan(g), feeds)
    for k in want:
        np.testing.assert_array_equal(got[k], want[k], err_msg=f"{k} vs kernel-call oracle")
    if sim:
        ref = gs.simulate_raw(g, feeds)
        for k in ref:
            np.testing.assert_array_equal(got[k], ref[k], err_msg=f"{k} vs numpy simulation")
    return got


@pytest.mark.parametrize("fuse", [True, False], ids=["fused", "unfused"])
@pytest.mark.parametrize("name", sorted(GRAPH_CASES))
def test_reference_graphs(name, fuse):
    say(f"scheduler graph {name} fuse={fuse}")
    g = OnnxGraph(ox.encode_model(GRAPH_CASES[name]()))
    check_session(g, feeds_for(g, len(name)), fuse=fuse)


@pytest.mark.parametrize("kind", om.SAT_KINDS)
def test_saturation_ramp(kind):
    say(f"scheduler saturation {kind}")
    g = OnnxGraph(ox.encode_model(om.sat_model(kind)))
    x = ramp_to_storage(np.arange(256)).reshape(1, 256)
    y = check_session(g, {"X": x})["Y"].reshape(-1)
    assert SAT_EXPECT[kind](y)


@pytest.mark.parametrize("name", sorted(om.MATMUL_CASES))
def test_matmul_graphs(name):
    say(f"scheduler matmul {name}")
    a, w = om.MATMUL_CASES[name]
    g = OnnxGraph(ox.encode_model(om.matmul(a, w, name)))
    check_session(g, {"X": wl.uniform_q88(wl.rng(63, len(name)), a, -2.0, 2.0)})


def test_session_reuse_and_input_copy():
    say("scheduler session reuse")
    g = OnnxGraph(ox.encode_model(om.reshape_input_to_output()))
    sess = InferenceSession(g)
    try:
        for seed in range(3):
            x = wl.uniform_q88(wl.rng(64, seed), (2, 8), -4.0, 4.0)
            out = sess.run({"X": x})
            np.testing.assert_array_equal(out["Z"], x.reshape(16))
            np.testing.assert_array_equal(out["R"], np.maximum(x, 0))
    finally:
        sess.close()


@pytest.mark.parametrize("fuse", [True, False], ids=["fused", "unfused"])
def test_mlp_full_size(fuse):
    """2-layer MLP, batch 64 (Gemm 784->256, Relu, Gemm 256->10)."""
    say(f"scheduler MLP b64 fuse={fuse}")
    g = OnnxGraph(ox.encode_model(wl.mlp_model()))
    check_session(g, {"X": wl.mlp_input()}, fuse=fuse)


def test_mobilenet_like_full_size():
    """MobileNetV2-like graph, batch 16 at 224x224: 36 convolutions, 5.06 GMAC."""
    say("scheduler MobileNetV2-like b16 224")
    g = OnnxGraph(ox.encode_model(wl.mobilenet_model()))
    y = check_session(g, {"X": wl.mobilenet_input()})["Y"]
    assert np.count_nonzero(y) > 0.9 * y.size


def test_mobilenet_like_small_unfused():
    say("scheduler MobileNetV2-like b2 32 unfused")
    g = OnnxGraph(ox.encode_model(wl.mobilenet_model(batch=2, hw=32)))
    check_session(g, {"X": wl.mobilenet_input(2, 32)}, fuse=False)


def test_run_helpers_reject_short_buffers():
    """cm_run_* check every touched element against the buffers' counts (nothing launches)."""
    from cormorant_amd import _native
    lib = _native.load()
    say("cm_run_* extent checks")
    a, b, c = lib.cm_buf_alloc(16), lib.cm_buf_alloc(16), lib.cm_buf_alloc(8)
    try:
        assert lib.cm_run_op(a, b, c, 16, 0, 1, 0, 0) == _native.CM_ERR_RANGE
        assert b"buffer c holds 8" in lib.cm_last_error()
        assert lib.cm_run_op(a, b, c, 4, 0, 3, 4, 0) == _native.CM_ERR_RANGE      # c needs 12
        assert lib.cm_run_matmul_at(a, 9, b, 0, c, 0, 2, 4, 2, 1, 0, 0, 0) == _native.CM_ERR_RANGE
        assert lib.cm_run_pool(a, c, 1, 1, 4, 4, 3, 3, 2, 2, 1, 1, 0, 0, 1, 1, 0, 2, 0) == \
            _native.CM_ERR_RANGE
        assert lib.cm_run_op(a, b, c, 8, 0, 1, 0, 0) == 0
        assert lib.cm_sync(None) == 0
    finally:
        for x in (a, b, c):
            lib.cm_buf_free(x)


def test_session_graph_replay_matches_eager():
    """The session's launch list (fused epilogues, split-K layers) captured in
    a HIP graph on a warmed-up stream: every replay, with eager work and
    synchronisations in between, reproduces the eager output."""
    import torch
    say("scheduler MobileNetV2-like b2 32 graph replay")
    g = OnnxGraph(ox.encode_model(wl.mobilenet_model(batch=2, hw=32)))
    x = wl.mobilenet_input(2, 32)
    sess = InferenceSession(g)
    try:
        want = sess.run({"X": x})["Y"]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            sess.launch(side.cuda_stream)       # eager run on the capture stream
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            sess.launch(side.cuda_stream)
        for rep in range(3):
            junk = torch.randint(-100, 100, (1 << 20,), dtype=torch.int16, device="cuda")
            junk.mul_(3)                           # unrelated eager work between replays
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(sess.read_output("Y"), want, err_msg=f"replay {rep}")
    finally:
        sess.close()
